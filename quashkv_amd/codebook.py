"""Lloyd-Max scalar codebooks for the rotated-coordinate distribution.

After a random rotation each coordinate of a unit vector in R^d follows a
Beta-type law that is close to N(0, 1/d).  The codebook is the continuous
1-D k-means (Lloyd-Max) fixed point for that law, solved once on the host
(parameters, not hot path) and shipped to the GPU as fp32 tables.

Solver (same iteration as quashkv/codebook.py:63-139, so the fp32 values are
identical): centroids start uniform on [-4 sigma, 4 sigma]; each step sets
boundaries to centroid midpoints, cells run from 5*lo to 5*hi, and each
centroid moves to its cell's conditional mean; stop after 300 steps or a
max shift < 1e-12.  Here the cell moments are CLOSED FORMS (Gaussian:
erf/erfc and exp; exact Beta law: the regularised incomplete beta function)
instead of numerical quadrature, and the law's symmetry is used exactly: the
upper half is solved and mirrored, so the middle boundary of an even codebook
is exactly 0.0.
"""

from __future__ import annotations

import math
from functools import lru_cache

import torch
from scipy import special

from .constants import LLOYD_MAX_ITER, LLOYD_MAX_RANGE_SIGMAS, LLOYD_MAX_TOL, SUPPORTED_BITS


# ---------------------------------------------------------------------------
# Closed-form cell moments
# ---------------------------------------------------------------------------

class _Gaussian:
    """N(0, sigma^2) cell mass and first/second moments in closed form."""

    def __init__(self, d: int):
        self.s = 1.0 / math.sqrt(d)
        self.r2 = math.sqrt(2.0) * self.s
        self.lo, self.hi = -LLOYD_MAX_RANGE_SIGMAS * self.s, LLOYD_MAX_RANGE_SIGMAS * self.s

    def _phi(self, x: float) -> float:
        return math.exp(-x * x / (2.0 * self.s * self.s)) / (self.s * math.sqrt(2.0 * math.pi))

    def mass(self, a: float, b: float) -> float:
        # use erfc in the tails to avoid cancellation
        if a >= 0.0:
            return 0.5 * (math.erfc(a / self.r2) - math.erfc(b / self.r2))
        if b <= 0.0:
            return 0.5 * (math.erfc(-b / self.r2) - math.erfc(-a / self.r2))
        return 0.5 * (math.erf(b / self.r2) - math.erf(a / self.r2))

    def m1(self, a: float, b: float) -> float:
        # int_a^b x phi = sigma^2 (phi(a) - phi(b))
        return self.s * self.s * (self._phi(a) - self._phi(b))

    def m2(self, a: float, b: float) -> float:
        # int_a^b x^2 phi = sigma^2 (mass + a phi(a) - b phi(b))
        s2 = self.s * self.s
        return s2 * (self.mass(a, b) + a * self._phi(a) - b * self._phi(b))


class _Beta:
    """Law of one coordinate of a uniform unit vector in R^d:
    f(x) = Gamma(d/2) / (sqrt(pi) Gamma((d-1)/2)) (1 - x^2)^((d-3)/2) on [-1, 1];
    x^2 ~ Beta(1/2, (d-1)/2)."""

    def __init__(self, d: int):
        self.d = d
        self.a_, self.b_ = 0.5, (d - 1) / 2.0
        self.lo, self.hi = -1.0, 1.0
        self.logc = special.gammaln(d / 2.0) - 0.5 * math.log(math.pi) - special.gammaln((d - 1) / 2.0)

    @staticmethod
    def _clip(x: float) -> float:
        return max(-1.0, min(1.0, x))

    def _cdf(self, x: float) -> float:
        x = self._clip(x)
        return 0.5 + math.copysign(0.5, x) * float(special.betainc(self.a_, self.b_, x * x))

    def mass(self, a: float, b: float) -> float:
        return self._cdf(b) - self._cdf(a)

    def m1(self, a: float, b: float) -> float:
        # antiderivative of x f(x) is -C (1 - x^2)^((d-1)/2) / (d - 1)
        a, b = self._clip(a), self._clip(b)
        e = (self.d - 1) / 2.0
        c = math.exp(self.logc) / (self.d - 1)
        return c * ((1.0 - a * a) ** e - (1.0 - b * b) ** e)

    def _half_m2(self, u: float) -> float:
        # int_0^u x^2 f(x) dx for u >= 0 = (1/2) E[x^2; x^2 <= u^2] = (1/(2d)) I_{u^2}(3/2, b)
        return 0.5 / self.d * float(special.betainc(self.a_ + 1.0, self.b_, min(u * u, 1.0)))

    def m2(self, a: float, b: float) -> float:
        a, b = self._clip(a), self._clip(b)
        fa = math.copysign(self._half_m2(abs(a)), a)
        fb = math.copysign(self._half_m2(abs(b)), b)
        return fb - fa


def _law(d: int, use_exact_pdf: bool):
    return _Beta(d) if use_exact_pdf else _Gaussian(d)


# ---------------------------------------------------------------------------
# Solver
# ---------------------------------------------------------------------------

def solve_lloyd_max(
    d: int,
    bits: int,
    *,
    use_exact_pdf: bool = False,
    max_iter: int = LLOYD_MAX_ITER,
    tol: float = LLOYD_MAX_TOL,
) -> tuple[list[float], list[float]]:
    """Lloyd-Max centroids (ascending, 2**bits) and midpoint boundaries.

    Same signature, iteration and stopping rule as the reference
    (quashkv/codebook.py:63-139); moments are exact closed forms.
    """
    if bits not in SUPPORTED_BITS:
        raise ValueError(f"bits must be in {SUPPORTED_BITS}, got {bits}")
    law = _law(d, use_exact_pdf)
    n = 1 << bits
    half = n // 2
    lo, hi = law.lo, law.hi
    # upper half of the symmetric initial grid; the lower half is its mirror
    up = [lo + (hi - lo) * (i + 0.5) / n for i in range(half, n)]
    for _ in range(max_iter):
        cents = [-c for c in reversed(up)] + up
        bnds = [(cents[i] + cents[i + 1]) / 2.0 for i in range(n - 1)]
        edges = [lo * 5] + bnds + [hi * 5]
        new = []
        for i in range(half, n):
            a, b = edges[i], edges[i + 1]
            den = law.mass(a, b)
            new.append(law.m1(a, b) / den if den > 1e-15 else cents[i])
        shift = max(abs(new[k] - up[k]) for k in range(half))
        up = new
        if shift < tol:
            break
    cents = [-c for c in reversed(up)] + up
    bnds = [(cents[i] + cents[i + 1]) / 2.0 for i in range(n - 1)]
    return cents, bnds


def compute_mse_cost(d: int, bits: int, *, use_exact_pdf: bool = False) -> float:
    """d * sum_i int_cell_i (x - c_i)^2 f(x) dx (quashkv/codebook.py:146-174)."""
    cents, bnds = solve_lloyd_max(d, bits, use_exact_pdf=use_exact_pdf)
    law = _law(d, use_exact_pdf)
    edges = [law.lo * 5] + bnds + [law.hi * 5]
    total = 0.0
    for i, c in enumerate(cents):
        a, b = edges[i], edges[i + 1]
        total += law.m2(a, b) - 2.0 * c * law.m1(a, b) + c * c * law.mass(a, b)
    return d * total


@lru_cache(maxsize=64)
def _solved(d: int, bits: int, exact: bool) -> tuple[tuple[float, ...], tuple[float, ...]]:
    c, t = solve_lloyd_max(d, bits, use_exact_pdf=exact)
    return tuple(c), tuple(t)


# ---------------------------------------------------------------------------
# Codebook
# ---------------------------------------------------------------------------

class LloydMaxCodebook:
    """Pre-solved Lloyd-Max codebook for (d, bits) (quashkv/codebook.py:181-276).

    ``centroids`` (2**bits,) and ``boundaries`` (2**bits - 1,) are fp32
    tensors; the quantise / dequantise methods run HIP kernels on GPU tensors.
    """

    def __init__(self, d: int, bits: int, *, use_exact_pdf: bool = False):
        self.d = d
        self.bits = bits
        self.n_levels = 1 << bits
        c, t = _solved(d, bits, bool(use_exact_pdf))
        self.centroids = torch.tensor(c, dtype=torch.float32)
        self.boundaries = torch.tensor(t, dtype=torch.float32)
        # fp32 values as Python floats: the attention entry points take the
        # centroids by value (no device round trip)
        self.centroids_host = tuple(self.centroids.tolist())
        self.boundaries_host = tuple(self.boundaries.tolist())

    def _tables_on(self, device: torch.device):
        if self.centroids.device != device:
            self.to(device)
        return self.centroids, self.boundaries

    def quantize(self, x: torch.Tensor) -> torch.Tensor:
        """Nearest-centroid index (first minimum), uint8."""
        from . import _native as N
        dev = N.require_gpu(x, what="LloydMaxCodebook.quantize")
        c, _ = self._tables_on(dev)
        xf = x.contiguous().float()
        out = torch.empty(x.shape, dtype=torch.uint8, device=dev)
        N.check(N.lib().qkv_quantize(xf.data_ptr(), xf.numel(), c.data_ptr(), self.n_levels, 1,
                                     out.data_ptr(), N.stream(dev)))
        return out

    def dequantize(self, indices: torch.Tensor) -> torch.Tensor:
        """Centroid values c[index], fp32."""
        from . import _native as N
        dev = N.require_gpu(indices, what="LloydMaxCodebook.dequantize")
        c, _ = self._tables_on(dev)
        idx = indices.contiguous()
        if idx.dtype != torch.uint8:
            if idx.numel() and (int(idx.min()) < 0 or int(idx.max()) >= self.n_levels):
                raise IndexError("codebook index out of range")
            idx = idx.to(torch.uint8)
        out = torch.empty(indices.shape, dtype=torch.float32, device=dev)
        N.check(N.lib().qkv_dequantize(idx.data_ptr(), idx.numel(), c.data_ptr(), self.n_levels,
                                       out.data_ptr(), N.stream(dev)))
        return out

    def quantize_boundary(self, x: torch.Tensor) -> torch.Tensor:
        """code = #{i : boundaries[i] < x} (ties go to the lower code), uint8."""
        from . import _native as N
        dev = N.require_gpu(x, what="LloydMaxCodebook.quantize_boundary")
        _, t = self._tables_on(dev)
        xf = x.contiguous().float()
        out = torch.empty(x.shape, dtype=torch.uint8, device=dev)
        N.check(N.lib().qkv_quantize(xf.data_ptr(), xf.numel(), t.data_ptr(), self.n_levels - 1, 0,
                                     out.data_ptr(), N.stream(dev)))
        return out

    def mse_cost(self) -> float:
        return compute_mse_cost(self.d, self.bits)

    def to(self, device) -> "LloydMaxCodebook":
        self.centroids = self.centroids.to(device)
        self.boundaries = self.boundaries.to(device)
        return self

    def __repr__(self) -> str:
        return (
            f"LloydMaxCodebook(d={self.d}, bits={self.bits}, "
            f"levels={self.n_levels}, "
            f"centroids=[{', '.join(f'{c:.6f}' for c in self.centroids.tolist())}])"
        )


@lru_cache(maxsize=32)
def get_codebook(d: int, bits: int) -> LloydMaxCodebook:
    return LloydMaxCodebook(d, bits)
