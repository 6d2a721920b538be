"""MSE and inner-product (MSE + QJL) quantizers on the HIP kernels.

Parameters follow the reference exactly so that a given (d, bits, seed)
yields the same Pi, S and codebooks (quashkv/quantizer.py:32-59, 85-103,
182-209).  compress / decompress run the fused kernels of libquashkv_hip.so.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _native as N
from .codebook import LloydMaxCodebook
from .constants import DEFAULT_SEED, DEFAULT_TOTAL_BITS, QJL_COEFF, SUPPORTED_HEAD_DIMS


def _default_device(device) -> torch.device:
    if device is None:
        return torch.device("cuda" if torch.cuda.is_available() else "cpu")
    return torch.device(device)


def _random_orthogonal(d: int, seed: int, device) -> torch.Tensor:
    """Pi = Q diag(sign(diag R)) of a seeded CPU Gaussian matrix.

    Same torch calls as quashkv/quantizer.py:32-44 (kept identical so a seed
    names the same rotation)."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    a = torch.randn(d, d, generator=gen, dtype=torch.float32)
    q, r = torch.linalg.qr(a)
    # LAPACK returns Q column-major; the kernels read Pi row-major
    return (q * torch.sign(torch.diag(r)).unsqueeze(0)).contiguous().to(device)


def _random_signs(d: int, seed: int, device) -> torch.Tensor:
    """S in {-1,+1}^d, CPU generator seeded with seed + 1_000_000
    (quashkv/quantizer.py:51-59)."""
    gen = torch.Generator(device="cpu").manual_seed(seed + 1_000_000)
    s = torch.randint(0, 2, (d,), generator=gen, dtype=torch.float32, device="cpu")
    return s.mul_(2).sub_(1).to(device)


def _flat_rows(x: torch.Tensor, d: int) -> torch.Tensor:
    if x.shape[-1] != d:
        raise ValueError(f"Expected last dim {d}, got {tuple(x.shape)}")
    x = x.reshape(-1, d)
    if x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        x = x.float()
    return x.contiguous()


def _host_tables(cb) -> tuple:
    """(centroids, boundaries) of a LloydMaxCodebook as host arrays, from
    the fp32 values it keeps on the host."""
    return N.HostFloats(cb.centroids_host), N.HostFloats(cb.boundaries_host)


def compress_into(mode: int, x: torch.Tensor, pi: torch.Tensor, boundaries: torch.Tensor,
                  centroids: torch.Tensor, bits: int, signs: Optional[torch.Tensor],
                  codes: torch.Tensor, qjl: Optional[torch.Tensor], norms: Optional[torch.Tensor],
                  packed: bool, out_seq: Optional[int] = None,
                  out_group_stride: Optional[int] = None, pre_rotated: bool = False,
                  host_tables: Optional[tuple] = None) -> None:
    """Run the fused compress, writing into caller-owned buffers.

    Rows of head_dim 128, 96 or 64 with a symmetric codebook run on the MFMA
    compress (qkv_compress_mfma; packed outputs through the bit packer after
    it); other shapes, pre-rotated rows and asymmetric tables on the VALU
    kernel (qkv_compress).  ``host_tables`` = (centroids, boundaries) host
    copies (N.HostFloats) spare the one-time copy of the device tables."""
    d = pi.shape[0]
    dev = N.require_gpu(x, pi, codes, what="compress")
    xf = _flat_rows(x, d)
    n = xf.shape[0]
    seq = out_seq if out_seq is not None else max(n, 1)
    gst = out_group_stride if out_group_stride is not None else seq
    flags = (N.QKV_FLAG_PACKED if packed else 0) | (N.QKV_FLAG_PRE_ROTATED if pre_rotated else 0)
    rows = N.grouped_rows(n, seq, gst)
    N.require_extent(codes, rows * (N.packed_row_bytes(d, bits) if packed else d), "compress codes")
    if mode == N.QKV_MODE_IP:
        N.require_extent(qjl, rows * (N.packed_row_bytes(d, 1) if packed else d), "compress qjl")
    if not pre_rotated:
        N.require_extent(norms, rows * 4, "compress norms")
    pi, boundaries, centroids, signs = N.dense(pi, boundaries, centroids, signs)
    L = N.lib()
    if (not pre_rotated and d in (64, 96, 128) and n > 0 and xf.data_ptr() % 16 == 0
            and (not packed or seq == n)):
        ip = mode == N.QKV_MODE_IP
        if host_tables is not None:
            ch, bh = host_tables
        else:   # the MSE search reads the boundaries only
            bh = N.host_table(boundaries)
            ch = N.host_table(centroids) if ip else bh
        if packed:   # unpacked codes first, then the bit packer
            c_out = torch.empty(n, d, dtype=torch.uint8, device=dev)
            q_out = torch.empty(n, d, dtype=torch.uint8, device=dev) if ip else None
        else:
            c_out, q_out = codes, qjl
        st = L.qkv_compress_mfma(mode, N.dtype_code(xf.dtype), xf.data_ptr(), n, d, pi.data_ptr(),
                                 ch.ptr, bh.ptr, bits, N.ptr(signs), c_out.data_ptr(),
                                 N.ptr(q_out), norms.data_ptr(), seq, gst, N.stream(dev))
        if st == N.QKV_OK:
            if packed:
                N.check(L.qkv_pack_bits(c_out.data_ptr(), codes.data_ptr(), n, d, bits,
                                        N.stream(dev)))
                if ip:
                    N.check(L.qkv_pack_bits(q_out.data_ptr(), qjl.data_ptr(), n, d, 1,
                                            N.stream(dev)))
            return
        if st != N.QKV_E_UNSUPPORTED:
            N.check(st)
    N.check(L.qkv_compress(
        mode, N.dtype_code(xf.dtype), flags, xf.data_ptr(), n, d, N.ptr(pi),
        boundaries.data_ptr(), centroids.data_ptr(), bits, N.ptr(signs), codes.data_ptr(),
        N.ptr(qjl), N.ptr(norms), seq, gst, N.stream(dev)))


def decompress_from(mode: int, codes: torch.Tensor, qjl: Optional[torch.Tensor],
                    norms: torch.Tensor, n: int, pi: torch.Tensor, centroids: torch.Tensor,
                    bits: int, signs: Optional[torch.Tensor], qjl_scale: float, fmt: int,
                    in_seq: Optional[int] = None, in_group_stride: Optional[int] = None,
                    out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Run the fused decompress kernel on codes in format ``fmt``
    (N.QKV_FMT_*); returns an (n, d) tensor."""
    d = pi.shape[0]
    dev = N.require_gpu(codes, norms, pi, what="decompress")
    out = torch.empty(n, d, dtype=out_dtype, device=dev)
    pi, centroids, signs = N.dense(pi, centroids, signs)
    seq = in_seq if in_seq is not None else max(n, 1)
    gst = in_group_stride if in_group_stride is not None else seq
    if fmt == N.QKV_FMT_VTILES:
        groups = (n + seq - 1) // seq
        N.require_extent(codes, ((groups - 1) * gst + (seq + 31) // 32) * bits * d * 4,
                         "decompress V tiles")
        N.require_extent(norms, ((groups - 1) * gst * 32 + seq) * 4, "decompress norms")
    else:
        rows = N.grouped_rows(n, seq, gst)
        rb = {N.QKV_FMT_UNPACKED: d, N.QKV_FMT_PACKED: N.packed_row_bytes(d, bits),
              N.QKV_FMT_KPLANES: (bits + 1) * d // 8}[fmt]
        N.require_extent(codes, rows * rb, "decompress codes")
        N.require_extent(norms, rows * 4, "decompress norms")
        if mode == N.QKV_MODE_IP and fmt != N.QKV_FMT_KPLANES:
            N.require_extent(qjl, rows * (N.packed_row_bytes(d, 1) if fmt == N.QKV_FMT_PACKED
                                          else d), "decompress qjl")
    N.check(N.lib().qkv_decompress(
        mode, int(fmt), codes.data_ptr(), N.ptr(qjl), norms.data_ptr(), n, d, bits,
        pi.data_ptr(), centroids.data_ptr(), N.ptr(signs), float(qjl_scale), seq, gst,
        out.data_ptr(), N.dtype_code(out_dtype), N.stream(dev)))
    return out


class MSEQuantizer:
    """Rotate by Pi, then Lloyd-Max quantise every coordinate (for values).

    API of quashkv/quantizer.py:66-153.  ``device`` defaults to the GPU;
    compress/decompress require GPU tensors (no CPU path).
    """

    def __init__(self, d: int, bits: int = 3, seed: int = DEFAULT_SEED,
                 device=None, use_exact_pdf: bool = False):
        self.d = d
        self.bits = bits
        self.seed = seed
        self.device = _default_device(device)
        self.Pi = _random_orthogonal(d, seed, self.device)
        self.codebook = LloydMaxCodebook(d, bits, use_exact_pdf=use_exact_pdf)
        self.codebook.to(self.device)

    def rotate(self, x: torch.Tensor) -> torch.Tensor:
        """x' = x Pi^T (a plain library GEMM)."""
        return x @ self.Pi.T

    def unrotate(self, x_rot: torch.Tensor) -> torch.Tensor:
        """x = x' Pi."""
        return x_rot @ self.Pi

    def compress(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """(uint8 codes (..., d), fp32 norms (...)) via the fused HIP kernel."""
        if self.d not in SUPPORTED_HEAD_DIMS:
            raise ValueError(f"head_dim {self.d} unsupported (64, 96 or 128)")
        dev = N.require_gpu(x, what="MSEQuantizer.compress")
        if self.Pi.device != dev:
            self.to(dev)
        lead = x.shape[:-1]
        n = int(torch.Size(lead).numel())
        codes = torch.empty(n, self.d, dtype=torch.uint8, device=dev)
        norms = torch.empty(n, dtype=torch.float32, device=dev)
        cb = self.codebook
        compress_into(N.QKV_MODE_MSE, x, self.Pi, cb.boundaries, cb.centroids, self.bits, None,
                      codes, None, norms, packed=False, host_tables=_host_tables(cb))
        return codes.reshape(*lead, self.d), norms.reshape(lead)

    def decompress(self, indices: torch.Tensor, norms: torch.Tensor) -> torch.Tensor:
        """(c[code] Pi) * norm via the fused HIP kernel; fp32."""
        dev = N.require_gpu(indices, norms, what="MSEQuantizer.decompress")
        if self.Pi.device != dev:
            self.to(dev)
        lead = indices.shape[:-1]
        n = int(torch.Size(lead).numel())
        out = decompress_from(N.QKV_MODE_MSE, indices.reshape(n, self.d).to(torch.uint8).contiguous(),
                              None, norms.reshape(n).float().contiguous(), n, self.Pi,
                              self.codebook.centroids, self.bits, None, 0.0,
                              fmt=N.QKV_FMT_UNPACKED)
        return out.reshape(*lead, self.d)

    def to(self, device) -> "MSEQuantizer":
        self.device = torch.device(device)
        self.Pi = self.Pi.to(self.device)
        self.codebook.to(self.device)
        return self


class InnerProductQuantizer:
    """(b-1)-bit MSE stage + 1-bit QJL residual sign (for keys).

    API of quashkv/quantizer.py:160-285.
    """

    def __init__(self, d: int, total_bits: int = DEFAULT_TOTAL_BITS, seed: int = DEFAULT_SEED,
                 device=None, use_exact_pdf: bool = False):
        if total_bits < 2:
            raise ValueError("InnerProductQuantizer needs at least 2 total bits")
        self.d = d
        self.total_bits = total_bits
        self.mse_bits = total_bits - 1
        self.seed = seed
        self.device = _default_device(device)
        self.mse_quantizer = MSEQuantizer(d, bits=self.mse_bits, seed=seed, device=self.device,
                                          use_exact_pdf=use_exact_pdf)
        self.S = _random_signs(d, seed, self.device)
        self.qjl_scale = QJL_COEFF / d

    def compress(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """(mse codes, QJL bits, norms); codes/bits uint8 (..., d)."""
        if self.d not in SUPPORTED_HEAD_DIMS:
            raise ValueError(f"head_dim {self.d} unsupported (64, 96 or 128)")
        dev = N.require_gpu(x, what="InnerProductQuantizer.compress")
        if self.S.device != dev:
            self.to(dev)
        lead = x.shape[:-1]
        n = int(torch.Size(lead).numel())
        codes = torch.empty(n, self.d, dtype=torch.uint8, device=dev)
        bits = torch.empty(n, self.d, dtype=torch.uint8, device=dev)
        norms = torch.empty(n, dtype=torch.float32, device=dev)
        mq = self.mse_quantizer
        compress_into(N.QKV_MODE_IP, x, mq.Pi, mq.codebook.boundaries, mq.codebook.centroids,
                      self.mse_bits, self.S, codes, bits, norms, packed=False,
                      host_tables=_host_tables(mq.codebook))
        return (codes.reshape(*lead, self.d), bits.reshape(*lead, self.d), norms.reshape(lead))

    def decompress_for_dot(self, mse_indices: torch.Tensor, qjl_signs: torch.Tensor,
                           norms: torch.Tensor, q_rot: torch.Tensor) -> torch.Tensor:
        """n (<q~, c[code]> + alpha sum |q~| (2b-1) S) per vector (HIP kernel)."""
        dev = N.require_gpu(mse_indices, qjl_signs, norms, q_rot,
                            what="InnerProductQuantizer.decompress_for_dot")
        if self.S.device != dev:
            self.to(dev)
        shape = torch.broadcast_shapes(mse_indices.shape, qjl_signs.shape, q_rot.shape)
        lead = shape[:-1]
        n = int(torch.Size(lead).numel())
        codes = mse_indices.expand(shape).reshape(n, self.d).to(torch.uint8).contiguous()
        bits = qjl_signs.expand(shape).reshape(n, self.d).to(torch.uint8).contiguous()
        qr = q_rot.expand(shape).reshape(n, self.d).float().contiguous()
        nr = norms.expand(lead).reshape(n).float().contiguous()
        out = torch.empty(n, dtype=torch.float32, device=dev)
        cb = self.mse_quantizer.codebook
        S, cents = N.dense(self.S, cb.centroids)
        N.check(N.lib().qkv_ip_dot(codes.data_ptr(), bits.data_ptr(), nr.data_ptr(), qr.data_ptr(),
                                   n, self.d, cents.data_ptr(), cb.n_levels,
                                   S.data_ptr(), float(self.qjl_scale), out.data_ptr(),
                                   N.stream(dev)))
        return out.reshape(lead)

    def to(self, device) -> "InnerProductQuantizer":
        self.device = torch.device(device)
        self.mse_quantizer.to(device)
        self.S = self.S.to(self.device)
        return self
