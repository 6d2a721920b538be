"""Mixed-precision quantizers with outlier channels (quashkv/mixed_precision.py).

Outlier channels of the rotated vector (the highest-variance ones, found by
``calibrate``) use a finer codebook than the rest.  Compress / decompress run
the generic HIP kernels with a per-coordinate codebook choice
(qkv_compress_mixed / qkv_decompress_mixed).  ``calibrate`` is set-up work:
one rotation (a library GEMM, like ``rotate``) and a variance / top-k on the
device.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _native as N
from .codebook import LloydMaxCodebook
from .constants import DEFAULT_SEED, QJL_COEFF, SUPPORTED_HEAD_DIMS
from .quantizer import _default_device, _flat_rows, _random_orthogonal, _random_signs


class MixedPrecisionMSEQuantizer:
    """Per-channel two-codebook MSE quantizer (quashkv/mixed_precision.py:25-197)."""

    def __init__(self, d: int, outlier_bits: int = 3, regular_bits: int = 2,
                 n_outliers: int = 32, seed: int = DEFAULT_SEED, device=None):
        if n_outliers < 0 or n_outliers > d:
            raise ValueError(f"n_outliers must be in [0, {d}], got {n_outliers}")
        if outlier_bits < regular_bits:
            raise ValueError("outlier_bits should be >= regular_bits")
        self.d = d
        self.outlier_bits = outlier_bits
        self.regular_bits = regular_bits
        self.n_outliers = n_outliers
        self.seed = seed
        self.device = _default_device(device)
        self.Pi = _random_orthogonal(d, seed, self.device)
        self.outlier_codebook = LloydMaxCodebook(d, outlier_bits)
        self.outlier_codebook.to(self.device)
        self.regular_codebook = LloydMaxCodebook(d, regular_bits)
        self.regular_codebook.to(self.device)
        self._outlier_indices: Optional[torch.Tensor] = None
        self._outlier_mask: Optional[torch.Tensor] = None

    @property
    def effective_bits(self) -> float:
        n_o = self.n_outliers
        return (n_o * self.outlier_bits + (self.d - n_o) * self.regular_bits) / self.d

    @property
    def calibrated(self) -> bool:
        return self._outlier_mask is not None

    def calibrate(self, data: torch.Tensor) -> None:
        """Outliers = the n_outliers highest-variance rotated channels
        (quashkv/mixed_precision.py:92-115)."""
        if data.dim() != 2 or data.shape[1] != self.d:
            raise ValueError(f"Expected (N, {self.d}) calibration data")
        data = data.to(self.device).float()
        norms = data.norm(dim=-1, keepdim=True).clamp(min=1e-8)
        x_rot = (data / norms) @ self.Pi.T
        _, top = x_rot.var(dim=0).topk(self.n_outliers)
        self.set_outlier_channels(top)

    def set_outlier_channels(self, indices: torch.Tensor) -> None:
        self._outlier_indices = indices.sort().values.to(self.device)
        mask = torch.zeros(self.d, dtype=torch.bool, device=self.device)
        mask[self._outlier_indices] = True
        self._outlier_mask = mask

    def rotate(self, x: torch.Tensor) -> torch.Tensor:
        return x @ self.Pi.T

    def unrotate(self, x_rot: torch.Tensor) -> torch.Tensor:
        return x_rot @ self.Pi

    # ------------------------------------------------------------- kernels

    def _sel(self, dev: torch.device) -> torch.Tensor:
        """Per-coordinate codebook choice (1 = outlier), uint8 on ``dev``."""
        if self._outlier_mask is None:
            return torch.zeros(self.d, dtype=torch.uint8, device=dev)
        return self._outlier_mask.to(dev, torch.uint8)

    def _tables(self, dev):
        for cb in (self.outlier_codebook, self.regular_codebook):
            if cb.centroids.device != dev:
                cb.to(dev)
        if self.Pi.device != dev:
            self.Pi = self.Pi.to(dev)
        return self.outlier_codebook, self.regular_codebook

    def _compress_into(self, mode: int, x: torch.Tensor, signs, pre_rotated: bool = False):
        if self.d not in SUPPORTED_HEAD_DIMS:
            raise ValueError(f"head_dim {self.d} unsupported (64, 96 or 128)")
        dev = N.require_gpu(x, what="MixedPrecision compress")
        oc, rc = self._tables(dev)
        xf = _flat_rows(x, self.d)
        n = xf.shape[0]
        codes = torch.empty(n, self.d, dtype=torch.uint8, device=dev)
        qjl = torch.empty_like(codes) if mode == N.QKV_MODE_IP else None
        norms = torch.empty(n, dtype=torch.float32, device=dev)
        sel = self._sel(dev)
        flags = N.QKV_FLAG_PRE_ROTATED if pre_rotated else 0
        pi, s = N.dense(self.Pi, signs)
        seq = max(n, 1)
        N.check(N.lib().qkv_compress_mixed(
            mode, N.dtype_code(xf.dtype), flags, xf.data_ptr(), n, self.d, pi.data_ptr(),
            sel.data_ptr(), oc.boundaries.data_ptr(), oc.centroids.data_ptr(), oc.bits,
            rc.boundaries.data_ptr(), rc.centroids.data_ptr(), rc.bits, N.ptr(s),
            codes.data_ptr(), N.ptr(qjl), norms.data_ptr(), seq, seq, N.stream(dev)))
        return codes, qjl, norms

    def compress(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """(uint8 codes (..., d) from each channel's codebook, fp32 norms (...))."""
        lead = x.shape[:-1]
        codes, _, norms = self._compress_into(N.QKV_MODE_MSE, x, None)
        return codes.reshape(*lead, self.d), norms.reshape(lead)

    def decompress(self, indices: torch.Tensor, norms: torch.Tensor) -> torch.Tensor:
        """(c_channel[code] Pi) * norm, fp32 (quashkv/mixed_precision.py:160-187)."""
        dev = N.require_gpu(indices, norms, what="MixedPrecisionMSEQuantizer.decompress")
        oc, rc = self._tables(dev)
        lead = indices.shape[:-1]
        n = int(torch.Size(lead).numel())
        codes = indices.reshape(n, self.d).to(torch.uint8).contiguous()
        nr = norms.reshape(n).float().contiguous()
        out = torch.empty(n, self.d, dtype=torch.float32, device=dev)
        if n:
            sel = self._sel(dev)
            pi = N.dense(self.Pi)[0]
            N.check(N.lib().qkv_decompress_mixed(
                N.QKV_MODE_MSE, codes.data_ptr(), None, nr.data_ptr(), n, self.d,
                sel.data_ptr(), oc.centroids.data_ptr(), oc.bits, rc.centroids.data_ptr(),
                rc.bits, pi.data_ptr(), None, 0.0, n, n, out.data_ptr(), N.QKV_F32,
                N.stream(dev)))
        return out.reshape(*lead, self.d)

    def to(self, device) -> "MixedPrecisionMSEQuantizer":
        self.device = torch.device(device)
        self.Pi = self.Pi.to(self.device)
        self.outlier_codebook.to(self.device)
        self.regular_codebook.to(self.device)
        if self._outlier_mask is not None:
            self._outlier_mask = self._outlier_mask.to(self.device)
            self._outlier_indices = self._outlier_indices.to(self.device)
        return self


class MixedPrecisionIPQuantizer:
    """Mixed-precision (bits - 1) MSE stage + 1-bit QJL on the residual
    (quashkv/mixed_precision.py:200-322)."""

    def __init__(self, d: int, outlier_bits: int = 3, regular_bits: int = 2,
                 n_outliers: int = 32, seed: int = DEFAULT_SEED, device=None):
        if regular_bits < 2:
            raise ValueError("IP quantizer needs at least 2 total bits")
        self.d = d
        self.outlier_bits = outlier_bits
        self.regular_bits = regular_bits
        self.n_outliers = n_outliers
        self.seed = seed
        self.device = _default_device(device)
        self.mse_quantizer = MixedPrecisionMSEQuantizer(
            d=d, outlier_bits=outlier_bits - 1, regular_bits=regular_bits - 1,
            n_outliers=n_outliers, seed=seed, device=self.device)
        self.S = _random_signs(d, seed, self.device)
        self.qjl_scale = QJL_COEFF / d

    @property
    def effective_bits(self) -> float:
        return self.mse_quantizer.effective_bits + 1.0

    @property
    def calibrated(self) -> bool:
        return self.mse_quantizer.calibrated

    def calibrate(self, data: torch.Tensor) -> None:
        self.mse_quantizer.calibrate(data)

    def set_outlier_channels(self, indices: torch.Tensor) -> None:
        self.mse_quantizer.set_outlier_channels(indices)

    def compress(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """(mse codes, qjl bits, norms): bit_j = [(y_j - c_j[code_j]) S_j >= 0]."""
        if self.S.device != x.device:
            self.S = self.S.to(x.device)
        lead = x.shape[:-1]
        codes, qjl, norms = self.mse_quantizer._compress_into(N.QKV_MODE_IP, x, self.S)
        return (codes.reshape(*lead, self.d), qjl.reshape(*lead, self.d), norms.reshape(lead))

    def _quantize_mixed(self, x_rot: torch.Tensor) -> torch.Tensor:
        """Per-channel boundary codes of rotated values."""
        lead = x_rot.shape[:-1]
        codes, _, _ = self.mse_quantizer._compress_into(N.QKV_MODE_MSE, x_rot, None,
                                                        pre_rotated=True)
        return codes.reshape(*lead, self.d)

    def _dequantize_mixed(self, indices: torch.Tensor) -> torch.Tensor:
        """Per-channel centroid values (rotated space), fp32."""
        mq = self.mse_quantizer
        rc = mq.regular_codebook
        if mq._outlier_mask is None:
            return rc.dequantize(indices)
        oc = mq.outlier_codebook
        out = oc.dequantize(indices.clamp(max=oc.n_levels - 1))
        reg = rc.dequantize(indices.clamp(max=rc.n_levels - 1))
        return torch.where(mq._outlier_mask.to(indices.device), out, reg)

    def to(self, device) -> "MixedPrecisionIPQuantizer":
        self.device = torch.device(device)
        self.mse_quantizer.to(device)
        self.S = self.S.to(device)
        return self
