"""quashkv.triton_kernels -> quashkv_amd.kernels (reference quashkv/triton_kernels/__init__.py:17-28).

The reference sets HAS_TRITON when its fused GPU kernels can run.  Here the
fused operators are HIP kernels for gfx950 and always the path taken on GPU
tensors (CPU tensors raise), so the flag is True whenever the library is
present.
"""
from quashkv_amd.kernels import (  # noqa: F401
    HAS_HIP, fused_compress_ip, fused_compress_mse, fused_decompress_ip, fused_decompress_mse,
    fused_quantized_attention)

HAS_TRITON = HAS_HIP

__all__ = [
    "HAS_TRITON",
    "fused_compress_mse",
    "fused_compress_ip",
    "fused_decompress_mse",
    "fused_decompress_ip",
    "fused_quantized_attention",
]
