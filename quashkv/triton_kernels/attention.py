"""quashkv.triton_kernels.attention -> quashkv_amd.kernels (reference attention.py:40-394)."""
from quashkv_amd.kernels import CompressedBlock, fused_quantized_attention  # noqa: F401
