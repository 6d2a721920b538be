"""quashkv.triton_kernels.decompress -> quashkv_amd.kernels (reference decompress.py:194-285)."""
from quashkv_amd.kernels import fused_decompress_ip, fused_decompress_mse  # noqa: F401
