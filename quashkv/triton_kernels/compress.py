"""quashkv.triton_kernels.compress -> quashkv_amd.kernels (reference compress.py:210-303)."""
from quashkv_amd.kernels import fused_compress_ip, fused_compress_mse  # noqa: F401
