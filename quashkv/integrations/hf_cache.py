"""quashkv.integrations.hf_cache -> quashkv_amd.integrations.hf_cache (reference hf_cache.py:19-203)."""
from quashkv_amd.integrations.hf_cache import QuashKVCache, QuashKVCacheConfig  # noqa: F401
