"""quashkv.integrations.vllm_backend -> quashkv_amd.integrations.vllm_backend (reference vllm_backend.py:68-341)."""
from quashkv_amd.integrations.vllm_backend import (  # noqa: F401
    HAS_VLLM, QuashKVModelManager, QuashKVPageConfig, QuashKVPageManager,
    quashkv_attention_forward, register_quashkv_backend)
