"""quashkv.engine -> quashkv_amd.engine (reference quashkv/engine.py)."""
from quashkv_amd.engine import CompressedKVBlock, QuashKVEngine  # noqa: F401
