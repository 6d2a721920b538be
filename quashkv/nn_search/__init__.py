"""quashkv.nn_search -> quashkv_amd.nn_search (reference nn_search/__init__.py)."""
from quashkv_amd.nn_search import QuashIndex  # noqa: F401

__all__ = ["QuashIndex"]
