"""quashkv.nn_search.index -> quashkv_amd.nn_search.index (reference nn_search/index.py)."""
from quashkv_amd.nn_search.index import QuashIndex  # noqa: F401
