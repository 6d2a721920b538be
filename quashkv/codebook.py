"""quashkv.codebook -> quashkv_amd.codebook (reference quashkv/codebook.py)."""
from quashkv_amd.codebook import (  # noqa: F401
    LloydMaxCodebook, compute_mse_cost, get_codebook, solve_lloyd_max)
