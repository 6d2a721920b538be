"""Defaults of the TurboQuant hot path (values from quashkv/constants.py:8-26)."""

import math

SUPPORTED_BITS = {1, 2, 3, 4}
DEFAULT_TOTAL_BITS = 3      # keys: 2-bit MSE + 1-bit QJL; values: 3-bit MSE
DEFAULT_SEED = 42

# QJL correction scale numerator: alpha = sqrt(pi/2) / d
QJL_COEFF = math.sqrt(math.pi / 2)

# Lloyd-Max solver parameters (iteration count and tolerance shape the exact
# fp32 codebook values, so they are kept identical)
LLOYD_MAX_ITER = 300
LLOYD_MAX_TOL = 1e-12
LLOYD_MAX_RANGE_SIGMAS = 4.0

# head dims with compiled kernels
SUPPORTED_HEAD_DIMS = (64, 96, 128)
