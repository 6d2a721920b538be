"""quashkv.mixed_precision -> quashkv_amd.mixed_precision (reference quashkv/mixed_precision.py)."""
from quashkv_amd.mixed_precision import (  # noqa: F401
    MixedPrecisionIPQuantizer, MixedPrecisionMSEQuantizer)
