"""quashkv.quantizer -> quashkv_amd.quantizer (reference quashkv/quantizer.py)."""
from quashkv_amd.quantizer import (  # noqa: F401
    InnerProductQuantizer, MSEQuantizer, _random_orthogonal, _random_signs)
