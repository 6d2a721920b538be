"""quashkv.constants -> quashkv_amd.constants (reference quashkv/constants.py)."""
from quashkv_amd.constants import *  # noqa: F401,F403
