"""quashkv.packing -> quashkv_amd.packing (reference quashkv/packing.py)."""
from quashkv_amd.packing import pack_bits, packed_size, unpack_bits  # noqa: F401
