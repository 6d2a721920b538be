"""quashkv_amd -- TurboQuant KV-cache compression hot path for AMD MI355X.

Drop-in for the reference package's public API (quashkv/__init__.py:5-22):
``import quashkv_amd as quashkv``.  Compression, packing, decompression and
attention run as hand-written HIP kernels (gfx950) in libquashkv_hip.so;
there is no CPU execution path.
"""

__version__ = "0.1.0"

from .codebook import LloydMaxCodebook
from .quantizer import MSEQuantizer, InnerProductQuantizer
from .engine import QuashKVEngine
from .packing import pack_bits, unpack_bits
from .nn_search import QuashIndex
from .mixed_precision import MixedPrecisionMSEQuantizer, MixedPrecisionIPQuantizer

__all__ = [
    "LloydMaxCodebook",
    "MSEQuantizer",
    "InnerProductQuantizer",
    "QuashKVEngine",
    "QuashIndex",
    "MixedPrecisionMSEQuantizer",
    "MixedPrecisionIPQuantizer",
    "pack_bits",
    "unpack_bits",
]
