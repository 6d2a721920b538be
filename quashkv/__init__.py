"""The reference package's import paths over quashkv_amd (quashkv/__init__.py:5-22).

``import quashkv`` and its submodules (``quashkv.engine``,
``quashkv.triton_kernels``, ``quashkv.integrations.hf_cache`` ...) resolve to
the same objects as ``quashkv_amd``: this package only lays the reference's
module tree over the HIP implementation, so code written against the
reference imports unchanged.  There is no second implementation here.
"""

from quashkv_amd import (  # noqa: F401
    __version__,
    LloydMaxCodebook,
    MSEQuantizer,
    InnerProductQuantizer,
    QuashKVEngine,
    QuashIndex,
    MixedPrecisionMSEQuantizer,
    MixedPrecisionIPQuantizer,
    pack_bits,
    unpack_bits,
)

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
