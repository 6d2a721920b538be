"""CPU test: every import the reference's own tests and benchmarks write
(tests/*.py, benchmarks/*.py of the reference) resolves under ``quashkv`` to
the quashkv_amd objects -- the module tree is laid over the HIP
implementation, not re-implemented."""

import importlib

import pytest

import quashkv_amd

# (module, names) as the reference's tests/benchmarks import them
IMPORTS = [
    ("quashkv", ["QuashKVEngine", "QuashIndex", "MSEQuantizer", "InnerProductQuantizer",
                 "pack_bits", "unpack_bits", "LloydMaxCodebook", "MixedPrecisionMSEQuantizer",
                 "MixedPrecisionIPQuantizer"]),
    ("quashkv.codebook", ["LloydMaxCodebook", "solve_lloyd_max", "compute_mse_cost"]),
    ("quashkv.quantizer", ["MSEQuantizer", "InnerProductQuantizer"]),
    ("quashkv.packing", ["pack_bits", "unpack_bits", "packed_size"]),
    ("quashkv.engine", ["QuashKVEngine", "CompressedKVBlock"]),
    ("quashkv.constants", ["SUPPORTED_BITS", "DEFAULT_TOTAL_BITS", "DEFAULT_SEED", "QJL_COEFF",
                           "LLOYD_MAX_ITER", "LLOYD_MAX_TOL", "LLOYD_MAX_RANGE_SIGMAS"]),
    ("quashkv.mixed_precision", ["MixedPrecisionMSEQuantizer", "MixedPrecisionIPQuantizer"]),
    ("quashkv.triton_kernels", ["HAS_TRITON", "fused_compress_mse", "fused_compress_ip",
                                "fused_decompress_mse", "fused_decompress_ip",
                                "fused_quantized_attention"]),
    ("quashkv.triton_kernels.compress", ["fused_compress_mse", "fused_compress_ip"]),
    ("quashkv.triton_kernels.decompress", ["fused_decompress_mse", "fused_decompress_ip"]),
    ("quashkv.triton_kernels.attention", ["fused_quantized_attention", "CompressedBlock"]),
    ("quashkv.integrations.hf_cache", ["QuashKVCache", "QuashKVCacheConfig"]),
    ("quashkv.integrations.vllm_backend", ["QuashKVPageConfig", "QuashKVPageManager",
                                           "QuashKVModelManager", "quashkv_attention_forward",
                                           "register_quashkv_backend", "HAS_VLLM"]),
    ("quashkv.nn_search", ["QuashIndex"]),
    ("quashkv.nn_search.index", ["QuashIndex"]),
]


@pytest.mark.parametrize("mod,names", IMPORTS, ids=[m for m, _ in IMPORTS])
def test_reference_import_paths_resolve(mod, names):
    m = importlib.import_module(mod)
    for n in names:
        assert hasattr(m, n), f"{mod}.{n}"


def test_same_objects_as_quashkv_amd():
    import quashkv
    from quashkv.engine import QuashKVEngine
    from quashkv.integrations.hf_cache import QuashKVCache
    from quashkv.triton_kernels import HAS_TRITON, fused_quantized_attention
    from quashkv_amd.integrations.hf_cache import QuashKVCache as HC
    from quashkv_amd.kernels import fused_quantized_attention as FQA

    assert QuashKVEngine is quashkv_amd.QuashKVEngine
    assert QuashKVCache is HC and fused_quantized_attention is FQA
    assert quashkv.__version__ == quashkv_amd.__version__
    assert HAS_TRITON is True
