"""Host side of the vLLM-style page manager (quashkv_amd.integrations.
vllm_backend), mirroring quashkv tests/test_vllm_backend.py where no GPU is
needed: config defaults, per-layer seeds, which store a layer gets, stats,
registration without vLLM, and that compute on CPU tensors fails loudly."""

import pytest
import torch

from quashkv_amd.integrations.vllm_backend import (
    HAS_VLLM, QuashKVModelManager, QuashKVPageConfig, QuashKVPageManager,
    register_quashkv_backend)
from quashkv_amd.paged import PagedQuashKVEngine

CPU = torch.device("cpu")


def test_config_defaults_and_custom():
    cfg = QuashKVPageConfig()
    assert (cfg.key_bits, cfg.value_bits, cfg.block_size, cfg.seed) == (3, 3, 16, 42)
    cfg = QuashKVPageConfig(key_bits=4, value_bits=4, block_size=32, seed=7)
    assert cfg.key_bits == 4 and cfg.block_size == 32


def test_page_manager_init_and_store_choice():
    pm = QuashKVPageManager(num_kv_heads=4, head_size=64, config=QuashKVPageConfig(), device=CPU)
    assert pm.total_tokens == 0 and pm.num_kv_heads == 4 and pm.head_size == 64
    assert pm.paged and isinstance(pm.engine, PagedQuashKVEngine)
    # every head_dim (64, 96, 128) and key/value width the config takes is paged
    for d in (64, 96, 128):
        for kb, vb in ((2, 1), (3, 3), (4, 4), (4, 2)):
            pm = QuashKVPageManager(num_kv_heads=2, head_size=d,
                                    config=QuashKVPageConfig(key_bits=kb, value_bits=vb),
                                    device=CPU)
            assert pm.paged and isinstance(pm.engine, PagedQuashKVEngine), (d, kb, vb)


def test_block_size_must_divide_page():
    with pytest.raises(ValueError, match="block_size"):
        QuashKVPageManager(4, 64, QuashKVPageConfig(block_size=48), CPU)


def test_layer_seed_offset():
    a = QuashKVPageManager(2, 64, QuashKVPageConfig(seed=42), CPU, layer_idx=0)
    b = QuashKVPageManager(2, 64, QuashKVPageConfig(seed=42), CPU, layer_idx=1)
    assert a.engine.seed != b.engine.seed
    assert not torch.equal(a.engine.key_quantizer.mse_quantizer.Pi,
                           b.engine.key_quantizer.mse_quantizer.Pi)


def test_attention_empty_raises():
    pm = QuashKVPageManager(4, 64, QuashKVPageConfig(), CPU)
    with pytest.raises(ValueError, match="No compressed"):
        pm.attention(torch.randn(1, 4, 1, 64))


def test_cpu_tensors_fail_loudly():
    pm = QuashKVPageManager(4, 64, QuashKVPageConfig(), CPU)
    with pytest.raises(Exception, match="(?i)gpu|hip|device"):
        pm.compress_and_store(torch.randn(1, 4, 8, 64), torch.randn(1, 4, 8, 64))
    assert pm.total_tokens == 0


def test_model_manager_stats_and_config():
    m = QuashKVModelManager(num_layers=4, num_kv_heads=8, head_size=64, device=CPU)
    assert m.num_layers == 4 and len(m.layers) == 4
    st = m.stats()
    assert st["num_layers"] == 4 and st["config"]["key_bits"] == 3
    assert st["tokens_per_layer"] == [0, 0, 0, 0]
    assert m.total_compressed_bytes() == 0
    m = QuashKVModelManager(2, 4, 128, config=QuashKVPageConfig(key_bits=4, value_bits=4,
                                                                seed=99), device=CPU)
    assert m.layers[0].engine.key_bits == 4 and m.layers[0].engine.value_bits == 4


def test_no_vllm_raises():
    if HAS_VLLM:
        pytest.skip("vLLM is installed")
    with pytest.raises(ImportError, match="vLLM is not installed"):
        register_quashkv_backend()


def test_paged_engine_rejects_uncovered_config():
    with pytest.raises(ValueError, match="paged cache"):
        PagedQuashKVEngine(head_dim=80, key_bits=3, device=CPU)
