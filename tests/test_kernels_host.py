"""Host-side argument checks of the fused operator API that run before any
device work (CPU tensors are fine: the checks raise first)."""

import pytest
import torch

from quashkv_amd.kernels import CompressedBlock, fused_quantized_attention


def _blocks(n):
    z = torch.zeros(1, 1, n, 8, dtype=torch.uint8)
    f = torch.ones(1, 1, n)
    return [CompressedBlock(z, z, f, z, f, n)]


def test_causal_total_kv_tokens_is_any_position():
    q = torch.zeros(1, 1, 2, 8)
    blocks = _blocks(5) + _blocks(3)
    args = (q, blocks, torch.eye(8), torch.zeros(4), torch.zeros(8), torch.ones(8), 0.1)
    with pytest.raises(ValueError, match="total_kv_tokens must be >= 0"):
        fused_quantized_attention(*args, causal=True, total_kv_tokens=-1)
    # any offset (0: the cache length) passes the check and reaches the device check
    for tk in (0, 6, 8, 11):
        with pytest.raises(RuntimeError, match="GPU"):
            fused_quantized_attention(*args, causal=True, total_kv_tokens=tk)
    with pytest.raises(RuntimeError, match="GPU"):
        fused_quantized_attention(*args, causal=False, total_kv_tokens=6)
