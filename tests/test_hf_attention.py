"""Host-side checks of the transformers attention hook: registration, the
cache class shape, and the error for a call without the compressed cache."""

import pytest
import torch

from quashkv_amd.integrations import hf_attention as HA


def test_registered_with_transformers():
    from transformers import AttentionInterface
    from transformers.masking_utils import AttentionMaskInterface
    assert AttentionInterface().get_interface(HA.ATTN_IMPLEMENTATION, None) is HA.quashkv_attention
    assert HA.ATTN_IMPLEMENTATION in AttentionMaskInterface()._global_mapping


def test_attention_needs_the_cache():
    q = torch.zeros(1, 2, 1, 64)
    k = torch.zeros(1, 1, 3, 64)
    with pytest.raises(ValueError, match="QuashKVHFCache"):
        HA.quashkv_attention(None, q, k, k, None, scaling=0.125)


def test_padded_batches_are_refused():
    # the 2-D padding mask transformers hands the mask interface: any padded
    # position raises; an all-ones mask (or none) builds no mask tensor
    pad = torch.tensor([[0, 1, 1], [1, 1, 1]], dtype=torch.bool)
    with pytest.raises(ValueError, match="unpadded"):
        HA._no_mask(batch_size=2, q_length=3, kv_length=3, attention_mask=pad)
    with pytest.raises(ValueError, match="unpadded"):
        HA._no_mask(batch_size=2, q_length=3, kv_length=3, attention_mask=pad.long())
    full = torch.ones(2, 3, dtype=torch.long)
    assert HA._no_mask(batch_size=2, q_length=3, kv_length=3, attention_mask=full) is None
    assert HA._no_mask(batch_size=2, q_length=3, kv_length=3, attention_mask=None) is None
