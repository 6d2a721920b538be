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


def test_padding_masks_become_key_ranges():
    # the 2-D padding mask transformers hands the mask interface: padding
    # before / after each row becomes that row's key range; an all-ones mask
    # (or none) builds nothing; a row with a hole raises
    pad = torch.tensor([[0, 0, 1, 1, 1], [1, 1, 1, 1, 1], [1, 1, 1, 0, 0], [0, 0, 0, 0, 0]],
                       dtype=torch.bool)
    for m in (pad, pad.long()):
        r = HA._range_mask(batch_size=4, q_length=5, kv_length=5, attention_mask=m)
        assert isinstance(r, HA.KVRanges)
        assert r.start.tolist() == [2, 0, 0, 0] and r.end.tolist() == [5, 5, 3, 0]
        assert r.start.dtype == torch.int32 and r.end.dtype == torch.int32
    full = torch.ones(2, 3, dtype=torch.long)
    assert HA._range_mask(batch_size=2, q_length=3, kv_length=3, attention_mask=full) is None
    assert HA._range_mask(batch_size=2, q_length=3, kv_length=3, attention_mask=None) is None
    holes = torch.tensor([[1, 0, 1]], dtype=torch.bool)
    with pytest.raises(ValueError, match="holes"):
        HA._range_mask(batch_size=1, q_length=3, kv_length=3, attention_mask=holes)
