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
