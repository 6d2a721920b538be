"""Fused decode attention behind HuggingFace models (transformers' attention
interface): the cache keeps every layer's K/V compressed and the model's
attention runs the fused kernel over it, so nothing is decompressed.

The reference's QuashKVCache hands the model fully decompressed K^, V^ on
every update (quashkv/integrations/hf_cache.py:123-152; its callers rebuild a
DynamicCache from them, generation_demo.py:202-215) and names fused
attention behind the generate path its biggest gap (README.md:364).  Here:

    from quashkv_amd.integrations.hf_attention import QuashKVHFCache, ATTN_IMPLEMENTATION
    model = AutoModelForCausalLM.from_config(cfg, attn_implementation=ATTN_IMPLEMENTATION)
    cache = QuashKVHFCache.from_model(model)
    model.generate(input_ids, past_key_values=cache, ...)

Each layer is a QuashKVEngine (seed + layer index, as QuashKVCache); its
update() appends the new K/V (fused compress into the packed store) and the
registered attention function calls ``engine.attention`` on the layer's
whole cache: scores from the IP keys (MSE codes + QJL bits) as
QuashKVEngine.attention computes them (quashkv/engine.py:204-299), causal
over the cache positions when a call brings several queries, GQA by kv-head
sharing.  A padded batch (HF's 2-D padding mask, left-padded as batched
generate makes it) becomes per-sequence key ranges [first kept, last kept + 1)
that the kernel masks, as the reference's HF attention masks its
reconstructed keys; padding must be a prefix and/or suffix of each row (a
mask with holes raises).  The engine's shape and dtype checks raise as usual.
"""

from __future__ import annotations

from typing import Optional

import torch

from ..engine import QuashKVEngine
from ..quantizer import _default_device
from .hf_cache import QuashKVCacheConfig

try:  # transformers >= 5: layered caches and a pluggable attention interface
    from transformers import AttentionInterface
    from transformers.cache_utils import Cache, CacheLayerMixin
    from transformers.masking_utils import AttentionMaskInterface
except ImportError as e:  # pragma: no cover - transformers is part of the image
    raise ImportError("quashkv_amd.integrations.hf_attention needs transformers >= 5") from e

ATTN_IMPLEMENTATION = "quashkv"


class QuashKVLayer(CacheLayerMixin):
    """One layer's compressed cache (a QuashKVEngine)."""

    is_sliding = False
    is_compileable = False

    def __init__(self, engine: QuashKVEngine):
        super().__init__()
        self.engine = engine

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        self.dtype, self.device = key_states.dtype, key_states.device
        self.is_initialized = True

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs):
        """Append the new tokens; returns the new K/V, the key tagged with this
        layer so that the attention function finds the compressed cache."""
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        self.engine.append(key_states, value_states)
        handle = key_states.view_as(key_states)
        handle._quashkv_layer = self
        return handle, value_states

    def get_seq_length(self) -> int:
        return self.engine.total_tokens

    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        return self.get_seq_length() + query_length, 0

    def get_max_length(self) -> int:
        return -1

    def reset(self) -> None:
        self.engine.clear()

    def reorder_cache(self, beam_idx: torch.LongTensor) -> None:
        raise NotImplementedError("QuashKVHFCache does not reorder (no beam search)")

    def offload(self) -> None:
        raise NotImplementedError("QuashKVHFCache stays on its device")

    def prefetch(self) -> None:
        pass


class QuashKVHFCache(Cache):
    """A transformers Cache of compressed layers, for models loaded with
    ``attn_implementation=ATTN_IMPLEMENTATION``."""

    def __init__(self, num_layers: int, head_dim: int,
                 config: Optional[QuashKVCacheConfig] = None, device=None):
        self.config = config or QuashKVCacheConfig()
        self.head_dim = head_dim
        dev = _default_device(device)
        self.engines = [
            QuashKVEngine(head_dim=head_dim, key_bits=self.config.key_bits,
                          value_bits=self.config.value_bits, seed=self.config.seed + i,
                          device=dev)
            for i in range(num_layers)
        ]
        super().__init__(layers=[QuashKVLayer(e) for e in self.engines])

    @classmethod
    def from_model(cls, model, config: Optional[QuashKVCacheConfig] = None, device=None):
        """num_hidden_layers / head_dim from a HF model config (as
        QuashKVCache.from_model, quashkv/integrations/hf_cache.py:69-94)."""
        mc = model.config
        num_layers = getattr(mc, "num_hidden_layers", None)
        if num_layers is None:
            raise ValueError("Cannot detect num_hidden_layers from model config")
        head_dim = getattr(mc, "head_dim", None) or mc.hidden_size // mc.num_attention_heads
        if device is None:
            device = next(model.parameters()).device
        return cls(num_layers, head_dim, config=config, device=device)


class KVRanges:
    """Per-sequence key ranges of a padded batch: sequence b attends to the
    cached keys [start[b], end[b]) ((B,) int32 device tensors)."""

    def __init__(self, start: torch.Tensor, end: torch.Tensor):
        self.start, self.end = start, end


def quashkv_attention(module, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                      attention_mask: Optional[torch.Tensor], scaling: Optional[float] = None,
                      dropout: float = 0.0, **kwargs):
    """Attention-interface function: (B, Hq, Q, d) queries over the layer's
    whole compressed cache; returns ((B, Q, Hq, d) in the query dtype, None)."""
    layer = getattr(key, "_quashkv_layer", None)
    if layer is None:
        raise ValueError(f"attn_implementation={ATTN_IMPLEMENTATION!r} needs a QuashKVHFCache "
                         "as past_key_values")
    if dropout:
        raise ValueError("quashkv attention has no dropout (inference only)")
    causal = query.shape[2] > 1
    if isinstance(attention_mask, KVRanges):
        eng = layer.engine
        out = eng.attention(query, scale=scaling, causal=causal, out_dtype=query.dtype,
                            kv_start=attention_mask.start, kv_end=attention_mask.end,
                            q_end=eng.total_tokens if causal else 0)
    else:
        out = layer.engine.attention(query, scale=scaling, causal=causal, out_dtype=query.dtype)
    return out.transpose(1, 2).contiguous(), None


def _range_mask(*args, attention_mask: Optional[torch.Tensor] = None, **kwargs):
    """The fused kernel masks causally itself, so no mask tensor is built.

    A 2-D padding mask with padded positions (any False, as left-padded
    batched generation passes) becomes per-sequence key ranges: each row must
    keep one contiguous run of positions [start, end) (padding before and/or
    after it); a row with holes raises ValueError."""
    if attention_mask is None or attention_mask.dim() != 2 or attention_mask.numel() == 0:
        return None
    m = attention_mask.bool()
    if bool(m.all()):
        return None
    n = m.shape[1]
    kept = m.sum(dim=1)
    start = torch.where(kept > 0, m.int().argmax(dim=1), torch.zeros_like(kept))
    pos = torch.arange(n, device=m.device)
    runs = (pos[None, :] >= start[:, None]) & (pos[None, :] < (start + kept)[:, None])
    if not bool((runs == m).all()):
        raise ValueError(
            f"attn_implementation={ATTN_IMPLEMENTATION!r} masks padding before and after each "
            "sequence; this attention mask has holes inside a sequence")
    return KVRanges(start.to(torch.int32), (start + kept).to(torch.int32))


def register() -> None:
    AttentionInterface.register(ATTN_IMPLEMENTATION, quashkv_attention)
    AttentionMaskInterface.register(ATTN_IMPLEMENTATION, _range_mask)


register()
