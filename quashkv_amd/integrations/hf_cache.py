"""QuashKVCache: per-layer compressed KV cache with HuggingFace-style update().

API of quashkv/integrations/hf_cache.py:19-203: one QuashKVEngine per layer
(seed + layer_idx); update() appends and returns the full reconstructed K/V
(keys from their MSE stage only, QJL bits dropped, as the reference does).
The reconstruction reads the engine's store directly with the fused
decompress kernel (one launch per tensor, no per-block loop or torch.cat).

Beyond the reference (its README's "biggest gap"): ``attention()`` runs the
fused decode-attention kernel on a layer's compressed cache, so a caller can
skip the full-cache reconstruction entirely.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from .. import _native as N
from ..engine import QuashKVEngine
from ..quantizer import _default_device, decompress_from


@dataclass
class QuashKVCacheConfig:
    """quashkv/integrations/hf_cache.py:19-24."""
    key_bits: int = 3
    value_bits: int = 3
    seed: int = 42


class QuashKVCache:
    """Drop-in for the reference QuashKVCache (quashkv/integrations/hf_cache.py:27-203)."""

    def __init__(self, num_layers: int, head_dim: int,
                 config: Optional[QuashKVCacheConfig] = None, device=None):
        self.config = config or QuashKVCacheConfig()
        self.num_layers = num_layers
        self.head_dim = head_dim
        self.device = _default_device(device)
        self.engines: list[QuashKVEngine] = [
            QuashKVEngine(head_dim=head_dim, key_bits=self.config.key_bits,
                          value_bits=self.config.value_bits, seed=self.config.seed + i,
                          device=self.device)
            for i in range(num_layers)
        ]

    @classmethod
    def from_model(cls, model, config: Optional[QuashKVCacheConfig] = None, device=None):
        """Read num_hidden_layers / head_dim from a HF model config (hf_cache.py:69-94)."""
        mc = model.config
        num_layers = getattr(mc, "num_hidden_layers", None)
        if num_layers is None:
            raise ValueError("Cannot detect num_hidden_layers from model config")
        head_dim = getattr(mc, "head_dim", None)
        if head_dim is None:
            head_dim = mc.hidden_size // mc.num_attention_heads
        if device is None:
            device = next(model.parameters()).device
        return cls(num_layers=num_layers, head_dim=head_dim, config=config, device=device)

    def _decompress_engine(self, engine: QuashKVEngine) -> tuple[torch.Tensor, torch.Tensor]:
        """Full (B, H, T, d) K^ (MSE stage only) and V^ (hf_cache.py:96-121)."""
        st = engine._store
        T = engine.total_tokens
        B, H, d = st.B, st.H, self.head_dim
        n = B * H * T
        kq, vq = engine.key_quantizer, engine.value_quantizer
        mq = kq.mse_quantizer
        k = decompress_from(N.QKV_MODE_MSE, st.kst, None, st.knorm, n, mq.Pi,
                            mq.codebook.centroids, kq.mse_bits, None, 0.0, N.QKV_FMT_KPLANES,
                            in_seq=T, in_group_stride=st.capacity)
        v = decompress_from(N.QKV_MODE_MSE, st.vst, None, st.vnorm, n, vq.Pi,
                            vq.codebook.centroids, vq.bits, None, 0.0, N.QKV_FMT_VTILES,
                            in_seq=T, in_group_stride=st.capacity // 32)
        return k.reshape(B, H, T, d), v.reshape(B, H, T, d)

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int,
               cache_kwargs: Optional[dict] = None) -> tuple[torch.Tensor, torch.Tensor]:
        """Append new K/V and return the full reconstructed cache (hf_cache.py:123-152)."""
        engine = self.engines[layer_idx]
        engine.append(key_states, value_states)
        return self._decompress_engine(engine)

    def attention(self, query_states: torch.Tensor, layer_idx: int,
                  scale: Optional[float] = None, causal: bool = False,
                  out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """Decode attention of (B, Hq, Q, d) queries on layer `layer_idx`'s
        compressed cache (fused kernel, no reconstruction; GQA allowed)."""
        return self.engines[layer_idx].attention(query_states, scale=scale, causal=causal,
                                                 out_dtype=out_dtype)

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self.engines[layer_idx].total_tokens

    def get_max_cache_length(self) -> Optional[int]:
        return None

    def __getitem__(self, layer_idx: int) -> tuple[torch.Tensor, torch.Tensor]:
        engine = self.engines[layer_idx]
        if not engine._blocks:
            return (torch.empty(0), torch.empty(0))
        return self._decompress_engine(engine)

    def __len__(self) -> int:
        return self.num_layers

    def __iter__(self):
        for i in range(self.num_layers):
            yield self[i]

    def reset(self) -> None:
        for engine in self.engines:
            engine.clear()

    def compression_stats(self) -> dict:
        """Bit totals over the layers (quashkv/integrations/hf_cache.py:179-203).

        A token costs 2 d 16 bits as fp16 K and V rows, and (key_bits +
        value_bits) d code bits plus two 32-bit norms compressed."""
        tokens = [e.total_tokens for e in self.engines]
        fp16_bits = sum(n * 32 * e.head_dim for n, e in zip(tokens, self.engines))
        code_bits = sum(n * ((e.key_bits + e.value_bits) * e.head_dim + 64)
                        for n, e in zip(tokens, self.engines))
        return {
            "num_layers": self.num_layers,
            "tokens_per_layer": tokens,
            "total_original_bits": fp16_bits,
            "total_compressed_bits": code_bits,
            "overall_compression_ratio": fp16_bits / code_bits if code_bits else 0,
        }
