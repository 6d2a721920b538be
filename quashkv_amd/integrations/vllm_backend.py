"""vLLM-style compressed KV page manager (quashkv/integrations/vllm_backend.py).

Same classes and functions as the reference module: QuashKVPageConfig,
QuashKVPageManager (one layer), quashkv_attention_forward (compress the new
K/V, then attend over the whole compressed history), QuashKVModelManager (all
layers) and register_quashkv_backend (raises ImportError without vLLM).

The reference's page manager wraps an engine of per-append tensors and never
uses ``block_size``.  Here a layer keeps its tokens in the paged store
(quashkv_amd.paged: pages of PAGE_TOKENS tokens from one pool, a device page
table per sequence) whenever the paged kernels cover the configuration (head_size 128
with key_bits 2..4, or 64 with key_bits 2 or 3), and a contiguous-store QuashKVEngine
otherwise; both
give the same codes and attention.  ``block_size`` must divide the page
(vLLM blocks then map onto page slots).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch

from ..engine import QuashKVEngine
from ..kernels import CompressedBlock
from ..quantizer import _default_device
from ..paged import PAGE_TOKENS, PagedQuashKVEngine, compressed_blocks

try:
    from vllm.v1.attention.backend import AttentionBackend, AttentionImpl  # noqa: F401
    from vllm.v1.attention.backends.registry import (  # noqa: F401
        AttentionBackendEnum, register_backend)
    HAS_VLLM = True
except ImportError:
    HAS_VLLM = False


@dataclass
class QuashKVPageConfig:
    """Compressed KV page configuration (quashkv/integrations/vllm_backend.py:68-75)."""
    key_bits: int = 3       # 2-bit MSE + 1-bit QJL
    value_bits: int = 3     # 3-bit MSE
    block_size: int = 16    # tokens per vLLM block; divides the 64-token page
    seed: int = 42


class QuashKVPageManager:
    """Compressed KV storage of one attention layer
    (quashkv/integrations/vllm_backend.py:82-195)."""

    def __init__(self, num_kv_heads: int, head_size: int, config: QuashKVPageConfig,
                 device: torch.device, layer_idx: int = 0):
        if config.block_size <= 0 or PAGE_TOKENS % config.block_size:
            raise ValueError(f"block_size {config.block_size} must divide the "
                             f"{PAGE_TOKENS}-token page")
        self.num_kv_heads = num_kv_heads
        self.head_size = head_size
        self.config = config
        self.device = device
        kw = dict(head_dim=head_size, key_bits=config.key_bits, value_bits=config.value_bits,
                  seed=config.seed + layer_idx, device=device)
        self.paged = PagedQuashKVEngine.covers(head_size, config.key_bits, config.value_bits)
        self.engine = PagedQuashKVEngine(**kw) if self.paged else QuashKVEngine(**kw)

    def compress_and_store(self, keys: torch.Tensor, values: torch.Tensor) -> None:
        """Compress (batch, num_kv_heads, seq_len, head_size) K/V into the cache."""
        if keys.dim() != 4 or keys.shape[1] != self.num_kv_heads:
            raise ValueError(f"expected (batch, {self.num_kv_heads}, seq_len, {self.head_size}) "
                             f"keys; got {tuple(keys.shape)}")
        self.engine.append(keys, values)

    def get_compressed_blocks(self) -> list[CompressedBlock]:
        """Unpacked per-append blocks (mse codes, QJL bits, norms, value codes)."""
        return compressed_blocks(self.engine)

    def attention(self, queries: torch.Tensor, scale: Optional[float] = None) -> torch.Tensor:
        """(batch, heads, q_len, head_size) queries over the whole compressed
        cache, no causal mask (as the reference); heads a multiple of the kv heads."""
        if scale is None:
            scale = 1.0 / math.sqrt(self.head_size)
        if self.engine.total_tokens == 0:
            raise ValueError("No compressed KV blocks stored yet")
        return self.engine.attention(queries, scale=scale)

    @property
    def total_tokens(self) -> int:
        return self.engine.total_tokens

    def clear(self) -> None:
        self.engine.clear()

    def compression_ratio(self) -> float:
        return self.engine.compression_ratio()


def quashkv_attention_forward(queries: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
                              page_manager: QuashKVPageManager,
                              scale: Optional[float] = None) -> torch.Tensor:
    """Compress and store the new K/V, then attend over the whole history
    (quashkv/integrations/vllm_backend.py:202-232)."""
    page_manager.compress_and_store(keys, values)
    return page_manager.attention(queries, scale=scale)


class QuashKVModelManager:
    """One QuashKVPageManager per layer (quashkv/integrations/vllm_backend.py:239-309)."""

    def __init__(self, num_layers: int, num_kv_heads: int, head_size: int,
                 config: Optional[QuashKVPageConfig] = None, device=None):
        self.num_layers = num_layers
        self.config = config or QuashKVPageConfig()
        self.device = _default_device(device)
        self.layers = [QuashKVPageManager(num_kv_heads=num_kv_heads, head_size=head_size,
                                          config=self.config, device=self.device, layer_idx=i)
                       for i in range(num_layers)]

    def forward_layer(self, layer_idx: int, queries: torch.Tensor, keys: torch.Tensor,
                      values: torch.Tensor, scale: Optional[float] = None) -> torch.Tensor:
        return quashkv_attention_forward(queries, keys, values, self.layers[layer_idx], scale)

    def clear(self) -> None:
        for layer in self.layers:
            layer.clear()

    def stats(self) -> dict:
        return {
            "num_layers": self.num_layers,
            "tokens_per_layer": [l.total_tokens for l in self.layers],
            "compression_ratios": [l.compression_ratio() for l in self.layers],
            "config": {"key_bits": self.config.key_bits, "value_bits": self.config.value_bits,
                       "block_size": self.config.block_size},
        }

    def total_compressed_bytes(self) -> int:
        return sum(l.engine.actual_memory_bytes() for l in self.layers)


def register_quashkv_backend() -> None:
    """vLLM backend registration (quashkv/integrations/vllm_backend.py:316-341):
    ImportError without vLLM; with it, use QuashKVModelManager directly, as the
    reference does."""
    if not HAS_VLLM:
        raise ImportError("vLLM is not installed. Install it with: pip install vllm>=0.6")
    raise NotImplementedError(
        "vLLM backend registration is not wired; use QuashKVModelManager directly, or "
        "quashkv_amd.integrations.hf_attention for HuggingFace models.")
