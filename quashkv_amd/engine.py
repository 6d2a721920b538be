"""QuashKVEngine: compressed KV cache + attention on the HIP kernels.

API of quashkv/engine.py:54-360.  What changes underneath:

* The cache is ONE preallocated device store per engine -- (B, H, capacity,
  row_bytes) code buffers and (B, H, capacity) norm buffers -- and append()
  compresses straight into it at offset total_tokens (no per-block tensors,
  no torch.cat).  Capacity grows by doubling.
* ``pack_storage`` keeps its meaning: True stores bit-packed rows (the
  pack_bits layout), False one uint8 per code.  The attention kernel reads
  either format directly.
* ``_cache`` still lists one CompressedKVBlock per append, as zero-copy views
  into the store, so code that walks blocks keeps working.
* attention() runs the split-K decode kernels; query heads may be a multiple
  of the cached kv heads (GQA, head h reads kv head h // G).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch

from . import _native as N
from .constants import DEFAULT_SEED, DEFAULT_TOTAL_BITS
from .kernels import attention_call
from .packing import pack_bits, unpack_bits
from .quantizer import InnerProductQuantizer, MSEQuantizer, _default_device, compress_into


@dataclass
class CompressedKVBlock:
    """One appended block (quashkv/engine.py:30-51); tensors are views of the store."""
    mse_indices: torch.Tensor
    qjl_signs: torch.Tensor
    key_norms: torch.Tensor
    val_indices: torch.Tensor
    val_norms: torch.Tensor
    seq_len: int
    packed: bool = False


class _KVStore:
    """Preallocated compressed KV buffers for one engine."""

    def __init__(self, B: int, H: int, d: int, kbits: int, vbits: int, packed: bool,
                 capacity: int, device: torch.device):
        self.B, self.H, self.d = B, H, d
        self.kbits, self.vbits, self.packed = kbits, vbits, packed
        self.device = device
        self.capacity = 0
        self.kcodes = self.kqjl = self.knorm = self.vcodes = self.vnorm = None
        self._alloc(capacity, 0)

    def row_bytes(self):
        if self.packed:
            return (N.packed_row_bytes(self.d, self.kbits), N.packed_row_bytes(self.d, 1),
                    N.packed_row_bytes(self.d, self.vbits))
        return self.d, self.d, self.d

    def _alloc(self, capacity: int, keep: int) -> None:
        pk, pq, pv = self.row_bytes()
        B, H, dev = self.B, self.H, self.device
        new = (
            torch.empty(B, H, capacity, pk, dtype=torch.uint8, device=dev),
            torch.empty(B, H, capacity, pq, dtype=torch.uint8, device=dev),
            torch.empty(B, H, capacity, dtype=torch.float32, device=dev),
            torch.empty(B, H, capacity, pv, dtype=torch.uint8, device=dev),
            torch.empty(B, H, capacity, dtype=torch.float32, device=dev),
        )
        if keep:
            old = (self.kcodes, self.kqjl, self.knorm, self.vcodes, self.vnorm)
            for n_, o_ in zip(new, old):
                n_[:, :, :keep].copy_(o_[:, :, :keep])
        self.kcodes, self.kqjl, self.knorm, self.vcodes, self.vnorm = new
        self.capacity = capacity

    def ensure(self, needed: int, keep: int) -> None:
        if needed > self.capacity:
            cap = max(needed, 2 * self.capacity, 256)
            self._alloc(cap, keep)

    def to(self, device) -> None:
        self.device = torch.device(device)
        for name in ("kcodes", "kqjl", "knorm", "vcodes", "vnorm"):
            setattr(self, name, getattr(self, name).to(self.device))

    def convert(self, packed: bool, used: int) -> None:
        """Re-encode the first `used` tokens in the other storage format."""
        if packed == self.packed:
            return
        old = (self.kcodes, self.kqjl, self.vcodes)
        old_bits = (self.kbits, 1, self.vbits)
        was_packed = self.packed
        self.packed = packed
        knorm, vnorm = self.knorm, self.vnorm
        self._alloc(self.capacity, 0)
        self.knorm, self.vnorm = knorm, vnorm
        for dst, src, bits in zip((self.kcodes, self.kqjl, self.vcodes), old, old_bits):
            if used == 0:
                continue
            view = src[:, :, :used]
            codes = unpack_bits(view.contiguous(), bits, self.d) if was_packed else view
            dst[:, :, :used].copy_(pack_bits(codes.contiguous(), bits) if packed else codes)


class QuashKVEngine:
    """TurboQuant KV-cache engine (quashkv/engine.py:54-360)."""

    def __init__(
        self,
        head_dim: int = 128,
        key_bits: int = DEFAULT_TOTAL_BITS,
        value_bits: int = DEFAULT_TOTAL_BITS,
        seed: int = DEFAULT_SEED,
        device=None,
        pack_storage: bool = False,
        capacity: int = 0,
    ):
        self.head_dim = head_dim
        self.key_bits = key_bits
        self.value_bits = value_bits
        self.seed = seed
        self.device = _default_device(device)
        self.pack_storage = pack_storage
        self.initial_capacity = capacity

        self.key_quantizer = InnerProductQuantizer(d=head_dim, total_bits=key_bits, seed=seed,
                                                   device=self.device)
        self.value_quantizer = MSEQuantizer(d=head_dim, bits=value_bits, seed=seed,
                                            device=self.device)
        self._store: Optional[_KVStore] = None
        self._blocks: list[tuple[int, int]] = []   # (start, seq_len) per append
        self._total_tokens = 0
        self._workspace: Optional[torch.Tensor] = None

    # ---------------------------------------------------------- compression

    def compress_keys(self, keys: torch.Tensor):
        """(mse codes, QJL bits, norms), unpacked uint8 (quashkv/engine.py:111-124)."""
        return self.key_quantizer.compress(keys)

    def compress_values(self, values: torch.Tensor):
        """(codes, norms), unpacked uint8 (quashkv/engine.py:126-139)."""
        return self.value_quantizer.compress(values)

    # -------------------------------------------------------------- storage

    def append(self, keys: torch.Tensor, values: torch.Tensor) -> None:
        """Compress (B, H, S, d) keys/values into the store (quashkv/engine.py:145-172)."""
        dev = N.require_gpu(keys, values, what="QuashKVEngine.append")
        if keys.dim() != 4 or keys.shape != values.shape or keys.shape[-1] != self.head_dim:
            raise ValueError(
                f"Expected keys and values of shape (batch, n_heads, seq_len, {self.head_dim}); "
                f"got {tuple(keys.shape)} and {tuple(values.shape)}")
        if self.key_quantizer.S.device != dev:
            self.to(dev)
        B, H, S, d = keys.shape
        st = self._store
        if st is not None and (st.B, st.H) != (B, H):
            raise ValueError(f"append shape (B={B}, H={H}) does not match the cache "
                             f"(B={st.B}, H={st.H})")
        if st is None:
            st = self._store = _KVStore(B, H, d, self.key_bits - 1, self.value_bits,
                                        bool(self.pack_storage),
                                        max(self.initial_capacity, S), dev)
        if st.packed != bool(self.pack_storage):
            st.convert(bool(self.pack_storage), self._total_tokens)
        t0 = self._total_tokens
        st.ensure(t0 + S, t0)
        if S > 0:
            kq, vq = self.key_quantizer, self.value_quantizer
            mq = kq.mse_quantizer
            k_rows = keys.reshape(B * H * S, d)
            v_rows = values.reshape(B * H * S, d)
            C = st.capacity
            # grouped rows: vector (bh, s) -> row bh * C + t0 + s
            compress_into(N.QKV_MODE_IP, k_rows, mq.Pi, mq.codebook.boundaries,
                          mq.codebook.centroids, kq.mse_bits, kq.S,
                          st.kcodes[:, :, t0:], st.kqjl[:, :, t0:], st.knorm[:, :, t0:],
                          packed=st.packed, out_seq=S, out_group_stride=C)
            compress_into(N.QKV_MODE_MSE, v_rows, vq.Pi, vq.codebook.boundaries,
                          vq.codebook.centroids, vq.bits, None,
                          st.vcodes[:, :, t0:], None, st.vnorm[:, :, t0:],
                          packed=st.packed, out_seq=S, out_group_stride=C)
        self._blocks.append((t0, S))
        self._total_tokens += S

    @property
    def _cache(self) -> list[CompressedKVBlock]:
        st = self._store
        out = []
        for t0, s in self._blocks:
            sl = slice(t0, t0 + s)
            out.append(CompressedKVBlock(
                mse_indices=st.kcodes[:, :, sl], qjl_signs=st.kqjl[:, :, sl],
                key_norms=st.knorm[:, :, sl], val_indices=st.vcodes[:, :, sl],
                val_norms=st.vnorm[:, :, sl], seq_len=s, packed=st.packed))
        return out

    def clear(self) -> None:
        self._blocks = []
        self._total_tokens = 0

    @property
    def total_tokens(self) -> int:
        return self._total_tokens

    @property
    def num_blocks(self) -> int:
        return len(self._blocks)

    def _unpack_block(self, block: CompressedKVBlock):
        """(mse codes, QJL bits, value codes) as uint8 (quashkv/engine.py:191-202)."""
        if not block.packed:
            return block.mse_indices, block.qjl_signs, block.val_indices
        d = self.head_dim
        return (unpack_bits(block.mse_indices.contiguous(), self.key_bits - 1, d),
                unpack_bits(block.qjl_signs.contiguous(), 1, d),
                unpack_bits(block.val_indices.contiguous(), self.value_bits, d))

    # ------------------------------------------------------------ attention

    def attention(self, queries: torch.Tensor, scale: Optional[float] = None,
                  causal: bool = False, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """Attention of (B, Hq, Q, d) queries over the whole compressed cache.

        Same result as quashkv/engine.py:204-299 (scores in the rotated domain,
        softmax over all cached tokens, values un-rotated), computed by the
        split-K HIP kernels.  Hq may be a multiple of the cached heads (GQA)."""
        if not self._blocks or self._total_tokens == 0:
            raise ValueError("No compressed KV blocks in cache. Call append() first.")
        st = self._store
        N.require_gpu(queries, what="QuashKVEngine.attention")
        B, Hq, Q, d = queries.shape
        if B != st.B or d != self.head_dim or Hq % st.H != 0:
            raise ValueError(f"queries {tuple(queries.shape)} do not match the cache "
                             f"(B={st.B}, kv heads={st.H}, head_dim={self.head_dim})")
        kq, vq = self.key_quantizer, self.value_quantizer
        L = N.lib()
        splits = L.qkv_attention_splits(B, Hq, st.H, Q, d, self._total_tokens)
        need = L.qkv_attention_workspace_bytes(B, Hq, st.H, Q, d, splits)
        if self._workspace is None or self._workspace.numel() < need \
                or self._workspace.device != queries.device:
            self._workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=queries.device)
        return attention_call(
            queries, st.kcodes, st.kqjl, st.knorm, st.vcodes, st.vnorm, self._total_tokens,
            kq.mse_quantizer.Pi, kq.mse_quantizer.codebook.centroids, vq.codebook.centroids,
            kq.S, kq.qjl_scale, kq.mse_bits, vq.bits, st.packed, scale=scale, causal=causal,
            out_dtype=out_dtype, workspace=self._workspace, n_splits=splits)

    # -------------------------------------------------------------- metrics

    def compression_ratio(self, original_dtype: torch.dtype = torch.float16) -> float:
        """2 d orig_bits / ((key_bits + value_bits) d + 64) (quashkv/engine.py:305-326)."""
        if not self._blocks:
            return 1.0
        orig_bits = torch.finfo(original_dtype).bits
        original = 2 * self.head_dim * orig_bits
        compressed = (self.key_bits * self.head_dim + 32 + self.value_bits * self.head_dim + 32)
        return original / compressed

    def actual_memory_bytes(self) -> int:
        """Bytes held by the appended blocks' codes and norms (quashkv/engine.py:328-337)."""
        total = 0
        for blk in self._cache:
            for t in (blk.mse_indices, blk.qjl_signs, blk.key_norms, blk.val_indices,
                      blk.val_norms):
                total += t.nelement() * t.element_size()
        return total

    def to(self, device) -> "QuashKVEngine":
        self.device = torch.device(device)
        self.key_quantizer.to(device)
        self.value_quantizer.to(device)
        if self._store is not None:
            self._store.to(device)
        self._workspace = None
        return self

    def __repr__(self) -> str:
        return (
            f"QuashKVEngine(head_dim={self.head_dim}, key_bits={self.key_bits}, "
            f"value_bits={self.value_bits}, cached_tokens={self._total_tokens}, "
            f"blocks={len(self._blocks)}, device={self.device})"
        )
