"""QuashKVEngine: compressed KV cache + attention on the HIP kernels.

API of quashkv/engine.py:54-360.  What changes underneath:

* The cache is ONE preallocated device store per engine (quashkv_amd.store:
  K bit-plane rows, V bit-plane tiles, fp32 norms) and append() compresses
  straight into it at offset total_tokens -- no per-block tensors, no
  torch.cat.  Capacity grows by doubling.
* ``pack_storage`` keeps its observable meaning: ``_cache`` blocks hold
  pack_bits rows when True and one uint8 per code when False, and
  actual_memory_bytes() reports the bytes those block tensors take.  The store
  itself is always bit-packed.
* ``_cache`` lists one CompressedKVBlock per append, decoded from the store
  on access, so code that walks blocks keeps working.
* attention() runs the split-K decode kernels; query heads may be a multiple
  of the cached kv heads (GQA, head h reads kv head h // G).
* ``key_quantizer=`` (an extension: the reference engine builds its own IP
  key quantizer) takes a mixed-precision key quantizer with 32 or 64 outlier
  channels at head_dim 128:

  - ``MixedPrecisionMSEQuantizer(128, 3, 2, n)`` keeps 2.25 / 2.5-bit MSE keys
    in the store's "kmixed" rows; attention scores them as the reference's
    decompress-then-attend would (quashkv/mixed_precision.py:160-187);
  - ``MixedPrecisionIPQuantizer(128, 3, 2, n)`` keeps its 2/1-bit MSE codes
    and QJL bits in "kipmixed" rows; attention scores them as
    decompress_for_dot does for IP keys (quashkv/quantizer.py:244-279) with
    each channel's MSE codebook.

  The outlier channels are fixed at the first append.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch

from . import _native as N
from .constants import DEFAULT_SEED, DEFAULT_TOTAL_BITS
from .kernels import attention_store, attention_store_kmixed
from .mixed_precision import MixedPrecisionIPQuantizer, MixedPrecisionMSEQuantizer
from .packing import pack_bits, unpack_bits
from .quantizer import InnerProductQuantizer, MSEQuantizer, _default_device, compress_into
from .store import KVStore


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
        key_quantizer=None,
    ):
        self.head_dim = head_dim
        self.key_bits = key_bits
        self.value_bits = value_bits
        self.seed = seed
        self.device = _default_device(device)
        self.pack_storage = pack_storage
        self.initial_capacity = capacity

        self._kmix = key_quantizer is not None
        self._kmix_ip = isinstance(key_quantizer, MixedPrecisionIPQuantizer)
        if self._kmix:
            kq = key_quantizer
            if not isinstance(kq, (MixedPrecisionMSEQuantizer, MixedPrecisionIPQuantizer)):
                raise ValueError("key_quantizer must be a MixedPrecisionMSEQuantizer or a "
                                 "MixedPrecisionIPQuantizer")
            if (kq.d != head_dim or head_dim != 128 or kq.outlier_bits != 3
                    or kq.regular_bits != 2 or kq.n_outliers not in (32, 64)):
                raise ValueError("mixed-precision keys run on head_dim 128 with outlier_bits 3 "
                                 "and regular_bits 2, 32 or 64 outliers")
            self.key_quantizer = kq.to(self.device)
            self.key_bits = kq.effective_bits
        else:
            self.key_quantizer = InnerProductQuantizer(d=head_dim, total_bits=key_bits,
                                                       seed=seed, device=self.device)
        self.value_quantizer = MSEQuantizer(d=head_dim, bits=value_bits, seed=seed,
                                            device=self.device)
        self._store: Optional[KVStore] = None
        self._blocks: list[tuple[int, int]] = []   # (start, seq_len) per append
        self._total_tokens = 0
        self._workspace: Optional[torch.Tensor] = None
        self._host_tables = None   # codebook tables passed by value to the store append
        self._app_ptrs = None      # (tensors, pointer arrays) of the one-layer store append
        self._attn_tables = None   # (key MSE, value) centroids for the decode entry points
        # mixed keys: (perm, pi_perm, n_out, host tables, S in slot order or None)
        self._kmix_tables = None

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
        if self.value_quantizer.Pi.device != dev:
            self.to(dev)
        B, H, S, d = keys.shape
        st = self._store
        if st is not None and (st.B, st.H) != (B, H):
            if self._total_tokens:
                raise ValueError(f"append shape (B={B}, H={H}) does not match the cache "
                                 f"(B={st.B}, H={st.H})")
            st = self._store = None  # empty (cleared): any shape, as the reference allows
        if st is None:
            kmix = None
            if self._kmix:
                perm, _, n_out, _ = self._kmix_setup()
                kmix = (perm, n_out, self._kmix_ip)
            st = self._store = KVStore(B, H, d, 2 if self._kmix else self.key_bits - 1,
                                       self.value_bits, max(self.initial_capacity, S), dev,
                                       kmix=kmix)
        t0 = self._total_tokens
        st.ensure(t0 + S, t0)
        if S > 0 and self._kmix:
            self._append_kmix(keys, values, t0)
        elif S > 0 and not self._append_fused(keys, values, t0):
            kq, vq = self.key_quantizer, self.value_quantizer
            mq = kq.mse_quantizer
            n = B * H * S
            kc = torch.empty(n, d, dtype=torch.uint8, device=dev)
            kb = torch.empty(n, d, dtype=torch.uint8, device=dev)
            vc = torch.empty(n, d, dtype=torch.uint8, device=dev)
            kn = torch.empty(n, dtype=torch.float32, device=dev)
            vn = torch.empty(n, dtype=torch.float32, device=dev)
            # codes and norms of the n = B*H*S new vectors, row-contiguous; the
            # bit-plane packers then place the codes at tokens [t0, t0 + S)
            compress_into(N.QKV_MODE_IP, keys.reshape(n, d), mq.Pi, mq.codebook.boundaries,
                          mq.codebook.centroids, kq.mse_bits, kq.S, kc, kb, kn, packed=False)
            compress_into(N.QKV_MODE_MSE, values.reshape(n, d), vq.Pi, vq.codebook.boundaries,
                          vq.codebook.centroids, vq.bits, None, vc, None, vn, packed=False)
            st.knorm[:, :, t0:t0 + S].copy_(kn.view(B, H, S))
            st.vnorm[:, :, t0:t0 + S].copy_(vn.view(B, H, S))
            st.write_codes(t0, S, kc, kb, vc)
        self._blocks.append((t0, S))
        self._total_tokens += S

    def _append_fused(self, keys: torch.Tensor, values: torch.Tensor, t0: int) -> bool:
        """bf16, fp16 or fp32 rows at head_dim 128, 96 or 64: compress straight into
        the store (qkv_store_append).  False when that kernel does not cover the
        call."""
        if (keys.dtype not in (torch.bfloat16, torch.float16, torch.float32)
                or values.dtype != keys.dtype
                or self.head_dim not in (64, 96, 128) or not 2 <= self.key_bits <= 4):
            return False
        B, H, S, d = keys.shape
        kq, vq = self.key_quantizer, self.value_quantizer
        mq = kq.mse_quantizer
        if self._host_tables is None:
            self._host_tables = (N.HostFloats(mq.codebook.centroids_host),
                                 N.HostFloats(mq.codebook.boundaries_host),
                                 N.HostFloats(vq.codebook.boundaries_host))
        kc, kb, vb = self._host_tables
        st = self._store
        k, v = keys.contiguous(), values.contiguous()
        # one layer through qkv_store_append_layers: the key and the value
        # kernel in one launch for small appends (each quantizer has its own Pi)
        ts = (mq.Pi, kq.S, vq.Pi, st.kst, st.knorm, st.vst, st.vnorm)
        a = self._app_ptrs
        if a is None or any(x is not y for x, y in zip(ts, a[0])):
            a = self._app_ptrs = (ts, N.ptr_array([0]), N.ptr_array([0]),
                                  *(N.ptr_array([t.data_ptr()]) for t in ts))
        _, ka, va, kpi, sg, vpi, kst, kn, vst, vn = a
        ka[0], va[0] = k.data_ptr(), v.data_ptr()
        status = N.lib().qkv_store_append_layers(
            1, N.dtype_code(k.dtype), ka, va, B * H, S, d, kq.mse_bits, vq.bits, kpi, sg, vpi,
            kc.ptr, kb.ptr, vb.ptr, kst, kn, vst, vn, st.capacity, t0, N.stream(k.device))
        if status == N.QKV_E_UNSUPPORTED:
            return False
        N.check(status)
        return True

    def _kmix_setup(self):
        """Slot order (outlier channels ascending, then the rest), Pi with its
        rows in that order, n_out and the host codebook tables (outlier and
        regular centroids and boundaries, value boundaries, and for IP keys S
        in slot order); fixed at the first append."""
        if self._kmix_tables is None:
            kq = self.key_quantizer
            mq = kq.mse_quantizer if self._kmix_ip else kq
            if not kq.calibrated:
                raise ValueError("mixed-precision keys need calibrate() or "
                                 "set_outlier_channels() before the first append")
            mask = mq._outlier_mask.cpu()
            out = [j for j in range(self.head_dim) if bool(mask[j])]
            reg = [j for j in range(self.head_dim) if not bool(mask[j])]
            perm = out + reg
            idx = torch.tensor(perm, device=mq.Pi.device)
            pi_perm = mq.Pi[idx].contiguous()
            oc, rc = mq.outlier_codebook, mq.regular_codebook
            host = (N.HostFloats(oc.centroids_host), N.HostFloats(rc.centroids_host),
                    N.HostFloats(oc.boundaries_host), N.HostFloats(rc.boundaries_host),
                    N.HostFloats(self.value_quantizer.codebook.boundaries_host))
            signs_perm = kq.S.to(mq.Pi.device)[idx].float().contiguous() if self._kmix_ip else None
            self._kmix_tables = (perm, pi_perm, len(out), host, signs_perm)
        return self._kmix_tables[:4]

    def _kmix_signs(self, device) -> Optional[torch.Tensor]:
        """S in slot order (IP mixed keys), on ``device``."""
        sp = self._kmix_tables[4]
        if sp is not None and sp.device != device:
            sp = sp.to(device)
            self._kmix_tables = self._kmix_tables[:4] + (sp,)
        return sp

    def _append_kmix(self, keys: torch.Tensor, values: torch.Tensor, t0: int) -> None:
        """Mixed-precision keys: bf16, fp16 or fp32 rows straight into kmixed /
        kipmixed rows, with the values, in one qkv_store_append_kmixed_kv
        call; other dtypes through qkv_compress_mixed and the row packers."""
        B, H, S, d = keys.shape
        st = self._store
        kq, vq = self.key_quantizer, self.value_quantizer
        perm, pi_perm, n_out, (oc, rc, ob, rb, vb) = self._kmix_setup()
        if pi_perm.device != keys.device:
            pi_perm = pi_perm.to(keys.device)
            self._kmix_tables = (perm, pi_perm, n_out) + self._kmix_tables[3:]
        sp = self._kmix_signs(keys.device)
        L = N.lib()
        stream = N.stream(keys.device)
        n = B * H * S
        fused = (keys.dtype in (torch.bfloat16, torch.float16, torch.float32)
                 and values.dtype == keys.dtype)
        if fused:
            k, v = keys.contiguous(), values.contiguous()
            # keys (kmixed / kipmixed rows) and values in one call, one launch
            # for chunk-sized appends
            N.check(L.qkv_store_append_kmixed_kv(
                N.dtype_code(k.dtype), k.data_ptr(), v.data_ptr(), B * H, S, d,
                pi_perm.data_ptr(), sp.data_ptr() if self._kmix_ip else None, n_out,
                int(self._kmix_ip), oc.ptr, ob.ptr, rc.ptr, rb.ptr, st.kst.data_ptr(),
                st.knorm.data_ptr(), vq.bits, vq.Pi.data_ptr(), vb.ptr, st.vst.data_ptr(),
                st.vnorm.data_ptr(), st.capacity, t0, stream))
            return
        if self._kmix_ip:
            kc, kb, kn = kq.compress(keys.reshape(n, d))
        else:
            kc, kn = kq.compress(keys.reshape(n, d))
            kb = None
        vc = torch.empty(n, d, dtype=torch.uint8, device=keys.device)
        vn = torch.empty(n, dtype=torch.float32, device=keys.device)
        compress_into(N.QKV_MODE_MSE, values.reshape(n, d), vq.Pi, vq.codebook.boundaries,
                      vq.codebook.centroids, vq.bits, None, vc, None, vn, packed=False)
        st.knorm[:, :, t0:t0 + S].copy_(kn.view(B, H, S))
        st.vnorm[:, :, t0:t0 + S].copy_(vn.view(B, H, S))
        st.write_codes(t0, S, kc, kb, vc)

    @property
    def _cache(self) -> list[CompressedKVBlock]:
        st = self._store
        out = []
        for t0, s in self._blocks:
            kc, kb, vc = st.read_codes(t0, s)
            if self.pack_storage and not self._kmix:
                kc = pack_bits(kc, self.key_bits - 1)
                kb = pack_bits(kb, 1)
                vc = pack_bits(vc, self.value_bits)
            elif self.pack_storage:   # mixed key codes stay one uint8 each
                vc = pack_bits(vc, self.value_bits)
            sl = slice(t0, t0 + s)
            out.append(CompressedKVBlock(
                mse_indices=kc, qjl_signs=kb, key_norms=st.knorm[:, :, sl],
                val_indices=vc, val_norms=st.vnorm[:, :, sl], seq_len=s,
                packed=bool(self.pack_storage)))
        return out

    def clear(self) -> None:
        """Drop every cached token (quashkv/engine.py:174-177).  The store is kept
        for reuse; the next append may have any (batch, heads) shape."""
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
        if self._kmix:
            return (block.mse_indices, block.qjl_signs,
                    unpack_bits(block.val_indices.contiguous(), self.value_bits, d))
        return (unpack_bits(block.mse_indices.contiguous(), self.key_bits - 1, d),
                unpack_bits(block.qjl_signs.contiguous(), 1, d),
                unpack_bits(block.val_indices.contiguous(), self.value_bits, d))

    # ------------------------------------------------------------ attention

    def attention(self, queries: torch.Tensor, scale: Optional[float] = None,
                  causal: bool = False, out_dtype: torch.dtype = torch.float32, *,
                  kv_start: Optional[torch.Tensor] = None, kv_end: Optional[torch.Tensor] = None,
                  q_end: int = 0) -> torch.Tensor:
        """Attention of (B, Hq, Q, d) queries over the whole compressed cache.

        Same result as quashkv/engine.py:204-299 (scores in the rotated domain,
        softmax over all cached tokens, values un-rotated), computed by the
        split-K HIP kernels.  Hq may be a multiple of the cached heads (GQA).

        Beyond the reference: ``kv_start`` / ``kv_end`` ((B,) int tensors)
        restrict sequence b to the cached keys [kv_start[b], kv_end[b]) -- the
        padding of a batch -- and with ``causal`` a ``q_end`` > 0 places query
        i at position q_end - Q + i instead of at the end of the cache."""
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
            self._workspace = torch.empty(max(need, 256), dtype=torch.uint8, device=queries.device)
        ranged = kv_start is not None or kv_end is not None or q_end != 0
        if self._kmix:
            if ranged:
                raise ValueError("key ranges are not supported with mixed-precision keys")
            _, pi_perm, n_out, (oc, rc, _, _, _) = self._kmix_setup()
            return attention_store_kmixed(
                queries, st, self._total_tokens, pi_perm, n_out, oc, rc, vq.Pi,
                vq.codebook.centroids_host, scale=scale, causal=causal, out_dtype=out_dtype,
                workspace=self._workspace, n_splits=splits,
                signs_perm=self._kmix_signs(queries.device),
                qjl_scale=kq.qjl_scale if self._kmix_ip else 0.0)
        if self._attn_tables is None:
            self._attn_tables = (N.HostFloats(kq.mse_quantizer.codebook.centroids_host),
                                 N.HostFloats(vq.codebook.centroids_host))
        kc, vc = self._attn_tables
        return attention_store(
            queries, st, self._total_tokens, kq.mse_quantizer.Pi, kc, vc, kq.S,
            kq.qjl_scale, scale=scale, causal=causal, out_dtype=out_dtype,
            workspace=self._workspace, n_splits=splits, kv_start=kv_start, kv_end=kv_end,
            q_end=q_end)

    # -------------------------------------------------------------- metrics

    def compression_ratio(self, original_dtype: torch.dtype = torch.float16) -> float:
        """2 d orig_bits / ((key_bits + value_bits) d + 64) (quashkv/engine.py:305-326)."""
        if not self._blocks:
            return 1.0
        orig_bits = torch.finfo(original_dtype).bits
        original = 2 * self.head_dim * orig_bits
        # key_bits is the effective (average) width with mixed-precision keys
        compressed = (self.key_bits * self.head_dim + 32 + self.value_bits * self.head_dim + 32)
        return original / compressed

    def actual_memory_bytes(self) -> int:
        """Bytes the reference's block tensors would take (quashkv/engine.py:328-337):
        pack_bits rows when pack_storage, else one byte per code, plus fp32 norms."""
        if not self._blocks:
            return 0
        B, H = self._heads()
        d = self.head_dim
        if self._kmix:   # one uint8 per key code (+ QJL bit), as the mixed quantizers keep them
            krow = 2 * d if self._kmix_ip else d
            row = krow + (N.packed_row_bytes(d, self.value_bits) if self.pack_storage else d)
            return B * H * self._total_tokens * (row + 8)
        if self.pack_storage:
            row = (N.packed_row_bytes(d, self.key_bits - 1) + N.packed_row_bytes(d, 1)
                   + N.packed_row_bytes(d, self.value_bits))
        else:
            row = 3 * d
        return B * H * self._total_tokens * (row + 8)

    def _heads(self) -> tuple[int, int]:
        """(batch, kv heads) of the cache."""
        return self._store.B, self._store.H

    def to(self, device) -> "QuashKVEngine":
        self.device = torch.device(device)
        self.key_quantizer.to(device)
        self.value_quantizer.to(device)
        if self._store is not None:
            self._store.to(device)
        if self._kmix_tables is not None:
            perm, pi_perm, n_out, host, sp = self._kmix_tables
            self._kmix_tables = (perm, pi_perm.to(self.device), n_out, host,
                                 None if sp is None else sp.to(self.device))
        self._workspace = None
        return self

    def __repr__(self) -> str:
        return (
            f"QuashKVEngine(head_dim={self.head_dim}, key_bits={self.key_bits}, "
            f"value_bits={self.value_bits}, cached_tokens={self._total_tokens}, "
            f"blocks={len(self._blocks)}, device={self.device})"
        )
