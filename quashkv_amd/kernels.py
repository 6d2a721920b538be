"""Fused operator API (same names and arguments as quashkv/triton_kernels/*).

The reference dispatches ``HAS_TRITON and x.is_cuda`` to Triton and falls
back to PyTorch otherwise (quashkv/triton_kernels/compress.py:230,275;
decompress.py:213,260; attention.py:344).  Here there is one path: the HIP
kernels of libquashkv_hip.so, on GPU tensors.  CPU tensors raise.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional, Sequence

import torch

from . import _native as N
from .quantizer import compress_into, decompress_from
from .store import KVStore, store_from_codes

HAS_HIP = True


def _lead(x: torch.Tensor):
    lead = x.shape[:-1]
    return lead, int(torch.Size(lead).numel())


def fused_compress_mse(x: torch.Tensor, Pi: torch.Tensor,
                       boundaries: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """normalise -> rotate -> boundary quantise; (codes uint8 (..., d), norms (...)).
    Replaces quashkv/triton_kernels/compress.py:210-249."""
    dev = N.require_gpu(x, Pi, boundaries, what="fused_compress_mse")
    d = x.shape[-1]
    lead, n = _lead(x)
    bits = int(round(math.log2(boundaries.numel() + 1)))
    if (1 << bits) - 1 != boundaries.numel():
        raise ValueError("boundaries must have 2**bits - 1 entries")
    codes = torch.empty(n, d, dtype=torch.uint8, device=dev)
    norms = torch.empty(n, dtype=torch.float32, device=dev)
    # centroids are not needed by the MSE stage; pass the boundaries as a
    # placeholder table of the right device
    cents = torch.zeros(1 << bits, dtype=torch.float32, device=dev)
    compress_into(N.QKV_MODE_MSE, x, Pi.float().contiguous(), boundaries.float().contiguous(),
                  cents, bits, None, codes, None, norms, packed=False)
    return codes.reshape(*lead, d), norms.reshape(lead)


def fused_compress_ip(x: torch.Tensor, Pi: torch.Tensor, boundaries: torch.Tensor,
                      S: torch.Tensor, centroids: torch.Tensor):
    """normalise -> rotate -> MSE quantise -> QJL sign of the residual.
    Replaces quashkv/triton_kernels/compress.py:252-303."""
    dev = N.require_gpu(x, Pi, boundaries, S, centroids, what="fused_compress_ip")
    d = x.shape[-1]
    lead, n = _lead(x)
    bits = int(round(math.log2(centroids.numel())))
    if (1 << bits) != centroids.numel() or boundaries.numel() != centroids.numel() - 1:
        raise ValueError("need 2**b centroids and 2**b - 1 boundaries")
    codes = torch.empty(n, d, dtype=torch.uint8, device=dev)
    qjl = torch.empty(n, d, dtype=torch.uint8, device=dev)
    norms = torch.empty(n, dtype=torch.float32, device=dev)
    compress_into(N.QKV_MODE_IP, x, Pi.float().contiguous(), boundaries.float().contiguous(),
                  centroids.float().contiguous(), bits, S.float().contiguous(), codes, qjl, norms,
                  packed=False)
    return codes.reshape(*lead, d), qjl.reshape(*lead, d), norms.reshape(lead)


def fused_decompress_mse(indices: torch.Tensor, norms: torch.Tensor, Pi: torch.Tensor,
                         centroids: torch.Tensor) -> torch.Tensor:
    """(c[code] Pi) * norm, fp32.  Replaces quashkv/triton_kernels/decompress.py:194-232."""
    N.require_gpu(indices, norms, Pi, centroids, what="fused_decompress_mse")
    d = indices.shape[-1]
    lead, n = _lead(indices)
    bits = max(1, int(math.ceil(math.log2(max(centroids.numel(), 2)))))
    out = decompress_from(N.QKV_MODE_MSE, indices.reshape(n, d).to(torch.uint8).contiguous(), None,
                          norms.reshape(n).float().contiguous(), n, Pi.float().contiguous(),
                          centroids.float().contiguous(), bits, None, 0.0,
                          fmt=N.QKV_FMT_UNPACKED)
    return out.reshape(*lead, d)


def fused_decompress_ip(mse_indices: torch.Tensor, qjl_signs: torch.Tensor, norms: torch.Tensor,
                        Pi: torch.Tensor, centroids: torch.Tensor, S: torch.Tensor,
                        qjl_scale: float) -> torch.Tensor:
    """((c[code] + alpha S (2b-1)) Pi) * norm, fp32.
    Replaces quashkv/triton_kernels/decompress.py:235-285."""
    N.require_gpu(mse_indices, qjl_signs, norms, Pi, centroids, S, what="fused_decompress_ip")
    d = mse_indices.shape[-1]
    lead, n = _lead(mse_indices)
    bits = max(1, int(math.ceil(math.log2(max(centroids.numel(), 2)))))
    out = decompress_from(N.QKV_MODE_IP, mse_indices.reshape(n, d).to(torch.uint8).contiguous(),
                          qjl_signs.reshape(n, d).to(torch.uint8).contiguous(),
                          norms.reshape(n).float().contiguous(), n, Pi.float().contiguous(),
                          centroids.float().contiguous(), bits, S.float().contiguous(),
                          qjl_scale, fmt=N.QKV_FMT_UNPACKED)
    return out.reshape(*lead, d)


@dataclass
class CompressedBlock:
    """View of one compressed KV block (quashkv/triton_kernels/attention.py:40-48)."""
    mse_indices: torch.Tensor   # (B, H, S, D) uint8
    qjl_signs: torch.Tensor     # (B, H, S, D) uint8
    key_norms: torch.Tensor     # (B, H, S) float32
    val_indices: torch.Tensor   # (B, H, S, D) uint8
    val_norms: torch.Tensor     # (B, H, S) float32
    seq_len: int


def attention_store(queries: torch.Tensor, store: KVStore, T: int, Pi: torch.Tensor,
                    key_centroids: Sequence[float], val_centroids: Sequence[float],
                    S: torch.Tensor, qjl_scale: float, scale: Optional[float] = None,
                    causal: bool = False, out_dtype: torch.dtype = torch.float32,
                    workspace: Optional[torch.Tensor] = None,
                    n_splits: Optional[int] = None, kv_start: Optional[torch.Tensor] = None,
                    kv_end: Optional[torch.Tensor] = None, q_end: int = 0) -> torch.Tensor:
    """Decode attention of (B, Hq, Q, d) queries over the first T tokens of a
    cache store.  ``key_centroids`` / ``val_centroids`` are the codebook values
    (host floats, or ``_native.HostFloats`` tables a caller keeps).  Returns
    (B, Hq, Q, d) in ``out_dtype``.

    ``kv_start`` / ``kv_end`` (B,) int32 on the device restrict sequence b to
    the keys [kv_start[b], kv_end[b]) (padding); with ``causal``, query i sits
    at ``q_end - Q + i`` when ``q_end > 0``, else at kv_end[b] - Q + i."""
    dev = N.require_gpu(queries, store.kst, Pi, what="attention")
    B, Hq, Q, d = queries.shape
    Hkv = store.H
    if B != store.B or d != store.d:
        raise ValueError(f"queries {tuple(queries.shape)} do not match the cache "
                         f"(B={store.B}, head_dim={store.d})")
    if Hq % Hkv != 0:
        raise ValueError(f"query heads ({Hq}) must be a multiple of kv heads ({Hkv})")
    if T <= 0:
        raise ValueError("No compressed KV blocks in cache. Call append() first.")
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    L = N.lib()
    if n_splits is None:
        n_splits = L.qkv_attention_splits(B, Hq, Hkv, Q, d, T)
    if workspace is None:   # (a caller's workspace is size-checked by the library)
        need = L.qkv_attention_workspace_bytes(B, Hq, Hkv, Q, d, n_splits)
        workspace = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
    q = queries.contiguous()
    if q.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        q = q.float()
    Pi, S = N.dense(Pi, S)
    kc = key_centroids if isinstance(key_centroids, N.HostFloats) else N.HostFloats(key_centroids)
    vc = val_centroids if isinstance(val_centroids, N.HostFloats) else N.HostFloats(val_centroids)
    out = torch.empty(B, Hq, Q, d, dtype=out_dtype, device=dev)
    if kv_start is None and kv_end is None and q_end == 0:
        N.check(L.qkv_decode_attention(
            q.data_ptr(), N.dtype_code(q.dtype), store.kst.data_ptr(), store.knorm.data_ptr(),
            store.vst.data_ptr(), store.vnorm.data_ptr(), store.capacity, T, B, Hq, Hkv, Q, d,
            store.mbits, store.vbits, Pi.data_ptr(), kc.ptr, vc.ptr, S.data_ptr(),
            float(qjl_scale), float(scale), 1 if causal else 0, out.data_ptr(),
            N.dtype_code(out_dtype), workspace.data_ptr(), workspace.numel(), n_splits,
            N.stream(dev)))
        return out
    rng = []
    for t in (kv_start, kv_end):
        if t is not None:
            t = t.to(device=dev, dtype=torch.int32).contiguous()
            if t.numel() != B:
                raise ValueError(f"key ranges need one entry per sequence ({B}), got {t.numel()}")
        rng.append(t)
    N.check(L.qkv_decode_attention_ranges(
        q.data_ptr(), N.dtype_code(q.dtype), store.kst.data_ptr(), store.knorm.data_ptr(),
        store.vst.data_ptr(), store.vnorm.data_ptr(), store.capacity, T, N.ptr(rng[0]),
        N.ptr(rng[1]), int(q_end), B, Hq, Hkv, Q, d, store.mbits, store.vbits, Pi.data_ptr(),
        kc.ptr, vc.ptr, S.data_ptr(), float(qjl_scale), float(scale), 1 if causal else 0,
        out.data_ptr(), N.dtype_code(out_dtype), workspace.data_ptr(), workspace.numel(),
        n_splits, N.stream(dev)))
    return out


def attention_store_kmixed(queries: torch.Tensor, store: KVStore, T: int,
                           pi_perm: torch.Tensor, n_out: int, out_centroids: "N.HostFloats",
                           reg_centroids: "N.HostFloats", Pi_v: torch.Tensor,
                           val_centroids: Sequence[float], scale: Optional[float] = None,
                           causal: bool = False, out_dtype: torch.dtype = torch.float32,
                           workspace: Optional[torch.Tensor] = None,
                           n_splits: Optional[int] = None,
                           signs_perm: Optional[torch.Tensor] = None,
                           qjl_scale: float = 0.0) -> torch.Tensor:
    """Decode attention over a store with mixed-precision K rows: scores
    n_k <q Pi^T, c_channel[code]> in the slot order of ``pi_perm`` (Pi's rows
    permuted outliers first), values un-rotated by ``Pi_v``.  With IP keys
    (the store's "kipmixed" rows) ``signs_perm`` (S in slot order) and
    ``qjl_scale`` add decompress_for_dot's QJL term
    (quashkv/quantizer.py:244-279)."""
    dev = N.require_gpu(queries, store.kst, pi_perm, Pi_v, what="attention")
    B, Hq, Q, d = queries.shape
    Hkv = store.H
    if B != store.B or d != store.d:
        raise ValueError(f"queries {tuple(queries.shape)} do not match the cache "
                         f"(B={store.B}, head_dim={store.d})")
    if Hq % Hkv != 0:
        raise ValueError(f"query heads ({Hq}) must be a multiple of kv heads ({Hkv})")
    if T <= 0:
        raise ValueError("No compressed KV blocks in cache. Call append() first.")
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    L = N.lib()
    if n_splits is None:
        n_splits = L.qkv_attention_splits(B, Hq, Hkv, Q, d, T)
    need = L.qkv_attention_workspace_bytes(B, Hq, Hkv, Q, d, n_splits)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
    q = queries.contiguous()
    if q.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        q = q.float()
    pi_perm, Pi_v = N.dense(pi_perm, Pi_v)
    vc = N.HostFloats(val_centroids)
    out = torch.empty(B, Hq, Q, d, dtype=out_dtype, device=dev)
    ip = store.kmix is not None and store.kmix[2]
    common = (q.data_ptr(), N.dtype_code(q.dtype), store.kst.data_ptr(), store.knorm.data_ptr(),
              store.vst.data_ptr(), store.vnorm.data_ptr(), store.capacity, T, B, Hq, Hkv, Q, d,
              store.vbits, pi_perm.data_ptr())
    tail = (Pi_v.data_ptr(), vc.ptr, float(scale), 1 if causal else 0, out.data_ptr(),
            N.dtype_code(out_dtype), workspace.data_ptr(), workspace.numel(), n_splits,
            N.stream(dev))
    if ip:
        if signs_perm is None:
            raise ValueError("IP mixed-precision keys need signs_perm")
        sp = N.dense(signs_perm)[0]
        N.check(L.qkv_decode_attention_kipmixed(*common, sp.data_ptr(), float(qjl_scale),
                                                int(n_out), out_centroids.ptr,
                                                reg_centroids.ptr, *tail))
    else:
        N.check(L.qkv_decode_attention_kmixed(*common, int(n_out), out_centroids.ptr,
                                              reg_centroids.ptr, *tail))
    return out


class LayerBatch:
    """Layer-batched decode over a fixed list of engines (a model's layers:
    one head_dim, bit widths, batch and kv heads), through
    qkv_decode_attention_layers, and the step's appends through
    qkv_store_append_layers (``batch.append``).  Per-layer constants (Pi, S, codebook tables)
    and the workspace are prepared once; each call reads the current stores,
    so appends between calls are seen.  ``batch(queries)`` returns one
    (B, Hq, Q, d) output per layer, as ``engines[l].attention(queries[l])``."""

    def __init__(self, engines: Sequence):
        n = len(engines)
        if n == 0 or n > 32:
            raise ValueError("1 to 32 engines per layer batch")
        e0 = engines[0]
        for e in engines:
            if (e._kmix or e.head_dim != e0.head_dim or e.key_bits != e0.key_bits
                    or e.value_bits != e0.value_bits):
                raise ValueError("attention_layers needs engines of one shape, bit widths and "
                                 "cached length")
        self.engines = list(engines)
        kq = [e.key_quantizer for e in engines]
        self._pi = [N.dense(k.mse_quantizer.Pi)[0] for k in kq]
        self._s = [N.dense(k.S)[0] for k in kq]
        self._pi_arr = N.ptr_array([t.data_ptr() for t in self._pi])
        self._s_arr = N.ptr_array([t.data_ptr() for t in self._s])
        self._kc = N.HostFloats(kq[0].mse_quantizer.codebook.centroids_host)
        self._vc = N.HostFloats(e0.value_quantizer.codebook.centroids_host)
        self._qjl = float(kq[0].qjl_scale)
        self._ws: Optional[torch.Tensor] = None
        self._stores = None   # (key, four pointer arrays) of the stores last seen
        self._app = None      # value Pi and the append's boundary tables, on first append

    def _store_arrays(self):
        sts = [e._store for e in self.engines]
        ptrs = tuple(tuple(getattr(st, f).data_ptr() for st in sts)
                     for f in ("kst", "knorm", "vst", "vnorm"))
        if self._stores is None or self._stores[0] != ptrs:
            self._stores = (ptrs, tuple(N.ptr_array(p) for p in ptrs))
        return self._stores[1]

    def append(self, keys: Sequence[torch.Tensor], values: Sequence[torch.Tensor]) -> None:
        """``engines[l].append(keys[l], values[l])`` for every layer.  When every
        engine already holds a store of one length and the rows take the fused
        append (bf16/fp16/fp32 rows of one shape, head_dim 64 or 128), all layers
        go through one K and one V launch (qkv_store_append_layers); otherwise
        each engine appends on its own."""
        engines = self.engines
        n = len(engines)
        if len(keys) != n or len(values) != n:
            raise ValueError("one key and one value tensor per engine")
        k0 = keys[0]
        e0 = engines[0]
        sts = [e._store for e in engines]
        T = e0.total_tokens
        fused = (k0.dim() == 4 and k0.is_cuda
                 and k0.dtype in (torch.bfloat16, torch.float16, torch.float32)
                 and e0.head_dim in (64, 96, 128) and 2 <= e0.key_bits <= 4
                 and all(k.shape == k0.shape and v.shape == k0.shape and k.dtype == k0.dtype
                         and v.dtype == k0.dtype and k.device == k0.device
                         and v.device == k0.device for k, v in zip(keys, values)))
        if fused:
            B, H, S, d = k0.shape
            fused = S > 0 and d == e0.head_dim and all(
                st is not None and (st.B, st.H) == (B, H) and e.total_tokens == T
                and st.kst.device == k0.device for e, st in zip(engines, sts))
        if fused:
            for st in sts:
                st.ensure(T + S, T)
            fused = len({st.capacity for st in sts}) == 1
        if fused:
            if self._app is None:
                vq = [e.value_quantizer for e in engines]
                mq0 = e0.key_quantizer.mse_quantizer
                vpi = [N.dense(q.Pi)[0] for q in vq]
                self._app = (vpi, N.ptr_array([t.data_ptr() for t in vpi]),
                             N.HostFloats(mq0.codebook.boundaries_host),
                             N.HostFloats(vq[0].codebook.boundaries_host))
            _, vpi_arr, kb, vb = self._app
            ks = [k.contiguous() for k in keys]
            vs = [v.contiguous() for v in values]
            kst, knorm, vst, vnorm = self._store_arrays()
            L = N.lib()
            status = L.qkv_store_append_layers(
                n, N.dtype_code(k0.dtype), N.ptr_array([k.data_ptr() for k in ks]),
                N.ptr_array([v.data_ptr() for v in vs]), B * H, S, d,
                e0.key_quantizer.mse_bits, e0.value_bits, self._pi_arr, self._s_arr, vpi_arr,
                self._kc.ptr, kb.ptr, vb.ptr, kst, knorm, vst, vnorm, sts[0].capacity, T,
                N.stream(k0.device))
            if status != N.QKV_E_UNSUPPORTED:
                N.check(status)
                for e in engines:
                    e._blocks.append((T, S))
                    e._total_tokens += S
                return
        for e, k, v in zip(engines, keys, values):
            e.append(k, v)

    def __call__(self, queries: Sequence[torch.Tensor], scale: Optional[float] = None,
                 causal: bool = False, out_dtype: torch.dtype = torch.float32,
                 n_splits: Optional[int] = None) -> list[torch.Tensor]:
        engines = self.engines
        n = len(engines)
        if len(queries) != n:
            raise ValueError("one query per engine, at least one engine")
        e0 = engines[0]
        st0 = e0._store
        T = e0.total_tokens
        if st0 is None or T == 0:
            raise ValueError("No compressed KV blocks in cache. Call append() first.")
        for e in engines:
            st = e._store
            if (st is None or e.total_tokens != T
                    or (st.B, st.H, st.capacity) != (st0.B, st0.H, st0.capacity)):
                raise ValueError("attention_layers needs engines of one shape, bit widths and "
                                 "cached length")
        q0 = queries[0]
        dev = N.require_gpu(q0, st0.kst, what="attention_layers")
        B, Hq, Q, d = q0.shape
        Hkv = st0.H
        if B != st0.B or d != e0.head_dim or Hq % Hkv != 0:
            raise ValueError(f"queries {tuple(q0.shape)} do not match the cache "
                             f"(B={st0.B}, kv heads={Hkv}, head_dim={e0.head_dim})")
        if any(q.shape != q0.shape for q in queries):
            raise ValueError("queries of one shape")
        dt = q0.dtype if q0.dtype in (torch.float32, torch.float16, torch.bfloat16) \
            else torch.float32
        qs = [q if (q.dtype == dt and q.is_contiguous()) else q.to(dt).contiguous()
              for q in queries]
        if scale is None:
            scale = 1.0 / math.sqrt(d)
        L = N.lib()
        if n_splits is None:
            n_splits = L.qkv_attention_splits(B * n, Hq, Hkv, Q, d, T)
        need = L.qkv_attention_workspace_bytes(B * n, Hq, Hkv, Q, d, n_splits)
        if self._ws is None or self._ws.numel() < need or self._ws.device != dev:
            self._ws = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
        out = torch.empty(n, B, Hq, Q, d, dtype=out_dtype, device=dev)
        step = out[0].numel() * out.element_size()
        kst, knorm, vst, vnorm = self._store_arrays()
        N.check(L.qkv_decode_attention_layers(
            n, N.ptr_array([q.data_ptr() for q in qs]), N.dtype_code(dt), kst, knorm, vst,
            vnorm, st0.capacity, T, B, Hq, Hkv, Q, d, st0.mbits, st0.vbits, self._pi_arr,
            self._kc.ptr, self._vc.ptr, self._s_arr, self._qjl, float(scale),
            1 if causal else 0, N.ptr_array([out.data_ptr() + l * step for l in range(n)]),
            N.dtype_code(out_dtype), self._ws.data_ptr(), self._ws.numel(), n_splits,
            N.stream(dev)))
        return list(out.unbind(0))


def attention_layers(engines: Sequence, queries: Sequence[torch.Tensor],
                     scale: Optional[float] = None, causal: bool = False,
                     out_dtype: torch.dtype = torch.float32,
                     n_splits: Optional[int] = None) -> list[torch.Tensor]:
    """One decode step over several layers' engines at once
    (qkv_decode_attention_layers): ``queries[l]`` (B, Hq, Q, d) attends the
    whole cache of ``engines[l]``; every engine must share head_dim, bit
    widths, batch, kv heads, cached length and store capacity (a model's
    layers).  Returns one output per layer, as ``engines[l].attention`` would.
    A decode loop keeps a ``LayerBatch`` instead, which prepares the per-layer
    constants once."""
    if len(engines) != len(queries):
        raise ValueError("one query per engine, at least one engine")
    return LayerBatch(engines)(queries, scale=scale, causal=causal, out_dtype=out_dtype,
                               n_splits=n_splits)


def _bits_of(centroids: torch.Tensor) -> int:
    n = centroids.numel()
    b = max(1, int(math.ceil(math.log2(max(n, 2)))))
    if (1 << b) != n:
        raise ValueError(f"a codebook needs 2**bits centroids, got {n}")
    return b


def fused_quantized_attention(queries: torch.Tensor, blocks: Sequence[CompressedBlock],
                              Pi: torch.Tensor, key_centroids: torch.Tensor,
                              val_centroids: torch.Tensor, S: torch.Tensor, qjl_scale: float,
                              scale: Optional[float] = None, causal: bool = False,
                              total_kv_tokens: int = 0) -> torch.Tensor:
    """Attention over unpacked compressed blocks (quashkv/triton_kernels/attention.py:307-394).

    Blocks hold one uint8 per code, as in the reference.  They are packed once
    into a cache store and attended by the decode kernels.  Query heads may be
    a multiple of the blocks' kv heads (GQA).  With ``causal``, query i sits at
    position total_kv_tokens - Q + i and sees the keys at positions <= it
    (quashkv/triton_kernels/attention.py:118-121); total_kv_tokens = 0, the
    default, places it at T - Q + i for the T cached tokens (the reference
    would mask every key then)."""
    if not blocks:
        raise ValueError("No compressed KV blocks in cache. Call append() first.")
    if total_kv_tokens < 0:
        raise ValueError(f"total_kv_tokens must be >= 0, got {total_kv_tokens}")
    N.require_gpu(queries, Pi, what="fused_quantized_attention")
    kc = torch.cat([b.mse_indices for b in blocks], dim=2)
    kq = torch.cat([b.qjl_signs for b in blocks], dim=2)
    kn = torch.cat([b.key_norms for b in blocks], dim=2).float()
    vc = torch.cat([b.val_indices for b in blocks], dim=2)
    vn = torch.cat([b.val_norms for b in blocks], dim=2).float()
    T = kc.shape[2]
    st = store_from_codes(kc, kq, kn, vc, vn, _bits_of(key_centroids), _bits_of(val_centroids))
    kh = key_centroids.detach().float().cpu().tolist()
    vh = val_centroids.detach().float().cpu().tolist()
    return attention_store(queries, st, T, Pi, kh, vh, S, qjl_scale, scale=scale, causal=causal,
                           q_end=int(total_kv_tokens) if causal else 0)
