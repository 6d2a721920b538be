"""Paged compressed KV cache: fixed-size pages from a shared pool and a page
table per sequence, the "preallocated, paged packed-cache format" the
reference's vLLM page manager leaves open (QuashKVPageManager,
quashkv/integrations/vllm_backend.py:82-195, whose ``block_size`` is unused:
it keeps one engine of per-append tensors).

A page holds ``page_tokens`` = 64 << k tokens (k = 0..5; 256 by default) of
all H kv heads of one sequence, in the store formats of quashkv_amd.store (C
ABI "Paged cache store"), with n = page_tokens:

* ``kpool`` (P, H, n, (mbits + 1) d / 8) uint8 -- K rows (MSE planes, QJL plane);
* ``knorm`` / ``vnorm`` (P, H, n) fp32;
* ``vpool`` (P, H, n / 32, vbits, d) int32 -- 32-token V bit-plane tiles.

``table`` (B, pages_per_seq) int32 on the device maps sequence b's token t to
page ``table[b, t // n]``.  Larger pages keep more of a sequence's K/V
contiguous in HBM (better DRAM locality when pages are scattered); smaller
ones waste less of the last page.  The append kernels (qkv_paged_store_append)
compress bf16, fp16 or fp32 K/V straight into the pages; the split-K decode kernel
(qkv_paged_decode_attention) follows the table per 32-token tile.  Pages come
from a free list and return to it on clear(); a reused page keeps its old
bits until tokens overwrite them (appends write whole K rows and merge V
tile bits under a token mask; decode masks tokens past the cached length).
The pool doubles when the free list runs dry (page ids stay valid).
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from . import _native as N
from .engine import CompressedKVBlock, QuashKVEngine
from .kernels import CompressedBlock
from .packing import pack_bits
from .quantizer import compress_into
from .store import KVStore

PAGE_TOKENS = 256          # default page size
PAGE_SIZES = tuple(64 << k for k in range(6))


def check_page_table(table: torch.Tensor, num_pages: int) -> None:
    """Host check of a page table (B, pages_per_seq) before it reaches the
    device: every entry must name a page of the pool, [0, num_pages).  (The
    kernels also never write through, and mask out, entries outside it.)"""
    t = table.detach()
    if t.dtype != torch.int32 or t.dim() != 2:
        raise ValueError("page table must be a 2-D int32 tensor")
    if t.numel() and (int(t.min()) < 0 or int(t.max()) >= num_pages):
        raise ValueError(f"page table entries must lie in [0, {num_pages}); got "
                         f"[{int(t.min())}, {int(t.max())}]")


class PagedKVStore:
    """Page pool + page table of B sequences with H kv heads each."""

    def __init__(self, B: int, H: int, d: int, mbits: int, vbits: int, num_pages: int,
                 device: torch.device, page_tokens: int = PAGE_TOKENS):
        if d % 32 != 0:
            raise ValueError(f"head_dim {d} must be a multiple of 32 for the cache store")
        if page_tokens not in PAGE_SIZES:
            raise ValueError(f"page_tokens {page_tokens} must be one of {PAGE_SIZES}")
        self.pt = page_tokens
        self.B, self.H, self.d = B, H, d
        self.mbits, self.vbits = mbits, vbits
        self.krb = (mbits + 1) * d // 8
        self.device = torch.device(device)
        self.num_pages = 0
        self.kpool = self.knorm = self.vpool = self.vnorm = None
        self.free: list[int] = []
        self.pages: list[list[int]] = [[] for _ in range(B)]   # page ids of each sequence
        self.table = torch.zeros(B, 1, dtype=torch.int32, device=self.device)
        self._grow_pool(max(int(num_pages), 1))

    # ------------------------------------------------------------- pool

    def _grow_pool(self, pages: int) -> None:
        H, d, dev = self.H, self.d, self.device
        old = self.num_pages
        n = self.pt
        kpool = torch.zeros(pages, H, n, self.krb, dtype=torch.uint8, device=dev)
        knorm = torch.zeros(pages, H, n, dtype=torch.float32, device=dev)
        vpool = torch.zeros(pages, H, n // 32, self.vbits, d, dtype=torch.int32, device=dev)
        vnorm = torch.zeros(pages, H, n, dtype=torch.float32, device=dev)
        if old:
            kpool[:old].copy_(self.kpool)
            knorm[:old].copy_(self.knorm)
            vpool[:old].copy_(self.vpool)
            vnorm[:old].copy_(self.vnorm)
        self.kpool, self.knorm, self.vpool, self.vnorm = kpool, knorm, vpool, vnorm
        self.free.extend(range(old, pages))
        self.num_pages = pages

    def _take(self, n: int) -> list[int]:
        if n > len(self.free):
            self._grow_pool(max(2 * self.num_pages, self.num_pages + n - len(self.free)))
        got, self.free = self.free[:n], self.free[n:]
        return got

    @property
    def pages_per_seq(self) -> int:
        return self.table.shape[1]

    def ensure(self, tokens: int) -> None:
        """Pages for tokens [0, tokens) of every sequence."""
        need = -(-tokens // self.pt)
        have = len(self.pages[0])
        if need <= have:
            return
        new = self._take(self.B * (need - have))
        for b in range(self.B):
            self.pages[b].extend(new[b * (need - have):(b + 1) * (need - have)])
        width = max(need, self.pages_per_seq)
        if width > self.pages_per_seq:
            width = max(width, 2 * self.pages_per_seq)
        tab = torch.zeros(self.B, width, dtype=torch.int32)
        for b in range(self.B):
            tab[b, :need] = torch.tensor(self.pages[b], dtype=torch.int32)
        check_page_table(tab, self.num_pages)
        self.table = tab.to(self.device)

    def release(self) -> None:
        """Every sequence's pages back to the free list."""
        for p in self.pages:
            self.free.extend(p)
            p.clear()

    def to(self, device) -> None:
        self.device = torch.device(device)
        for name in ("kpool", "knorm", "vpool", "vnorm", "table"):
            setattr(self, name, getattr(self, name).to(self.device))

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size()
                   for t in (self.kpool, self.knorm, self.vpool, self.vnorm))

    # ------------------------------------------------ token <-> page rows

    def _rows(self, t0: int, S: int) -> torch.Tensor:
        """(B, H, S) flat row ids (pool row (p H + h) n + slot) of tokens [t0, t0 + S)."""
        n = self.pt
        t = torch.arange(t0, t0 + S, device=self.device)
        page = self.table.long()[:, t // n]                                 # (B, S)
        h = torch.arange(self.H, device=self.device)
        return (page[:, None, :] * self.H + h[None, :, None]) * n + (t % n)[None, None, :]

    def _tiles(self, t0: int, S: int) -> tuple[torch.Tensor, int, int]:
        """Flat V tile ids (B, H, n) of the 32-token tiles covering [t0, t0 + S),
        with the first tile index j0 = t0 // 32 and n."""
        j0, j1 = t0 // 32, (t0 + S - 1) // 32 + 1
        tp = self.pt // 32                                                  # tiles per page
        j = torch.arange(j0, j1, device=self.device)
        page = self.table.long()[:, j // tp]
        h = torch.arange(self.H, device=self.device)
        return (page[:, None, :] * self.H + h[None, :, None]) * tp + (j % tp)[None, None, :], \
            j0, j1 - j0

    def write_from(self, tmp: KVStore, t0: int, S: int) -> None:
        """Tokens [t0 % n, t0 % n + S) of a contiguous store into the pages at
        [t0, t0 + S): K rows and norms by row, V tile words merged under the
        mask of those tokens' bits."""
        o = t0 % self.pt
        rows = self._rows(t0, S).reshape(-1)
        self.kpool.view(-1, self.krb)[rows] = tmp.kst[:, :, o:o + S].reshape(-1, self.krb)
        self.knorm.view(-1)[rows] = tmp.knorm[:, :, o:o + S].reshape(-1)
        self.vnorm.view(-1)[rows] = tmp.vnorm[:, :, o:o + S].reshape(-1)
        tiles, j0, n = self._tiles(t0, S)
        jt = j0 - (t0 - o) // 32                   # tmp tile of global tile j0
        flat = self.vpool.view(-1, self.vbits, self.d)
        tiles = tiles.reshape(-1)
        j = torch.arange(j0, j0 + n, device=self.device, dtype=torch.int64)
        lo = (t0 - 32 * j).clamp(0, 32)
        hi = (t0 + S - 32 * j).clamp(0, 32)
        m = (torch.ones_like(j) << hi) - (torch.ones_like(j) << lo)       # bits [lo, hi)
        m = torch.where(m >= 1 << 31, m - (1 << 32), m).to(torch.int32)
        m = m.view(1, 1, n, 1, 1)
        src = tmp.vst[:, :, jt:jt + n] & m
        dst = flat[tiles].view(self.B, self.H, n, self.vbits, self.d)
        flat[tiles] = ((dst & ~m) | src).reshape(-1, self.vbits, self.d)

    def gather(self, T: int) -> KVStore:
        """Tokens [0, T) as a contiguous KVStore (capacity T rounded to 64)."""
        st = KVStore(self.B, self.H, self.d, self.mbits, self.vbits, max(T, 1), self.device)
        if T == 0:
            return st
        rows = self._rows(0, T).reshape(-1)
        st.kst[:, :, :T] = self.kpool.view(-1, self.krb)[rows].view(self.B, self.H, T, self.krb)
        st.knorm[:, :, :T] = self.knorm.view(-1)[rows].view(self.B, self.H, T)
        st.vnorm[:, :, :T] = self.vnorm.view(-1)[rows].view(self.B, self.H, T)
        tiles, _, n = self._tiles(0, T)
        st.vst[:, :, :n] = self.vpool.view(-1, self.vbits, self.d)[tiles.reshape(-1)].view(
            self.B, self.H, n, self.vbits, self.d)
        return st


class PagedQuashKVEngine(QuashKVEngine):
    """QuashKVEngine (quashkv/engine.py:54-360) over a paged store.

    Same quantizers, append / attention / clear / metrics semantics; tokens
    live in pages of ``page_tokens`` tokens from one pool (``num_pages`` to start with).  bf16 /
    fp16 K/V compress straight into the pages; other dtypes go through the
    generic compress kernel and are scattered into the pages.  Attention runs
    the integer-MFMA split-K kernel, which covers head_dim 64 / 128 with keys
    of 2 or 3 total bits (``covers``)."""

    def __init__(self, head_dim: int = 128, key_bits: int = 3, value_bits: int = 3,
                 seed: int = 42, device=None, num_pages: int = 0,
                 page_tokens: int = PAGE_TOKENS):
        super().__init__(head_dim=head_dim, key_bits=key_bits, value_bits=value_bits, seed=seed,
                         device=device)
        if not self.covers(head_dim, key_bits, value_bits):
            raise ValueError("the paged cache runs head_dim 128, 96 or 64 with key_bits 2..4 and "
                             "value_bits 1..4")
        if page_tokens not in PAGE_SIZES:
            raise ValueError(f"page_tokens {page_tokens} must be one of {PAGE_SIZES}")
        self.initial_pages = num_pages
        self.page_tokens = page_tokens
        self._paged: Optional[PagedKVStore] = None

    @staticmethod
    def covers(head_dim: int, key_bits: int, value_bits: int) -> bool:
        return head_dim in (128, 96, 64) and key_bits in (2, 3, 4) and 1 <= value_bits <= 4

    # -------------------------------------------------------------- storage

    def append(self, keys: torch.Tensor, values: torch.Tensor) -> None:
        """Compress (B, H, S, d) keys/values into the pages (quashkv/engine.py:145-172)."""
        dev = N.require_gpu(keys, values, what="PagedQuashKVEngine.append")
        if keys.dim() != 4 or keys.shape != values.shape or keys.shape[-1] != self.head_dim:
            raise ValueError(
                f"Expected keys and values of shape (batch, n_heads, seq_len, {self.head_dim}); "
                f"got {tuple(keys.shape)} and {tuple(values.shape)}")
        if self.value_quantizer.Pi.device != dev:
            self.to(dev)
        B, H, S, d = keys.shape
        st = self._paged
        if st is not None and (st.B, st.H) != (B, H):
            if self._total_tokens:
                raise ValueError(f"append shape (B={B}, H={H}) does not match the cache "
                                 f"(B={st.B}, H={st.H})")
            st = self._paged = None  # empty (cleared): any shape, as the reference allows
        if st is None:
            pages = self.initial_pages or B * max(1, -(-S // self.page_tokens))
            st = self._paged = PagedKVStore(B, H, d, self.key_bits - 1, self.value_bits, pages,
                                            dev, self.page_tokens)
        t0 = self._total_tokens
        st.ensure(t0 + S)
        if S > 0 and not self._append_paged(keys, values, t0):
            self._append_scatter(keys, values, t0)
        self._blocks.append((t0, S))
        self._total_tokens += S

    def _append_paged(self, keys: torch.Tensor, values: torch.Tensor, t0: int) -> bool:
        """bf16, fp16 or fp32 K/V straight into the pages (qkv_paged_store_append_kv)."""
        if (keys.dtype not in (torch.bfloat16, torch.float16, torch.float32)
                or values.dtype != keys.dtype):
            return False
        B, H, S, d = keys.shape
        kq, vq = self.key_quantizer, self.value_quantizer
        mq = kq.mse_quantizer
        if self._host_tables is None:
            self._host_tables = (N.HostFloats(mq.codebook.centroids_host),
                                 N.HostFloats(mq.codebook.boundaries_host),
                                 N.HostFloats(vq.codebook.boundaries_host))
        kc, kb, vb = self._host_tables
        st = self._paged
        k, v = keys.contiguous(), values.contiguous()
        dt = N.dtype_code(k.dtype)
        stream = N.stream(k.device)
        L = N.lib()
        # keys and values in one call (one launch for a decode step's tokens)
        N.check(L.qkv_paged_store_append_kv(
            dt, k.data_ptr(), v.data_ptr(), B, H, S, d, kq.mse_bits, vq.bits, mq.Pi.data_ptr(),
            kq.S.data_ptr(), vq.Pi.data_ptr(), kc.ptr, kb.ptr, vb.ptr, st.kpool.data_ptr(),
            st.knorm.data_ptr(), st.vpool.data_ptr(), st.vnorm.data_ptr(), st.table.data_ptr(),
            st.pages_per_seq, st.pt, st.num_pages, t0, stream))
        return True

    def _append_scatter(self, keys: torch.Tensor, values: torch.Tensor, t0: int) -> None:
        """Other dtypes: the generic compress kernel into a contiguous store at
        the pages' token offset, then rows and tiles into the pages."""
        B, H, S, d = keys.shape
        kq, vq = self.key_quantizer, self.value_quantizer
        mq = kq.mse_quantizer
        dev = keys.device
        n = B * H * S
        kc = torch.empty(n, d, dtype=torch.uint8, device=dev)
        kb = torch.empty(n, d, dtype=torch.uint8, device=dev)
        vc = torch.empty(n, d, dtype=torch.uint8, device=dev)
        kn = torch.empty(n, dtype=torch.float32, device=dev)
        vn = torch.empty(n, dtype=torch.float32, device=dev)
        compress_into(N.QKV_MODE_IP, keys.reshape(n, d), mq.Pi, mq.codebook.boundaries,
                      mq.codebook.centroids, kq.mse_bits, kq.S, kc, kb, kn, packed=False)
        compress_into(N.QKV_MODE_MSE, values.reshape(n, d), vq.Pi, vq.codebook.boundaries,
                      vq.codebook.centroids, vq.bits, None, vc, None, vn, packed=False)
        st = self._paged
        o = t0 % st.pt
        tmp = KVStore(B, H, d, st.mbits, st.vbits, o + S, dev)
        tmp.knorm[:, :, o:o + S].copy_(kn.view(B, H, S))
        tmp.vnorm[:, :, o:o + S].copy_(vn.view(B, H, S))
        tmp.write_codes(o, S, kc, kb, vc)
        st.write_from(tmp, t0, S)

    @property
    def _store(self):
        """Tokens so far as a contiguous store (gathered from the pages), for
        code that reads codes back; None before the first append."""
        if self._paged is None:
            return None
        return self._paged.gather(self._total_tokens)

    @_store.setter
    def _store(self, value) -> None:
        if value is not None:
            raise AttributeError("PagedQuashKVEngine keeps its tokens in pages")

    @property
    def paged_store(self) -> Optional[PagedKVStore]:
        return self._paged

    @property
    def _cache(self) -> list:
        st = self._store
        out = []
        for t0, s in self._blocks:
            kc, kb, vc = st.read_codes(t0, s)
            sl = slice(t0, t0 + s)
            if self.pack_storage:
                kc, kb, vc = pack_bits(kc, self.key_bits - 1), pack_bits(kb, 1), \
                    pack_bits(vc, self.value_bits)
            out.append(CompressedKVBlock(
                mse_indices=kc, qjl_signs=kb, key_norms=st.knorm[:, :, sl],
                val_indices=vc, val_norms=st.vnorm[:, :, sl], seq_len=s,
                packed=bool(self.pack_storage)))
        return out

    def _heads(self) -> tuple[int, int]:
        return self._paged.B, self._paged.H

    def clear(self) -> None:
        if self._paged is not None:
            self._paged.release()
        super().clear()

    # ------------------------------------------------------------ attention

    def attention(self, queries: torch.Tensor, scale: Optional[float] = None,
                  causal: bool = False, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """Attention of (B, Hq, Q, d) queries over every cached token
        (quashkv/engine.py:204-299), Hq a multiple of the kv heads."""
        if not self._blocks or self._total_tokens == 0:
            raise ValueError("No compressed KV blocks in cache. Call append() first.")
        st = self._paged
        dev = N.require_gpu(queries, what="PagedQuashKVEngine.attention")
        B, Hq, Q, d = queries.shape
        if B != st.B or d != self.head_dim or Hq % st.H != 0:
            raise ValueError(f"queries {tuple(queries.shape)} do not match the cache "
                             f"(B={st.B}, kv heads={st.H}, head_dim={self.head_dim})")
        if scale is None:
            scale = 1.0 / math.sqrt(d)
        T = self._total_tokens
        kq, vq = self.key_quantizer, self.value_quantizer
        mq = kq.mse_quantizer
        L = N.lib()
        splits = L.qkv_attention_splits(B, Hq, st.H, Q, d, T)
        need = L.qkv_attention_workspace_bytes(B, Hq, st.H, Q, d, splits)
        if self._workspace is None or self._workspace.numel() < need \
                or self._workspace.device != dev:
            self._workspace = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
        q = queries.contiguous()
        if q.dtype not in (torch.float32, torch.float16, torch.bfloat16):
            q = q.float()
        kc = N.HostFloats(mq.codebook.centroids_host)
        vc = N.HostFloats(vq.codebook.centroids_host)
        out = torch.empty(B, Hq, Q, d, dtype=out_dtype, device=dev)
        N.check(L.qkv_paged_decode_attention(
            q.data_ptr(), N.dtype_code(q.dtype), st.kpool.data_ptr(), st.knorm.data_ptr(),
            st.vpool.data_ptr(), st.vnorm.data_ptr(), st.table.data_ptr(), st.pages_per_seq, st.pt,
            st.num_pages, T, B, Hq, st.H, Q, d, st.mbits, st.vbits, mq.Pi.data_ptr(), kc.ptr, vc.ptr,
            kq.S.data_ptr(), float(kq.qjl_scale), float(scale), 1 if causal else 0,
            out.data_ptr(), N.dtype_code(out_dtype), self._workspace.data_ptr(),
            self._workspace.numel(), splits, N.stream(dev)))
        return out

    # -------------------------------------------------------------- metrics

    def pool_bytes(self) -> int:
        """Device bytes of the page pool."""
        return 0 if self._paged is None else self._paged.nbytes()

    def to(self, device) -> "PagedQuashKVEngine":
        self.device = torch.device(device)
        self.key_quantizer.to(device)
        self.value_quantizer.to(device)
        if self._paged is not None:
            self._paged.to(device)
        self._workspace = None
        return self

    def __repr__(self) -> str:
        pages = 0 if self._paged is None else self._paged.num_pages
        return (f"PagedQuashKVEngine(head_dim={self.head_dim}, key_bits={self.key_bits}, "
                f"value_bits={self.value_bits}, cached_tokens={self._total_tokens}, "
                f"pages={pages}, device={self.device})")


def compressed_blocks(engine: QuashKVEngine) -> list[CompressedBlock]:
    """The engine's blocks as unpacked CompressedBlocks (quashkv/integrations/
    vllm_backend.py:116-129)."""
    out = []
    for blk in engine._cache:
        mse, qjl, val = engine._unpack_block(blk)
        out.append(CompressedBlock(mse_indices=mse, qjl_signs=qjl, key_norms=blk.key_norms,
                                   val_indices=val, val_norms=blk.val_norms,
                                   seq_len=blk.seq_len))
    return out
