"""TurboQuant maximum-inner-product search index (quashkv/nn_search/index.py).

Vectors are compressed with the inner-product quantizer (``bits - 1``-bit MSE
codes + 1-bit QJL signs) into one K row each -- the key-store layout of the
engine, (bits) * dim / 8 bytes -- plus an fp32 norm.  ``search`` runs the
integer-MFMA scoring and a streaming top-k on the GPU (qkv_mips_search); the
(M, N) score matrix the reference materialises is never formed.
"""

from __future__ import annotations

from typing import Optional

import torch

from .. import _native as N
from ..quantizer import InnerProductQuantizer, _default_device, compress_into


class QuashIndex:
    """Approximate MIPS over TurboQuant codes (quashkv/nn_search/index.py:21-252)."""

    def __init__(self, dim: int, bits: int = 3, seed: int = 42, device=None,
                 pack_storage: bool = False):
        self.dim = dim
        self.bits = bits
        self.seed = seed
        self.device = _default_device(device)
        self.pack_storage = pack_storage
        self.quantizer = InnerProductQuantizer(d=dim, total_bits=bits, seed=seed,
                                               device=self.device)
        self._rows: Optional[torch.Tensor] = None    # (capacity, bits * dim / 8) uint8
        self._norms: Optional[torch.Tensor] = None   # (capacity,) fp32
        self._n_vectors = 0
        self._tables = None
        self._workspace: Optional[torch.Tensor] = None

    # ------------------------------------------------------------ properties

    @property
    def n_vectors(self) -> int:
        return self._n_vectors

    def __len__(self) -> int:
        return self._n_vectors

    @property
    def _row_bytes(self) -> int:
        return self.bits * self.dim // 8

    # ------------------------------------------------------------------ add

    def _ensure(self, needed: int, dev: torch.device) -> None:
        cap = 0 if self._rows is None else self._rows.shape[0]
        if needed <= cap and self._rows.device == dev:
            return
        new_cap = max(64, needed, 2 * cap)
        new_cap = (new_cap + 63) // 64 * 64
        rows = torch.zeros(new_cap, self._row_bytes, dtype=torch.uint8, device=dev)
        norms = torch.zeros(new_cap, dtype=torch.float32, device=dev)
        if self._n_vectors:
            rows[:self._n_vectors].copy_(self._rows[:self._n_vectors])
            norms[:self._n_vectors].copy_(self._norms[:self._n_vectors])
        self._rows, self._norms = rows, norms

    def add(self, vectors: torch.Tensor) -> None:
        """Compress (N, dim) vectors into the index (quashkv/nn_search/index.py:77-107)."""
        if vectors.dim() != 2 or vectors.shape[1] != self.dim:
            raise ValueError(
                f"Expected (N, {self.dim}) tensor, got shape {tuple(vectors.shape)}")
        dev = N.require_gpu(vectors, what="QuashIndex.add")
        if self.quantizer.S.device != dev:
            self.quantizer.to(dev)
            self.device = dev
        n = vectors.shape[0]
        t0 = self._n_vectors
        self._ensure(t0 + n, dev)
        if n == 0:
            return
        q = self.quantizer
        mq = q.mse_quantizer
        x = vectors.contiguous()
        L = N.lib()
        stream = N.stream(dev)
        done = False
        if (x.dtype in (torch.bfloat16, torch.float16, torch.float32) and self.dim in (64, 96, 128)
                and 2 <= self.bits <= 4):
            kc, kb, _ = self._host_tables()
            st = L.qkv_store_append(N.dtype_code(x.dtype), x.data_ptr(), None, 1, n, self.dim,
                                    q.mse_bits, 1, mq.Pi.data_ptr(), q.S.data_ptr(), kc.ptr,
                                    kb.ptr, None, self._rows.data_ptr(), self._norms.data_ptr(),
                                    None, None, self._rows.shape[0], t0, stream)
            if st != N.QKV_E_UNSUPPORTED:
                N.check(st)
                done = True
        if not done:
            codes = torch.empty(n, self.dim, dtype=torch.uint8, device=dev)
            qjl = torch.empty_like(codes)
            compress_into(N.QKV_MODE_IP, x, mq.Pi, mq.codebook.boundaries, mq.codebook.centroids,
                          q.mse_bits, q.S, codes, qjl, self._norms[t0:], packed=False)
            N.check(L.qkv_kplanes_pack(codes.data_ptr(), qjl.data_ptr(), n, self.dim, q.mse_bits,
                                       self._rows[t0:].data_ptr(), self._row_bytes, n, n,
                                       stream))
        self._n_vectors += n

    def _host_tables(self):
        if self._tables is None:
            cb = self.quantizer.mse_quantizer.codebook
            self._tables = (N.HostFloats(cb.centroids_host), N.HostFloats(cb.boundaries_host),
                            None)
        return self._tables

    # --------------------------------------------------------------- search

    def _get_unpacked(self) -> tuple[torch.Tensor, torch.Tensor]:
        """(mse codes, qjl bits) as (N, dim) uint8."""
        n, d = self._n_vectors, self.dim
        mse = torch.empty(n, d, dtype=torch.uint8, device=self._rows.device)
        qjl = torch.empty_like(mse)
        if n:
            N.check(N.lib().qkv_kplanes_unpack(self._rows.data_ptr(), self._row_bytes, n, d,
                                               self.bits - 1, n, n, mse.data_ptr(),
                                               qjl.data_ptr(), N.stream(mse.device)))
        return mse, qjl

    def search(self, queries: torch.Tensor, k: int = 10):
        """(scores, indices) of the k largest approximate inner products per query,
        descending (quashkv/nn_search/index.py:121-163; ties: lower index first)."""
        if self._n_vectors == 0:
            raise ValueError("Index is empty. Call add() first.")
        k = min(k, self._n_vectors)
        dev = N.require_gpu(queries, what="QuashIndex.search")
        if queries.dim() != 2 or queries.shape[1] != self.dim:
            raise ValueError(
                f"Expected (M, {self.dim}) queries, got shape {tuple(queries.shape)}")
        q = queries.contiguous()
        if q.dtype not in (torch.float32, torch.float16, torch.bfloat16):
            q = q.float()
        M = q.shape[0]
        scores = torch.empty(M, k, dtype=torch.float32, device=dev)
        indices = torch.empty(M, k, dtype=torch.int64, device=dev)
        if M == 0:
            return torch.return_types.topk((scores, indices))
        quant = self.quantizer
        mq = quant.mse_quantizer
        L = N.lib()
        need = L.qkv_mips_workspace_bytes(M, self.dim, self.bits - 1, k, self._n_vectors)
        if need < 0:
            raise ValueError(f"QuashIndex.search: unsupported dim {self.dim} / bits {self.bits}")
        if self._workspace is None or self._workspace.numel() < need \
                or self._workspace.device != dev:
            self._workspace = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
        kc, _, _ = self._host_tables()
        pi, s = N.dense(mq.Pi, quant.S)
        N.check(L.qkv_mips_search(q.data_ptr(), N.dtype_code(q.dtype), M, self.dim,
                                  self.bits - 1, pi.data_ptr(), s.data_ptr(), kc.ptr,
                                  float(quant.qjl_scale), self._rows.data_ptr(),
                                  self._norms.data_ptr(), self._n_vectors, k,
                                  scores.data_ptr(), indices.data_ptr(),
                                  self._workspace.data_ptr(), self._workspace.numel(),
                                  N.stream(dev)))
        return torch.return_types.topk((scores, indices))

    # ----------------------------------------------------- ground truth etc.

    @staticmethod
    def brute_force(queries: torch.Tensor, database: torch.Tensor, k: int = 10):
        """Exact MIPS for ground truth (quashkv/nn_search/index.py:169-188)."""
        k = min(k, database.shape[0])
        return torch.topk(queries @ database.T, k, dim=1)

    def recall_at_k(self, queries: torch.Tensor, database: torch.Tensor, k: int = 10) -> float:
        """Mean recall@k against exact search (quashkv/nn_search/index.py:190-219)."""
        _, approx = self.search(queries, k)
        _, exact = self.brute_force(queries, database, k)
        m = queries.shape[0]
        hits = 0
        a, e = approx.cpu().tolist(), exact.cpu().tolist()
        for i in range(m):
            hits += len(set(a[i]) & set(e[i]))
        return hits / (m * k)

    # ---------------------------------------------------------------- stats

    def memory_bytes(self) -> int:
        """Bytes of the reference's storage for these codes
        (quashkv/nn_search/index.py:225-232): pack_bits rows when pack_storage,
        else one byte per code, plus fp32 norms."""
        if self._n_vectors == 0:
            return 0
        d = self.dim
        if self.pack_storage:
            row = N.packed_row_bytes(d, self.bits - 1) + N.packed_row_bytes(d, 1)
        else:
            row = 2 * d
        return self._n_vectors * (row + 4)

    def compression_ratio(self, original_dtype: torch.dtype = torch.float32) -> float:
        if self._n_vectors == 0:
            return 1.0
        element_bytes = torch.finfo(original_dtype).bits // 8
        original = self._n_vectors * self.dim * element_bytes
        compressed = self.memory_bytes()
        return original / compressed if compressed > 0 else float("inf")

    def reset(self) -> None:
        self._rows = self._norms = None
        self._n_vectors = 0

    def __repr__(self) -> str:
        return (f"QuashIndex(dim={self.dim}, bits={self.bits}, n_vectors={self._n_vectors}, "
                f"pack_storage={self.pack_storage}, device={self.device})")
