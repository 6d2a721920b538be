"""The engine's compressed KV cache store (device buffers, bit-plane formats).

The reference keeps a Python list of per-append tensors (quashkv/engine.py:
104, 145-172) and re-concatenates them on every attention call
(quashkv/triton_kernels/attention.py:348-352).  Here one preallocated store
per engine holds every appended token in the layouts the decode kernels
stream (C ABI "Cache store formats"):

* ``kst``   (B, H, C, (mbits + 1) d / 8) uint8 -- K rows: MSE bit planes, then
  the QJL plane;
* ``knorm`` (B, H, C) fp32;
* ``vst``   (B, H, C / 32, vbits, d) int32 -- V bit-plane tiles of 32 tokens;
* ``vnorm`` (B, H, C) fp32.

With mixed-precision keys (``kmix = (perm, n_out, ip)``) ``kst`` holds rows
over coordinates permuted outliers first (slot j = rotated channel perm[j]):

* MSE keys ("kmixed", 3/2-bit): planes b0 and b1 of every slot, then b2 and
  the parity b0^b1^b2 of the n_out outlier slots -- 32 + n_out / 4 bytes;
* IP keys ("kipmixed", 2/1-bit MSE stage + QJL): plane b0 and the QJL plane
  of every slot, then b1 of the outlier slots -- 32 + n_out / 8 bytes.

The capacity C is a multiple of 64 and doubles when an append needs room.
Writes and reads go through the store converters of libquashkv_hip.so.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _native as N

ALIGN = 64


def round_capacity(n: int) -> int:
    return max(ALIGN, (n + ALIGN - 1) // ALIGN * ALIGN)


class KVStore:
    def __init__(self, B: int, H: int, d: int, mbits: int, vbits: int, capacity: int,
                 device: torch.device, kmix: Optional[tuple] = None):
        if d % 32 != 0:
            raise ValueError(f"head_dim {d} must be a multiple of 32 for the cache store")
        self.B, self.H, self.d = B, H, d
        self.mbits, self.vbits = mbits, vbits
        self.kmix = None
        if kmix is not None:
            perm, n_out, ip = kmix
            if d != 128 or n_out not in (32, 64):
                raise ValueError("mixed-precision keys need head_dim 128 and 32 or 64 outliers")
            self.kmix = (N.HostInts(perm), int(n_out), bool(ip))
            self.mbits = 2
            self.krb = 32 + (n_out // 8 if ip else n_out // 4)
        else:
            self.krb = (mbits + 1) * d // 8
        self.device = torch.device(device)
        self.capacity = 0
        self.kst = self.knorm = self.vst = self.vnorm = None
        self._alloc(round_capacity(capacity), 0)

    # ----------------------------------------------------------- storage

    def _alloc(self, capacity: int, keep: int) -> None:
        B, H, d, dev = self.B, self.H, self.d, self.device
        kst = torch.zeros(B, H, capacity, self.krb, dtype=torch.uint8, device=dev)
        knorm = torch.zeros(B, H, capacity, dtype=torch.float32, device=dev)
        vst = torch.zeros(B, H, capacity // 32, self.vbits, d, dtype=torch.int32, device=dev)
        vnorm = torch.zeros(B, H, capacity, dtype=torch.float32, device=dev)
        if keep:
            kst[:, :, :keep].copy_(self.kst[:, :, :keep])
            knorm[:, :, :keep].copy_(self.knorm[:, :, :keep])
            nt = (keep + 31) // 32
            vst[:, :, :nt].copy_(self.vst[:, :, :nt])
            vnorm[:, :, :keep].copy_(self.vnorm[:, :, :keep])
        self.kst, self.knorm, self.vst, self.vnorm = kst, knorm, vst, vnorm
        self.capacity = capacity

    def ensure(self, needed: int, keep: int) -> None:
        if needed > self.capacity:
            self._alloc(round_capacity(max(needed, 2 * self.capacity)), keep)

    def to(self, device) -> None:
        self.device = torch.device(device)
        for name in ("kst", "knorm", "vst", "vnorm"):
            setattr(self, name, getattr(self, name).to(self.device))

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.kst, self.knorm, self.vst, self.vnorm))

    # ----------------------------------------------------- code transfers

    def k_row_ptr(self, t0: int) -> int:
        return self.kst.data_ptr() + t0 * self.krb

    def write_codes(self, t0: int, S: int, kcodes: torch.Tensor, kqjl: Optional[torch.Tensor],
                    vcodes: torch.Tensor) -> None:
        """Unpacked uint8 codes (B*H*S, d) of tokens [t0, t0 + S) into the store
        (``kqjl`` None with mixed-precision MSE keys)."""
        L = N.lib()
        n = self.B * self.H * S
        stream = N.stream(self.device)
        if self.kmix is not None:
            perm, n_out, ip = self.kmix
            if ip:
                N.check(L.qkv_kipmixed_pack(kcodes.data_ptr(), kqjl.data_ptr(), n, perm.ptr,
                                            n_out, self.k_row_ptr(t0), S, self.capacity, stream))
            else:
                N.check(L.qkv_kmixed_pack(kcodes.data_ptr(), n, perm.ptr, n_out,
                                          self.k_row_ptr(t0), S, self.capacity, stream))
        else:
            N.check(L.qkv_kplanes_pack(kcodes.data_ptr(), kqjl.data_ptr(), n, self.d, self.mbits,
                                       self.k_row_ptr(t0), self.krb, S, self.capacity, stream))
        N.check(L.qkv_vtiles_pack(vcodes.data_ptr(), self.B * self.H, S, self.d, self.vbits,
                                  self.vst.data_ptr(), self.capacity // 32, t0, stream))

    def read_codes(self, t0: int, S: int):
        """(kcodes, kqjl, vcodes) of tokens [t0, t0 + S) as (B, H, S, d) uint8
        (kqjl None with mixed-precision MSE keys)."""
        L = N.lib()
        B, H, d = self.B, self.H, self.d
        kc = torch.empty(B, H, S, d, dtype=torch.uint8, device=self.device)
        kq = torch.empty_like(kc) if self.kmix is None or self.kmix[2] else None
        vc = torch.empty_like(kc)
        if S == 0:
            return kc, kq, vc
        stream = N.stream(self.device)
        if self.kmix is not None:
            perm, n_out, ip = self.kmix
            if ip:
                N.check(L.qkv_kipmixed_unpack(self.k_row_ptr(t0), B * H * S, perm.ptr, n_out, S,
                                              self.capacity, kc.data_ptr(), kq.data_ptr(),
                                              stream))
            else:
                N.check(L.qkv_kmixed_unpack(self.k_row_ptr(t0), B * H * S, perm.ptr, n_out, S,
                                            self.capacity, kc.data_ptr(), stream))
        else:
            N.check(L.qkv_kplanes_unpack(self.k_row_ptr(t0), self.krb, B * H * S, d, self.mbits,
                                         S, self.capacity, kc.data_ptr(), kq.data_ptr(), stream))
        N.check(L.qkv_vtiles_unpack(self.vst.data_ptr(), B * H, S, d, self.vbits,
                                    self.capacity // 32, t0, vc.data_ptr(), stream))
        return kc, kq, vc


def store_from_codes(kcodes: torch.Tensor, kqjl: torch.Tensor, knorm: torch.Tensor,
                     vcodes: torch.Tensor, vnorm: torch.Tensor, mbits: int, vbits: int,
                     capacity: Optional[int] = None) -> KVStore:
    """Build a store from unpacked (B, H, T, d) codes and (B, H, T) norms."""
    B, H, T, d = kcodes.shape
    st = KVStore(B, H, d, mbits, vbits, capacity or T, kcodes.device)
    st.knorm[:, :, :T].copy_(knorm)
    st.vnorm[:, :, :T].copy_(vnorm)
    if T:
        st.write_codes(0, T, kcodes.reshape(-1, d).to(torch.uint8).contiguous(),
                       kqjl.reshape(-1, d).to(torch.uint8).contiguous(),
                       vcodes.reshape(-1, d).to(torch.uint8).contiguous())
    return st
