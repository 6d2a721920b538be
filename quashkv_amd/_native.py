"""ctypes boundary to libquashkv_hip.so (the C ABI in include/quashkv_amd.h).

The Python layer owns every allocation (outputs and workspaces are torch
tensors on the GPU) and passes raw device pointers plus the current HIP
stream.  There is exactly one execution path: the HIP kernels.  If the
library is missing, or a tensor is not on the GPU, the call raises -- the
package has no CPU fallback.
"""

from __future__ import annotations

import ctypes
import os
import weakref
from typing import Optional

import torch  # loads torch's HIP runtime first; the library binds to the same one

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libquashkv_hip.so")
_lib: Optional[ctypes.CDLL] = None

QKV_OK, QKV_E_INVALID, QKV_E_UNSUPPORTED, QKV_E_HIP = 0, 1, 2, 3
QKV_F32, QKV_F16, QKV_BF16 = 0, 1, 2
QKV_MODE_MSE, QKV_MODE_IP = 0, 1
QKV_FMT_UNPACKED, QKV_FMT_PACKED, QKV_FMT_KPLANES, QKV_FMT_VTILES = 0, 1, 2, 3
QKV_FLAG_PACKED, QKV_FLAG_PRE_ROTATED = 1, 2
NOALLOC_SCRATCH_BYTES = 16 << 20  # QKV_NOALLOC_SCRATCH_BYTES

_DTYPE = {torch.float32: QKV_F32, torch.float16: QKV_F16, torch.bfloat16: QKV_BF16}

_i32, _i64, _f32, _p = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p

# name -> (restype, argtypes); mirrors include/quashkv_amd.h
_SIGS = {
    "qkv_abi_version": (_i32, []),
    "qkv_last_error": (ctypes.c_char_p, []),
    "qkv_packed_row_bytes": (_i64, [_i32, _i32]),
    "qkv_pack_bits": (_i32, [_p, _p, _i64, _i32, _i32, _p]),
    "qkv_unpack_bits": (_i32, [_p, _i64, _p, _i64, _i32, _i32, _p]),
    "qkv_quantize": (_i32, [_p, _i64, _p, _i32, _i32, _p, _p]),
    "qkv_dequantize": (_i32, [_p, _i64, _p, _i32, _p, _p]),
    "qkv_ip_dot": (_i32, [_p, _p, _p, _p, _i64, _i32, _p, _i32, _p, _f32, _p, _p]),
    "qkv_compress": (_i32, [_i32, _i32, _i32, _p, _i64, _i32, _p, _p, _p, _i32, _p,
                            _p, _p, _p, _i64, _i64, _p]),
    "qkv_decompress": (_i32, [_i32, _i32, _p, _p, _p, _i64, _i32, _i32, _p, _p, _p, _f32,
                              _i64, _i64, _p, _i32, _p]),
    "qkv_compress_mfma": (_i32, [_i32, _i32, _p, _i64, _i32, _p, _p, _p, _i32, _p, _p, _p, _p,
                                 _i64, _i64, _p]),
    "qkv_kplanes_row_bytes": (_i64, [_i32, _i32, _i32]),
    "qkv_vtiles_bytes": (_i64, [_i32, _i32, _i64]),
    "qkv_kplanes_pack": (_i32, [_p, _p, _i64, _i32, _i32, _p, _i64, _i64, _i64, _p]),
    "qkv_kplanes_unpack": (_i32, [_p, _i64, _i64, _i32, _i32, _i64, _i64, _p, _p, _p]),
    "qkv_vtiles_pack": (_i32, [_p, _i64, _i64, _i32, _i32, _p, _i64, _i64, _p]),
    "qkv_vtiles_unpack": (_i32, [_p, _i64, _i64, _i32, _i32, _i64, _i64, _p, _p]),
    "qkv_store_append": (_i32, [_i32, _p, _p, _i64, _i64, _i32, _i32, _i32, _p, _p, _p, _p, _p,
                                _p, _p, _p, _p, _i64, _i64, _p]),
    "qkv_compress_mixed": (_i32, [_i32, _i32, _i32, _p, _i64, _i32, _p, _p, _p, _p, _i32, _p, _p,
                                  _i32, _p, _p, _p, _p, _i64, _i64, _p]),
    "qkv_decompress_mixed": (_i32, [_i32, _p, _p, _p, _i64, _i32, _p, _p, _i32, _p, _i32, _p, _p,
                                    _f32, _i64, _i64, _p, _i32, _p]),
    "qkv_decode_attention_layers": (_i32, [_i32, _p, _i32, _p, _p, _p, _p, _i64, _i64, _i32,
                                           _i32, _i32, _i32, _i32, _i32, _i32, _p, _p, _p, _p,
                                           _f32, _f32, _i32, _p, _i32, _p, _i64, _i32, _p]),
    "qkv_kmixed_pack": (_i32, [_p, _i64, _p, _i32, _p, _i64, _i64, _p]),
    "qkv_kmixed_unpack": (_i32, [_p, _i64, _p, _i32, _i64, _i64, _p, _p]),
    "qkv_store_append_kmixed": (_i32, [_i32, _p, _i64, _i64, _i32, _p, _i32, _p, _p, _p, _p,
                                       _i64, _i64, _p]),
    "qkv_store_append_layers": (_i32, [_i32, _i32, _p, _p, _i64, _i64, _i32, _i32, _i32, _p, _p,
                                       _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _p]),
    "qkv_store_append_rotated": (_i32, [_p, _p, _p, _p, _i64, _i64, _i32, _i32, _i32, _p, _p, _p,
                                        _p, _p, _p, _p, _p, _i64, _i64, _p]),
    "qkv_store_append_kmixed_rotated": (_i32, [_p, _p, _i64, _i64, _i32, _i32, _p, _p, _p, _p,
                                               _i64, _i64, _p]),
    "qkv_kipmixed_pack": (_i32, [_p, _p, _i64, _p, _i32, _p, _i64, _i64, _p]),
    "qkv_kipmixed_unpack": (_i32, [_p, _i64, _p, _i32, _i64, _i64, _p, _p, _p]),
    "qkv_store_append_kipmixed": (_i32, [_i32, _p, _i64, _i64, _i32, _p, _p, _i32, _p, _p, _p,
                                         _p, _p, _p, _i64, _i64, _p]),
    "qkv_store_append_kmixed_kv": (_i32, [_i32, _p, _p, _i64, _i64, _i32, _p, _p, _i32, _i32, _p,
                                          _p, _p, _p, _p, _p, _i32, _p, _p, _p, _p, _i64, _i64,
                                          _p]),
    "qkv_store_append_kipmixed_rotated": (_i32, [_p, _p, _i64, _i64, _i32, _p, _i32, _p, _p, _p,
                                                 _p, _p, _p, _i64, _i64, _p]),
    "qkv_decode_attention_kipmixed": (_i32, [_p, _i32, _p, _p, _p, _p, _i64, _i64, _i32, _i32,
                                             _i32, _i32, _i32, _i32, _p, _p, _f32, _i32, _p, _p,
                                             _p, _p, _f32, _i32, _p, _i32, _p, _i64, _i32, _p]),
    "qkv_decode_attention_kmixed": (_i32, [_p, _i32, _p, _p, _p, _p, _i64, _i64, _i32, _i32,
                                           _i32, _i32, _i32, _i32, _p, _i32, _p, _p, _p, _p,
                                           _f32, _i32, _p, _i32, _p, _i64, _i32, _p]),
    "qkv_mips_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32, _i64]),
    "qkv_mips_search": (_i32, [_p, _i32, _i32, _i32, _i32, _p, _p, _p, _f32, _p, _p, _i64, _i32,
                               _p, _p, _p, _i64, _p]),
    "qkv_attention_splits": (_i32, [_i32, _i32, _i32, _i32, _i32, _i64]),
    "qkv_attention_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "qkv_attention_path": (_i32, [_i32, _i32, _i32, _p, _p, _i64, _i64, _i32]),
    "qkv_decode_attention": (_i32, [_p, _i32, _p, _p, _p, _p, _i64, _i64, _i32, _i32, _i32,
                                    _i32, _i32, _i32, _i32, _p, _p, _p, _p, _f32, _f32, _i32,
                                    _p, _i32, _p, _i64, _i32, _p]),
    "qkv_decode_attention_ranges": (_i32, [_p, _i32, _p, _p, _p, _p, _i64, _i64, _p, _p, _i64,
                                           _i32, _i32, _i32, _i32, _i32, _i32, _i32, _p, _p, _p,
                                           _p, _f32, _f32, _i32, _p, _i32, _p, _i64, _i32, _p]),
    "qkv_decode_attention_noalloc": (_i32, [_p, _i32, _p, _p, _p, _p, _i64, _i64, _i32, _i32,
                                            _i32, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _f32,
                                            _f32, _i32, _p, _i32, _i32, _p]),
    "qkv_attention_prepare": (_i32, [_p, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _p,
                                     _p, _p, _p, _f32, _p, _i64, _i32, _p]),
    "qkv_attention_partial": (_i32, [_p, _p, _p, _p, _i64, _i64, _i32, _i32, _i32, _i32, _i32,
                                     _i32, _i32, _p, _p, _f32, _i32, _p, _i64, _i32, _p]),
    "qkv_attention_combine": (_i32, [_i32, _i32, _i32, _i32, _i32, _p, _p, _i32, _p, _i64, _i32,
                                     _p]),
    "qkv_attention_run": (_i32, [_p, _p, _p, _p, _i64, _i64, _i32, _i32, _i32, _i32, _i32,
                                 _i32, _i32, _p, _p, _p, _f32, _i32, _p, _i32, _p, _i64, _i32,
                                 _p]),
    "qkv_paged_store_append": (_i32, [_i32, _p, _p, _i32, _i32, _i64, _i32, _i32, _i32, _p, _p,
                                      _p, _p, _p, _p, _p, _p, _p, _p, _i32, _i32, _i32, _i64,
                                      _p]),
    "qkv_paged_store_append_kv": (_i32, [_i32, _p, _p, _i32, _i32, _i64, _i32, _i32, _i32, _p, _p,
                                         _p, _p, _p, _p, _p, _p, _p, _p, _p, _i32, _i32, _i32,
                                         _i64, _p]),
    "qkv_paged_decode_attention": (_i32, [_p, _i32, _p, _p, _p, _p, _p, _i32, _i32, _i32, _i64,
                                          _i32,
                                          _i32, _i32, _i32, _i32, _i32, _i32, _p, _p, _p, _p,
                                          _f32, _f32, _i32, _p, _i32, _p, _i64, _i32, _p]),
    "qkv_hbm_read_probe": (_i32, [_p, _i64, _p, _i32, _i32, _i32, _p]),
    "qkv_paged_decode_attention_layers": (_i32, [_i32, _p, _i32, _p, _p, _p, _p, _p, _i32, _i32,
                                                 _i32, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                                 _p, _p, _p, _p, _f32, _f32, _i32, _p, _i32, _p,
                                                 _i64, _i32, _p]),
}

EXPORTED = tuple(_SIGS)


class NativeLibraryMissing(ImportError):
    pass


def library_path() -> str:
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raise if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise NativeLibraryMissing(
                f"quashkv_amd: {_LIB_PATH} is not built; run `python -m quashkv_amd.build` "
                "(or __graft_entry__.build()).  There is no CPU fallback.")
        handle = ctypes.CDLL(_LIB_PATH, mode=ctypes.RTLD_GLOBAL)
        for name, (res, args) in _SIGS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(status: int) -> None:
    if status == QKV_OK:
        return
    msg = lib().qkv_last_error().decode(errors="replace")
    if status in (QKV_E_INVALID, QKV_E_UNSUPPORTED):
        raise ValueError(msg)
    raise RuntimeError(f"quashkv_amd HIP failure: {msg}")


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE[dt]
    except KeyError:
        raise ValueError(f"unsupported dtype {dt}; expected float32, float16 or bfloat16")


def require_gpu(*tensors: torch.Tensor, what: str = "quashkv_amd") -> torch.device:
    """All tensors must live on the same HIP device.  No CPU fallback exists."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                f"{what} runs on the GPU (HIP); got a tensor on {t.device}. "
                "Move inputs to the GPU (e.g. .to('cuda')); there is no CPU path.")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"{what}: tensors on different devices ({dev} vs {t.device})")
    return dev


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def extent(t: torch.Tensor) -> int:
    """Bytes addressable from t.data_ptr() to the end of t's storage."""
    st = t.untyped_storage()
    return st.nbytes() - (t.data_ptr() - st.data_ptr())


def require_extent(t: Optional[torch.Tensor], nbytes: int, what: str) -> None:
    """Host-side bounds check before a kernel writes or reads `nbytes` bytes
    from t's first element (kernels address raw pointers)."""
    if t is not None and nbytes > extent(t):
        raise ValueError(f"{what}: kernel would touch {nbytes} bytes but the buffer has "
                         f"{extent(t)} from its first element")


def grouped_rows(n: int, seq: int, gstride: int) -> int:
    """Rows spanned by n vectors under grouped-row addressing."""
    if n <= 0:
        return 0
    last = n - 1
    return (last // seq) * gstride + (last % seq) + 1


def dense(*tensors: Optional[torch.Tensor]):
    """Row-major fp32 copies (when needed) of parameter tensors whose raw
    pointers the kernels read as dense arrays (Pi, S, codebook tables).
    torch.linalg.qr hands back a column-major Q, so a strided Pi is common."""
    out = []
    for t in tensors:
        if t is not None:
            if t.dtype != torch.float32:
                t = t.float()
            t = t.contiguous()
        out.append(t)
    return out


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream(device: torch.device) -> int:
    """The current HIP stream of ``device`` as an integer handle (the raw
    query skips building a torch Stream object on every kernel call)."""
    if _RAW_STREAM is not None:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        return _RAW_STREAM(idx)
    return torch.cuda.current_stream(device).cuda_stream


class HostFloats:
    """A small fp32 table as a ctypes array (codebook centroids passed by
    value to the attention entry points)."""

    def __init__(self, values):
        vals = [float(v) for v in values]
        self.n = len(vals)
        self.arr = (ctypes.c_float * max(self.n, 1))(*vals)

    @property
    def ptr(self) -> int:
        return ctypes.addressof(self.arr)


_HOST_TABLES: dict = {}


def host_table(t: torch.Tensor) -> HostFloats:
    """A host copy of a small device table (codebook centroids / boundaries),
    cached per tensor object: the first use of a table costs one
    device-to-host copy, later calls with the same tensor none.

    An entry holds a weak reference to the tensor it was made from and the
    tensor's version counter (shared by its views, bumped by every in-place
    write); it is used only while that same tensor is alive and unmodified,
    and dropped when the tensor is freed.  A table that is freed and replaced
    by another at the same address is therefore copied afresh."""
    key = id(t)
    ent = _HOST_TABLES.get(key)
    if ent is not None:
        ref, version, h = ent
        if ref() is t and version == t._version:
            return h
    h = HostFloats(t.detach().float().cpu().reshape(-1).tolist())

    def _drop(r, key=key):
        e = _HOST_TABLES.get(key)
        if e is not None and e[0] is r:
            del _HOST_TABLES[key]

    _HOST_TABLES[key] = (weakref.ref(t, _drop), t._version, h)
    return h


class HostInts:
    """A small int32 table as a ctypes array (passed by value, like HostFloats)."""

    def __init__(self, values):
        vals = [int(v) for v in values]
        self.n = len(vals)
        self.arr = (ctypes.c_int32 * max(self.n, 1))(*vals)

    @property
    def ptr(self) -> int:
        return ctypes.addressof(self.arr)


def ptr_array(ptrs) -> "ctypes.Array":
    """Device pointers (ints) as a host array of void* (per-layer arguments)."""
    return (ctypes.c_void_p * max(len(ptrs), 1))(*[ctypes.c_void_p(int(x)) for x in ptrs])


def packed_row_bytes(d: int, bits: int) -> int:
    if bits == 8:
        return d
    if bits == 3:
        return 3 * ((d + 7) // 8)
    if bits in (1, 2, 4):
        return (d * bits + 7) // 8
    raise ValueError(f"Unsupported bits: {bits}")
