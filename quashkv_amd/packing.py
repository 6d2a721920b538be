"""Bit-packing of low-bit codes on the GPU (layout of quashkv/packing.py:1-14).

1-bit: 8 codes per byte; 2-bit: 4 per byte; 4-bit: 2 per byte (low nibble
first); 3-bit: 8 codes form a little-endian 24-bit word stored as 3 bytes.
Packing is along the last dimension, LSB first; rows are zero-padded to a
whole group; bits = 8 passes the tensor through unchanged.
"""

from __future__ import annotations

import torch

from . import _native as N


def packed_size(d: int, bits: int) -> int:
    """ceil(d * bits / 8) (quashkv/packing.py:162-165).

    This is the reference helper's value; for 3-bit codes the rows that
    pack_bits produces are 3 * ceil(d / 8) bytes (see packed_row_bytes)."""
    return (d * bits + 7) // 8


def packed_row_bytes(d: int, bits: int) -> int:
    """Bytes per row that pack_bits actually produces."""
    return N.packed_row_bytes(d, bits)


def pack_bits(indices: torch.Tensor, bits: int) -> torch.Tensor:
    """Pack uint8 codes (..., d) into (..., packed_row_bytes(d, bits)) bytes
    (quashkv/packing.py:22-94)."""
    if bits == 8:
        return indices
    if bits not in (1, 2, 3, 4):
        raise ValueError(f"Unsupported bits: {bits}")
    dev = N.require_gpu(indices, what="pack_bits")
    *lead, d = indices.shape
    rows = int(torch.Size(lead).numel())
    src = indices.reshape(rows, d).to(torch.uint8).contiguous()
    pb = N.packed_row_bytes(d, bits)
    out = torch.empty(rows, pb, dtype=torch.uint8, device=dev)
    N.check(N.lib().qkv_pack_bits(src.data_ptr(), out.data_ptr(), rows, d, bits, N.stream(dev)))
    return out.reshape(*lead, pb)


def unpack_bits(packed: torch.Tensor, bits: int, d: int) -> torch.Tensor:
    """Unpack (..., P) bytes back into uint8 codes (..., d)
    (quashkv/packing.py:97-159)."""
    if bits == 8:
        return packed
    if bits not in (1, 2, 3, 4):
        raise ValueError(f"Unsupported bits: {bits}")
    dev = N.require_gpu(packed, what="unpack_bits")
    *lead, p = packed.shape
    rows = int(torch.Size(lead).numel())
    src = packed.reshape(rows, p).contiguous()
    out = torch.empty(rows, d, dtype=torch.uint8, device=dev)
    N.check(N.lib().qkv_unpack_bits(src.data_ptr(), p, out.data_ptr(), rows, d, bits,
                                    N.stream(dev)))
    return out.reshape(*lead, d)
