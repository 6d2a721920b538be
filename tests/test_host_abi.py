"""CPU tests: the C ABI library loads and exports every declared symbol, host
validation rejects bad arguments before any launch, and the product's host-side
parameters (codebooks, Pi, S) equal the reference's golden values bit-for-bit."""

import math
import os
import re

import numpy as np
import pytest
import torch

import quashkv_amd as Q
from quashkv_amd import _native as N
from quashkv_amd.codebook import LloydMaxCodebook, compute_mse_cost, solve_lloyd_max
from quashkv_amd.quantizer import _random_orthogonal, _random_signs

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "quashkv_amd.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qkv_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_header_symbol():
    lib = N.lib()
    names = header_functions()
    assert len(names) >= 12
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(N.EXPORTED)
    assert lib.qkv_abi_version() == 1


@pytest.mark.parametrize("d,bits,expect", [(128, 1, 16), (128, 2, 32), (128, 3, 48), (128, 4, 64),
                                           (65, 3, 27), (63, 2, 16), (100, 4, 50), (8, 8, 8)])
def test_packed_row_bytes(d, bits, expect):
    assert N.lib().qkv_packed_row_bytes(d, bits) == expect
    assert N.packed_row_bytes(d, bits) == expect


def test_abi_rejects_before_launch():
    lib = N.lib()
    assert lib.qkv_pack_bits(None, None, 4, 128, 5, None) == N.QKV_E_INVALID
    assert "Unsupported bits" in lib.qkv_last_error().decode()
    assert lib.qkv_unpack_bits(None, 10, None, 1, 128, 3, None) == N.QKV_E_INVALID
    assert "cannot hold" in lib.qkv_last_error().decode()
    # bad head dim -> unsupported
    st = lib.qkv_compress(0, 0, 0, None, 4, 80, None, None, None, 3, None, None, None, None, 4, 4, None)
    assert st == N.QKV_E_UNSUPPORTED
    st = lib.qkv_compress(0, 0, 0, None, 4, 128, None, None, None, 7, None, None, None, None, 4, 4, None)
    assert st == N.QKV_E_INVALID and "bits must be in" in lib.qkv_last_error().decode()
    # empty cache
    st = lib.qkv_decode_attention(None, 0, None, None, None, None, 0, 0, 1, 8, 8, 1, 128, 2, 3,
                                  None, None, None, None, 0.1, 0.1, 0, None, 0, None, 0, 1, None)
    assert st == N.QKV_E_INVALID and "No compressed KV blocks" in lib.qkv_last_error().decode()
    # workspace too small
    st = lib.qkv_decode_attention(1, 0, 1, 1, 1, 1, 64, 64, 1, 8, 8, 1, 128, 2, 3, 1, 1, 1, 1,
                                  0.1, 0.1, 0, 1, 0, 256, 8, 1, None)
    assert st == N.QKV_E_INVALID and "workspace too small" in lib.qkv_last_error().decode()
    # GQA divisibility
    st = lib.qkv_decode_attention(1, 0, 1, 1, 1, 1, 64, 64, 1, 6, 4, 1, 128, 2, 3, 1, 1, 1, 1,
                                  0.1, 0.1, 0, 1, 0, 256, 1 << 30, 1, None)
    assert st == N.QKV_E_INVALID and "multiple of kv heads" in lib.qkv_last_error().decode()
    # store converters validate shapes
    assert lib.qkv_kplanes_pack(None, None, 4, 80, 2, None, 30, 4, 4, None) == N.QKV_E_UNSUPPORTED
    assert lib.qkv_vtiles_pack(1, 1, 40, 128, 3, 1, 1, 0, None) == N.QKV_E_INVALID
    assert "exceed" in lib.qkv_last_error().decode()


def test_store_append_validation():
    lib = N.lib()
    # unknown input dtypes are refused, head_dims other than 128 / 96 / 64 not covered
    assert lib.qkv_store_append(7, 16, None, 1, 1, 128, 2, 3, 16, 16, 16, 16, 16, 16,
                                16, 16, 16, 64, 0, None) == N.QKV_E_INVALID
    assert lib.qkv_store_append(N.QKV_BF16, 16, None, 1, 1, 80, 2, 3, 16, 16, 16, 16, 16, 16,
                                16, 16, 16, 64, 0, None) == N.QKV_E_UNSUPPORTED
    # capacity must hold the appended tokens
    st = lib.qkv_store_append(N.QKV_BF16, 16, None, 1, 10, 128, 2, 3, 16, 16, 16, 16, 16, 16,
                              16, 16, 16, 64, 60, None)
    assert st == N.QKV_E_INVALID and "capacity" in lib.qkv_last_error().decode()
    # an asymmetric key codebook is refused (the sign folding needs symmetry)
    kc = N.HostFloats([-1.0, -0.4, 0.5, 1.0])
    kb = N.HostFloats([-0.7, 0.05, 0.75])
    st = lib.qkv_store_append(N.QKV_BF16, 16, None, 1, 1, 128, 2, 3, 16, 16, kc.ptr, kb.ptr,
                              16, 16, 16, 16, 16, 64, 0, None)
    assert st == N.QKV_E_UNSUPPORTED and "symmetric" in lib.qkv_last_error().decode()


def test_kmixed_host_validation():
    lib = N.lib()
    perm = N.HostInts(list(range(128)))
    bad = N.HostInts([0] * 128)
    assert lib.qkv_kmixed_pack(16, 4, bad.ptr, 32, 16, 4, 4, None) == N.QKV_E_INVALID
    assert "permutation" in lib.qkv_last_error().decode()
    assert lib.qkv_kmixed_pack(16, 4, perm.ptr, 48, 16, 4, 4, None) == N.QKV_E_INVALID
    assert lib.qkv_kmixed_unpack(16, 4, perm.ptr, 32, 4, 2, 16, None) == N.QKV_E_INVALID
    # unknown input dtypes are refused, other outlier counts not covered
    ob, rb = N.HostFloats([-3, -2, -1, 0, 1, 2, 3]), N.HostFloats([-1, 0, 1])
    assert lib.qkv_store_append_kmixed(7, 16, 1, 1, 128, 16, 32, ob.ptr, rb.ptr, 16, 16,
                                       64, 0, None) == N.QKV_E_INVALID
    assert lib.qkv_store_append_kmixed(N.QKV_BF16, 16, 1, 1, 128, 16, 16, ob.ptr, rb.ptr, 16,
                                       16, 64, 0, None) == N.QKV_E_UNSUPPORTED
    asym = N.HostFloats([-3, -2, -1, 0.1, 1, 2, 3])
    assert lib.qkv_store_append_kmixed(N.QKV_BF16, 16, 1, 1, 128, 16, 32, asym.ptr, rb.ptr, 16,
                                       16, 64, 0, None) == N.QKV_E_UNSUPPORTED
    # attention: only the MFMA path reads kmixed rows (capacity a multiple of 64)
    oc = N.HostFloats([-4, -3, -2, -1, 1, 2, 3, 4])
    rc, vc = N.HostFloats([-2, -1, 1, 2]), N.HostFloats([-2, -1, 1, 2])
    st = lib.qkv_decode_attention_kmixed(256, 0, 256, 256, 256, 256, 96, 90, 1, 8, 8, 1, 128, 2,
                                         256, 32, oc.ptr, rc.ptr, 256, vc.ptr, 0.1, 0, 256, 0,
                                         256, 1 << 30, 1, None)
    assert st == N.QKV_E_UNSUPPORTED and "multiple of 64" in lib.qkv_last_error().decode()


def test_compress_mfma_host_validation():
    lib = N.lib()
    c2, t2 = N.HostFloats([-1.5, -0.5, 0.5, 1.5]), N.HostFloats([-1.0, 0.0, 1.0])
    # other head dims and bit widths are not covered (the VALU qkv_compress is)
    assert lib.qkv_compress_mfma(N.QKV_MODE_IP, N.QKV_F32, 16, 4, 80, 16, c2.ptr, t2.ptr, 2, 16,
                                 16, 16, 16, 4, 4, None) == N.QKV_E_UNSUPPORTED
    assert lib.qkv_compress_mfma(N.QKV_MODE_IP, N.QKV_F32, 16, 4, 128, 16, c2.ptr, t2.ptr, 4, 16,
                                 16, 16, 16, 4, 4, None) == N.QKV_E_UNSUPPORTED
    # asymmetric tables, and a fine list that does not interleave
    ta = N.HostFloats([-1.0, 0.1, 1.0])
    assert lib.qkv_compress_mfma(N.QKV_MODE_MSE, N.QKV_F32, 16, 4, 128, 16, None, ta.ptr, 2, None,
                                 16, None, 16, 4, 4, None) == N.QKV_E_UNSUPPORTED
    cb = N.HostFloats([-1.5, -1.2, 1.2, 1.5])
    assert lib.qkv_compress_mfma(N.QKV_MODE_IP, N.QKV_F32, 16, 4, 128, 16, cb.ptr, t2.ptr, 2, 16,
                                 16, 16, 16, 4, 4, None) == N.QKV_E_UNSUPPORTED
    assert "symmetric" in lib.qkv_last_error().decode()
    assert lib.qkv_compress_mfma(N.QKV_MODE_IP, 9, 16, 4, 128, 16, c2.ptr, t2.ptr, 2, 16,
                                 16, 16, 16, 4, 4, None) == N.QKV_E_INVALID
    # IP needs the QJL output and the signs
    assert lib.qkv_compress_mfma(N.QKV_MODE_IP, N.QKV_F32, 16, 4, 128, 16, c2.ptr, t2.ptr, 2, None,
                                 16, 16, 16, 4, 4, None) == N.QKV_E_INVALID
    assert lib.qkv_compress_mfma(N.QKV_MODE_IP, N.QKV_F32, 16, 4, 128, 16, c2.ptr, t2.ptr, 2, 16,
                                 16, None, 16, 4, 4, None) == N.QKV_E_INVALID


def test_kipmixed_host_validation():
    lib = N.lib()
    perm = N.HostInts(list(range(128)))
    bad = N.HostInts([0] * 128)
    assert lib.qkv_kipmixed_pack(16, 16, 4, bad.ptr, 32, 16, 4, 4, None) == N.QKV_E_INVALID
    assert "permutation" in lib.qkv_last_error().decode()
    assert lib.qkv_kipmixed_pack(16, None, 4, perm.ptr, 32, 16, 4, 4, None) == N.QKV_E_INVALID
    assert lib.qkv_kipmixed_unpack(16, 4, perm.ptr, 32, 4, 4, 16, None, None) == N.QKV_E_INVALID
    oc, ob = N.HostFloats([-1.5, -0.5, 0.5, 1.5]), N.HostFloats([-1, 0, 1])
    rc, rb = N.HostFloats([-0.8, 0.8]), N.HostFloats([0.0])
    # unknown input dtypes are refused, other outlier counts not covered
    assert lib.qkv_store_append_kipmixed(7, 16, 1, 1, 128, 16, 16, 32, oc.ptr, ob.ptr,
                                         rc.ptr, rb.ptr, 16, 16, 64, 0, None) == \
        N.QKV_E_INVALID
    assert lib.qkv_store_append_kipmixed(N.QKV_BF16, 16, 1, 1, 128, 16, 16, 48, oc.ptr, ob.ptr,
                                         rc.ptr, rb.ptr, 16, 16, 64, 0, None) == \
        N.QKV_E_UNSUPPORTED
    # the fine list c_0 < t_0 < c_1 ... must interleave
    oc_bad = N.HostFloats([-1.5, -1.2, 1.2, 1.5])
    assert lib.qkv_store_append_kipmixed(N.QKV_BF16, 16, 1, 1, 128, 16, 16, 32, oc_bad.ptr,
                                         ob.ptr, rc.ptr, rb.ptr, 16, 16, 64, 0, None) == \
        N.QKV_E_UNSUPPORTED
    assert "fine lists" in lib.qkv_last_error().decode()
    assert lib.qkv_store_append_kipmixed(N.QKV_BF16, 16, 1, 1, 128, 16, None, 32, oc.ptr, ob.ptr,
                                         rc.ptr, rb.ptr, 16, 16, 64, 0, None) == N.QKV_E_INVALID
    vc = N.HostFloats([-2, -1, 1, 2])
    st = lib.qkv_decode_attention_kipmixed(256, 0, 256, 256, 256, 256, 96, 90, 1, 8, 8, 1, 128,
                                           2, 256, 256, 0.01, 32, oc.ptr, rc.ptr, 256, vc.ptr,
                                           0.1, 0, 256, 0, 256, 1 << 30, 1, None)
    assert st == N.QKV_E_UNSUPPORTED and "multiple of 64" in lib.qkv_last_error().decode()
    st = lib.qkv_decode_attention_kipmixed(256, 0, 256, 256, 256, 256, 128, 90, 1, 8, 8, 1, 128,
                                           2, 256, None, 0.01, 32, oc.ptr, rc.ptr, 256, vc.ptr,
                                           0.1, 0, 256, 0, 256, 1 << 30, 1, None)
    assert st == N.QKV_E_INVALID


def test_layers_host_validation():
    lib = N.lib()
    a = N.ptr_array([256] * 33)
    kc = N.HostFloats(LloydMaxCodebook(64, 2).centroids_host)
    vc = N.HostFloats(LloydMaxCodebook(64, 3).centroids_host)
    args = lambda n, k: (n, a, 0, a, a, a, a, 128, 100, 1, 8, 8, 1, 64, 2, 3, a, k.ptr, vc.ptr,
                         a, 0.1, 0.1, 0, a, 0, 256, 1 << 30, 1, None)
    assert lib.qkv_decode_attention_layers(*args(0, kc)) == N.QKV_E_INVALID
    assert lib.qkv_decode_attention_layers(*args(33, kc)) == N.QKV_E_INVALID
    assert "n_layers" in lib.qkv_last_error().decode()
    asym = N.HostFloats([-1.0, -0.25, 0.5, 1.0])
    assert lib.qkv_decode_attention_layers(*args(2, asym)) == N.QKV_E_UNSUPPORTED
    assert "MFMA path" in lib.qkv_last_error().decode()


def test_store_append_layers_host_validation():
    """Argument checks of qkv_store_append_layers (all before any launch)."""
    lib = N.lib()
    a = N.ptr_array([256] * 33)
    cb = LloydMaxCodebook(64, 2)
    kc, kb = N.HostFloats(cb.centroids_host), N.HostFloats(cb.boundaries_host)
    vb = N.HostFloats(LloydMaxCodebook(64, 3).boundaries_host)
    args = lambda n, dt=2, d=64, cap=128, k=kc, arr=a: (
        n, dt, arr, arr, 4, 1, d, 2, 3, arr, arr, arr, k.ptr, kb.ptr, vb.ptr, arr, arr, arr, arr,
        cap, 100, None)
    assert lib.qkv_store_append_layers(*args(0)) == N.QKV_E_INVALID
    assert lib.qkv_store_append_layers(*args(33)) == N.QKV_E_INVALID
    assert "n_layers" in lib.qkv_last_error().decode()
    assert lib.qkv_store_append_layers(*args(2, dt=7)) == N.QKV_E_INVALID
    assert lib.qkv_store_append_layers(*args(2, cap=100)) == N.QKV_E_INVALID   # capacity
    assert lib.qkv_store_append_layers(*args(2, d=80)) == N.QKV_E_UNSUPPORTED
    assert lib.qkv_store_append_layers(*args(2, arr=None)) == N.QKV_E_INVALID
    nul = N.ptr_array([256, 0])
    assert lib.qkv_store_append_layers(*args(2, arr=nul)) == N.QKV_E_INVALID
    assert "layer 1" in lib.qkv_last_error().decode()
    asym = N.HostFloats([-1.0, -0.25, 0.5, 1.0])
    assert lib.qkv_store_append_layers(*args(2, k=asym)) == N.QKV_E_UNSUPPORTED
    assert "symmetric" in lib.qkv_last_error().decode()


def test_mips_host_validation():
    lib = N.lib()
    assert lib.qkv_mips_workspace_bytes(10, 80, 2, 10, 100) == -1      # dim
    assert lib.qkv_mips_workspace_bytes(10, 128, 4, 10, 100) == -1     # 5-bit codes
    assert lib.qkv_mips_workspace_bytes(10, 128, 2, 10, 100) > 0
    st = lib.qkv_mips_search(16, 0, 4, 128, 2, 16, 16, 16, 0.1, 16, 16, 0, 10, 16, 16, 256,
                             1 << 20, None)
    assert st == N.QKV_E_INVALID and "Index is empty" in lib.qkv_last_error().decode()
    from quashkv_amd.nn_search import QuashIndex
    idx = QuashIndex(dim=64, bits=3, device="cpu")
    with pytest.raises(ValueError, match="Expected"):
        idx.add(torch.randn(5, 32))
    with pytest.raises(ValueError, match="Index is empty"):
        idx.search(torch.randn(2, 64))


def test_check_maps_status_to_exceptions():
    N.lib().qkv_pack_bits(None, None, 4, 128, 9, None)
    with pytest.raises(ValueError, match="Unsupported bits"):
        N.check(N.QKV_E_INVALID)


def test_workspace_and_split_policy_are_consistent():
    lib = N.lib()
    for (B, Hq, Hkv, Q_, d) in [(32, 32, 8, 1, 128), (1, 32, 8, 1, 128), (16, 14, 2, 1, 64)]:
        ws = lib.qkv_attention_workspace_bytes(B, Hq, Hkv, Q_, d, 4)
        R = (Hq // Hkv) * Q_
        ch = (R + 3) // 4
        assert ws == (4 * B * Hkv * R * 2 * d + B * Hkv * ch * 6 * 64 * 16 + B * Hkv * ch * 4 * 2 * 4
                      + 4 * (4 * B * Hkv * R * d + 4 * B * Hkv * R * 2))
    # d = 128 (fused kernel, any split length): one split per row group once
    # the groups cover the CUs (256 here: no device), else splits of >= ~1024
    # tokens up to one workgroup per CU
    for T_ in (1, 63, 64, 2048, 2049, 8192, 131072):
        assert lib.qkv_attention_splits(32, 32, 8, 1, 128, T_) == 1
        s = lib.qkv_attention_splits(1, 32, 8, 1, 128, T_)
        assert s == max(1, min(32, -(-T_ // 1024)))
    # d = 64 (split_mfma): every split within the LDS-resident length
    for T_ in (1, 63, 64, 2048, 2049, 8192, 131072):
        s = lib.qkv_attention_splits(16, 14, 2, 1, 64, T_)
        assert 1 <= s <= max(1, (T_ + 63) // 64)
        assert -(-T_ // s) <= 2048 or s == 1024


def test_attention_path_selection():
    lib = N.lib()
    k2 = LloydMaxCodebook(128, 2).centroids_host
    v3 = LloydMaxCodebook(128, 3).centroids_host
    kc, vc = N.HostFloats(k2), N.HostFloats(v3)
    assert lib.qkv_attention_path(128, 2, 3, kc.ptr, vc.ptr, 8192, 8192, 4) == 1
    assert lib.qkv_attention_path(128, 2, 3, kc.ptr, vc.ptr, 8192, 8192, 1) == 1   # fused: any split
    assert lib.qkv_attention_path(128, 2, 3, kc.ptr, vc.ptr, 8160, 8150, 8) == 0   # stride % 64
    assert lib.qkv_attention_path(96, 2, 3, kc.ptr, vc.ptr, 8192, 8192, 4) == 1   # fused, padded
    assert lib.qkv_attention_path(96, 2, 3, kc.ptr, vc.ptr, 8160, 8150, 4) == 0
    k64 = N.HostFloats(LloydMaxCodebook(64, 2).centroids_host)
    v64 = N.HostFloats(LloydMaxCodebook(64, 3).centroids_host)
    assert lib.qkv_attention_path(64, 2, 3, k64.ptr, v64.ptr, 2048, 2048, 2) == 1
    assert lib.qkv_attention_path(64, 2, 3, k64.ptr, v64.ptr, 2048, 2048, 1) == 1
    assert lib.qkv_attention_path(64, 2, 3, k64.ptr, v64.ptr, 4096, 4096, 1) == 1   # fused: any split
    assert lib.qkv_attention_path(64, 2, 3, k64.ptr, v64.ptr, 4064, 4000, 1) == 0   # stride % 64
    for vb in (1, 2, 4):
        v = N.HostFloats(LloydMaxCodebook(128, vb).centroids_host)
        assert lib.qkv_attention_path(128, 2, vb, kc.ptr, v.ptr, 256, 256, 1) == 1
    k1 = N.HostFloats(LloydMaxCodebook(128, 1).centroids_host)
    assert lib.qkv_attention_path(128, 1, 3, k1.ptr, vc.ptr, 256, 256, 1) == 1
    k3 = N.HostFloats(LloydMaxCodebook(128, 3).centroids_host)
    assert lib.qkv_attention_path(128, 3, 3, k3.ptr, vc.ptr, 256, 256, 1) == 1   # parity plane
    k3_64 = N.HostFloats(LloydMaxCodebook(64, 3).centroids_host)
    assert lib.qkv_attention_path(64, 3, 3, k3_64.ptr, v64.ptr, 256, 256, 1) == 1   # parity plane
    asym = N.HostFloats([-1.0, -0.25, 0.5, 1.0])
    assert lib.qkv_attention_path(128, 2, 3, asym.ptr, vc.ptr, 256, 256, 1) == 0


# -------------------------------------------------- product host parameters

@pytest.mark.parametrize("d", [64, 96, 128])
@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_codebook_solver_bit_exact(golden, d, bits):
    cb = golden("codebooks")
    c = LloydMaxCodebook(d, bits)
    assert torch.equal(c.centroids, torch.from_numpy(cb[f"c_d{d}_b{bits}"]))
    assert torch.equal(c.boundaries, torch.from_numpy(cb[f"t_d{d}_b{bits}"]))
    c64, t64 = solve_lloyd_max(d, bits)
    assert np.allclose(c64, cb[f"c64_d{d}_b{bits}"], rtol=0, atol=1e-14)


@pytest.mark.parametrize("d,bits", [(64, 2), (64, 3), (128, 2)])
def test_codebook_exact_pdf_bit_exact(golden, d, bits):
    cb = golden("codebooks")
    c = LloydMaxCodebook(d, bits, use_exact_pdf=True)
    assert torch.equal(c.centroids, torch.from_numpy(cb[f"ce_d{d}_b{bits}"]))
    assert torch.equal(c.boundaries, torch.from_numpy(cb[f"te_d{d}_b{bits}"]))


def test_codebook_closed_forms():
    # 1-bit Gaussian Lloyd-Max: +-sigma sqrt(2/pi); distortions (Max 1960)
    for d in (64, 128):
        c, _ = solve_lloyd_max(d, 1)
        assert abs(c[1] - math.sqrt(2 / math.pi) / math.sqrt(d)) < 1e-12
    assert abs(compute_mse_cost(128, 1) - (1 - 2 / math.pi)) < 1e-9
    assert abs(compute_mse_cost(128, 2) - 0.11748) < 1e-4
    assert abs(compute_mse_cost(128, 3) - 0.03455) < 1e-4
    for bits in (1, 2, 3):
        m = compute_mse_cost(128, bits)
        assert 0.9 * 4 ** -bits < m < 2.8 * 4 ** -bits
    with pytest.raises(ValueError, match="bits must be in"):
        solve_lloyd_max(128, 5)


@pytest.mark.parametrize("d,seed", [(64, 42), (64, 65), (96, 42), (128, 42), (128, 7)])
def test_rotation_and_signs_bit_exact(golden, d, seed):
    g = golden("rotations")
    assert torch.equal(_random_orthogonal(d, seed, "cpu"), torch.from_numpy(g[f"Pi_d{d}_s{seed}"]))
    assert torch.equal(_random_signs(d, seed, "cpu"), torch.from_numpy(g[f"S_d{d}_s{seed}"]))


# ---------------------------------------------------------------- host API

def test_engine_host_logic_and_errors():
    e = Q.QuashKVEngine(head_dim=64, device="cpu")
    assert e.total_tokens == 0 and e.num_blocks == 0
    assert e.compression_ratio() == 1.0
    assert "head_dim=64" in repr(e) and "key_bits=3" in repr(e)
    with pytest.raises(ValueError, match="No compressed KV blocks"):
        e.attention(torch.zeros(1, 2, 1, 64))
    with pytest.raises(RuntimeError, match="runs on the GPU"):
        e.append(torch.zeros(1, 2, 4, 64), torch.zeros(1, 2, 4, 64))
    with pytest.raises(ValueError, match="at least 2"):
        Q.InnerProductQuantizer(d=128, total_bits=1, device="cpu")


def test_cpu_tensors_raise_no_fallback():
    q = Q.MSEQuantizer(64, device="cpu")
    with pytest.raises(RuntimeError, match="runs on the GPU"):
        q.compress(torch.randn(2, 64))
    with pytest.raises(RuntimeError, match="runs on the GPU"):
        Q.pack_bits(torch.zeros(2, 64, dtype=torch.uint8), 3)
    assert Q.pack_bits(torch.zeros(2, 8, dtype=torch.uint8), 8).shape == (2, 8)  # passthrough
    with pytest.raises(ValueError, match="Unsupported bits"):
        Q.pack_bits(torch.zeros(2, 8, dtype=torch.uint8), 5)


def test_hf_cache_host_logic():
    from quashkv_amd.integrations.hf_cache import QuashKVCache, QuashKVCacheConfig
    c = QuashKVCache(num_layers=4, head_dim=64, device="cpu")
    assert [e.seed for e in c.engines] == [42, 43, 44, 45]
    assert len(c) == 4 and c.get_max_cache_length() is None
    k, v = c[0]
    assert k.numel() == 0 and v.numel() == 0
    st = c.compression_stats()
    assert st["overall_compression_ratio"] == 0 and st["tokens_per_layer"] == [0] * 4
    cfg = QuashKVCacheConfig(key_bits=4, value_bits=4, seed=7)
    c2 = QuashKVCache(num_layers=2, head_dim=128, config=cfg, device="cpu")
    assert c2.engines[0].key_bits == 4 and c2.engines[1].seed == 8


def test_store_append_kmixed_kv_host_validation():
    """Argument checks of qkv_store_append_kmixed_kv: every one before any
    launch (fake device pointers; a call that passes them launches nothing
    only when there is nothing to append)."""
    lib = N.lib()
    ob = N.HostFloats(LloydMaxCodebook(128, 3).boundaries_host)
    rb = N.HostFloats(LloydMaxCodebook(128, 2).boundaries_host)
    vb = N.HostFloats(LloydMaxCodebook(128, 4).boundaries_host)
    P = 256

    def call(groups=2, S=1, d=128, n_out=32, vbits=4, values=P, vstore=P, cap=128, dt=2):
        return lib.qkv_store_append_kmixed_kv(dt, P, values, groups, S, d, P, None, n_out, 0,
                                              None, ob.ptr, None, rb.ptr, P, P, vbits, P, vb.ptr,
                                              vstore, P, cap, 0, None)

    assert call(groups=0) == N.QKV_OK            # nothing to append: checks only
    assert call(d=96) == N.QKV_E_UNSUPPORTED
    assert call(n_out=16) == N.QKV_E_UNSUPPORTED
    assert call(vbits=5) == N.QKV_E_INVALID
    assert call(values=None) == N.QKV_E_INVALID
    assert call(vstore=None) == N.QKV_E_INVALID
    assert call(cap=100, S=1) == N.QKV_E_INVALID  # capacity not a multiple of 32
    assert call(cap=64, S=65) == N.QKV_E_INVALID
    assert call(dt=7) == N.QKV_E_INVALID


def test_paged_store_append_kv_host_validation():
    """Argument checks of qkv_paged_store_append_kv, all before any launch."""
    lib = N.lib()
    cb = LloydMaxCodebook(128, 2)
    kc, kb = N.HostFloats(cb.centroids_host), N.HostFloats(cb.boundaries_host)
    vb = N.HostFloats(LloydMaxCodebook(128, 3).boundaries_host)
    P = 256

    def call(keys=P, values=P, B=2, S=1, d=128, vbits=3, table=P, pt=64, npages=8, dt=2):
        return lib.qkv_paged_store_append_kv(dt, keys, values, B, 2, S, d, 2, vbits, P, P, P,
                                             kc.ptr, kb.ptr, vb.ptr, P, P, P, P, table, 4, pt,
                                             npages, 0, None)

    assert call(B=0) == N.QKV_OK                   # nothing to append: checks only
    assert call(values=None) == N.QKV_E_INVALID
    assert call(keys=None) == N.QKV_E_INVALID
    assert call(table=None) == N.QKV_E_INVALID
    assert call(pt=48) == N.QKV_E_INVALID           # pages of 64 * 2^k tokens
    assert call(npages=0) == N.QKV_E_INVALID
    assert call(S=4 * 64 + 1) == N.QKV_E_INVALID    # beyond the table's pages
    assert call(d=80) == N.QKV_E_UNSUPPORTED
    assert call(vbits=5) == N.QKV_E_INVALID
    assert call(dt=7) == N.QKV_E_INVALID


def test_host_table_cache_follows_the_tensor_not_its_address():
    """N.host_table's cached host copy belongs to one live tensor: a table
    freed and replaced by another of the same size (often at the same
    address) is copied afresh, and an in-place write to a live table is seen."""
    for i in range(200):
        t = torch.full((7,), float(i))
        assert list(N.host_table(t).arr) == [float(i)] * 7
        del t
    t = torch.arange(5, dtype=torch.float32)
    assert list(N.host_table(t).arr) == [0.0, 1.0, 2.0, 3.0, 4.0]
    t.view(5)[2] = 9.0            # a write through a view bumps the shared version
    assert list(N.host_table(t).arr) == [0.0, 1.0, 9.0, 3.0, 4.0]
    n_before = len(N._HOST_TABLES)
    del t
    assert len(N._HOST_TABLES) == n_before - 1   # the entry goes with its tensor
