"""GPU parity: the HIP kernels against the CPU oracle and the reference's golden
vectors.  Bars: bit-exact for packing and for codes from identical rotated
inputs; rel-err <= 1e-3 (fp32) / 1e-2 (bf16 inputs) and cosine >= 0.9999 for
reconstructions and attention outputs (tighter where the math allows)."""

import math

import numpy as np
import pytest
import torch

import quashkv_amd as Q
from quashkv_amd import _native as N
from quashkv_amd import kernels as K
from quashkv_amd.quantizer import compress_into
from quashkv_amd.store import KVStore
from oracle import ref_math as R

pytestmark = pytest.mark.gpu

DEV = "cuda"


def T(a):
    return torch.from_numpy(np.asarray(a))


def rel_err(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return float((a - b).norm() / b.norm().clamp(min=1e-30))


def cosine(a, b):
    a, b = a.double().cpu().flatten(), b.double().cpu().flatten()
    return float(a @ b / (a.norm() * b.norm()).clamp(min=1e-30))


def assert_close(out, ref, rel=1e-3, cos=0.9999):
    e, c = rel_err(out, ref), cosine(out, ref)
    assert e <= rel and c >= cos, f"rel_err={e:.3e} cosine={c:.7f}"


@pytest.fixture(autouse=True, scope="module")
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")
    N.lib()


# ------------------------------------------------------------------ packing

@pytest.mark.parametrize("d", [8, 63, 64, 65, 100, 128])
@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_pack_unpack_golden(golden, d, bits):
    g = golden("packing")
    codes = T(g[f"codes_d{d}_b{bits}"]).to(DEV)
    packed = Q.pack_bits(codes, bits)
    assert np.array_equal(packed.cpu().numpy(), g[f"packed_d{d}_b{bits}"])
    assert torch.equal(Q.unpack_bits(packed, bits, d), codes)


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_pack_unpack_large_vs_oracle(bits):
    gen = torch.Generator().manual_seed(bits)
    codes = torch.randint(0, 1 << bits, (3, 7, 1111, 128), generator=gen, dtype=torch.uint8)
    packed = Q.pack_bits(codes.to(DEV), bits)
    assert np.array_equal(packed.cpu().numpy(), R.pack_bits(codes.numpy(), bits))
    assert torch.equal(Q.unpack_bits(packed, bits, 128).cpu(), codes)


def test_pack_edge_cases():
    e = torch.empty(0, 128, dtype=torch.uint8, device=DEV)
    assert Q.pack_bits(e, 3).shape == (0, 48)
    assert Q.unpack_bits(Q.pack_bits(e, 2), 2, 128).shape == (0, 128)
    k = torch.arange(8, dtype=torch.uint8, device=DEV)[None]
    assert Q.pack_bits(k, 3).cpu().tolist() == [[0x88, 0xC6, 0xFA]]


# ------------------------------------------------------------- codebooks

@pytest.mark.parametrize("d,bits", [(128, 2), (128, 3), (64, 4), (128, 1)])
def test_quantize_boundary_ties(golden, d, bits):
    g = golden("compress")
    cb = Q.LloydMaxCodebook(d, bits)
    y = T(g[f"tie_y_d{d}_b{bits}"]).to(DEV)
    assert torch.equal(cb.quantize_boundary(y).cpu(), T(g[f"tie_code_d{d}_b{bits}"]))


def test_quantize_argmin_and_dequantize():
    cb = Q.LloydMaxCodebook(128, 3)
    y = (torch.randn(50000) / math.sqrt(128)).to(DEV)
    assert torch.equal(cb.quantize(y), cb.quantize_boundary(y))
    assert torch.equal(cb.quantize(y).cpu(), R.quantize_argmin(y.cpu(), cb.centroids.cpu()))
    codes = torch.randint(0, 8, (33, 17), dtype=torch.uint8)
    assert torch.equal(cb.dequantize(codes.to(DEV)).cpu(), cb.centroids.cpu()[codes.long()])


# -------------------------------------------------------------- compress

def _pi_s(golden, d, seed=42):
    rot = golden("rotations")
    return T(rot[f"Pi_d{d}_s{seed}"]), T(rot[f"S_d{d}_s{seed}"])


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_compress_mse_vs_golden(golden, d, bits):
    g = golden("compress")
    x = T(g[f"x_d{d}"])
    q = Q.MSEQuantizer(d, bits=bits, seed=42, device=DEV)
    codes, norms = q.compress(x.to(DEV))
    ref_codes = T(g[f"mse_idx_d{d}_b{bits}"])
    agree = (codes.cpu() == ref_codes).float().mean().item()
    assert agree >= 0.999, agree
    assert torch.allclose(norms.cpu(), T(g[f"mse_norm_d{d}_b{bits}"]), rtol=1e-6, atol=0)
    # identical rotated inputs -> bit-exact codes
    y = T(g[f"mse_y_d{d}_b{bits}"]).to(DEV)
    n = y.numel() // d
    out = torch.empty(n, d, dtype=torch.uint8, device=DEV)
    compress_into(N.QKV_MODE_MSE, y, q.Pi, q.codebook.boundaries, q.codebook.centroids, bits,
                  None, out, None, None, packed=False, pre_rotated=True)
    assert torch.equal(out.cpu().reshape(ref_codes.shape), T(g[f"mse_qb_d{d}_b{bits}"]))
    # decompress of the reference's codes
    xh = q.decompress(ref_codes.to(DEV), T(g[f"mse_norm_d{d}_b{bits}"]).to(DEV))
    assert_close(xh, T(g[f"mse_xhat_d{d}_b{bits}"]), rel=1e-5, cos=0.99999)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("tb", [2, 3, 4])
def test_compress_ip_vs_golden(golden, d, tb):
    g = golden("compress")
    x = T(g[f"x_d{d}"])
    q = Q.InnerProductQuantizer(d, total_bits=tb, seed=42, device=DEV)
    codes, bits, norms = q.compress(x.to(DEV))
    assert (codes.cpu() == T(g[f"ip_mse_d{d}_b{tb}"])).float().mean() >= 0.999
    assert (bits.cpu() == T(g[f"ip_qjl_d{d}_b{tb}"])).float().mean() >= 0.999
    assert torch.allclose(norms.cpu(), T(g[f"ip_norm_d{d}_b{tb}"]), rtol=1e-6, atol=0)
    # pre-rotated: codes and QJL bits equal the oracle's from the same y
    pi, s = _pi_s(golden, d)
    mq = q.mse_quantizer
    xcpu = x.reshape(-1, d)
    y = (xcpu / xcpu.norm(dim=-1, keepdim=True).clamp(min=1e-8)) @ pi.T
    c_ref, b_ref = R.compress_ip_from_y(y, mq.codebook.boundaries.cpu(), s,
                                        mq.codebook.centroids.cpu())
    n = y.shape[0]
    oc = torch.empty(n, d, dtype=torch.uint8, device=DEV)
    ob = torch.empty(n, d, dtype=torch.uint8, device=DEV)
    compress_into(N.QKV_MODE_IP, y.to(DEV), mq.Pi, mq.codebook.boundaries, mq.codebook.centroids,
                  tb - 1, q.S, oc, ob, None, packed=False, pre_rotated=True)
    assert torch.equal(oc.cpu(), c_ref) and torch.equal(ob.cpu(), b_ref)
    # decompress_for_dot on the reference's codes
    qv = T(g[f"ip_q_d{d}_b{tb}"])
    q_rot = (qv.unsqueeze(0) @ pi.T).expand(*x.shape[:-1], d)
    dot = q.decompress_for_dot(T(g[f"ip_mse_d{d}_b{tb}"]).to(DEV), T(g[f"ip_qjl_d{d}_b{tb}"]).to(DEV),
                               T(g[f"ip_norm_d{d}_b{tb}"]).to(DEV), q_rot.to(DEV))
    assert_close(dot, T(g[f"ip_dot_d{d}_b{tb}"]), rel=1e-5, cos=0.99999)
    # fused decompress_ip of the reference's codes
    xh = K.fused_decompress_ip(T(g[f"ip_mse_d{d}_b{tb}"]).to(DEV), T(g[f"ip_qjl_d{d}_b{tb}"]).to(DEV),
                               T(g[f"ip_norm_d{d}_b{tb}"]).to(DEV), mq.Pi, mq.codebook.centroids,
                               q.S, q.qjl_scale)
    assert_close(xh, T(g[f"fip_xhat_d{d}_b{tb}"]), rel=1e-5, cos=0.99999)


@pytest.mark.parametrize("d", [64, 96, 128])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_compress_packed_grouped_vs_oracle(d, dtype):
    gen = torch.Generator().manual_seed(d)
    B, H, S, C, t0 = 2, 3, 37, 100, 11
    x = torch.randn(B, H, S, d, generator=gen).to(dtype)
    q = Q.InnerProductQuantizer(d, total_bits=3, seed=5, device=DEV)
    mq = q.mse_quantizer
    pk, pq = N.packed_row_bytes(d, 2), N.packed_row_bytes(d, 1)
    codes = torch.zeros(B, H, C, pk, dtype=torch.uint8, device=DEV)
    qjl = torch.zeros(B, H, C, pq, dtype=torch.uint8, device=DEV)
    norms = torch.zeros(B, H, C, device=DEV)
    compress_into(N.QKV_MODE_IP, x.to(DEV), mq.Pi, mq.codebook.boundaries, mq.codebook.centroids,
                  2, q.S, codes[:, :, t0:], qjl[:, :, t0:], norms[:, :, t0:], packed=True,
                  out_seq=S, out_group_stride=C)
    oc, ob, on = R.compress_ip(x.float(), mq.Pi.cpu(), mq.codebook.boundaries.cpu(), q.S.cpu(),
                               mq.codebook.centroids.cpu())
    got_c = R.unpack_bits(codes[:, :, t0:t0 + S].cpu().numpy(), 2, d)
    got_b = R.unpack_bits(qjl[:, :, t0:t0 + S].cpu().numpy(), 1, d)
    assert (torch.from_numpy(got_c) == oc).float().mean() >= 0.999
    assert (torch.from_numpy(got_b) == ob).float().mean() >= 0.999
    assert torch.allclose(norms[:, :, t0:t0 + S].cpu(), on, rtol=1e-5)
    # untouched rows stay zero
    assert int(codes[:, :, :t0].sum()) == 0 and int(codes[:, :, t0 + S:].sum()) == 0


# ------------------------------------------------------------ decompress

@pytest.mark.parametrize("d", [64, 96, 128])
@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("mode", ["mse", "ip"])
def test_decompress_vs_oracle(d, packed, mode):
    gen = torch.Generator().manual_seed(7 * d + packed)
    n, bits = 777, 3 if mode == "mse" else 2
    codes = torch.randint(0, 1 << bits, (n, d), generator=gen, dtype=torch.uint8)
    qb = torch.randint(0, 2, (n, d), generator=gen, dtype=torch.uint8)
    norms = torch.rand(n, generator=gen) * 3 + 0.1
    pi = R.random_orthogonal(d, 9)
    s = R.random_signs(d, 9)
    cents = Q.LloydMaxCodebook(d, bits).centroids
    alpha = R.QJL_COEFF / d
    if mode == "mse":
        ref = R.decompress_mse(codes, norms, pi, cents)
    else:
        ref = R.decompress_ip(codes, qb, norms, pi, cents, s, alpha)
    c_in = torch.from_numpy(R.pack_bits(codes.numpy(), bits)) if packed else codes
    b_in = torch.from_numpy(R.pack_bits(qb.numpy(), 1)) if packed else qb
    from quashkv_amd.quantizer import decompress_from
    out = decompress_from(N.QKV_MODE_MSE if mode == "mse" else N.QKV_MODE_IP, c_in.to(DEV),
                          b_in.to(DEV), norms.to(DEV), n, pi.to(DEV), cents.to(DEV), bits,
                          s.to(DEV), alpha, fmt=N.QKV_FMT_PACKED if packed else N.QKV_FMT_UNPACKED)
    assert_close(out, ref, rel=1e-5, cos=0.99999)


# ------------------------------------------------------------ cache store

def kplanes_ref(codes, qjl, mbits):
    """Expected K store rows: plane r of every coordinate, then the QJL plane,
    each as LSB-first 1-bit rows (numpy)."""
    planes = [(codes >> r) & 1 for r in range(mbits)] + [qjl & 1]
    return np.concatenate([R.pack_bits(p.astype(np.uint8), 1) for p in planes], axis=-1)


def vtiles_ref(codes, vbits):
    """Expected V store words (G, S/32, vbits, d) for codes (G, S, d), S % 32 == 0."""
    G, S, d = codes.shape
    c = codes.astype(np.uint64).reshape(G, S // 32, 32, d)
    out = np.zeros((G, S // 32, vbits, d), dtype=np.uint64)
    for k in range(vbits):
        bits = (c >> k) & 1
        out[:, :, k, :] = (bits << np.arange(32, dtype=np.uint64)[None, None, :, None]).sum(axis=2)
    return out.astype(np.uint32)


@pytest.mark.parametrize("d,mbits", [(64, 2), (96, 3), (128, 1), (128, 2)])
def test_kplanes_pack_layout_and_roundtrip(d, mbits):
    gen = torch.Generator().manual_seed(d + mbits)
    G, S, C, t0 = 3, 37, 128, 5
    codes = torch.randint(0, 1 << mbits, (G * S, d), generator=gen, dtype=torch.uint8)
    qjl = torch.randint(0, 2, (G * S, d), generator=gen, dtype=torch.uint8)
    krb = (mbits + 1) * d // 8
    dst = torch.zeros(G, C, krb, dtype=torch.uint8, device=DEV)
    L = N.lib()
    codes_d, qjl_d = codes.to(DEV), qjl.to(DEV)   # keep the device copies alive
    N.check(L.qkv_kplanes_pack(codes_d.data_ptr(), qjl_d.data_ptr(), G * S, d, mbits,
                               dst.data_ptr() + t0 * krb, krb, S, C, 0))
    torch.cuda.synchronize()
    ref = kplanes_ref(codes.numpy(), qjl.numpy(), mbits).reshape(G, S, krb)
    got = dst.cpu().numpy()
    assert np.array_equal(got[:, t0:t0 + S], ref)
    assert not got[:, :t0].any() and not got[:, t0 + S:].any()
    c2 = torch.empty_like(codes, device=DEV)
    q2 = torch.empty_like(qjl, device=DEV)
    N.check(L.qkv_kplanes_unpack(dst.data_ptr() + t0 * krb, krb, G * S, d, mbits, S, C,
                                 c2.data_ptr(), q2.data_ptr(), 0))
    assert torch.equal(c2.cpu(), codes) and torch.equal(q2.cpu(), qjl)


@pytest.mark.parametrize("vbits", [1, 2, 3, 4])
def test_vtiles_pack_layout_rmw_and_roundtrip(vbits):
    gen = torch.Generator().manual_seed(vbits)
    G, d, C = 5, 128, 192
    full = torch.randint(0, 1 << vbits, (G, C, d), generator=gen, dtype=torch.uint8)
    dst = torch.zeros(G, C // 32, vbits, d, dtype=torch.int32, device=DEV)
    L = N.lib()
    # append in ragged pieces that straddle tiles (read-modify-write of shared words)
    t0 = 0
    for S in (1, 30, 2, 64, 33, 7, 55):
        part = full[:, t0:t0 + S].contiguous().to(DEV)
        N.check(L.qkv_vtiles_pack(part.data_ptr(), G, S, d, vbits, dst.data_ptr(), C // 32, t0, 0))
        t0 += S
    assert t0 == C
    got = dst.cpu().numpy().view(np.uint32)
    ref = vtiles_ref(full[:, :t0].numpy() if t0 % 32 == 0 else
                     np.pad(full[:, :t0].numpy(), ((0, 0), (0, (-t0) % 32), (0, 0))), vbits)
    nt = ref.shape[1]
    assert np.array_equal(got[:, :nt], ref)
    out = torch.empty(G, t0 - 3, d, dtype=torch.uint8, device=DEV)
    N.check(L.qkv_vtiles_unpack(dst.data_ptr(), G, t0 - 3, d, vbits, C // 32, 3, out.data_ptr(), 0))
    assert torch.equal(out.cpu(), full[:, 3:t0])


@pytest.mark.parametrize("d", [64, 128])
def test_decompress_from_store_vs_oracle(d):
    gen = torch.Generator().manual_seed(d)
    B, H, T_ = 2, 3, 77
    k = torch.randn(B, H, T_, d, generator=gen)
    v = torch.randn(B, H, T_, d, generator=gen)
    eng = Q.QuashKVEngine(head_dim=d, seed=5, device=DEV)
    eng.append(k[:, :, :40].to(DEV), v[:, :, :40].to(DEV))
    eng.append(k[:, :, 40:].to(DEV), v[:, :, 40:].to(DEV))
    st = eng._store
    kq, vq = eng.key_quantizer, eng.value_quantizer
    mq = kq.mse_quantizer
    from quashkv_amd.quantizer import decompress_from
    n = B * H * T_
    kh = decompress_from(N.QKV_MODE_MSE, st.kst, None, st.knorm, n, mq.Pi, mq.codebook.centroids,
                         2, None, 0.0, N.QKV_FMT_KPLANES, in_seq=T_, in_group_stride=st.capacity)
    kip = decompress_from(N.QKV_MODE_IP, st.kst, None, st.knorm, n, mq.Pi, mq.codebook.centroids,
                          2, kq.S, kq.qjl_scale, N.QKV_FMT_KPLANES, in_seq=T_,
                          in_group_stride=st.capacity)
    vh = decompress_from(N.QKV_MODE_MSE, st.vst, None, st.vnorm, n, vq.Pi, vq.codebook.centroids,
                         3, None, 0.0, N.QKV_FMT_VTILES, in_seq=T_,
                         in_group_stride=st.capacity // 32)
    kc, kb, vc = st.read_codes(0, T_)
    pi = mq.Pi.cpu()
    kn, vn = st.knorm[:, :, :T_].cpu(), st.vnorm[:, :, :T_].cpu()
    assert_close(kh.reshape(B, H, T_, d), R.decompress_mse(kc.cpu(), kn, pi, mq.codebook.centroids.cpu()),
                 rel=1e-5, cos=0.99999)
    assert_close(kip.reshape(B, H, T_, d),
                 R.decompress_ip(kc.cpu(), kb.cpu(), kn, pi, mq.codebook.centroids.cpu(), kq.S.cpu(),
                                 kq.qjl_scale), rel=1e-5, cos=0.99999)
    assert_close(vh.reshape(B, H, T_, d), R.decompress_mse(vc.cpu(), vn, vq.Pi.cpu(),
                                                           vq.codebook.centroids.cpu()),
                 rel=1e-5, cos=0.99999)
    # the store holds exactly the oracle's codes of the same inputs (from identical y)
    oc, ob, on = R.compress_ip(k, pi, mq.codebook.boundaries.cpu(), kq.S.cpu(),
                               mq.codebook.centroids.cpu())
    assert (kc.cpu() == oc).float().mean() > 0.999
    assert torch.allclose(kn, on, rtol=1e-6)


# -------------------------------------------------------------- attention

CASES = ["single64", "multi64", "single128q1", "multi128", "bits44_d96", "bits23_d64", "bits34_d128"]


@pytest.mark.parametrize("name", CASES)
def test_engine_attention_vs_golden(golden, name):
    g = golden("attention")
    d, H, Qn, kb, vb, packed = [int(v) for v in g[f"{name}_cfg"]]
    seqs = [int(v) for v in g[f"{name}_seqs"]]
    k, v, q = T(g[f"{name}_k"]), T(g[f"{name}_v"]), T(g[f"{name}_q"])
    eng = Q.QuashKVEngine(head_dim=d, key_bits=kb, value_bits=vb, seed=42, device=DEV,
                          pack_storage=bool(packed))
    off = 0
    for sl in seqs:
        eng.append(k[:, :, off:off + sl].to(DEV), v[:, :, off:off + sl].to(DEV))
        off += sl
    out = eng.attention(q.to(DEV))
    assert_close(out, T(g[f"{name}_out"]), rel=1e-3, cos=0.9999)
    outc = eng.attention(q.to(DEV), causal=True)
    assert_close(outc, T(g[f"{name}_out_causal"]), rel=1e-3, cos=0.9999)
    assert abs(eng.compression_ratio() - float(g[f"{name}_ratio"])) < 1e-12
    assert eng.actual_memory_bytes() == int(g[f"{name}_membytes"])
    # identical caches: kernel vs oracle (online softmax) at fp32 tolerance
    blocks = _oracle_blocks(eng)
    kq = eng.key_quantizer
    ref = R.attention_online(q, blocks, kq.mse_quantizer.Pi.cpu(),
                             kq.mse_quantizer.codebook.centroids.cpu(),
                             eng.value_quantizer.codebook.centroids.cpu(), kq.S.cpu(), kq.qjl_scale)
    assert_close(out, ref, rel=2e-5, cos=0.999999)


def _oracle_blocks(eng):
    out = []
    for blk in eng._cache:
        mi, qj, vi = eng._unpack_block(blk)
        out.append(dict(kcodes=mi.cpu(), kbits=qj.cpu(), knorm=blk.key_norms.cpu(),
                        vcodes=vi.cpu(), vnorm=blk.val_norms.cpu()))
    return out


def test_gqa_vs_golden(golden):
    g = golden("attention")
    eng = Q.QuashKVEngine(head_dim=128, seed=42, device=DEV, pack_storage=True)
    eng.append(T(g["gqa_k"]).to(DEV), T(g["gqa_v"]).to(DEV))
    out = eng.attention(T(g["gqa_q"]).to(DEV))
    assert_close(out, T(g["gqa_out"]), rel=1e-3, cos=0.9999)


@pytest.mark.parametrize("d,Hkv,G,Qn,T_,causal,qdt,kb", [
    (128, 8, 4, 1, 3000, False, torch.bfloat16, 3),
    (64, 2, 7, 1, 2049, False, torch.float16, 3),
    (128, 2, 4, 3, 700, True, torch.float32, 3),
    (96, 3, 2, 2, 513, True, torch.float32, 3),
    (128, 1, 40, 1, 300, False, torch.float32, 3),     # 40 rows -> two row chunks
    (128, 8, 4, 1, 3000, False, torch.bfloat16, 4),    # 3-bit key MSE: parity plane
    (128, 2, 4, 3, 700, True, torch.float32, 4),
    (128, 1, 40, 1, 2100, False, torch.float16, 4),
    (96, 4, 4, 1, 2500, False, torch.bfloat16, 3),     # d = 96: zero-padded operands
    (96, 2, 1, 3, 900, True, torch.float32, 4),
    (96, 2, 7, 1, 1100, False, torch.float16, 2),
])
def test_attention_random_vs_oracle(d, Hkv, G, Qn, T_, causal, qdt, kb):
    gen = torch.Generator().manual_seed(T_)
    B = 2
    k = torch.randn(B, Hkv, T_, d, generator=gen)
    k[..., 3] *= 10.0
    v = torch.randn(B, Hkv, T_, d, generator=gen)
    q = torch.randn(B, Hkv * G, Qn, d, generator=gen).to(qdt)
    eng = Q.QuashKVEngine(head_dim=d, key_bits=kb, seed=3, device=DEV, pack_storage=True)
    half = T_ // 3
    eng.append(k[:, :, :half].to(DEV), v[:, :, :half].to(DEV))
    eng.append(k[:, :, half:].to(DEV), v[:, :, half:].to(DEV))
    out = eng.attention(q.to(DEV), causal=causal)
    blocks = _oracle_blocks(eng)
    kq = eng.key_quantizer
    args = (kq.mse_quantizer.Pi.cpu(), kq.mse_quantizer.codebook.centroids.cpu(),
            eng.value_quantizer.codebook.centroids.cpu(), kq.S.cpu(), kq.qjl_scale)
    qr = q.float().reshape(B, Hkv, G * Qn, d)
    if causal:
        assert G == 1 or True
        outs = []
        # rows (g, qi) share a causal position only through qi; evaluate per group member
        for gi in range(G):
            qg = q.float().reshape(B, Hkv, G, Qn, d)[:, :, gi]
            outs.append(R.attention_naive(qg, blocks, *args, causal=True))
        ref = torch.stack(outs, dim=2).reshape(B, Hkv * G, Qn, d)
    else:
        ref = R.attention_online(qr, blocks, *args).reshape(B, Hkv * G, Qn, d)
    assert_close(out, ref, rel=2e-5, cos=0.999999)


def test_attention_split_invariance_full_size():
    """cfg3 shape (B=32, Hq=32, Hkv=8, d=128, T=8192): the fused decode kernel's
    result is independent of the number of splits (size-independent property):
    one split (the kernel merges and un-rotates itself) against 4, 7 and 32
    splits (partials merged by the combine kernel)."""
    gen = torch.Generator(device="cpu").manual_seed(2)
    B, Hkv, G, d, T_ = 32, 8, 4, 128, 8192
    eng = Q.QuashKVEngine(head_dim=d, seed=42, device=DEV, pack_storage=True)
    for c in range(4):
        k = torch.randn(B, Hkv, T_ // 4, d, generator=gen, dtype=torch.float32)
        k[..., [11, 47, 83, 119]] *= 10
        v = torch.randn(B, Hkv, T_ // 4, d, generator=gen, dtype=torch.float32)
        eng.append(k.to(DEV, torch.bfloat16), v.to(DEV, torch.bfloat16))
    q = torch.randn(B, Hkv * G, 1, d, generator=gen).to(DEV, torch.bfloat16)
    st = eng._store
    kq, vq = eng.key_quantizer, eng.value_quantizer
    kh, vh = kq.mse_quantizer.codebook.centroids_host, vq.codebook.centroids_host
    L = N.lib()
    paths = []
    outs = []
    kc_h, vc_h = N.HostFloats(kh), N.HostFloats(vh)   # keep the host tables alive
    for ns in (1, 4, 7, 32):
        paths.append(L.qkv_attention_path(d, 2, 3, kc_h.ptr, vc_h.ptr, st.capacity, T_, ns))
        outs.append(K.attention_store(q, st, T_, kq.mse_quantizer.Pi, kh, vh, kq.S, kq.qjl_scale,
                                      n_splits=ns))
    assert paths == [1, 1, 1, 1]
    # split counts agree with each other over the whole batch
    for o in outs[1:]:
        assert_close(o, outs[0], rel=2e-5, cos=0.999999)
    for o in outs:
        assert torch.isfinite(o).all()
    # every configuration against the oracle on a slice of the batch
    kc, kb, vc = (t[:4] for t in st.read_codes(0, T_))
    blocks = [dict(kcodes=kc.cpu(), kbits=kb.cpu(), knorm=st.knorm[:4, :, :T_].cpu(),
                   vcodes=vc.cpu(), vnorm=st.vnorm[:4, :, :T_].cpu())]
    ref = R.attention_online(q[:4].float().cpu().reshape(4, Hkv, G, d), blocks,
                             kq.mse_quantizer.Pi.cpu(), kq.mse_quantizer.codebook.centroids.cpu(),
                             vq.codebook.centroids.cpu(), kq.S.cpu(), kq.qjl_scale)
    ref = ref.reshape(4, Hkv * G, 1, d)
    for o in outs:
        assert_close(o[:4], ref, rel=2e-5, cos=0.999999)


def test_attention_d64_cfg2_shape_splits_and_paths():
    """cfg2 shape (B=16, Hq=14, Hkv=2, d=64, T=2048, fp16 K/V with log-normal
    token norms): the 64-dim MFMA kernel at several split counts agrees with
    itself, with the VALU kernel (forced by a 32-multiple capacity), and with
    the oracle on a slice of the batch."""
    gen = torch.Generator(device="cpu").manual_seed(5)
    B, Hkv, G, d, T_ = 16, 2, 7, 64, 2048
    k = torch.randn(B, Hkv, T_, d, generator=gen) * torch.exp(0.5 * torch.randn(B, Hkv, T_, 1, generator=gen))
    v = torch.randn(B, Hkv, T_, d, generator=gen) * torch.exp(0.5 * torch.randn(B, Hkv, T_, 1, generator=gen))
    q = torch.randn(B, Hkv * G, 1, d, generator=gen).to(DEV, torch.float16)
    eng = Q.QuashKVEngine(head_dim=d, seed=42, device=DEV)
    eng.append(k.to(DEV, torch.float16), v.to(DEV, torch.float16))
    st = eng._store
    kq, vq = eng.key_quantizer, eng.value_quantizer
    kh, vh = kq.mse_quantizer.codebook.centroids_host, vq.codebook.centroids_host
    kc_h, vc_h = N.HostFloats(kh), N.HostFloats(vh)
    L = N.lib()
    outs = []
    for ns in (1, 2, 5, 16):
        assert L.qkv_attention_path(d, 2, 3, kc_h.ptr, vc_h.ptr, st.capacity, T_, ns) == 1
        outs.append(K.attention_store(q, st, T_, kq.mse_quantizer.Pi, kh, vh, kq.S, kq.qjl_scale,
                                      n_splits=ns))
    for o in outs[1:]:
        assert_close(o, outs[0], rel=2e-5, cos=0.999999)
    # the VALU kernel over a copy of the store whose capacity is not a multiple of 64
    kc, kb, vc = st.read_codes(0, T_)
    st2 = KVStore(B, Hkv, d, 2, 3, 64, st.device)
    st2._alloc(T_ + 32, 0)
    st2.knorm[:, :, :T_].copy_(st.knorm[:, :, :T_])
    st2.vnorm[:, :, :T_].copy_(st.vnorm[:, :, :T_])
    st2.write_codes(0, T_, kc.reshape(-1, d).contiguous(), kb.reshape(-1, d).contiguous(),
                    vc.reshape(-1, d).contiguous())
    assert L.qkv_attention_path(d, 2, 3, kc_h.ptr, vc_h.ptr, st2.capacity, T_, 2) == 0
    valu = K.attention_store(q, st2, T_, kq.mse_quantizer.Pi, kh, vh, kq.S, kq.qjl_scale,
                             n_splits=2)
    assert_close(outs[0], valu, rel=2e-5, cos=0.999999)
    kc, kb, vc = (t[:3] for t in st.read_codes(0, T_))
    blocks = [dict(kcodes=kc.cpu(), kbits=kb.cpu(), knorm=st.knorm[:3, :, :T_].cpu(),
                   vcodes=vc.cpu(), vnorm=st.vnorm[:3, :, :T_].cpu())]
    ref = R.attention_online(q[:3].float().cpu().reshape(3, Hkv, G, d), blocks,
                             kq.mse_quantizer.Pi.cpu(), kq.mse_quantizer.codebook.centroids.cpu(),
                             vq.codebook.centroids.cpu(), kq.S.cpu(), kq.qjl_scale)
    assert_close(outs[0][:3], ref.reshape(3, Hkv * G, 1, d), rel=2e-5, cos=0.999999)


@pytest.mark.parametrize("d,key_bits,value_bits", [
    (d, kb, vb) for d in (128, 64) for kb, vb in ((2, 1), (2, 2), (2, 4), (3, 1), (3, 2), (3, 4))
] + [(128, 4, vb) for vb in (1, 2, 3, 4)] + [(96, kb, vb) for kb in (2, 3, 4) for vb in (1, 4)])
def test_mfma_bit_widths_vs_oracle(key_bits, value_bits, d):
    gen = torch.Generator().manual_seed(10 * key_bits + value_bits + d)
    B, Hkv, G, T_ = 2, 2, 3, 1000
    k = torch.randn(B, Hkv, T_, d, generator=gen)
    v = torch.randn(B, Hkv, T_, d, generator=gen) * torch.exp(torch.randn(B, Hkv, T_, 1, generator=gen))
    q = torch.randn(B, Hkv * G, 1, d, generator=gen)
    eng = Q.QuashKVEngine(head_dim=d, key_bits=key_bits, value_bits=value_bits, seed=7, device=DEV)
    eng.append(k.to(DEV), v.to(DEV))
    st = eng._store
    kq, vq = eng.key_quantizer, eng.value_quantizer
    kh, vh = kq.mse_quantizer.codebook.centroids_host, vq.codebook.centroids_host
    ns = N.lib().qkv_attention_splits(B, Hkv * G, Hkv, 1, d, T_)
    kc_h, vc_h = N.HostFloats(kh), N.HostFloats(vh)
    assert N.lib().qkv_attention_path(d, key_bits - 1, value_bits, kc_h.ptr, vc_h.ptr,
                                      st.capacity, T_, ns) == 1
    out = eng.attention(q.to(DEV))
    blocks = _oracle_blocks(eng)
    ref = R.attention_online(q.reshape(B, Hkv, G, d), blocks, kq.mse_quantizer.Pi.cpu(),
                             kq.mse_quantizer.codebook.centroids.cpu(),
                             vq.codebook.centroids.cpu(), kq.S.cpu(), kq.qjl_scale)
    assert_close(out, ref.reshape(B, Hkv * G, 1, d), rel=2e-5, cos=0.999999)


def test_fused_attention_api_vs_golden(golden):
    g = golden("attention")
    name = "multi64"
    d = 64
    k, v, q = T(g[f"{name}_k"]), T(g[f"{name}_v"]), T(g[f"{name}_q"])
    eng = Q.QuashKVEngine(head_dim=d, seed=42, device=DEV)
    eng.append(k[:, :, :16].to(DEV), v[:, :, :16].to(DEV))
    eng.append(k[:, :, 16:].to(DEV), v[:, :, 16:].to(DEV))
    blocks = []
    for blk in eng._cache:
        mi, qj, vi = eng._unpack_block(blk)
        blocks.append(K.CompressedBlock(mi, qj, blk.key_norms, vi, blk.val_norms, blk.seq_len))
    kq = eng.key_quantizer
    out = K.fused_quantized_attention(q.to(DEV), blocks, kq.mse_quantizer.Pi,
                                      kq.mse_quantizer.codebook.centroids,
                                      eng.value_quantizer.codebook.centroids, kq.S, kq.qjl_scale,
                                      total_kv_tokens=eng.total_tokens)
    assert_close(out, T(g[f"{name}_fused_out"]), rel=1e-3, cos=0.9999)


# ------------------------------------------------------ engine / hf cache

def test_packed_vs_unpacked_engine_identical():
    gen = torch.Generator().manual_seed(42)
    k, v = torch.randn(1, 2, 32, 64, generator=gen), torch.randn(1, 2, 32, 64, generator=gen)
    q = torch.randn(1, 2, 4, 64, generator=gen)
    eu = Q.QuashKVEngine(head_dim=64, seed=42, device=DEV, pack_storage=False)
    ep = Q.QuashKVEngine(head_dim=64, seed=42, device=DEV, pack_storage=True)
    eu.append(k.to(DEV), v.to(DEV))
    ep.append(k.to(DEV), v.to(DEV))
    assert torch.allclose(eu.attention(q.to(DEV)), ep.attention(q.to(DEV)), atol=1e-6)
    assert ep.actual_memory_bytes() < eu.actual_memory_bytes()
    # switching format mid-stream converts the store
    eu.pack_storage = True
    eu.append(k[:, :, :5].to(DEV), v[:, :, :5].to(DEV))
    ep.append(k[:, :, :5].to(DEV), v[:, :, :5].to(DEV))
    assert torch.allclose(eu.attention(q.to(DEV)), ep.attention(q.to(DEV)), atol=1e-6)


def test_engine_growth_and_decode_steps():
    gen = torch.Generator().manual_seed(1)
    eng = Q.QuashKVEngine(head_dim=64, seed=42, device=DEV, pack_storage=True)
    ks, vs = [], []
    eng.append(*(t.to(DEV) for t in (torch.randn(1, 4, 16, 64, generator=gen),) * 2))
    ks.append(eng._cache[0])
    for _ in range(300):   # crosses the initial capacity several times
        k = torch.randn(1, 4, 1, 64, generator=gen)
        eng.append(k.to(DEV), k.to(DEV))
    assert eng.total_tokens == 316 and eng.num_blocks == 301
    out = eng.attention(torch.randn(1, 4, 1, 64, generator=gen).to(DEV))
    assert torch.isfinite(out).all()


def test_hf_cache_vs_golden(golden):
    from quashkv_amd.integrations.hf_cache import QuashKVCache
    g = golden("hf_cache")
    cache = QuashKVCache(num_layers=2, head_dim=64, device=DEV)
    cache.update(T(g["k0"]).to(DEV), T(g["v0"]).to(DEV), layer_idx=1)
    fk, fv = cache.update(T(g["k1"]).to(DEV), T(g["v1"]).to(DEV), layer_idx=1)
    assert_close(fk, T(g["fk"]), rel=1e-3, cos=0.9999)
    assert_close(fv, T(g["fv"]), rel=1e-3, cos=0.9999)
    assert abs(cache.compression_stats()["overall_compression_ratio"] - float(g["stats_ratio"])) < 1e-12
    k1, v1 = cache[1]
    assert torch.equal(k1, fk) and torch.equal(v1, fv)
    for eng in cache.engines:
        eng.pack_storage = True
    fk2, fv2 = cache.update(T(g["k1"]).to(DEV), T(g["v1"]).to(DEV), layer_idx=1)
    assert torch.allclose(fk2[:, :, :13], fk, atol=1e-5)


def test_kernels_api_compress_vs_golden(golden):
    g = golden("compress")
    x = T(g["x_d64"])
    q = Q.MSEQuantizer(64, bits=3, seed=42, device=DEV)
    idx, nr = K.fused_compress_mse(x.to(DEV), q.Pi, q.codebook.boundaries)
    assert (idx.cpu() == T(g["fmse_idx_d64_b3"])).float().mean() >= 0.999
    assert torch.allclose(nr.cpu(), T(g["fmse_norm_d64_b3"]), rtol=1e-6)
    ip = Q.InnerProductQuantizer(64, total_bits=3, seed=42, device=DEV)
    mq = ip.mse_quantizer
    mi, qj, n2 = K.fused_compress_ip(x.to(DEV), mq.Pi, mq.codebook.boundaries, ip.S,
                                     mq.codebook.centroids)
    assert (mi.cpu() == T(g["fip_mse_d64_b3"])).float().mean() >= 0.999
    assert (qj.cpu() == T(g["fip_qjl_d64_b3"])).float().mean() >= 0.999
    xh = K.fused_decompress_mse(T(g["mse_idx_d64_b3"]).to(DEV), T(g["mse_norm_d64_b3"]).to(DEV),
                                q.Pi, q.codebook.centroids)
    assert_close(xh, T(g["fmse_xhat_d64_b3"]), rel=1e-5, cos=0.99999)


@pytest.mark.parametrize("paged", [False, True])
def test_clear_then_new_batch_shape(paged):
    """clear() empties the cache and the next append may have another (B, H)
    (quashkv/engine.py:174-177): append B=2, clear, append B=3 with other kv
    heads, attention against the oracle on the new cache."""
    from quashkv_amd.paged import PagedQuashKVEngine
    gen = torch.Generator().manual_seed(31)
    d = 128
    cls = PagedQuashKVEngine if paged else Q.QuashKVEngine
    eng = cls(head_dim=d, seed=42, device=DEV)
    k = torch.randn(2, 2, 70, d, generator=gen)
    eng.append(k.to(DEV, torch.bfloat16), k.to(DEV, torch.bfloat16))
    with pytest.raises(ValueError, match="does not match"):
        eng.append(k[:1].to(DEV, torch.bfloat16), k[:1].to(DEV, torch.bfloat16))
    eng.clear()
    assert eng.total_tokens == 0
    B, H, G, T_ = 3, 4, 2, 150
    k2 = torch.randn(B, H, T_, d, generator=gen)
    v2 = torch.randn(B, H, T_, d, generator=gen)
    eng.append(k2.to(DEV, torch.bfloat16), v2.to(DEV, torch.bfloat16))
    q = torch.randn(B, H * G, 1, d, generator=gen)
    out = eng.attention(q.to(DEV)).cpu()
    blocks = []
    for blk in eng._cache:
        mi, qj, vi = eng._unpack_block(blk)
        blocks.append(dict(kcodes=mi.cpu(), kbits=qj.cpu(), knorm=blk.key_norms.cpu(),
                           vcodes=vi.cpu(), vnorm=blk.val_norms.cpu()))
    kq, vq = eng.key_quantizer, eng.value_quantizer
    ref = R.attention_online(q.reshape(B, H, G, d), blocks, kq.mse_quantizer.Pi.cpu(),
                             kq.mse_quantizer.codebook.centroids.cpu(),
                             vq.codebook.centroids.cpu(), kq.S.cpu(),
                             kq.qjl_scale).reshape(B, H * G, 1, d)
    assert out.shape == (B, H * G, 1, d)
    assert_close(out, ref, rel=2e-5, cos=0.999999)
