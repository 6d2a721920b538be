"""Pin the CPU oracle (oracle/ref_math.py) to the reference.

Golden vectors were written by the reference itself (tests/golden/make_golden.py);
closed forms and invariants cover what the vectors leave open.  CPU only.
"""

import math

import numpy as np
import pytest
import torch

from oracle import ref_math as R


def T(a):
    return torch.from_numpy(np.asarray(a))


# ---------------------------------------------------------------- parameters

@pytest.mark.parametrize("d,seed", [(64, 42), (64, 43), (64, 65), (96, 42), (128, 42), (128, 43), (128, 7)])
def test_rotation_and_signs_match_golden(golden, d, seed):
    g = golden("rotations")
    assert torch.equal(R.random_orthogonal(d, seed), T(g[f"Pi_d{d}_s{seed}"]))
    assert torch.equal(R.random_signs(d, seed), T(g[f"S_d{d}_s{seed}"]))


@pytest.mark.parametrize("d,seed", [(64, 42), (128, 42)])
def test_rotation_is_sign_fixed_qr(d, seed):
    # Pi is the unique Q of A = Q R with diag(R) > 0: Pi^T A upper triangular
    # with a positive diagonal, and Pi orthogonal.
    gen = torch.Generator().manual_seed(seed)
    a = torch.randn(d, d, generator=gen, dtype=torch.float32).double()
    pi = R.random_orthogonal(d, seed).double()
    r = pi.T @ a
    assert torch.allclose(torch.tril(r, -1), torch.zeros_like(r), atol=1e-4)
    assert (torch.diag(r) > 0).all()
    assert torch.allclose(pi.T @ pi, torch.eye(d, dtype=torch.float64), atol=1e-5)


def test_signs_are_pm1_and_seed_offset():
    s = R.random_signs(128, 42)
    assert set(s.tolist()) <= {-1.0, 1.0}
    # seed + 1e6 offset: the signs of seed 42 are NOT those of a plain seed-42 randint
    gen = torch.Generator().manual_seed(42)
    plain = torch.randint(0, 2, (128,), generator=gen, dtype=torch.float32) * 2 - 1
    assert not torch.equal(s, plain)


# ------------------------------------------------------------------- packing

def test_packing_known_answers():
    assert R.pack_bits(np.arange(8, dtype=np.uint8)[None], 3).tolist() == [[0x88, 0xC6, 0xFA]]
    assert R.pack_bits(np.array([[0, 1, 2, 3]], np.uint8), 2).tolist() == [[0xE4]]
    assert R.pack_bits(np.array([[1, 2]], np.uint8), 4).tolist() == [[0x21]]
    assert R.pack_bits(np.array([[1, 0, 1, 1, 0, 0, 0, 1]], np.uint8), 1).tolist() == [[0x8D]]


@pytest.mark.parametrize("d", [8, 63, 64, 65, 100, 128])
@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_packing_matches_golden(golden, d, bits):
    g = golden("packing")
    codes = g[f"codes_d{d}_b{bits}"]
    packed = R.pack_bits(codes, bits)
    assert np.array_equal(packed, g[f"packed_d{d}_b{bits}"])
    assert np.array_equal(R.unpack_bits(packed, bits, d), codes)
    assert R.packed_size(d, bits) == int(g[f"psize_d{d}_b{bits}"])
    assert packed.shape[-1] == R.packed_row_bytes(d, bits)


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_packing_bruteforce_bits(bits):
    rng = np.random.default_rng(bits)
    codes = rng.integers(0, 1 << bits, (3, 19), dtype=np.uint8)
    packed = R.pack_bits(codes, bits)
    # brute force: bit k of value j lives at stream position j*bits + k (LSB first)
    for r in range(codes.shape[0]):
        for j in range(codes.shape[1]):
            for k in range(bits):
                pos = j * bits + k
                assert ((packed[r, pos // 8] >> (pos % 8)) & 1) == ((codes[r, j] >> k) & 1)


def test_packing_8bit_passthrough():
    c = np.arange(256, dtype=np.uint8).reshape(2, 128)
    assert np.array_equal(R.pack_bits(c, 8), c)
    assert np.array_equal(R.unpack_bits(c, 8, 128), c)


# ------------------------------------------------------------ boundary search

@pytest.mark.parametrize("d,bits", [(128, 2), (128, 3), (64, 4), (128, 1)])
def test_quantize_boundary_ties_golden(golden, d, bits):
    g = golden("compress")
    cb = golden("codebooks")
    y = T(g[f"tie_y_d{d}_b{bits}"])
    t = T(cb[f"t_d{d}_b{bits}"])
    out = R.quantize_boundary(y, t)
    assert torch.equal(out, T(g[f"tie_code_d{d}_b{bits}"]))
    assert torch.equal(out, T(g[f"tie_bucket_d{d}_b{bits}"]))


def test_quantize_boundary_equals_argmin(golden):
    cb = golden("codebooks")
    for bits in (1, 2, 3, 4):
        c, t = T(cb[f"c_d128_b{bits}"]), T(cb[f"t_d128_b{bits}"])
        y = torch.randn(4000) / math.sqrt(128)
        assert torch.equal(R.quantize_boundary(y, t), R.quantize_argmin(y, c))


# ----------------------------------------------------------- compress/decomp

@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_compress_mse_golden(golden, d, bits):
    g, cb, rot = golden("compress"), golden("codebooks"), golden("rotations")
    x = T(g[f"x_d{d}"])
    pi = T(rot[f"Pi_d{d}_s42"])
    t, c = T(cb[f"t_d{d}_b{bits}"]), T(cb[f"c_d{d}_b{bits}"])
    codes, norms = R.compress_mse(x, pi, t)
    assert torch.equal(codes, T(g[f"mse_idx_d{d}_b{bits}"]))
    assert torch.equal(codes, T(g[f"fmse_idx_d{d}_b{bits}"]))
    assert torch.equal(norms, T(g[f"mse_norm_d{d}_b{bits}"]))
    # codes from the reference's own y are reproduced exactly
    assert torch.equal(R.quantize_boundary(T(g[f"mse_y_d{d}_b{bits}"]), t),
                       T(g[f"mse_qb_d{d}_b{bits}"]))
    xh = R.decompress_mse(codes, norms, pi, c)
    assert torch.allclose(xh, T(g[f"mse_xhat_d{d}_b{bits}"]), rtol=1e-5, atol=1e-6)
    assert torch.allclose(xh, T(g[f"fmse_xhat_d{d}_b{bits}"]), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("tb", [2, 3, 4])
def test_compress_ip_golden(golden, d, tb):
    g, cb, rot = golden("compress"), golden("codebooks"), golden("rotations")
    x = T(g[f"x_d{d}"])
    pi, s = T(rot[f"Pi_d{d}_s42"]), T(rot[f"S_d{d}_s42"])
    t, c = T(cb[f"t_d{d}_b{tb - 1}"]), T(cb[f"c_d{d}_b{tb - 1}"])
    codes, bits, norms = R.compress_ip(x, pi, t, s, c)
    assert torch.equal(codes, T(g[f"ip_mse_d{d}_b{tb}"]))
    assert torch.equal(bits, T(g[f"ip_qjl_d{d}_b{tb}"]))
    assert torch.equal(norms, T(g[f"ip_norm_d{d}_b{tb}"]))
    assert torch.equal(codes, T(g[f"fip_mse_d{d}_b{tb}"]))
    assert torch.equal(bits, T(g[f"fip_qjl_d{d}_b{tb}"]))
    alpha = R.QJL_COEFF / d
    xh = R.decompress_ip(codes, bits, norms, pi, c, s, alpha)
    assert torch.allclose(xh, T(g[f"fip_xhat_d{d}_b{tb}"]), rtol=1e-5, atol=1e-6)
    qv = T(g[f"ip_q_d{d}_b{tb}"])
    q_rot = (qv.unsqueeze(0) @ pi.T).expand(*x.shape[:-1], d)
    dot = R.decompress_for_dot(codes, bits, norms, q_rot, c, s, alpha)
    assert torch.allclose(dot, T(g[f"ip_dot_d{d}_b{tb}"]), rtol=1e-5, atol=1e-5)


def test_compress_orientation_unit_vectors(golden):
    # x = e_k  =>  y = Pi[:, k]: pins the y = u Pi^T orientation.
    rot, cb = golden("rotations"), golden("codebooks")
    pi, t = T(rot["Pi_d64_s42"]), T(cb["t_d64_b3"])
    x = torch.eye(64)
    codes, norms = R.compress_mse(x, pi, t)
    assert torch.equal(codes, R.quantize_boundary(pi.T.contiguous(), t))
    assert torch.equal(norms, torch.ones(64))


def test_zero_vector_norm_clamp(golden):
    g = golden("compress")
    assert float(g["mse_norm_d128_b3"][0, 0, 0]) == np.float32(1e-8)


# ----------------------------------------------------------------- attention

def _blocks_from(golden_name_k, golden_name_v, seqs, d, kb, vb, seed=42):
    """Build oracle blocks by compressing the stored K/V per block."""
    from oracle.ref_math import compress_ip, compress_mse
    import tests.conftest as C
    cb = C.load_golden("codebooks")
    pi, s = R.random_orthogonal(d, seed), R.random_signs(d, seed)
    kt, kc = T(cb[f"t_d{d}_b{kb - 1}"]), T(cb[f"c_d{d}_b{kb - 1}"])
    vt, vc = T(cb[f"t_d{d}_b{vb}"]), T(cb[f"c_d{d}_b{vb}"])
    blocks, off = [], 0
    for sl in seqs:
        k = golden_name_k[:, :, off:off + sl]
        v = golden_name_v[:, :, off:off + sl]
        kcodes, kbits, kn = compress_ip(k, pi, kt, s, kc)
        vcodes, vn = compress_mse(v, pi, vt)
        blocks.append(dict(kcodes=kcodes, kbits=kbits, knorm=kn, vcodes=vcodes, vnorm=vn))
        off += sl
    return blocks, pi, s, kc, vc


CASES = ["single64", "multi64", "single128q1", "multi128", "bits44_d96", "bits23_d64", "bits34_d128"]


@pytest.mark.parametrize("name", CASES)
def test_attention_golden(golden, name):
    g = golden("attention")
    d, H, Q, kb, vb, packed = [int(v) for v in g[f"{name}_cfg"]]
    seqs = [int(v) for v in g[f"{name}_seqs"]]
    blocks, pi, s, kc, vc = _blocks_from(T(g[f"{name}_k"]), T(g[f"{name}_v"]), seqs, d, kb, vb)
    q = T(g[f"{name}_q"])
    alpha = R.QJL_COEFF / d
    out = R.attention_naive(q, blocks, pi, kc, vc, s, alpha)
    assert torch.allclose(out, T(g[f"{name}_out"]), rtol=1e-5, atol=1e-6)
    outc = R.attention_naive(q, blocks, pi, kc, vc, s, alpha, causal=True)
    assert torch.allclose(outc, T(g[f"{name}_out_causal"]), rtol=1e-5, atol=1e-6)
    on = R.attention_online(q, blocks, pi, kc, vc, s, alpha)
    assert torch.allclose(on, T(g[f"{name}_fused_out"]), rtol=1e-5, atol=1e-6)
    assert torch.allclose(on, out, atol=1e-5)
    assert abs(R.compression_ratio(d, kb, vb) - float(g[f"{name}_ratio"])) < 1e-12


def test_attention_gqa_golden(golden):
    g = golden("attention")
    blocks, pi, s, kc, vc = _blocks_from(T(g["gqa_k"]), T(g["gqa_v"]), [48], 128, 3, 3)
    out = R.attention_gqa(T(g["gqa_q"]), blocks, pi, kc, vc, s, R.QJL_COEFF / 128, online=False)
    assert torch.allclose(out, T(g["gqa_out"]), rtol=1e-5, atol=1e-6)


def test_attention_bruteforce_tiny():
    torch.manual_seed(3)
    d, T_ = 8, 5
    pi = R.random_orthogonal(d, 5)
    s = R.random_signs(d, 5)
    kc = torch.tensor([-0.5, -0.1, 0.1, 0.5])
    vc = torch.linspace(-0.7, 0.7, 8)
    kcodes = torch.randint(0, 4, (T_, d), dtype=torch.uint8)
    kbits = torch.randint(0, 2, (T_, d), dtype=torch.uint8)
    vcodes = torch.randint(0, 8, (T_, d), dtype=torch.uint8)
    kn, vn = torch.rand(T_) + 0.5, torch.rand(T_) + 0.5
    q = torch.randn(2, d)
    alpha = R.QJL_COEFF / d
    bf = R.attention_bruteforce(q, kcodes, kbits, kn, vcodes, vn, pi, kc, vc, s, alpha)
    blk = dict(kcodes=kcodes[None, None], kbits=kbits[None, None], knorm=kn[None, None],
               vcodes=vcodes[None, None], vnorm=vn[None, None])
    out = R.attention_naive(q[None, None], [blk], pi, kc, vc, s, alpha)[0, 0]
    assert torch.allclose(out.double(), bf, atol=1e-5)


def test_attention_empty_raises():
    with pytest.raises(ValueError, match="No compressed KV blocks"):
        R.attention_naive(torch.zeros(1, 1, 1, 8), [], None, None, None, None, 0.1)


# --------------------------------------------------------- mixed and index

def test_mixed_golden(golden):
    g, cb = golden("mixed"), golden("codebooks")
    pi = R.random_orthogonal(128, 42)
    out = R.mixed_calibrate(T(g["calib"]), pi, 32)
    assert torch.equal(out, T(g["outliers"]))
    codes, norms = R.mixed_compress(T(g["x"]), pi, out, T(cb["t_d128_b3"]), T(cb["t_d128_b2"]))
    assert torch.equal(codes, T(g["idx"]))
    assert torch.equal(norms, T(g["norm"]))
    xh = R.mixed_decompress(codes, norms, pi, out, T(cb["c_d128_b3"]), T(cb["c_d128_b2"]))
    assert torch.allclose(xh, T(g["xhat"]), rtol=1e-5, atol=1e-6)
    pi2 = R.random_orthogonal(64, 43)
    c2, n2 = R.mixed_compress(T(g["x2"]), pi2, None, None, T(cb["t_d64_b2"]))
    assert torch.equal(c2, T(g["idx2"]))
    xh2 = R.mixed_decompress(c2, n2, pi2, None, None, T(cb["c_d64_b2"]))
    assert torch.allclose(xh2, T(g["xhat2"]), rtol=1e-5, atol=1e-6)


def test_attention_mixed_keys_pinned(golden):
    """attention_mixed_keys (decompress-then-attend) against a scalar fp64 loop
    of softmax(q k / sqrt(d)) v over keys from the golden-pinned
    mixed_decompress, with GQA head h -> kv head h // G."""
    cb = golden("codebooks")
    g = torch.Generator().manual_seed(4)
    B, H, G, Tn, d = 1, 2, 3, 9, 128
    pi_k, pi_v = R.random_orthogonal(d, 42), R.random_orthogonal(d, 7)
    out_idx = torch.arange(0, 128, 4)
    kc = torch.randint(0, 4, (B, H, Tn, d), generator=g, dtype=torch.uint8)
    kc[..., out_idx] = torch.randint(0, 8, (B, H, Tn, 32), generator=g, dtype=torch.uint8)
    vc = torch.randint(0, 16, (B, H, Tn, d), generator=g, dtype=torch.uint8)
    kn = torch.rand(B, H, Tn, generator=g) + 0.5
    vn = torch.rand(B, H, Tn, generator=g) + 0.5
    q = torch.randn(B, H * G, 1, d, generator=g)
    c_out, c_reg, c_v = T(cb["c_d128_b3"]), T(cb["c_d128_b2"]), T(cb["c_d128_b4"])
    got = R.attention_mixed_keys(q, kc, kn, vc, vn, pi_k, out_idx, c_out, c_reg, pi_v, c_v)
    k = R.mixed_decompress(kc, kn, pi_k, out_idx, c_out, c_reg).double()
    v = ((c_v[vc.long()] @ pi_v) * vn.unsqueeze(-1)).double()
    ref = torch.zeros(B, H * G, 1, d, dtype=torch.float64)
    for h in range(H * G):
        kv = h // G
        s = [float(q[0, h, 0].double() @ k[0, kv, t]) / math.sqrt(d) for t in range(Tn)]
        m = max(s)
        p = [math.exp(x - m) for x in s]
        ref[0, h, 0] = sum(p[t] * v[0, kv, t] for t in range(Tn)) / sum(p)
    assert torch.allclose(got.double(), ref, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("tag", ["a", "b", "c", "d"])
def test_mixed_ip_golden(golden, tag):
    """mixed_ip_compress against MixedPrecisionIPQuantizer.compress's own
    outputs (codes, QJL bits and norms bit for bit): d 128 with 32 and 64
    outliers, d 64 with 4/3-bit channels, and an uncalibrated quantizer
    (regular codebook everywhere)."""
    g, cb = golden("mixed_ip"), golden("codebooks")
    d, ob, rb, n_out, seed, calibrated = (int(v) for v in g[f"{tag}_cfg"])
    pi, s = R.random_orthogonal(d, seed), R.random_signs(d, seed)
    assert torch.equal(s, T(g[f"{tag}_S"]))
    out_idx = T(g[f"{tag}_outliers"]) if calibrated else None
    if calibrated:
        assert out_idx.numel() == n_out
    tabs = (T(cb[f"c_d{d}_b{ob - 1}"]), T(cb[f"t_d{d}_b{ob - 1}"]),
            T(cb[f"c_d{d}_b{rb - 1}"]), T(cb[f"t_d{d}_b{rb - 1}"]))
    codes, bits, norms = R.mixed_ip_compress(T(g[f"{tag}_x"]), pi, out_idx, *tabs, s)
    assert torch.equal(codes, T(g[f"{tag}_codes"]))
    assert torch.equal(bits, T(g[f"{tag}_qjl"]))
    assert torch.equal(norms, T(g[f"{tag}_norm"]))


def test_attention_mixed_ip_keys_pinned(golden):
    """attention_mixed_ip_keys against the golden-pinned routines: with every
    channel in one codebook (no outliers, or all outliers) it is
    attention_naive over IP blocks, causal and not; mixed, its scores are the
    sum of decompress_for_dot over the outlier channels with the outlier
    codebook and over the rest with the regular one (the other channels'
    query zeroed), through an fp64 softmax with GQA head h -> kv head h // G."""
    cb = golden("codebooks")
    g = torch.Generator().manual_seed(9)
    B, H, G, Q, Tn, d = 2, 2, 3, 2, 11, 128
    pi_k, pi_v = R.random_orthogonal(d, 42), R.random_orthogonal(d, 7)
    s = R.random_signs(d, 42)
    alpha = R.QJL_COEFF / d
    c_out, c_reg, c_v = T(cb["c_d128_b2"]), T(cb["c_d128_b1"]), T(cb["c_d128_b3"])
    kb = torch.randint(0, 2, (B, H, Tn, d), generator=g, dtype=torch.uint8)
    vc = torch.randint(0, 8, (B, H, Tn, d), generator=g, dtype=torch.uint8)
    kn = torch.rand(B, H, Tn, generator=g) + 0.5
    vn = torch.rand(B, H, Tn, generator=g) + 0.5
    # one codebook everywhere (G = 1, values un-rotated by the key Pi as the
    # IP engine does): attention_naive, pinned by attention.npz
    q1 = torch.randn(B, H, Q, d, generator=g)
    for outl, c_all in ((None, c_reg), (torch.arange(d), c_out)):
        codes = torch.randint(0, c_all.numel(), (B, H, Tn, d), generator=g, dtype=torch.uint8)
        blk = dict(kcodes=codes, kbits=kb, knorm=kn, vcodes=vc, vnorm=vn)
        for causal in (False, True):
            got = R.attention_mixed_ip_keys(q1, codes, kb, kn, vc, vn, pi_k, outl, c_out, c_reg,
                                            s, alpha, pi_k, c_v, causal=causal)
            ref = R.attention_naive(q1, [blk], pi_k, c_all, c_v, s, alpha, causal=causal)
            assert torch.allclose(got, ref, rtol=1e-5, atol=1e-6)
    # mixed: per-codebook decompress_for_dot, fp64 softmax
    out_idx = torch.arange(1, 128, 4)
    mask = torch.zeros(d, dtype=torch.bool)
    mask[out_idx] = True
    kc = torch.randint(0, 2, (B, H, Tn, d), generator=g, dtype=torch.uint8)
    kc[..., out_idx] = torch.randint(0, 4, (B, H, Tn, 32), generator=g, dtype=torch.uint8)
    q = torch.randn(B, H * G, Q, d, generator=g)
    got = R.attention_mixed_ip_keys(q, kc, kb, kn, vc, vn, pi_k, out_idx, c_out, c_reg, s,
                                    alpha, pi_v, c_v)
    q_rot = (q @ pi_k.T).reshape(B, H, G * Q, 1, d)
    one = torch.ones(B, H, 1, Tn)
    kc5, kb5 = kc.unsqueeze(2), kb.unsqueeze(2)
    sc = (R.decompress_for_dot(kc5, kb5, one, q_rot * mask, c_out, s * mask, alpha)
          + R.decompress_for_dot(kc5.clamp(max=1), kb5, one, q_rot * ~mask, c_reg, s * ~mask,
                                 alpha))
    sc = (kn.unsqueeze(2) * sc).double() / math.sqrt(d)
    w = torch.softmax(sc, dim=-1)
    v = ((c_v[vc.long()] @ pi_v) * vn.unsqueeze(-1)).double()
    ref = (w @ v).reshape(B, H * G, Q, d)
    assert torch.allclose(got.double(), ref, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("d,bits", [(64, 3), (128, 3), (128, 4)])
def test_index_golden(golden, d, bits):
    g, cb = golden("index"), golden("codebooks")
    pi, s = R.random_orthogonal(d, 42), R.random_signs(d, 42)
    t, c = T(cb[f"t_d{d}_b{bits - 1}"]), T(cb[f"c_d{d}_b{bits - 1}"])
    db = T(g[f"db_d{d}_b{bits}"])
    codes, qb, norms = R.compress_ip(db, pi, t, s, c)
    sc, ix = R.index_search(T(g[f"q_d{d}_b{bits}"]), codes, qb, norms, pi, c, s,
                            R.QJL_COEFF / d, 10, chunk=7)
    assert torch.equal(ix, T(g[f"ids_d{d}_b{bits}"]))
    assert torch.allclose(sc, T(g[f"scores_d{d}_b{bits}"]), rtol=1e-5, atol=1e-5)
