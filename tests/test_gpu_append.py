"""GPU parity of the fused store append (qkv_store_append: bf16 / fp16 K and V
rows at head_dim 128 or 64 compressed straight into the K-row / V-tile store).

Its rotation carries ~16 (bf16) / ~22 (fp16) significant bits of Pi, so codes
agree with the fp32 reference except where the rotated value sits within
~1e-5 relative of a boundary or centroid: the bar is a mismatch rate
<= 1e-4 per code stream, every mismatch one code step, norms to 2e-6, and
bit-exact preservation of the store outside the appended tokens."""

import numpy as np
import pytest
import torch

import quashkv_amd as Q
from quashkv_amd import _native as N
from oracle import ref_math as R

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(autouse=True, scope="module")
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")
    N.lib()


def _rows(gen, shape, dtype, outliers=True):
    x = torch.randn(*shape, generator=gen)
    if outliers:
        x[..., [c for c in (11, 47, 83, 119) if c < shape[-1]]] *= 10.0
    return x.to(dtype)


def _engines(key_bits, value_bits, seed=5, d=128):
    fused = Q.QuashKVEngine(head_dim=d, key_bits=key_bits, value_bits=value_bits, seed=seed,
                            device=DEV)
    generic = Q.QuashKVEngine(head_dim=d, key_bits=key_bits, value_bits=value_bits, seed=seed,
                              device=DEV)
    generic._append_fused = lambda *a: False   # the unfused compress + converters path
    return fused, generic


def _mismatch(a, b):
    a, b = a.cpu().to(torch.int16), b.cpu().to(torch.int16)
    diff = (a - b).abs()
    return float((diff != 0).double().mean()), int(diff.max()) if diff.numel() else 0


@pytest.mark.parametrize("d", [128, 96, 64])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("key_bits,value_bits", [(3, 3), (2, 1), (4, 4), (3, 2)])
def test_store_append_matches_unfused_path(dtype, key_bits, value_bits, d):
    gen = torch.Generator().manual_seed(key_bits * 10 + value_bits + d)
    B, H = 2, 3
    fused, generic = _engines(key_bits, value_bits, d=d)
    total = 0
    for S in (150, 37, 1, 64, 0, 95):        # ragged sizes, unaligned starts
        k = _rows(gen, (B, H, S, d), dtype)
        v = _rows(gen, (B, H, S, d), dtype, outliers=False)
        fused.append(k.to(DEV), v.to(DEV))
        generic.append(k.to(DEV), v.to(DEV))
        total += S
    sf, sg = fused._store, generic._store
    for a, b in zip(sf.read_codes(0, total), sg.read_codes(0, total)):
        rate, step = _mismatch(a, b)
        assert rate <= 1e-4 and step <= 1, (rate, step)
    for a, b in ((sf.knorm, sg.knorm), (sf.vnorm, sg.vnorm)):
        a, b = a[:, :, :total].cpu().double(), b[:, :, :total].cpu().double()
        assert float(((a - b).abs() / b).max()) <= 2e-6


@pytest.mark.parametrize("d", [128, 96, 64])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_store_append_vs_oracle(dtype, d):
    """Codes and norms against the CPU restatement of compress_ip / compress_mse
    (quashkv/quantizer.py:113-131, 211-242) on the same (upcast) inputs."""
    gen = torch.Generator().manual_seed(3)
    B, H, S = 2, 4, 700
    k = _rows(gen, (B, H, S, d), dtype)
    v = _rows(gen, (B, H, S, d), dtype, outliers=False)
    eng = Q.QuashKVEngine(head_dim=d, seed=42, device=DEV)
    eng.append(k.to(DEV), v.to(DEV))
    st = eng._store
    kc, kb, vc = st.read_codes(0, S)
    kq, vq = eng.key_quantizer, eng.value_quantizer
    mq = kq.mse_quantizer
    okc, okb, okn = R.compress_ip(k.float().reshape(-1, d), mq.Pi.cpu(),
                                  mq.codebook.boundaries.cpu(), kq.S.cpu(),
                                  mq.codebook.centroids.cpu())
    ovc, ovn = R.compress_mse(v.float().reshape(-1, d), vq.Pi.cpu(),
                              vq.codebook.boundaries.cpu())
    # fp32 rows are split hi + lo for the fp16 MFMA: ~22 bits, fewer near-ties
    bar = 2e-5 if dtype == torch.float32 else 1e-4
    for got, ref in ((kc, okc), (kb, okb), (vc, ovc)):
        rate, step = _mismatch(got.reshape(-1, d), ref.reshape(-1, d))
        assert rate <= bar and step <= 1, (rate, step)
    for got, ref in ((st.knorm[:, :, :S], okn), (st.vnorm[:, :, :S], ovn)):
        got, ref = got.cpu().double().reshape(-1), ref.double().reshape(-1)
        assert float(((got - ref).abs() / ref).max()) <= 2e-6


def test_store_append_keeps_other_tokens():
    """Tokens outside [t0, t0 + S) keep their bytes (K rows, norms) and bits (the
    partially covered V tiles are read-modify-written)."""
    gen = torch.Generator().manual_seed(9)
    B, H = 1, 3
    eng = Q.QuashKVEngine(head_dim=128, seed=42, device=DEV, capacity=256)
    eng.append(*(_rows(gen, (B, H, 70, 128), torch.bfloat16).to(DEV) for _ in range(2)))
    st = eng._store
    g = torch.Generator(device="cpu").manual_seed(1)
    # scribble over everything past token 70, then append 45 tokens at t0 = 70
    st.kst[:, :, 70:] = torch.randint(0, 256, st.kst[:, :, 70:].shape, generator=g,
                                      dtype=torch.uint8).to(DEV)
    st.knorm[:, :, 70:] = 7.0
    st.vnorm[:, :, 70:] = 7.0
    tail = torch.randint(-2**31, 2**31 - 1, st.vst[:, :, 2:].shape, generator=g,
                         dtype=torch.int64).to(torch.int32).to(DEV)
    st.vst[:, :, 2:] = tail
    before = [t.clone() for t in (st.kst, st.knorm, st.vst, st.vnorm)]
    k = _rows(gen, (B, H, 45, 128), torch.bfloat16)
    eng.append(k.to(DEV), k.to(DEV))
    kst, knorm, vst, vnorm = st.kst, st.knorm, st.vst, st.vnorm
    assert torch.equal(kst[:, :, :70], before[0][:, :, :70])
    assert torch.equal(kst[:, :, 115:], before[0][:, :, 115:])
    for cur, old in ((knorm, before[1]), (vnorm, before[3])):
        assert torch.equal(cur[:, :, :70], old[:, :, :70])
        assert torch.equal(cur[:, :, 115:], old[:, :, 115:])
        assert bool((cur[:, :, 70:115] != 7.0).all())
    # V tiles: tile 2 = tokens 64..95 (bits 0..5 kept), tile 3 = 96..127 (bits 19.. kept)
    w_old = before[2].view(torch.int32).cpu().numpy().view(np.uint32)
    w_new = vst.view(torch.int32).cpu().numpy().view(np.uint32)
    keep2 = np.uint32((1 << 6) - 1)
    keep3 = np.uint32(0xFFFFFFFF ^ ((1 << 19) - 1))
    assert np.array_equal(w_new[:, :, :2], w_old[:, :, :2])
    assert np.array_equal(w_new[:, :, 2] & keep2, w_old[:, :, 2] & keep2)
    assert np.array_equal(w_new[:, :, 3] & keep3, w_old[:, :, 3] & keep3)
    assert np.array_equal(w_new[:, :, 4:], w_old[:, :, 4:])
    # and the appended codes agree with the unfused path on the same rows
    ref = Q.QuashKVEngine(head_dim=128, seed=42, device=DEV)
    ref._append_fused = lambda *a: False
    ref.append(k.to(DEV), k.to(DEV))
    for a, b in zip(st.read_codes(70, 45), ref._store.read_codes(0, 45)):
        rate, step = _mismatch(a, b)
        assert rate <= 1e-4 and step <= 1


def test_fused_append_engine_attention_vs_oracle():
    """Engine over bf16 appends (fused store path) against the oracle's
    attention on the oracle's own codes of the same inputs: the end-to-end
    bar for bf16 inputs (rel-err <= 1e-2, cosine >= 0.9999)."""
    gen = torch.Generator().manual_seed(11)
    B, Hkv, G, S = 2, 2, 4, 600
    k = _rows(gen, (B, Hkv, S, 128), torch.bfloat16)
    v = _rows(gen, (B, Hkv, S, 128), torch.bfloat16, outliers=False)
    q = torch.randn(B, Hkv * G, 1, 128, generator=gen).to(torch.bfloat16)
    eng = Q.QuashKVEngine(head_dim=128, seed=42, device=DEV)
    eng.append(k.to(DEV), v.to(DEV))
    out = eng.attention(q.to(DEV)).cpu().double()
    kq, vq = eng.key_quantizer, eng.value_quantizer
    mq = kq.mse_quantizer
    okc, okb, okn = R.compress_ip(k.float(), mq.Pi.cpu(), mq.codebook.boundaries.cpu(),
                                  kq.S.cpu(), mq.codebook.centroids.cpu())
    ovc, ovn = R.compress_mse(v.float(), vq.Pi.cpu(), vq.codebook.boundaries.cpu())
    blocks = [dict(kcodes=okc, kbits=okb, knorm=okn, vcodes=ovc, vnorm=ovn)]
    ref = R.attention_online(q.float().reshape(B, Hkv, G, 128), blocks, mq.Pi.cpu(),
                             mq.codebook.centroids.cpu(), vq.codebook.centroids.cpu(),
                             kq.S.cpu(), kq.qjl_scale).reshape(B, Hkv * G, 1, 128).double()
    err = float((out - ref).norm() / ref.norm())
    cos = float((out.flatten() @ ref.flatten()) / (out.norm() * ref.norm()))
    assert err <= 1e-2 and cos >= 0.9999, (err, cos)


# ---------------------------------------------------------------- from y
#
# qkv_store_append_rotated / qkv_store_append_kmixed_rotated run the search,
# QJL and store code of the fused append on a given rotated y: codes equal the
# reference's quantize_boundary / [(y - c[code]) S >= 0] bit for bit, on
# values chosen to hit every tie: each boundary and centroid, its neighbours
# one ulp away on both sides, both signs, +-0, denormals and huge values.

def _specials(values):
    sp = [0.0, -0.0, 1e-45, -1e-45, 1e-30, -1e-30, 1e30, -1e30, 1.0, -1.0]
    for v in values:
        v = np.float32(v)
        for w in (v, -v):
            sp += [w, np.nextafter(w, np.float32(np.inf)), np.nextafter(w, np.float32(-np.inf))]
    return np.asarray(sp, dtype=np.float32)


def _special_rows(seed, shape, values, n_random=0):
    """Rows of special values at random coordinates (each value lands on
    coordinates of both QJL signs), plus n_random rows of random unit y."""
    sp = _specials(values)
    rng = np.random.default_rng(seed)
    y = sp[rng.integers(0, len(sp), size=shape)]
    if n_random:
        r = rng.standard_normal((*shape[:-2], n_random, shape[-1])).astype(np.float32)
        r /= np.linalg.norm(r, axis=-1, keepdims=True)
        y[..., :n_random, :] = r
    return torch.from_numpy(y)


@pytest.mark.parametrize("d", [128, 96, 64])
@pytest.mark.parametrize("mbits,vbits", [(1, 1), (2, 3), (3, 4), (2, 2), (1, 4), (3, 1)])
def test_store_append_rotated_bit_exact(d, mbits, vbits):
    from quashkv_amd.store import KVStore
    groups_b, H, S = 2, 3, 300
    kq = Q.InnerProductQuantizer(d=d, total_bits=mbits + 1, seed=17, device=DEV)
    vq = Q.MSEQuantizer(d=d, bits=vbits, seed=17, device=DEV)
    mq = kq.mse_quantizer
    kcb, vcb = mq.codebook, vq.codebook
    yk = _special_rows(mbits * 7 + d, (groups_b, H, S, d),
                       list(kcb.centroids_host) + list(kcb.boundaries_host), n_random=40)
    yv = _special_rows(vbits * 5 + d, (groups_b, H, S, d), list(vcb.boundaries_host),
                       n_random=40)
    g = torch.Generator().manual_seed(d)
    kn = torch.rand(groups_b, H, S, generator=g) + 0.5
    vn = torch.rand(groups_b, H, S, generator=g) + 0.5
    st = KVStore(groups_b, H, d, mbits, vbits, S, DEV)
    t0 = 0
    yk_d, yv_d, kn_d, vn_d = (t.contiguous().to(DEV) for t in (yk, yv, kn, vn))
    kc_h, kb_h, vb_h = (N.HostFloats(kcb.centroids_host), N.HostFloats(kcb.boundaries_host),
                        N.HostFloats(vcb.boundaries_host))
    N.check(N.lib().qkv_store_append_rotated(
        yk_d.data_ptr(), kn_d.data_ptr(), yv_d.data_ptr(), vn_d.data_ptr(), groups_b * H, S, d,
        mbits, vbits, kq.S.data_ptr(), kc_h.ptr, kb_h.ptr, vb_h.ptr, st.kst.data_ptr(),
        st.knorm.data_ptr(), st.vst.data_ptr(), st.vnorm.data_ptr(), st.capacity, t0,
        N.stream(torch.device(DEV))))
    kc, kb, vc = (t.cpu() for t in st.read_codes(0, S))
    okc, okb = R.compress_ip_from_y(yk, kcb.boundaries.cpu(), kq.S.cpu(), kcb.centroids.cpu())
    ovc = R.quantize_boundary(yv, vcb.boundaries.cpu())
    assert torch.equal(kc, okc.to(torch.uint8))
    assert torch.equal(kb, okb.to(torch.uint8))
    assert torch.equal(vc, ovc.to(torch.uint8))
    assert torch.equal(st.knorm[:, :, :S].cpu(), kn)
    assert torch.equal(st.vnorm[:, :, :S].cpu(), vn)
    # the r = 0 cases are present with both signs of S, and resolve to 1
    r0 = yk == kcb.centroids.cpu()[okc.long()]
    sgn = kq.S.cpu().expand_as(yk)
    assert bool(r0[sgn > 0].any()) and bool(r0[sgn < 0].any())
    assert bool((kb[r0] == 1).all())


@pytest.mark.parametrize("n_out", [32, 64])
def test_store_append_kmixed_rotated_bit_exact(n_out):
    from quashkv_amd.store import KVStore
    kq = Q.MixedPrecisionMSEQuantizer(128, outlier_bits=3, regular_bits=2, n_outliers=n_out,
                                      seed=3, device=DEV)
    g = torch.Generator().manual_seed(n_out)
    out_idx = torch.randperm(128, generator=g)[:n_out].sort().values
    kq.set_outlier_channels(out_idx.to(DEV))
    oc, rc = kq.outlier_codebook, kq.regular_codebook
    B, H, S = 2, 2, 260
    y = _special_rows(n_out, (B, H, S, 128),
                      list(oc.boundaries_host) + list(rc.boundaries_host), n_random=30)
    nrm = torch.rand(B, H, S, generator=g) + 0.5
    o = [int(i) for i in out_idx]
    perm = o + [j for j in range(128) if j not in set(o)]
    st = KVStore(B, H, 128, 2, 4, S, DEV, kmix=(perm, n_out, False))
    ys = y[..., perm].contiguous().to(DEV)
    nd = nrm.to(DEV)
    ob_h, rb_h = N.HostFloats(oc.boundaries_host), N.HostFloats(rc.boundaries_host)
    N.check(N.lib().qkv_store_append_kmixed_rotated(
        ys.data_ptr(), nd.data_ptr(), B * H, S, 128, n_out, ob_h.ptr, rb_h.ptr,
        st.kst.data_ptr(), st.knorm.data_ptr(), st.capacity, 0, N.stream(torch.device(DEV))))
    kc = st.read_codes(0, S)[0].cpu()
    mask = torch.zeros(128, dtype=torch.bool)
    mask[out_idx] = True
    ref = torch.empty(B, H, S, 128, dtype=torch.uint8)
    ref[..., mask] = R.quantize_boundary(y[..., mask], oc.boundaries.cpu()).to(torch.uint8)
    ref[..., ~mask] = R.quantize_boundary(y[..., ~mask], rc.boundaries.cpu()).to(torch.uint8)
    assert torch.equal(kc, ref)
    assert torch.equal(st.knorm[:, :, :S].cpu(), nrm)


def test_store_append_cfg3_size_vs_oracle():
    """The fused append from bf16 x at the full cfg3 shape (B=32, 8 kv heads,
    8192 tokens, d=128, 3-bit keys with 4 outlier channels x10, 3-bit values):
    codes against the oracle's compress_ip / compress_mse of the same inputs,
    mismatch rate <= 1e-4 per stream, every mismatch one code step."""
    B, H, T, d = 32, 8, 8192, 128
    g = torch.Generator(device=DEV).manual_seed(2)
    k = torch.randn(B, H, T, d, device=DEV, generator=g)
    k[..., [11, 47, 83, 119]] *= 10.0
    k = k.to(torch.bfloat16)
    v = torch.randn(B, H, T, d, device=DEV, generator=g).to(torch.bfloat16)
    eng = Q.QuashKVEngine(head_dim=d, key_bits=3, value_bits=3, seed=42, device=DEV, capacity=T)
    eng.append(k, v)
    st = eng._store
    kq, vq = eng.key_quantizer, eng.value_quantizer
    mq = kq.mse_quantizer
    tabs = (mq.Pi.cpu(), mq.codebook.boundaries.cpu(), kq.S.cpu(), mq.codebook.centroids.cpu())
    bad = [0, 0, 0]
    total = 0
    for b0 in range(0, B, 4):
        kc, kb, vc = (t[b0:b0 + 4].cpu() for t in st.read_codes(0, T))
        okc, okb, _ = R.compress_ip(k[b0:b0 + 4].cpu().float(), *tabs)
        ovc, _ = R.compress_mse(v[b0:b0 + 4].cpu().float(), vq.Pi.cpu(),
                                vq.codebook.boundaries.cpu())
        for i, (a, r) in enumerate(((kc, okc), (kb, okb), (vc, ovc))):
            diff = (a.to(torch.int16) - r.to(torch.int16)).abs()
            assert int(diff.max()) <= 1
            bad[i] += int((diff != 0).sum())
        total += kc.numel()
    rates = [x / total for x in bad]
    print("cfg3 code mismatch rates (mse, qjl, value):", rates)
    assert max(rates) <= 1e-4, rates


def _kv_stores_equal(a, b, T):
    assert torch.equal(a.kst[:, :, :T], b.kst[:, :, :T])
    assert torch.equal(a.knorm[:, :, :T], b.knorm[:, :, :T])
    assert torch.equal(a.vnorm[:, :, :T], b.vnorm[:, :, :T])
    nt = (T + 31) // 32
    va, vb = a.vst[:, :, :nt].clone(), b.vst[:, :, :nt].clone()
    if T % 32:   # bits past T in the last tile are not part of the cache
        va[:, :, -1] &= (1 << (T % 32)) - 1
        vb[:, :, -1] &= (1 << (T % 32)) - 1
    assert torch.equal(va, vb)


@pytest.mark.parametrize("d", [128, 96, 64])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("mbits", [1, 2, 3])
@pytest.mark.parametrize("shape", ["few", "many", "xcd"])
def test_one_launch_append_equals_two_launches(d, dtype, mbits, shape):
    """Small appends with value bits = key MSE bits + 1 run the key and the
    value kernel as one launch (qkv_store_append_layers at one layer, and
    qkv_store_append given keys and values under one Pi): a wave per
    32-coordinate block of a tile for few tiles ("few": 6 groups), a wave per
    tile for more ("many": 64 groups, up to 10 tiles each); "xcd": 8 groups
    of 8 tiles, where the block workgroups of a tile group are placed on one
    XCD (a whole number of rounds of 8 tile groups), then 7 tiles per group
    (not), then an unaligned start.  The stores must be bit-identical to a
    key-only call followed by a value-only call (two launches), over ragged
    sizes and unaligned starts."""
    vbits = mbits + 1
    gen = torch.Generator().manual_seed(100 * mbits + d)
    (B, H), sizes = {"few": ((2, 3), (1, 5, 37, 64, 1, 100, 3)),
                     "many": ((8, 8), (160, 7, 300)),
                     "xcd": ((1, 8), (256, 200, 256))}[shape]
    cap = 1024 if shape == "xcd" else 512
    kq = Q.InnerProductQuantizer(d, mbits + 1, seed=7, device=DEV)
    vq = Q.MSEQuantizer(d, vbits, seed=8, device=DEV)
    mq = kq.mse_quantizer
    kc = N.HostFloats(mq.codebook.centroids_host)
    kb = N.HostFloats(mq.codebook.boundaries_host)
    vb = N.HostFloats(vq.codebook.boundaries_host)
    L = N.lib()
    dt = N.dtype_code(dtype)
    st = {name: Q.store.KVStore(B, H, d, mbits, vbits, cap, torch.device(DEV))
          for name in ("one", "two", "one_pi", "two_pi")}
    stream = N.stream(torch.device(DEV))

    def arr(t):
        return N.ptr_array([t.data_ptr()])

    t0 = 0
    for S in sizes:
        k = _rows(gen, (B, H, S, d), dtype).to(DEV)
        v = _rows(gen, (B, H, S, d), dtype, outliers=False).to(DEV)
        s = st["one"]
        N.check(L.qkv_store_append_layers(
            1, dt, arr(k), arr(v), B * H, S, d, mbits, vbits, arr(mq.Pi), arr(kq.S), arr(vq.Pi),
            kc.ptr, kb.ptr, vb.ptr, arr(s.kst), arr(s.knorm), arr(s.vst), arr(s.vnorm), cap, t0,
            stream))
        for name, kpi, vpi, both in (("two", mq.Pi, vq.Pi, False), ("one_pi", mq.Pi, mq.Pi, True),
                                     ("two_pi", mq.Pi, mq.Pi, False)):
            s = st[name]
            calls = [(k, v, kpi)] if both else [(k, None, kpi), (None, v, vpi)]
            for kk, vv, pi in calls:
                N.check(L.qkv_store_append(
                    dt, kk.data_ptr() if kk is not None else None,
                    vv.data_ptr() if vv is not None else None, B * H, S, d, mbits, vbits,
                    pi.data_ptr(), kq.S.data_ptr(), kc.ptr, kb.ptr, vb.ptr, s.kst.data_ptr(),
                    s.knorm.data_ptr(), s.vst.data_ptr(), s.vnorm.data_ptr(), cap, t0, stream))
        t0 += S
    torch.cuda.synchronize()
    _kv_stores_equal(st["one"], st["two"], t0)
    _kv_stores_equal(st["one_pi"], st["two_pi"], t0)
    assert st["one"].knorm[:, :, :t0].abs().min() > 0   # every token was written
