"""GPU parity of mixed-precision IP keys (MixedPrecisionIPQuantizer with
outlier_bits 3 / regular_bits 2: a 2-bit outlier / 1-bit regular MSE stage
plus a QJL bit per coordinate) in the engine's store: kipmixed rows
(qkv_kipmixed_pack / _unpack), the fused bf16 / fp16 key append
(qkv_store_append_kipmixed, and its _rotated twin from given y) and decode
attention over them (qkv_decode_attention_kipmixed), against the CPU oracle's
mixed_ip_compress (pinned to the reference's own outputs) and
attention_mixed_ip_keys (decompress_for_dot scores with each channel's
codebook).

Bars: the row format bit-exact (round trip and an independent bit model);
codes and QJL bits from identical y bit-exact, ties included; from x as the
IP-key append (mismatch rate <= 1e-4); attention from the store's own codes
within 1e-3 relative (fp32 queries), end to end from bf16 inputs within 1e-2
with cosine >= 0.9999."""

import numpy as np
import pytest
import torch

import quashkv_amd as Q
from quashkv_amd import _native as N
from oracle import ref_math as R

from .test_gpu_append import _special_rows

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(autouse=True, scope="module")
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")
    N.lib()


def _outliers(n_out, seed=1):
    g = torch.Generator().manual_seed(seed)
    return torch.randperm(128, generator=g)[:n_out].sort().values


def _perm(out_idx):
    o = [int(i) for i in out_idx]
    return o + [j for j in range(128) if j not in set(o)]


def _engine(n_out, vbits=4, seed=42, out_idx=None, capacity=0):
    kq = Q.MixedPrecisionIPQuantizer(128, outlier_bits=3, regular_bits=2, n_outliers=n_out,
                                     seed=seed, device=DEV)
    kq.set_outlier_channels((out_idx if out_idx is not None else _outliers(n_out)).to(DEV))
    return Q.QuashKVEngine(head_dim=128, value_bits=vbits, seed=seed, device=DEV,
                           key_quantizer=kq, capacity=capacity)


def _tabs(kq):
    mq = kq.mse_quantizer
    oc, rc = mq.outlier_codebook, mq.regular_codebook
    return (oc.centroids.cpu(), oc.boundaries.cpu(), rc.centroids.cpu(), rc.boundaries.cpu())


def _mismatch(a, b):
    a, b = a.cpu().to(torch.int16), b.cpu().to(torch.int16)
    diff = (a - b).abs()
    return float((diff != 0).double().mean()), int(diff.max()) if diff.numel() else 0


@pytest.mark.parametrize("n_out", [32, 64])
def test_kipmixed_rows_round_trip_and_bit_model(n_out):
    gen = torch.Generator().manual_seed(n_out + 1)
    out_idx = _outliers(n_out, seed=n_out)
    n, seq, gstride = 70, 35, 64          # 2 groups of 35 rows in a 64-row stride
    codes = torch.randint(0, 2, (n, 128), generator=gen, dtype=torch.uint8)
    codes[:, out_idx] = torch.randint(0, 4, (n, n_out), generator=gen, dtype=torch.uint8)
    qjl = torch.randint(0, 2, (n, 128), generator=gen, dtype=torch.uint8)
    perm = _perm(out_idx)
    ph = N.HostInts(perm)
    L = N.lib()
    rb = 32 + n_out // 8                  # row bytes: b0, QJL, outlier b1
    dst = torch.zeros(2 * gstride, rb, dtype=torch.uint8, device=DEV)
    cd, qd = codes.to(DEV), qjl.to(DEV)   # held: the kernel reads them after the call
    N.check(L.qkv_kipmixed_pack(cd.data_ptr(), qd.data_ptr(), n, ph.ptr, n_out, dst.data_ptr(),
                                seq, gstride, N.stream(dst.device)))
    back = torch.empty(n, 128, dtype=torch.uint8, device=DEV)
    bq = torch.empty(n, 128, dtype=torch.uint8, device=DEV)
    N.check(L.qkv_kipmixed_unpack(dst.data_ptr(), n, ph.ptr, n_out, seq, gstride,
                                  back.data_ptr(), bq.data_ptr(), N.stream(dst.device)))
    assert torch.equal(back.cpu(), codes) and torch.equal(bq.cpu(), qjl)
    # independent model of the row: bit (slot % 8) of byte slot / 8 per plane
    rows = dst.cpu().numpy()
    c = codes.numpy()[:, perm].astype(np.uint32)
    b = qjl.numpy()[:, perm].astype(np.uint32)
    for r in range(n):
        bits = np.unpackbits(rows[(r // seq) * gstride + r % seq], bitorder="little")
        assert len(bits) == 256 + n_out
        assert np.array_equal(bits[0:128], c[r] & 1)
        assert np.array_equal(bits[128:256], b[r])
        assert np.array_equal(bits[256:], (c[r, :n_out] >> 1) & 1)
    assert not dst.cpu()[seq:gstride].any() and not dst.cpu()[gstride + seq:].any()


@pytest.mark.parametrize("n_out", [32, 64])
def test_store_append_kipmixed_rotated_bit_exact(n_out):
    """The fused append's search, QJL and row store on given y: codes and
    bits equal mixed_ip_compress_from_y bit for bit on every centroid and
    boundary of both codebooks, their one-ulp neighbours, +-0, denormals and
    huge values, with r = 0 present under both signs of S."""
    from quashkv_amd.store import KVStore
    kq = Q.MixedPrecisionIPQuantizer(128, outlier_bits=3, regular_bits=2, n_outliers=n_out,
                                     seed=5, device=DEV)
    g = torch.Generator().manual_seed(n_out + 3)
    out_idx = torch.randperm(128, generator=g)[:n_out].sort().values
    kq.set_outlier_channels(out_idx.to(DEV))
    mq = kq.mse_quantizer
    oc, rc = mq.outlier_codebook, mq.regular_codebook
    B, H, S = 2, 2, 260
    y = _special_rows(n_out + 11, (B, H, S, 128),
                      list(oc.centroids_host) + list(oc.boundaries_host)
                      + list(rc.centroids_host) + list(rc.boundaries_host), n_random=30)
    nrm = torch.rand(B, H, S, generator=g) + 0.5
    perm = _perm(out_idx)
    st = KVStore(B, H, 128, 2, 4, S, DEV, kmix=(perm, n_out, True))
    ys = y[..., perm].contiguous().to(DEV)
    sp = kq.S.cpu()[perm].contiguous().to(DEV)
    nd = nrm.to(DEV)
    hs = [N.HostFloats(t) for t in (oc.centroids_host, oc.boundaries_host, rc.centroids_host,
                                    rc.boundaries_host)]
    N.check(N.lib().qkv_store_append_kipmixed_rotated(
        ys.data_ptr(), nd.data_ptr(), B * H, S, 128, sp.data_ptr(), n_out, *[h.ptr for h in hs],
        st.kst.data_ptr(), st.knorm.data_ptr(), st.capacity, 0, N.stream(torch.device(DEV))))
    kc, kb, _ = (t.cpu() if t is not None else None for t in st.read_codes(0, S))
    s = kq.S.cpu()
    okc, okb = R.mixed_ip_compress_from_y(y, out_idx, *_tabs(kq), s)
    assert torch.equal(kc, okc)
    assert torch.equal(kb, okb)
    assert torch.equal(st.knorm[:, :, :S].cpu(), nrm)
    mask = torch.zeros(128, dtype=torch.bool)
    mask[out_idx] = True
    cent = torch.where(mask, oc.centroids.cpu()[okc.long().clamp(max=3)],
                       rc.centroids.cpu()[okc.long().clamp(max=1)])
    r0 = y == cent
    sgn = s.expand_as(y)
    for m in (mask, ~mask):
        assert bool(r0[(sgn > 0) & m].any()) and bool(r0[(sgn < 0) & m].any())
    assert bool((kb[r0] == 1).all())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("n_out", [32, 64])
def test_kipmixed_append_vs_oracle(dtype, n_out):
    """Codes, QJL bits and norms in the store against the oracle's
    mixed_ip_compress on the same (upcast) keys; ragged appends with unaligned
    starts (fp32 keys take the generic compress kernel and the row packer)."""
    gen = torch.Generator().manual_seed(17 + n_out)
    B, H = 2, 3
    eng = _engine(n_out)
    kq = eng.key_quantizer
    mq = kq.mse_quantizer
    out_idx = mq._outlier_indices.cpu()
    pi = mq.Pi.cpu()
    ks, vs, total = [], [], 0
    for S in (150, 37, 1, 64, 0, 95):
        y = torch.randn(B, H, S, 128, generator=gen)
        y[..., out_idx] *= 8.0
        k = (y @ pi).to(dtype)
        v = torch.randn(B, H, S, 128, generator=gen).to(dtype)
        eng.append(k.to(DEV), v.to(DEV))
        ks.append(k)
        vs.append(v)
        total += S
    k = torch.cat(ks, dim=2)
    st = eng._store
    kc, kb, _ = st.read_codes(0, total)
    okc, okb, okn = R.mixed_ip_compress(k.float().reshape(-1, 128), pi, out_idx, *_tabs(kq),
                                        kq.S.cpu())
    for got, ref in ((kc, okc), (kb, okb)):
        rate, step = _mismatch(got.reshape(-1, 128), ref.reshape(-1, 128))
        assert rate <= 1e-4 and step <= 1, (rate, step)
    got, ref = st.knorm[:, :, :total].cpu().double().reshape(-1), okn.double().reshape(-1)
    assert float(((got - ref).abs() / ref).max()) <= 2e-6
    mask = torch.ones(128, dtype=torch.bool)
    mask[out_idx] = False
    assert int(kc[..., out_idx].max()) == 3 and int(kc[..., mask].max()) <= 1


@pytest.mark.parametrize("n_out,G,Q_,causal", [(32, 4, 1, False), (64, 4, 1, False),
                                               (32, 1, 3, True), (64, 2, 2, False)])
def test_kipmixed_attention_from_store_codes(n_out, G, Q_, causal):
    """The decode kernel alone: the oracle's attention_mixed_ip_keys on the
    codes, bits and norms read back from the store, fp32 queries,
    rel-err <= 1e-3."""
    gen = torch.Generator().manual_seed(5 * n_out + G + Q_)
    B, Hkv, S = 2, 2, 777
    eng = _engine(n_out)
    kq, vq = eng.key_quantizer, eng.value_quantizer
    mq = kq.mse_quantizer
    out_idx = mq._outlier_indices.cpu()
    y = torch.randn(B, Hkv, S, 128, generator=gen)
    y[..., out_idx] *= 8.0
    k = (y @ mq.Pi.cpu()).to(torch.bfloat16)
    v = torch.randn(B, Hkv, S, 128, generator=gen).to(torch.bfloat16)
    eng.append(k[:, :, :500].to(DEV), v[:, :, :500].to(DEV))
    eng.append(k[:, :, 500:].to(DEV), v[:, :, 500:].to(DEV))
    q = torch.randn(B, Hkv * G, Q_, 128, generator=gen)
    out = eng.attention(q.to(DEV), causal=causal).cpu().double()
    st = eng._store
    kc, kb, vc = st.read_codes(0, S)
    ref = R.attention_mixed_ip_keys(
        q, kc.cpu(), kb.cpu(), st.knorm[:, :, :S].cpu(), vc.cpu(), st.vnorm[:, :, :S].cpu(),
        mq.Pi.cpu(), out_idx, mq.outlier_codebook.centroids.cpu(),
        mq.regular_codebook.centroids.cpu(), kq.S.cpu(), kq.qjl_scale, vq.Pi.cpu(),
        vq.codebook.centroids.cpu(), causal=causal).double()
    err = float((out - ref).norm() / ref.norm())
    assert err <= 1e-3, err


def test_kipmixed_engine_attention_end_to_end():
    """bf16 keys, values and query through the fused append and the decode
    kernel, against the oracle on its own codes of the same inputs; then the
    reference-shaped views: _cache blocks, _unpack_block, memory figures."""
    gen = torch.Generator().manual_seed(6)
    B, Hkv, G, S = 1, 4, 4, 1500
    eng = _engine(32)
    kq, vq = eng.key_quantizer, eng.value_quantizer
    mq = kq.mse_quantizer
    out_idx = mq._outlier_indices.cpu()
    y = torch.randn(B, Hkv, S, 128, generator=gen)
    y[..., out_idx] *= 8.0
    k = (y @ mq.Pi.cpu()).to(torch.bfloat16)
    v = torch.randn(B, Hkv, S, 128, generator=gen).to(torch.bfloat16)
    q = torch.randn(B, Hkv * G, 1, 128, generator=gen).to(torch.bfloat16)
    for a in range(0, S, 512):
        eng.append(k[:, :, a:a + 512].to(DEV), v[:, :, a:a + 512].to(DEV))
    out = eng.attention(q.to(DEV)).cpu().double()
    tabs = _tabs(kq)
    kc, kb, kn = R.mixed_ip_compress(k.float(), mq.Pi.cpu(), out_idx, *tabs, kq.S.cpu())
    vc, vn = R.compress_mse(v.float(), vq.Pi.cpu(), vq.codebook.boundaries.cpu())
    ref = R.attention_mixed_ip_keys(q.float(), kc, kb, kn, vc, vn, mq.Pi.cpu(), out_idx,
                                    tabs[0], tabs[2], kq.S.cpu(), kq.qjl_scale, vq.Pi.cpu(),
                                    vq.codebook.centroids.cpu()).double()
    err = float((out - ref).norm() / ref.norm())
    cos = float((out.flatten() @ ref.flatten()) / (out.norm() * ref.norm()))
    assert err <= 1e-2 and cos >= 0.9999, (err, cos)
    assert eng.key_bits == 2.25 and eng.total_tokens == S
    assert eng._store.krb == 36
    blocks = eng._cache
    assert len(blocks) == 3 and sum(b.seq_len for b in blocks) == S
    c0, b0, _ = eng._unpack_block(blocks[0])
    got_c, got_b, _ = eng._store.read_codes(0, 512)
    assert torch.equal(c0, got_c) and torch.equal(b0, got_b)
    assert eng.actual_memory_bytes() == B * Hkv * S * (2 * 128 + 128 + 8)


def test_kipmixed_engine_errors():
    kq = Q.MixedPrecisionIPQuantizer(128, outlier_bits=3, regular_bits=2, n_outliers=32,
                                     device=DEV)
    eng = Q.QuashKVEngine(head_dim=128, value_bits=4, device=DEV, key_quantizer=kq)
    x = torch.randn(1, 1, 8, 128, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="calibrate"):
        eng.append(x, x)
    with pytest.raises(ValueError, match="32 or 64 outliers"):
        Q.QuashKVEngine(head_dim=128, device=DEV, key_quantizer=Q.MixedPrecisionIPQuantizer(
            128, outlier_bits=4, regular_bits=3, n_outliers=32, device=DEV))


def test_kipmixed_long_context():
    """A long single-sequence cache at the long-context workload's head
    layout (32 query heads over 8 kv heads, 32768 bf16 tokens appended in
    chunks of 2048, 32 calibrated outliers, 4-bit values): per kv head the
    kernel against the oracle on the store's codes (rel <= 1e-3) and end to
    end on the oracle's own codes (rel <= 1e-2, cosine >= 0.9999)."""
    B, Hq, Hkv, TT, CH = 1, 32, 8, 32768, 2048
    G = Hq // Hkv
    gen = torch.Generator().manual_seed(45)
    out_ch = list(range(2, 128, 4))
    cal = torch.randn(16384, 128, generator=gen)
    cal[:, out_ch] *= 8.0
    kq = Q.MixedPrecisionIPQuantizer(128, outlier_bits=3, regular_bits=2, n_outliers=32,
                                     seed=42, device=DEV)
    kq.calibrate(cal.to(DEV))
    eng = Q.QuashKVEngine(head_dim=128, value_bits=4, seed=42, device=DEV, key_quantizer=kq,
                          capacity=TT)
    vq = eng.value_quantizer
    mq = kq.mse_quantizer
    k = torch.randn(B, Hkv, TT, 128, generator=gen)
    k[..., out_ch] *= 8.0
    k = k.to(torch.bfloat16)
    v = torch.randn(B, Hkv, TT, 128, generator=gen).to(torch.bfloat16)
    q = torch.randn(B, Hq, 1, 128, generator=gen).to(torch.bfloat16)
    kd, vd = k.to(DEV), v.to(DEV)
    for a in range(0, TT, CH):
        eng.append(kd[:, :, a:a + CH], vd[:, :, a:a + CH])
    out = eng.attention(q.to(DEV)).cpu().double()
    st = eng._store
    kc, kb, vc = (t.cpu() for t in st.read_codes(0, TT))
    kn, vn = st.knorm[:, :, :TT].cpu(), st.vnorm[:, :, :TT].cpu()
    out_idx = mq._outlier_indices.cpu()
    tabs = _tabs(kq)
    errs, e2e = [], []
    for h in range(Hkv):
        hs, qs = slice(h, h + 1), slice(G * h, G * h + G)
        qh = q[:, qs].float()
        common = (mq.Pi.cpu(), out_idx, tabs[0], tabs[2], kq.S.cpu(), kq.qjl_scale, vq.Pi.cpu(),
                  vq.codebook.centroids.cpu())
        ref = R.attention_mixed_ip_keys(qh, kc[:, hs], kb[:, hs], kn[:, hs], vc[:, hs],
                                        vn[:, hs], *common).double()
        mine = out[:, qs]
        errs.append(float((mine - ref).norm() / ref.norm()))
        okc, okb, okn = R.mixed_ip_compress(k[:, hs].float(), mq.Pi.cpu(), out_idx, *tabs,
                                            kq.S.cpu())
        ovc, ovn = R.compress_mse(v[:, hs].float(), vq.Pi.cpu(), vq.codebook.boundaries.cpu())
        ref2 = R.attention_mixed_ip_keys(qh, okc, okb, okn, ovc, ovn, *common).double()
        e2e.append((float((mine - ref2).norm() / ref2.norm()),
                    float((mine.flatten() @ ref2.flatten()) / (mine.norm() * ref2.norm()))))
    assert max(errs) <= 1e-3, errs
    assert max(e for e, _ in e2e) <= 1e-2 and min(c for _, c in e2e) >= 0.9999, e2e
