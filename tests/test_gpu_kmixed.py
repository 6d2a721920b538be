"""GPU parity of mixed-precision keys in the engine's store: kmixed rows
(qkv_kmixed_pack / _unpack), the fused bf16 / fp16 key append
(qkv_store_append_kmixed) and decode attention over them
(qkv_decode_attention_kmixed), against the CPU oracle's mixed_compress and
decompress-then-attend attention.

Bars: the row format bit-exact (round trip and an independent bit model);
fused codes as in the IP-key append (mismatch rate <= 1e-4, one code step);
attention from the store's own codes within 1e-3 relative (fp32 queries),
end to end from bf16 inputs within 1e-2 with cosine >= 0.9999."""

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


def _outliers(n_out, seed=1):
    g = torch.Generator().manual_seed(seed)
    return torch.randperm(128, generator=g)[:n_out].sort().values


def _engine(n_out, vbits=4, seed=42, out_idx=None, capacity=0):
    kq = Q.MixedPrecisionMSEQuantizer(128, outlier_bits=3, regular_bits=2, n_outliers=n_out,
                                      seed=seed, device=DEV)
    kq.set_outlier_channels((out_idx if out_idx is not None else _outliers(n_out)).to(DEV))
    return Q.QuashKVEngine(head_dim=128, value_bits=vbits, seed=seed, device=DEV,
                           key_quantizer=kq, capacity=capacity)


def _mismatch(a, b):
    a, b = a.cpu().to(torch.int16), b.cpu().to(torch.int16)
    diff = (a - b).abs()
    return float((diff != 0).double().mean()), int(diff.max()) if diff.numel() else 0


def _perm(out_idx):
    o = [int(i) for i in out_idx]
    return o + [j for j in range(128) if j not in set(o)]


@pytest.mark.parametrize("n_out", [32, 64])
def test_kmixed_rows_round_trip_and_bit_model(n_out):
    gen = torch.Generator().manual_seed(n_out)
    out_idx = _outliers(n_out, seed=n_out)
    n, seq, gstride = 70, 35, 64          # 2 groups of 35 rows in a 64-row stride
    codes = torch.randint(0, 4, (n, 128), generator=gen, dtype=torch.uint8)
    codes[:, out_idx] = torch.randint(0, 8, (n, n_out), generator=gen, dtype=torch.uint8)
    perm = _perm(out_idx)
    ph = N.HostInts(perm)
    L = N.lib()
    rb = 32 + n_out // 4                 # row bytes: b0, b1, outlier b2, outlier parity
    dst = torch.zeros(2 * gstride, rb, dtype=torch.uint8, device=DEV)
    N.check(L.qkv_kmixed_pack(codes.to(DEV).data_ptr(), n, ph.ptr, n_out, dst.data_ptr(), seq,
                              gstride, N.stream(dst.device)))
    back = torch.empty(n, 128, dtype=torch.uint8, device=DEV)
    N.check(L.qkv_kmixed_unpack(dst.data_ptr(), n, ph.ptr, n_out, seq, gstride,
                                back.data_ptr(), N.stream(dst.device)))
    assert torch.equal(back.cpu(), codes)
    # independent model of the row: bit (slot % 8) of byte slot / 8 per plane
    rows = dst.cpu().numpy()
    c = codes.numpy()[:, perm].astype(np.uint32)
    for r in range(n):
        row = rows[(r // seq) * gstride + r % seq]
        bits = np.unpackbits(row, bitorder="little")
        assert np.array_equal(bits[0:128], c[r] & 1)
        assert np.array_equal(bits[128:256], (c[r] >> 1) & 1)
        co = c[r, :n_out]
        assert np.array_equal(bits[256:256 + n_out], (co >> 2) & 1)
        assert np.array_equal(bits[256 + n_out:256 + 2 * n_out], (co ^ (co >> 1) ^ (co >> 2)) & 1)
        assert len(bits) == 256 + 2 * n_out
    # rows outside the groups' first 35 stay zero
    assert not dst.cpu()[seq:gstride].any() and not dst.cpu()[gstride + seq:].any()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("n_out", [32, 64])
def test_kmixed_append_vs_oracle(dtype, n_out):
    """Codes and norms in the store against the oracle's mixed_compress
    (quashkv/mixed_precision.py:132-158) on the same (upcast) keys; ragged
    appends with unaligned starts."""
    gen = torch.Generator().manual_seed(7 + n_out)
    B, H = 2, 3
    eng = _engine(n_out)
    kq = eng.key_quantizer
    out_idx = kq._outlier_indices.cpu()
    pi = kq.Pi.cpu()
    ks, vs, total = [], [], 0
    for S in (150, 37, 1, 64, 0, 95):
        y = torch.randn(B, H, S, 128, generator=gen)
        y[..., out_idx] *= 8.0
        k = (y @ pi).to(dtype)                     # rotated outliers -> key space
        v = torch.randn(B, H, S, 128, generator=gen).to(dtype)
        eng.append(k.to(DEV), v.to(DEV))
        ks.append(k)
        vs.append(v)
        total += S
    k, v = torch.cat(ks, dim=2), torch.cat(vs, dim=2)
    st = eng._store
    kc, kb, vc = st.read_codes(0, total)
    assert kb is None
    kc, vc = kc.cpu(), vc.cpu()
    oc, on = R.mixed_compress(k.float().reshape(-1, 128), pi, out_idx,
                              kq.outlier_codebook.boundaries.cpu(),
                              kq.regular_codebook.boundaries.cpu())
    vq = eng.value_quantizer
    ovc, ovn = R.compress_mse(v.float().reshape(-1, 128), vq.Pi.cpu(),
                              vq.codebook.boundaries.cpu())
    for got, ref in ((kc, oc), (vc, ovc)):
        rate, step = _mismatch(got.reshape(-1, 128), ref.reshape(-1, 128))
        assert rate <= 1e-4 and step <= 1, (rate, step)
    for got, ref in ((st.knorm[:, :, :total], on), (st.vnorm[:, :, :total], ovn)):
        got, ref = got.cpu().double().reshape(-1), ref.double().reshape(-1)
        assert float(((got - ref).abs() / ref).max()) <= 2e-6
    # outlier codes reach the top of 8 levels, regular ones stay within 4
    assert int(kc[..., out_idx].max()) == 7
    mask = torch.ones(128, dtype=torch.bool)
    mask[out_idx] = False
    assert int(kc[..., mask].max()) <= 3


@pytest.mark.parametrize("n_out,G,Q_", [(32, 4, 1), (64, 4, 1), (32, 1, 2)])
def test_kmixed_attention_from_store_codes(n_out, G, Q_):
    """Attention kernel alone: the oracle's decompress-then-attend on the
    codes and norms read back from the store, fp32 queries, rel-err <= 1e-3."""
    gen = torch.Generator().manual_seed(3 * n_out + G)
    B, Hkv, S = 2, 2, 777
    eng = _engine(n_out)
    kq, vq = eng.key_quantizer, eng.value_quantizer
    out_idx = kq._outlier_indices.cpu()
    y = torch.randn(B, Hkv, S, 128, generator=gen)
    y[..., out_idx] *= 8.0
    k = (y @ kq.Pi.cpu()).to(torch.bfloat16)
    v = torch.randn(B, Hkv, S, 128, generator=gen).to(torch.bfloat16)
    eng.append(k[:, :, :500].to(DEV), v[:, :, :500].to(DEV))
    eng.append(k[:, :, 500:].to(DEV), v[:, :, 500:].to(DEV))
    q = torch.randn(B, Hkv * G, Q_, 128, generator=gen)
    out = eng.attention(q.to(DEV)).cpu().double()
    st = eng._store
    kc, _, vc = st.read_codes(0, S)
    ref = R.attention_mixed_keys(q, kc.cpu(), st.knorm[:, :, :S].cpu(), vc.cpu(),
                                 st.vnorm[:, :, :S].cpu(), kq.Pi.cpu(), out_idx,
                                 kq.outlier_codebook.centroids.cpu(),
                                 kq.regular_codebook.centroids.cpu(), vq.Pi.cpu(),
                                 vq.codebook.centroids.cpu()).double()
    err = float((out - ref).norm() / ref.norm())
    assert err <= 1e-3, err


def test_kmixed_engine_attention_end_to_end():
    """bf16 keys, values and query through the fused append and the decode
    kernel, against the oracle on its own codes of the same inputs."""
    gen = torch.Generator().manual_seed(5)
    B, Hkv, G, S = 1, 4, 4, 1500
    eng = _engine(32)
    kq, vq = eng.key_quantizer, eng.value_quantizer
    out_idx = kq._outlier_indices.cpu()
    y = torch.randn(B, Hkv, S, 128, generator=gen)
    y[..., out_idx] *= 8.0
    k = (y @ kq.Pi.cpu()).to(torch.bfloat16)
    v = torch.randn(B, Hkv, S, 128, generator=gen).to(torch.bfloat16)
    q = torch.randn(B, Hkv * G, 1, 128, generator=gen).to(torch.bfloat16)
    for a in range(0, S, 512):
        eng.append(k[:, :, a:a + 512].to(DEV), v[:, :, a:a + 512].to(DEV))
    out = eng.attention(q.to(DEV)).cpu().double()
    kc, kn = R.mixed_compress(k.float(), kq.Pi.cpu(), out_idx,
                              kq.outlier_codebook.boundaries.cpu(),
                              kq.regular_codebook.boundaries.cpu())
    vc, vn = R.compress_mse(v.float(), vq.Pi.cpu(), vq.codebook.boundaries.cpu())
    ref = R.attention_mixed_keys(q.float(), kc, kn, vc, vn, kq.Pi.cpu(), out_idx,
                                 kq.outlier_codebook.centroids.cpu(),
                                 kq.regular_codebook.centroids.cpu(), vq.Pi.cpu(),
                                 vq.codebook.centroids.cpu()).double()
    err = float((out - ref).norm() / ref.norm())
    cos = float((out.flatten() @ ref.flatten()) / (out.norm() * ref.norm()))
    assert err <= 1e-2 and cos >= 0.9999, (err, cos)
    assert eng.key_bits == 2.25 and eng.total_tokens == S


def test_kmixed_engine_errors():
    kq = Q.MixedPrecisionMSEQuantizer(128, outlier_bits=3, regular_bits=2, n_outliers=32,
                                      device=DEV)
    eng = Q.QuashKVEngine(head_dim=128, value_bits=4, device=DEV, key_quantizer=kq)
    x = torch.randn(1, 1, 8, 128, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="calibrate"):
        eng.append(x, x)
    with pytest.raises(ValueError, match="32 or 64 outliers"):
        Q.QuashKVEngine(head_dim=128, device=DEV, key_quantizer=Q.MixedPrecisionMSEQuantizer(
            128, outlier_bits=3, regular_bits=2, n_outliers=16, device=DEV))


def test_kmixed_cfg4_full_size():
    """The long-context mixed-precision workload at its full size: B=1, 32
    query heads over 8 kv heads, 131072 bf16 tokens appended in 64 chunks of
    2048, keys MixedPrecisionMSE 3/2 bits with 32 outliers calibrated on 65536
    keys whose raw channels 0, 4, .., 124 have sigma 8, values 4-bit MSE, one
    bf16 query.  Per kv head: the kernel against the oracle's attention on the
    store's own codes (fp32 arithmetic from the same bf16 query, rel <= 1e-3),
    and end to end against the oracle's own codes of the same bf16 inputs
    (rel <= 1e-2, cosine >= 0.9999)."""
    B, Hq, Hkv, TT, CH = 1, 32, 8, 131072, 2048
    G = Hq // Hkv
    gen = torch.Generator().manual_seed(44)
    out_ch = list(range(0, 128, 4))
    cal = torch.randn(65536, 128, generator=gen)
    cal[:, out_ch] *= 8.0
    kq = Q.MixedPrecisionMSEQuantizer(128, outlier_bits=3, regular_bits=2, n_outliers=32,
                                      seed=42, device=DEV)
    kq.calibrate(cal.to(DEV))
    eng = Q.QuashKVEngine(head_dim=128, value_bits=4, seed=42, device=DEV, key_quantizer=kq,
                          capacity=TT)
    vq = eng.value_quantizer
    k = torch.randn(B, Hkv, TT, 128, generator=gen)
    k[..., out_ch] *= 8.0
    k = k.to(torch.bfloat16)
    v = torch.randn(B, Hkv, TT, 128, generator=gen).to(torch.bfloat16)
    q = torch.randn(B, Hq, 1, 128, generator=gen).to(torch.bfloat16)
    kd, vd = k.to(DEV), v.to(DEV)
    for a in range(0, TT, CH):
        eng.append(kd[:, :, a:a + CH], vd[:, :, a:a + CH])
    out = eng.attention(q.to(DEV)).cpu().double()
    assert eng.total_tokens == TT
    st = eng._store
    kc, _, vc = st.read_codes(0, TT)
    kc, vc = kc.cpu(), vc.cpu()
    kn, vn = st.knorm[:, :, :TT].cpu(), st.vnorm[:, :, :TT].cpu()
    del kd, vd
    out_idx = kq._outlier_indices.cpu()
    tabs = (kq.Pi.cpu(), out_idx, kq.outlier_codebook.centroids.cpu(),
            kq.regular_codebook.centroids.cpu(), vq.Pi.cpu(), vq.codebook.centroids.cpu())
    pi_k, t_out, t_reg = (kq.Pi.cpu(), kq.outlier_codebook.boundaries.cpu(),
                          kq.regular_codebook.boundaries.cpu())
    errs, e2e = [], []
    for h in range(Hkv):
        hs, qs = slice(h, h + 1), slice(G * h, G * h + G)
        qh = q[:, qs].float()
        ref = R.attention_mixed_keys(qh, kc[:, hs], kn[:, hs], vc[:, hs], vn[:, hs],
                                     *tabs).double()
        mine = out[:, qs]
        errs.append(float((mine - ref).norm() / ref.norm()))
        okc, okn = R.mixed_compress(k[:, hs].float(), pi_k, out_idx, t_out, t_reg)
        ovc, ovn = R.compress_mse(v[:, hs].float(), vq.Pi.cpu(), vq.codebook.boundaries.cpu())
        ref2 = R.attention_mixed_keys(qh, okc, okn, ovc, ovn, *tabs).double()
        e2e.append((float((mine - ref2).norm() / ref2.norm()),
                    float((mine.flatten() @ ref2.flatten()) / (mine.norm() * ref2.norm()))))
    assert max(errs) <= 1e-3, errs
    assert all(e <= 1e-2 and c >= 0.9999 for e, c in e2e), e2e


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


@pytest.mark.parametrize("ip", [False, True])
@pytest.mark.parametrize("n_out", [32, 64])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("vbits", [4, 2, 1])
@pytest.mark.parametrize("shape", ["few", "many", "chunk"])
def test_kmixed_kv_append_equals_two_calls(ip, n_out, dtype, vbits, shape):
    """qkv_store_append_kmixed_kv (keys and values in one launch for chunk-sized
    appends: a wave per 32-slot block of a tile while two workgroups per CU
    hold the grid, a wave per tile for more; value bits 1 take the two-kernel
    path inside) writes the same store, bit for bit, as
    qkv_store_append_kmixed / _kipmixed followed by the value-only
    qkv_store_append, over ragged sizes and unaligned starts.  "chunk": cfg4's
    2048-token chunks of 8 kv heads (the block workgroups of a tile group on
    one XCD), then shorter appends that are not whole rounds."""
    cls = Q.MixedPrecisionIPQuantizer if ip else Q.MixedPrecisionMSEQuantizer
    kq = cls(128, outlier_bits=3, regular_bits=2, n_outliers=n_out, seed=42, device=DEV)
    out_idx = _outliers(n_out, seed=3)
    kq.set_outlier_channels(out_idx.to(DEV))
    eng = Q.QuashKVEngine(head_dim=128, value_bits=vbits, seed=42, device=DEV, key_quantizer=kq)
    perm, pi_perm, no, (oc, rc, ob, rb, vb) = eng._kmix_setup()
    pi_perm = pi_perm.to(DEV)
    sp = eng._kmix_signs(torch.device(DEV))
    vq = eng.value_quantizer
    (B, H), sizes = {"few": ((2, 3), (1, 37, 64, 5, 100)), "many": ((8, 8), (160, 7, 300)),
                     "chunk": ((1, 8), (2048, 256, 200))}[shape]
    cap = 4096 if shape == "chunk" else 512
    dev = torch.device(DEV)
    one = Q.store.KVStore(B, H, 128, 2, vbits, cap, dev, kmix=(perm, no, ip))
    two = Q.store.KVStore(B, H, 128, 2, vbits, cap, dev, kmix=(perm, no, ip))
    L = N.lib()
    dt = N.dtype_code(dtype)
    stream = N.stream(dev)
    gen = torch.Generator().manual_seed(n_out + vbits + 10 * int(ip))
    t0 = 0
    for S in sizes:
        k = torch.randn(B, H, S, 128, generator=gen)
        k[..., out_idx] *= 8.0
        k = k.to(dtype).to(DEV)
        v = torch.randn(B, H, S, 128, generator=gen).to(dtype).to(DEV)
        N.check(L.qkv_store_append_kmixed_kv(
            dt, k.data_ptr(), v.data_ptr(), B * H, S, 128, pi_perm.data_ptr(),
            sp.data_ptr() if ip else None, no, int(ip), oc.ptr, ob.ptr, rc.ptr, rb.ptr,
            one.kst.data_ptr(), one.knorm.data_ptr(), vbits, vq.Pi.data_ptr(), vb.ptr,
            one.vst.data_ptr(), one.vnorm.data_ptr(), cap, t0, stream))
        if ip:
            N.check(L.qkv_store_append_kipmixed(
                dt, k.data_ptr(), B * H, S, 128, pi_perm.data_ptr(), sp.data_ptr(), no, oc.ptr,
                ob.ptr, rc.ptr, rb.ptr, two.kst.data_ptr(), two.knorm.data_ptr(), cap, t0,
                stream))
        else:
            N.check(L.qkv_store_append_kmixed(
                dt, k.data_ptr(), B * H, S, 128, pi_perm.data_ptr(), no, ob.ptr, rb.ptr,
                two.kst.data_ptr(), two.knorm.data_ptr(), cap, t0, stream))
        N.check(L.qkv_store_append(dt, None, v.data_ptr(), B * H, S, 128, 2, vbits,
                                   vq.Pi.data_ptr(), None, None, None, vb.ptr, None, None,
                                   two.vst.data_ptr(), two.vnorm.data_ptr(), cap, t0, stream))
        t0 += S
    torch.cuda.synchronize()
    _kv_stores_equal(one, two, t0)
    assert one.knorm[:, :, :t0].abs().min() > 0
