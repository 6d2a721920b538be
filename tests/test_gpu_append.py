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


@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
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


@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
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
    for got, ref in ((kc, okc), (kb, okb), (vc, ovc)):
        rate, step = _mismatch(got.reshape(-1, d), ref.reshape(-1, d))
        assert rate <= 1e-4 and step <= 1, (rate, step)
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
