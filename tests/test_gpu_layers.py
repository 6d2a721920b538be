"""GPU parity of the layer-batched decode step (qkv_decode_attention_layers):
several layers' engines (own Pi, S, store, query) attended in three launches
agree with each layer's own decode call and with the oracle."""

import pytest
import torch

import quashkv_amd as Q
from quashkv_amd import _native as N
from quashkv_amd import kernels as K
from oracle import ref_math as R

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(autouse=True, scope="module")
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")
    N.lib()


def _close(a, b, rel):
    a, b = a.detach().cpu().double(), b.detach().cpu().double()
    err = float((a - b).norm() / b.norm())
    assert err <= rel, err


@pytest.mark.parametrize("d,G,Qn,causal,kb", [
    (64, 7, 1, False, 3), (128, 4, 1, False, 3), (128, 2, 3, True, 3),
    (64, 7, 1, False, 4),       # 3-bit key MSE at d = 64: decode_fused (parity plane)
    (64, 2, 3, True, 4),
    (96, 4, 1, False, 3), (96, 2, 3, True, 4)])
def test_layers_match_per_layer_and_oracle(d, G, Qn, causal, kb):
    gen = torch.Generator().manual_seed(d + G + kb)
    n, B, Hkv, T = 5, 3, 2, 700
    engines = [Q.QuashKVEngine(head_dim=d, key_bits=kb, seed=42 + l, device=DEV)
               for l in range(n)]
    for e in engines:
        k = torch.randn(B, Hkv, T, d, generator=gen) * torch.exp(0.5 * torch.randn(B, Hkv, T, 1, generator=gen))
        v = torch.randn(B, Hkv, T, d, generator=gen)
        e.append(k[:, :, :300].to(DEV, torch.float16), v[:, :, :300].to(DEV, torch.float16))
        e.append(k[:, :, 300:].to(DEV, torch.float16), v[:, :, 300:].to(DEV, torch.float16))
    qs = [torch.randn(B, Hkv * G, Qn, d, generator=gen).to(DEV, torch.float16) for _ in range(n)]
    L = N.lib()
    ns = L.qkv_attention_splits(B * n, Hkv * G, Hkv, Qn, d, T)
    outs = K.attention_layers(engines, qs, causal=causal, n_splits=ns)
    assert len(outs) == n and outs[0].shape == (B, Hkv * G, Qn, d)
    for e, q, o in zip(engines, qs, outs):
        st, kq, vq = e._store, e.key_quantizer, e.value_quantizer
        ref = K.attention_store(q, st, T, kq.mse_quantizer.Pi, kq.mse_quantizer.codebook.centroids_host,
                                vq.codebook.centroids_host, kq.S, kq.qjl_scale, causal=causal,
                                n_splits=ns)
        # at d = 64 with 1-2 key MSE bits the batch runs split_mfma (exact
        # integer scores) and the single call decode_fused (fp8 query
        # digits): both sit within 2e-5 of the oracle, not bit-identical
        _close(o, ref, 1e-6 if d != 64 or kb == 4 else 2e-5)
    # one layer against the oracle on its stored codes
    e, q, o = engines[2], qs[2], outs[2]
    st, kq, vq = e._store, e.key_quantizer, e.value_quantizer
    kc, kb, vc = st.read_codes(0, T)
    blocks = [dict(kcodes=kc.cpu(), kbits=kb.cpu(), knorm=st.knorm[:, :, :T].cpu(),
                   vcodes=vc.cpu(), vnorm=st.vnorm[:, :, :T].cpu())]
    args = (kq.mse_quantizer.Pi.cpu(), kq.mse_quantizer.codebook.centroids.cpu(),
            vq.codebook.centroids.cpu(), kq.S.cpu(), kq.qjl_scale)
    if causal:
        qg = q.float().cpu().reshape(B, Hkv, G, Qn, d)
        ref = torch.stack([R.attention_naive(qg[:, :, g], blocks, *args, causal=True)
                           for g in range(G)], dim=2).reshape(B, Hkv * G, Qn, d)
    else:
        ref = R.attention_online(q.float().cpu().reshape(B, Hkv, G * Qn, d), blocks,
                                 *args).reshape(B, Hkv * G, Qn, d)
    _close(o, ref, 2e-5)


def test_layers_default_splits_and_errors():
    gen = torch.Generator().manual_seed(1)
    engines = [Q.QuashKVEngine(head_dim=64, seed=7 + l, device=DEV) for l in range(3)]
    for e in engines:
        x = torch.randn(2, 2, 130, 64, generator=gen).to(DEV, torch.float16)
        e.append(x, x)
    qs = [torch.randn(2, 14, 1, 64, generator=gen).to(DEV, torch.float16) for _ in range(3)]
    outs = K.attention_layers(engines, qs)
    for e, q, o in zip(engines, qs, outs):
        _close(o, e.attention(q), 2e-5)
    engines[1].append(x[:, :, :1], x[:, :, :1])     # lengths differ
    with pytest.raises(ValueError, match="one shape"):
        K.attention_layers(engines, qs)
    with pytest.raises(ValueError, match="one query per engine"):
        K.attention_layers(engines[:2], qs)


def test_layer_batch_follows_appends_and_store_growth():
    """A LayerBatch kept across decode steps sees each step's appends, also
    when an append reallocates the stores (capacity doubling)."""
    gen = torch.Generator().manual_seed(2)
    engines = [Q.QuashKVEngine(head_dim=64, seed=11 + l, device=DEV) for l in range(4)]
    for e in engines:
        x = torch.randn(2, 2, 100, 64, generator=gen).to(DEV, torch.float16)
        e.append(x, x)
    batch = K.LayerBatch(engines)
    caps = [e._store.capacity for e in engines]
    for step in range(3):
        qs = [torch.randn(2, 14, 1, 64, generator=gen).to(DEV, torch.float16) for _ in range(4)]
        outs = batch(qs)
        for e, q, o in zip(engines, qs, outs):
            _close(o, e.attention(q), 2e-5)
        for e in engines:   # 60 more tokens per step: the stores outgrow their capacity
            x = torch.randn(2, 2, 60, 64, generator=gen).to(DEV, torch.float16)
            e.append(x, x)
    assert engines[0]._store.capacity > caps[0]


def _stores_equal(a, b, T):
    sa, sb = a._store, b._store
    assert a.total_tokens == b.total_tokens == T and a.num_blocks == b.num_blocks
    assert torch.equal(sa.kst[:, :, :T], sb.kst[:, :, :T])
    assert torch.equal(sa.knorm[:, :, :T], sb.knorm[:, :, :T])
    nt = (T + 31) // 32
    if T % 32:   # bits of the last tile past T are not part of the cache
        ta, tb = sa.vst[:, :, :nt].clone(), sb.vst[:, :, :nt].clone()
        m = (1 << (T % 32)) - 1
        ta[:, :, -1] &= m
        tb[:, :, -1] &= m
        assert torch.equal(ta, tb)
    else:
        assert torch.equal(sa.vst[:, :, :nt], sb.vst[:, :, :nt])
    assert torch.equal(sa.vnorm[:, :, :T], sb.vnorm[:, :, :T])


@pytest.mark.parametrize("d,key_bits,value_bits,dtype", [
    (64, 3, 3, torch.bfloat16), (128, 3, 3, torch.float16), (128, 4, 4, torch.float32),
    (64, 2, 2, torch.float32)])
def test_layer_batch_append_matches_per_engine(d, key_bits, value_bits, dtype):
    """batch.append (one K and one V launch over all layers) writes the same
    store bytes, norms and bookkeeping as each engine's own append: one-token
    decode steps, a multi-token append crossing a V tile, and a store growth."""
    gen = torch.Generator().manual_seed(d + key_bits)
    n, B, H = 6, 3, 2
    mk = lambda: [Q.QuashKVEngine(head_dim=d, key_bits=key_bits, value_bits=value_bits,
                                  seed=5 + l, device=DEV) for l in range(n)]
    ea, eb = mk(), mk()
    T = 61
    for a, b in zip(ea, eb):   # prefill per engine (creates the stores)
        x = torch.randn(B, H, T, d, generator=gen).to(DEV, dtype)
        y = torch.randn(B, H, T, d, generator=gen).to(DEV, dtype)
        a.append(x, y)
        b.append(x, y)
    batch = K.LayerBatch(ea)
    for S in (1, 1, 1, 5, 1, 64):
        ks = [torch.randn(B, H, S, d, generator=gen).to(DEV, dtype) for _ in range(n)]
        vs = [torch.randn(B, H, S, d, generator=gen).to(DEV, dtype) for _ in range(n)]
        batch.append(ks, vs)
        for e, k, v in zip(eb, ks, vs):
            e.append(k, v)
        T += S
        for a, b in zip(ea, eb):
            _stores_equal(a, b, T)
    qs = [torch.randn(B, H * 4, 1, d, generator=gen).to(DEV, torch.float16) for _ in range(n)]
    for o, e, q in zip(batch(qs), eb, qs):
        _close(o, e.attention(q), 2e-5)


def test_layer_batch_append_falls_back():
    """Engines without a store yet, or of different lengths, append one by one."""
    gen = torch.Generator().manual_seed(3)
    engines = [Q.QuashKVEngine(head_dim=64, seed=20 + l, device=DEV) for l in range(3)]
    batch = K.LayerBatch(engines)
    x = torch.randn(2, 2, 40, 64, generator=gen).to(DEV, torch.bfloat16)
    batch.append([x] * 3, [x] * 3)            # no stores yet: per engine
    assert all(e.total_tokens == 40 for e in engines)
    engines[0].append(x[:, :, :1], x[:, :, :1])
    batch.append([x[:, :, :2]] * 3, [x[:, :, :2]] * 3)   # lengths differ: per engine
    assert [e.total_tokens for e in engines] == [43, 42, 42]
    with pytest.raises(ValueError, match="one key and one value"):
        batch.append([x] * 2, [x] * 3)
