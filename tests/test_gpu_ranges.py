"""Per-sequence key ranges and causal query positions in decode attention
(qkv_decode_attention_ranges; QuashKVEngine.attention(kv_start=, kv_end=,
q_end=); fused_quantized_attention(causal=True, total_kv_tokens=...)).

The reference places causal queries at total_kv_tokens - Q + i
(quashkv/triton_kernels/attention.py:118-121) and HF's attention masks the
padding of a batch on the reference's reconstructed keys
(quashkv/integrations/hf_cache.py:123-152).  The oracle: the reference's
scores (oracle _block_scores, quashkv/engine.py:250-271) over all T cached
keys, keys outside [start, end) and causally hidden keys set to -inf, softmax,
values c_v[code] Pi n_v (engine.py:284-297); a row with no visible key is 0.
Bars: rel-err <= 1e-4 against it on the store's own codes (fp32 queries),
bit-identical to the plain entry point when the ranges cover everything."""

import math

import numpy as np
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


def _oracle(eng, q, start, end, causal, q_end):
    """(B, Hq, Q, d) reference attention with per-sequence key ranges."""
    st = eng._store
    T = eng.total_tokens
    kc, kb, vc = (t.cpu() for t in st.read_codes(0, T))
    kn, vn = st.knorm[:, :, :T].cpu(), st.vnorm[:, :, :T].cpu()
    kq, vq = eng.key_quantizer, eng.value_quantizer
    pi = kq.mse_quantizer.Pi.cpu()
    B, Hq, Qn, d = q.shape
    Hkv = kc.shape[1]
    G = Hq // Hkv
    qr = (q.float().reshape(B, Hkv, G * Qn, d)) @ pi.T
    sc = R._block_scores(qr, kc, kb, kn, kq.mse_quantizer.codebook.centroids.cpu(), kq.S.cpu(),
                         kq.qjl_scale, 1.0 / math.sqrt(d)).double()     # (B, Hkv, G Q, T)
    t = torch.arange(T)
    qi = torch.arange(G * Qn) % Qn
    for b in range(B):
        lo, hi = max(0, int(start[b])), min(T, int(end[b]))
        hide = (t < lo) | (t >= hi)
        sc[b, :, :, hide] = float("-inf")
        if causal:
            cp = q_end if q_end > 0 else hi
            sc[b][:, t[None, :] > (cp - Qn + qi)[:, None]] = float("-inf")
    w = torch.softmax(sc, dim=-1)
    w = torch.nan_to_num(w, nan=0.0)                     # rows without a visible key: 0
    v = (vq.codebook.centroids.cpu()[vc.long()] @ vq.Pi.cpu()).double() * vn.double()[..., None]
    return (w @ v).reshape(B, Hq, Qn, d).float()


def _engine(d, T, B, Hkv, seed, capacity=0):
    gen = torch.Generator().manual_seed(seed)
    k = torch.randn(B, Hkv, T, d, generator=gen)
    k[..., 3] *= 8.0
    v = torch.randn(B, Hkv, T, d, generator=gen)
    eng = Q.QuashKVEngine(head_dim=d, seed=seed, device=DEV, capacity=capacity)
    eng.append(k.to(DEV), v.to(DEV))
    return eng, gen


def _rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return float((a - b).norm() / b.norm().clamp(min=1e-30))


@pytest.mark.parametrize("d", [128, 64, 96])
@pytest.mark.parametrize("causal,Qn", [(False, 1), (True, 3)])
@pytest.mark.parametrize("splits", [1, 5])
def test_ranges_vs_oracle(d, causal, Qn, splits):
    B, Hkv, G, T = 5, 2, 4, 1500
    eng, gen = _engine(d, T, B, Hkv, seed=d + Qn + splits)
    q = torch.randn(B, Hkv * G, Qn, d, generator=gen)
    start = torch.tensor([0, 37, 300, 1499, 700], dtype=torch.int32)
    end = torch.tensor([1500, 1500, 1111, 1500, 700], dtype=torch.int32)   # last: empty
    st = eng._store
    kq, vq = eng.key_quantizer, eng.value_quantizer
    for q_end in ((0, 1490) if causal else (0,)):
        out = K.attention_store(q.to(DEV), st, T, kq.mse_quantizer.Pi,
                                kq.mse_quantizer.codebook.centroids_host,
                                vq.codebook.centroids_host, kq.S, kq.qjl_scale, causal=causal,
                                n_splits=splits, kv_start=start.to(DEV), kv_end=end.to(DEV),
                                q_end=q_end)
        ref = _oracle(eng, q, start, end, causal, q_end)
        assert torch.isfinite(out).all()
        assert out[4].abs().max() == 0            # no key in range: zeros
        assert _rel(out[:4], ref[:4]) <= 1e-4, (q_end, _rel(out[:4], ref[:4]))


def test_ranges_generic_path_vs_oracle():
    """A copy of the store whose capacity is a multiple of 32 but not of 64
    runs the VALU kernel; the ranges and the causal position apply there too."""
    from quashkv_amd.store import KVStore
    B, Hkv, G, T, d = 3, 2, 2, 576, 128
    eng, gen = _engine(d, T, B, Hkv, seed=11)
    st = eng._store
    kc, kb, vc = st.read_codes(0, T)
    st2 = KVStore(B, Hkv, d, 2, 3, 64, st.device)
    st2._alloc(T + 32, 0)
    assert st2.capacity % 64 != 0
    st2.knorm[:, :, :T].copy_(st.knorm[:, :, :T])
    st2.vnorm[:, :, :T].copy_(st.vnorm[:, :, :T])
    st2.write_codes(0, T, kc.reshape(-1, d).contiguous(), kb.reshape(-1, d).contiguous(),
                    vc.reshape(-1, d).contiguous())
    kq, vq = eng.key_quantizer, eng.value_quantizer
    kh, vh = kq.mse_quantizer.codebook.centroids_host, vq.codebook.centroids_host
    L = N.lib()
    assert L.qkv_attention_path(d, 2, 3, N.HostFloats(kh).ptr, N.HostFloats(vh).ptr,
                                st2.capacity, T, 2) == 0
    q = torch.randn(B, Hkv * G, 2, d, generator=gen)
    start = torch.tensor([5, 0, 100], dtype=torch.int32)
    end = torch.tensor([576, 333, 500], dtype=torch.int32)
    out = K.attention_store(q.to(DEV), st2, T, kq.mse_quantizer.Pi, kh, vh, kq.S, kq.qjl_scale,
                            causal=True, n_splits=2, kv_start=start.to(DEV),
                            kv_end=end.to(DEV), q_end=450)
    ref = _oracle(eng, q, start, end, True, 450)
    assert _rel(out, ref) <= 1e-4, _rel(out, ref)


def test_full_ranges_equal_plain_call():
    B, Hkv, G, T, d = 4, 2, 4, 2000, 128
    eng, gen = _engine(d, T, B, Hkv, seed=3)
    q = torch.randn(B, Hkv * G, 1, d, generator=gen).to(DEV, torch.bfloat16)
    plain = eng.attention(q)
    ranged = eng.attention(q, kv_start=torch.zeros(B, dtype=torch.int32, device=DEV),
                           kv_end=torch.full((B,), T, dtype=torch.int32, device=DEV))
    assert torch.equal(plain, ranged)


@pytest.mark.parametrize("offset", [-5, 7, 0])
def test_fused_quantized_attention_causal_offsets(offset):
    """fused_quantized_attention(causal=True, total_kv_tokens=T + offset) puts
    query i at T + offset - Q + i, as the reference's online attention
    (oracle attention_naive with total_tokens; offset 0 means T)."""
    gen = torch.Generator().manual_seed(20 + offset)
    B, H, T, Qn, d = 2, 3, 300, 4, 128
    kq = Q.InnerProductQuantizer(d, 3, seed=5, device=DEV)
    vq = Q.MSEQuantizer(d, 3, seed=5, device=DEV)
    k = torch.randn(B, H, T, d, generator=gen).to(DEV)
    v = torch.randn(B, H, T, d, generator=gen).to(DEV)
    kc, kb, kn = kq.compress(k)
    vc, vn = vq.compress(v)
    blk = K.CompressedBlock(kc, kb, kn, vc, vn, T)
    q = torch.randn(B, H, Qn, d, generator=gen)
    tot = T + offset
    out = K.fused_quantized_attention(q.to(DEV), [blk], kq.mse_quantizer.Pi,
                                      kq.mse_quantizer.codebook.centroids,
                                      vq.codebook.centroids, kq.S, kq.qjl_scale, causal=True,
                                      total_kv_tokens=tot if offset else 0)
    blocks = [dict(kcodes=kc.cpu(), kbits=kb.cpu(), knorm=kn.cpu(), vcodes=vc.cpu(),
                   vnorm=vn.cpu())]
    ref = R.attention_naive(q, blocks, kq.mse_quantizer.Pi.cpu(),
                            kq.mse_quantizer.codebook.centroids.cpu(),
                            vq.codebook.centroids.cpu(), kq.S.cpu(), kq.qjl_scale, causal=True,
                            total_tokens=tot)
    assert _rel(out, ref) <= 1e-4, _rel(out, ref)


def test_hf_left_padded_batch_matches_unpadded_sequences():
    """Left-padded batched prefill + decode through the registered attention
    (HF's 2-D padding mask -> per-sequence key ranges) gives each sequence the
    logits it gets alone, unpadded, through the same compressed path."""
    from transformers import AutoModelForCausalLM, Qwen2Config
    from quashkv_amd.integrations import hf_attention as HA
    cfg = Qwen2Config(vocab_size=512, hidden_size=4 * 64, intermediate_size=256,
                      num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                      max_position_embeddings=256, tie_word_embeddings=False)
    torch.manual_seed(0)
    model = AutoModelForCausalLM.from_config(cfg, attn_implementation=HA.ATTN_IMPLEMENTATION,
                                             dtype=torch.float32).to(DEV).eval()
    g = torch.Generator().manual_seed(9)
    lens = [20, 13]
    seqs = [torch.randint(1, 512, (n,), generator=g) for n in lens]
    Tm = max(lens)
    ids = torch.zeros(2, Tm, dtype=torch.long)
    mask = torch.zeros(2, Tm, dtype=torch.long)
    for b, s in enumerate(seqs):
        ids[b, Tm - len(s):] = s
        mask[b, Tm - len(s):] = 1
    ids, mask = ids.to(DEV), mask.to(DEV)
    pos = (mask.cumsum(-1) - 1).clamp(min=0)
    cache = HA.QuashKVHFCache.from_model(model)
    with torch.no_grad():
        out = model(input_ids=ids, attention_mask=mask, position_ids=pos, past_key_values=cache,
                    use_cache=True)
        nxt = out.logits[:, -1:].argmax(-1)
        mask2 = torch.cat([mask, torch.ones(2, 1, dtype=torch.long, device=DEV)], dim=1)
        out2 = model(input_ids=nxt, attention_mask=mask2, position_ids=pos[:, -1:] + 1,
                     past_key_values=cache, use_cache=True)
    for b, s in enumerate(seqs):
        solo = HA.QuashKVHFCache.from_model(model)
        with torch.no_grad():
            o = model(input_ids=s[None].to(DEV), past_key_values=solo, use_cache=True)
            o2 = model(input_ids=nxt[b:b + 1], past_key_values=solo, use_cache=True)
        for got, ref in ((out.logits[b, -1], o.logits[0, -1]), (out2.logits[b, -1], o2.logits[0, -1])):
            rel = float((got - ref).norm() / ref.norm())
            assert rel <= 1e-3, (b, rel)
