"""GPU parity of the paged cache (quashkv_amd.paged: 64-token pages from one
pool, a device page table per sequence; qkv_paged_store_append and
qkv_paged_decode_attention) against the contiguous store and the oracle.

Bars: the codes and norms read back from the pages are bit-identical to a
contiguous-store engine fed the same K/V (same seed), and so is every
attention output (same kernels, same split count: only the addressing
differs); attention of the paged engine against the oracle's engine
attention (quashkv/engine.py:204-299 restated) within rel-err 1e-3 and
cosine >= 0.9999 on fp32 outputs.  Cases: ragged appends crossing page and
tile edges, shuffled page ids, pool and table growth, bf16 / fp16 / fp32
inputs (fp32 through the generic compress kernel), GQA, causal Q > 1, pages
reused after clear(); the reference's page-manager tests
(quashkv tests/test_vllm_backend.py) on the GPU."""

import math
import random

import pytest
import torch

import quashkv_amd as Q
from quashkv_amd import _native as N
from quashkv_amd.engine import QuashKVEngine
from quashkv_amd.paged import PagedKVStore, PagedQuashKVEngine
from quashkv_amd.integrations.vllm_backend import (
    QuashKVModelManager, QuashKVPageConfig, QuashKVPageManager, quashkv_attention_forward)
from oracle import ref_math as R

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(autouse=True, scope="module")
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")
    N.lib()


def _pair(d, key_bits, value_bits, B, H, seed, pool_pages=5, page_tokens=64):
    cont = QuashKVEngine(head_dim=d, key_bits=key_bits, value_bits=value_bits, seed=seed,
                         device=DEV)
    paged = PagedQuashKVEngine(head_dim=d, key_bits=key_bits, value_bits=value_bits, seed=seed,
                               device=DEV)
    paged._paged = PagedKVStore(B, H, d, key_bits - 1, value_bits, pool_pages, torch.device(DEV),
                                page_tokens)
    random.Random(seed).shuffle(paged._paged.free)      # page ids out of order
    return cont, paged


def _same_codes(cont, paged):
    T = cont.total_tokens
    assert paged.total_tokens == T
    a, b = cont._store, paged._store
    for x, y in zip(a.read_codes(0, T), b.read_codes(0, T)):
        assert torch.equal(x, y)
    assert torch.equal(a.knorm[:, :, :T], b.knorm[:, :, :T])
    assert torch.equal(a.vnorm[:, :, :T], b.vnorm[:, :, :T])


def _oracle(q, eng, causal):
    st = eng._store
    T = eng.total_tokens
    kc, kb, vc = st.read_codes(0, T)
    G = q.shape[1] // st.H
    rep = lambda t: t.cpu().repeat_interleave(G, dim=1)
    blk = dict(kcodes=rep(kc), kbits=rep(kb), knorm=rep(st.knorm[:, :, :T]), vcodes=rep(vc),
               vnorm=rep(st.vnorm[:, :, :T]))
    kq, vq = eng.key_quantizer, eng.value_quantizer
    return R.attention_naive(q.float().cpu(), [blk], kq.mse_quantizer.Pi.cpu(),
                             kq.mse_quantizer.codebook.centroids.cpu(),
                             vq.codebook.centroids.cpu(), kq.S.cpu(), kq.qjl_scale,
                             scale=1.0 / math.sqrt(q.shape[-1]), causal=causal, total_tokens=T)


def _close(got, ref):
    got, ref = got.double().cpu(), ref.double()
    err = float((got - ref).norm() / ref.norm())
    cos = float((got.flatten() @ ref.flatten()) / (got.norm() * ref.norm()))
    assert err <= 1e-3 and cos >= 0.9999, (err, cos)


@pytest.mark.parametrize("page_tokens", [64, 256])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("d,key_bits,value_bits", [
    (d, kb, vb) for d in (64, 128) for kb, vb in ((3, 3), (2, 4))] + [(128, 4, 3), (64, 4, 3),
                                                         (96, 3, 3), (96, 4, 2)])
def test_paged_matches_contiguous(d, dtype, key_bits, value_bits, page_tokens):
    B, H, G = 3, 2, 4
    seed = d + key_bits * 10 + value_bits
    cont, paged = _pair(d, key_bits, value_bits, B, H, seed, page_tokens=page_tokens)
    gen = torch.Generator(device=DEV).manual_seed(seed)
    for step, S in enumerate([70, 1, 1, 57, 33, 1, 100]):   # crosses page and tile edges
        k = torch.randn(B, H, S, d, generator=gen, device=DEV).to(dtype)
        v = torch.randn(B, H, S, d, generator=gen, device=DEV).to(dtype)
        cont.append(k, v)
        paged.append(k, v)
        _same_codes(cont, paged)
        Q = 1 if step % 2 else 4
        q = torch.randn(B, H * G, Q, d, generator=gen, device=DEV).to(dtype)
        for causal in ((False, True) if Q > 1 else (False,)):
            a = cont.attention(q, causal=causal)
            b = paged.attention(q, causal=causal)
            assert torch.equal(a, b), (step, causal, float((a - b).abs().max()))
    st = paged.paged_store
    per_seq = -(-263 // page_tokens)
    assert st.num_pages >= B * per_seq > 5 and st.pages_per_seq >= per_seq   # pool grew
    assert sorted(sum(st.pages, []) + st.free) == list(range(st.num_pages))
    _close(paged.attention(q, causal=True), _oracle(q, paged, causal=True))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_paged_clear_reuses_pages(dtype):
    B, H, d = 2, 4, 128
    cont, paged = _pair(d, 3, 3, B, H, seed=9, pool_pages=2, page_tokens=128)
    gen = torch.Generator(device=DEV).manual_seed(9)
    kv = lambda S: [torch.randn(B, H, S, d, generator=gen, device=DEV, dtype=dtype)
                    for _ in range(2)]
    paged.append(*kv(150))
    pages_before = paged.paged_store.num_pages
    paged.clear()
    assert paged.total_tokens == 0 and not any(paged.paged_store.pages)
    with pytest.raises(ValueError, match="No compressed"):
        paged.attention(torch.randn(B, H, 1, d, device=DEV))
    for S in (40, 1, 30):               # reused pages hold the old tokens' bits
        k, v = kv(S)
        cont.append(k, v)
        paged.append(k, v)
    assert paged.paged_store.num_pages == pages_before
    _same_codes(cont, paged)
    q = torch.randn(B, H, 1, d, generator=gen, device=DEV)
    assert torch.equal(cont.attention(q), paged.attention(q))
    _close(paged.attention(q), _oracle(q, paged, causal=False))


@pytest.mark.parametrize("page_tokens", [64, 2048])
def test_paged_long_split_matches_contiguous(page_tokens):
    """One split streaming 4,133 tokens (nine 512-token chunks, the last one
    partial) over shuffled pages: qkv_paged_decode_attention equals
    qkv_decode_attention on the contiguous store bit for bit at the same
    split count (each wave reads a chunk's page entries a chunk ahead)."""
    B, Hq, H, d, T = 2, 32, 8, 128, 4133
    cont, paged = _pair(d, 3, 3, B, H, seed=5, pool_pages=B * -(-T // page_tokens) + 2,
                        page_tokens=page_tokens)
    gen = torch.Generator(device=DEV).manual_seed(5)
    k = torch.randn(B, H, T, d, generator=gen, device=DEV, dtype=torch.bfloat16)
    v = torch.randn(B, H, T, d, generator=gen, device=DEV, dtype=torch.bfloat16)
    cont.append(k, v)
    paged.append(k, v)
    q = torch.randn(B, Hq, 1, d, generator=gen, device=DEV, dtype=torch.bfloat16)
    L = N.lib()
    stream = N.stream(torch.device(DEV))
    kq = cont.key_quantizer
    kc = N.HostFloats(kq.mse_quantizer.codebook.centroids_host)
    vc = N.HostFloats(cont.value_quantizer.codebook.centroids_host)
    ws_bytes = L.qkv_attention_workspace_bytes(B, Hq, H, 1, d, 1)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    outs = []
    for eng in (cont, paged):
        out = torch.empty(B, Hq, 1, d, device=DEV)
        common = (T, B, Hq, H, 1, d, 2, 3, kq.mse_quantizer.Pi.data_ptr(), kc.ptr, vc.ptr,
                  kq.S.data_ptr(), float(kq.qjl_scale), 1.0 / math.sqrt(d), 0, out.data_ptr(),
                  N.QKV_F32, ws.data_ptr(), ws_bytes, 1, stream)
        if eng is cont:
            st = cont._store
            N.check(L.qkv_decode_attention(q.data_ptr(), N.QKV_BF16, st.kst.data_ptr(),
                                           st.knorm.data_ptr(), st.vst.data_ptr(),
                                           st.vnorm.data_ptr(), st.capacity, *common))
        else:
            st = paged.paged_store
            N.check(L.qkv_paged_decode_attention(
                q.data_ptr(), N.QKV_BF16, st.kpool.data_ptr(), st.knorm.data_ptr(),
                st.vpool.data_ptr(), st.vnorm.data_ptr(), st.table.data_ptr(), st.pages_per_seq,
                st.pt, st.num_pages, *common))
        torch.cuda.synchronize()
        outs.append(out)
    assert torch.equal(outs[0], outs[1]), float((outs[0] - outs[1]).abs().max())
    _close(outs[1], _oracle(q, paged, causal=False))


def test_paged_cfg3_shape_decode_matches_contiguous():
    """cfg3's head layout (32 query / 8 kv heads, d = 128) at 4 sequences of
    1000 tokens appended as a prefill and decode steps."""
    B, Hq, H, d = 4, 32, 8, 128
    cont, paged = _pair(d, 3, 3, B, H, seed=42, pool_pages=B * 4, page_tokens=256)
    gen = torch.Generator(device=DEV).manual_seed(1)
    for S in (997, 1, 1, 1):
        k = torch.randn(B, H, S, d, generator=gen, device=DEV, dtype=torch.bfloat16)
        v = torch.randn(B, H, S, d, generator=gen, device=DEV, dtype=torch.bfloat16)
        cont.append(k, v)
        paged.append(k, v)
        q = torch.randn(B, Hq, 1, d, generator=gen, device=DEV, dtype=torch.bfloat16)
        assert torch.equal(cont.attention(q, out_dtype=torch.bfloat16),
                           paged.attention(q, out_dtype=torch.bfloat16))
    _same_codes(cont, paged)


def test_paged_shape_errors():
    paged = PagedQuashKVEngine(head_dim=64, device=DEV)
    paged.append(torch.randn(2, 2, 5, 64, device=DEV), torch.randn(2, 2, 5, 64, device=DEV))
    with pytest.raises(ValueError, match="does not match"):
        paged.append(torch.randn(3, 2, 1, 64, device=DEV), torch.randn(3, 2, 1, 64, device=DEV))
    with pytest.raises(ValueError, match="do not match"):
        paged.attention(torch.randn(2, 3, 1, 64, device=DEV))
    with pytest.raises(ValueError, match="Expected keys"):
        paged.append(torch.randn(2, 2, 1, 32, device=DEV), torch.randn(2, 2, 1, 32, device=DEV))


# --- the reference's page-manager tests (quashkv tests/test_vllm_backend.py), on the GPU


def test_manager_append_attention_blocks():
    pm = QuashKVPageManager(4, 64, QuashKVPageConfig(), torch.device(DEV))
    pm.compress_and_store(torch.randn(1, 4, 8, 64, device=DEV), torch.randn(1, 4, 8, 64, device=DEV))
    pm.compress_and_store(torch.randn(1, 4, 4, 64, device=DEV), torch.randn(1, 4, 4, 64, device=DEV))
    assert pm.total_tokens == 12
    out = pm.attention(torch.randn(1, 4, 4, 64, device=DEV))
    assert out.shape == (1, 4, 4, 64)
    blocks = pm.get_compressed_blocks()
    assert [b.seq_len for b in blocks] == [8, 4]
    assert blocks[0].mse_indices.shape == (1, 4, 8, 64) and blocks[0].mse_indices.max() < 4
    assert pm.compression_ratio() > 3.0
    pm.clear()
    assert pm.total_tokens == 0


def test_manager_attention_quality():
    torch.manual_seed(42)
    B, H, KV, Q, D = 1, 2, 32, 4, 64
    keys, values = torch.randn(B, H, KV, D), torch.randn(B, H, KV, D)
    queries = torch.randn(B, H, Q, D)
    s = (queries @ keys.transpose(-1, -2)) / math.sqrt(D)
    exact = torch.softmax(s, dim=-1) @ values
    pm = QuashKVPageManager(H, D, QuashKVPageConfig(seed=42), torch.device(DEV))
    out = quashkv_attention_forward(queries.to(DEV), keys.to(DEV), values.to(DEV), pm)
    cos = torch.nn.functional.cosine_similarity(exact.flatten(), out.cpu().flatten(), dim=0)
    assert float(cos) > 0.6
    assert pm.total_tokens == KV


def test_model_manager_generation():
    m = QuashKVModelManager(num_layers=4, num_kv_heads=8, head_size=64, device=DEV)
    B, H, D = 1, 8, 64
    for layer in range(4):
        m.forward_layer(layer, torch.randn(B, H, 32, D, device=DEV),
                        torch.randn(B, H, 32, D, device=DEV), torch.randn(B, H, 32, D, device=DEV))
    for _ in range(5):
        for layer in range(4):
            out = m.forward_layer(layer, torch.randn(B, H, 1, D, device=DEV),
                                  torch.randn(B, H, 1, D, device=DEV),
                                  torch.randn(B, H, 1, D, device=DEV))
            assert out.shape == (B, H, 1, D)
    assert m.stats()["tokens_per_layer"] == [37] * 4
    assert m.total_compressed_bytes() > 0
    m.clear()
    assert all(l.total_tokens == 0 for l in m.layers)


@pytest.mark.parametrize("d,page_tokens", [(128, 64), (64, 256), (96, 64)])
def test_paged_layers_match_single_layer_calls(d, page_tokens):
    """qkv_paged_decode_attention_layers (per-layer pools, one shared page
    table) against one qkv_paged_decode_attention call per layer with the same
    split count: identical outputs."""
    NL, B, H, Hq, Q = 3, 2, 2, 8, 1
    L = N.lib()
    engs = []
    gen = torch.Generator(device=DEV).manual_seed(d + page_tokens)
    for l in range(NL):
        e = PagedQuashKVEngine(head_dim=d, seed=42 + l, device=DEV, page_tokens=page_tokens)
        e._paged = PagedKVStore(B, H, d, 2, 3, 3, torch.device(DEV), page_tokens)
        random.Random(7).shuffle(e._paged.free)          # the same page order in every layer
        for S in (200, 1, 99):
            e.append(torch.randn(B, H, S, d, generator=gen, device=DEV, dtype=torch.bfloat16),
                     torch.randn(B, H, S, d, generator=gen, device=DEV, dtype=torch.bfloat16))
        engs.append(e)
    tab = engs[0].paged_store.table
    assert all(torch.equal(e.paged_store.table, tab) for e in engs)
    T = engs[0].total_tokens
    qs = [torch.randn(B, Hq, Q, d, generator=gen, device=DEV, dtype=torch.bfloat16)
          for _ in range(NL)]
    splits = L.qkv_attention_splits(B * NL, Hq, H, Q, d, T)
    ws_bytes = L.qkv_attention_workspace_bytes(B * NL, Hq, H, Q, d, splits)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    outs = [torch.empty(B, Hq, Q, d, device=DEV) for _ in range(NL)]
    st0, kq0 = engs[0].paged_store, engs[0].key_quantizer
    kc = N.HostFloats(kq0.mse_quantizer.codebook.centroids_host)
    vc = N.HostFloats(engs[0].value_quantizer.codebook.centroids_host)
    arr = lambda ts: N.ptr_array([t.data_ptr() for t in ts])
    sts = [e.paged_store for e in engs]
    N.check(L.qkv_paged_decode_attention_layers(
        NL, arr(qs), N.QKV_BF16, arr([s.kpool for s in sts]), arr([s.knorm for s in sts]),
        arr([s.vpool for s in sts]), arr([s.vnorm for s in sts]), tab.data_ptr(),
        st0.pages_per_seq, page_tokens, min(s.num_pages for s in sts), T, B, Hq, H, Q, d, 2, 3,
        arr([e.key_quantizer.mse_quantizer.Pi for e in engs]), kc.ptr, vc.ptr,
        arr([e.key_quantizer.S for e in engs]), float(kq0.qjl_scale), 1.0 / math.sqrt(d), 0,
        arr(outs), N.QKV_F32, ws.data_ptr(), ws_bytes, splits, N.stream(torch.device(DEV))))
    for e, q, o in zip(engs, qs, outs):
        st, kq = e.paged_store, e.key_quantizer
        ref = torch.empty_like(o)
        N.check(L.qkv_paged_decode_attention(
            q.data_ptr(), N.QKV_BF16, st.kpool.data_ptr(), st.knorm.data_ptr(),
            st.vpool.data_ptr(), st.vnorm.data_ptr(), tab.data_ptr(), st.pages_per_seq,
            page_tokens, st.num_pages, T, B, Hq, H, Q, d, 2, 3, kq.mse_quantizer.Pi.data_ptr(), kc.ptr, vc.ptr,
            kq.S.data_ptr(), float(kq.qjl_scale), 1.0 / math.sqrt(d), 0, ref.data_ptr(),
            N.QKV_F32, ws.data_ptr(), ws_bytes, splits, N.stream(torch.device(DEV))))
        if d == 64:
            # the batch runs split_mfma (exact integer scores), the single call
            # decode_fused (fp8 query digits): both within 2e-5 of the oracle
            err = float((o - ref).double().norm() / ref.double().norm())
            assert err <= 2e-5, err
        else:
            assert torch.equal(o, ref)
        _close(o, _oracle(q, e, causal=False))


@pytest.mark.parametrize("d", [128, 96, 64])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("key_bits,value_bits", [(3, 3), (4, 4), (3, 2)])
@pytest.mark.parametrize("shape", ["few", "many"])
def test_paged_kv_append_equals_two_calls(d, dtype, key_bits, value_bits, shape):
    """qkv_paged_store_append_kv (keys and values in one launch for small
    appends when value bits = key bits: a wave per 32-coordinate block of a
    tile for few tiles, a wave per tile for more; 3/2 bits take two launches
    inside) writes the same pool, bit for bit, as qkv_paged_store_append for
    the keys and then for the values, over ragged sizes and unaligned starts
    on shuffled pages."""
    (B, H), sizes = ((2, 3), (1, 5, 37, 64, 1, 100)) if shape == "few" else \
        ((8, 8), (160, 7, 300))
    dev = torch.device(DEV)
    kq = Q.InnerProductQuantizer(d, key_bits, seed=7, device=DEV)
    vq = Q.MSEQuantizer(d, value_bits, seed=8, device=DEV)
    mq = kq.mse_quantizer
    kc = N.HostFloats(mq.codebook.centroids_host)
    kb = N.HostFloats(mq.codebook.boundaries_host)
    vb = N.HostFloats(vq.codebook.boundaries_host)
    total = sum(sizes)
    stores = []
    for _ in range(2):
        st = PagedKVStore(B, H, d, key_bits - 1, value_bits, B * 32 + 3, dev, 64)
        st.ensure(total)
        stores.append(st)
    g = torch.Generator().manual_seed(11)
    assert stores[0].num_pages >= B * stores[0].table.shape[1]
    perm = torch.randperm(stores[0].num_pages, generator=g)[:B * stores[0].table.shape[1]]
    tab = perm.view(B, -1).to(torch.int32).to(dev)   # shuffled pages, same table for both
    for st in stores:
        st.table = tab.clone()
    L = N.lib()
    dt = N.dtype_code(dtype)
    stream = N.stream(dev)
    t0 = 0
    for S in sizes:
        k = torch.randn(B, H, S, d, generator=g).to(dtype).to(DEV)
        v = torch.randn(B, H, S, d, generator=g).to(dtype).to(DEV)
        a, b = stores
        N.check(L.qkv_paged_store_append_kv(
            dt, k.data_ptr(), v.data_ptr(), B, H, S, d, key_bits - 1, value_bits,
            mq.Pi.data_ptr(), kq.S.data_ptr(), vq.Pi.data_ptr(), kc.ptr, kb.ptr, vb.ptr,
            a.kpool.data_ptr(), a.knorm.data_ptr(), a.vpool.data_ptr(), a.vnorm.data_ptr(),
            a.table.data_ptr(), a.table.shape[1], a.pt, a.num_pages, t0, stream))
        N.check(L.qkv_paged_store_append(
            dt, k.data_ptr(), None, B, H, S, d, key_bits - 1, value_bits, mq.Pi.data_ptr(),
            kq.S.data_ptr(), kc.ptr, kb.ptr, vb.ptr, b.kpool.data_ptr(), b.knorm.data_ptr(),
            b.vpool.data_ptr(), b.vnorm.data_ptr(), b.table.data_ptr(), b.table.shape[1], b.pt,
            b.num_pages, t0, stream))
        N.check(L.qkv_paged_store_append(
            dt, None, v.data_ptr(), B, H, S, d, key_bits - 1, value_bits, vq.Pi.data_ptr(),
            None, None, None, vb.ptr, None, None, b.vpool.data_ptr(), b.vnorm.data_ptr(),
            b.table.data_ptr(), b.table.shape[1], b.pt, b.num_pages, t0, stream))
        t0 += S
    torch.cuda.synchronize()
    a, b = stores
    ga, gb = a.gather(t0), b.gather(t0)       # contiguous copies of tokens [0, t0)
    assert torch.equal(ga.kst[:, :, :t0], gb.kst[:, :, :t0])
    assert torch.equal(ga.knorm[:, :, :t0], gb.knorm[:, :, :t0])
    assert torch.equal(ga.vnorm[:, :, :t0], gb.vnorm[:, :, :t0])
    nt = (t0 + 31) // 32
    va, vb2 = ga.vst[:, :, :nt].clone(), gb.vst[:, :, :nt].clone()
    if t0 % 32:
        va[:, :, -1] &= (1 << (t0 % 32)) - 1
        vb2[:, :, -1] &= (1 << (t0 % 32)) - 1
    assert torch.equal(va, vb2)
    assert ga.knorm[:, :, :t0].abs().min() > 0


@pytest.mark.parametrize("d", [128, 96, 64])
@pytest.mark.parametrize("n_splits", [1, 0])
def test_paged_decode_masks_pages_off_the_pool(d, n_splits):
    """qkv_paged_decode_attention gives no weight to the tokens of a page whose
    table entry lies outside the pool (-1 or >= num_pages): each sequence
    attends like the oracle over its other tokens.  1,500 tokens in 64-token
    pages: one split streams three 512-token chunks (n_splits 1), or the
    library's split count (0).  The masked pages sit inside a chunk, on a
    chunk's first tile and on the last, partial page."""
    B, H, G, S, pt = 3, 2, 2, 1500, 64
    dev = torch.device(DEV)
    e = PagedQuashKVEngine(head_dim=d, seed=31, device=DEV, page_tokens=pt)
    e._paged = PagedKVStore(B, H, d, 2, 3, 8, dev, pt)
    random.Random(3).shuffle(e._paged.free)
    gen = torch.Generator(device=DEV).manual_seed(d + n_splits)
    e.append(torch.randn(B, H, S, d, generator=gen, device=DEV, dtype=torch.bfloat16),
             torch.randn(B, H, S, d, generator=gen, device=DEV, dtype=torch.bfloat16))
    st, kq = e.paged_store, e.key_quantizer
    per = st.pages_per_seq
    off = {0: [(3, -1)], 1: [(8, st.num_pages), (17, -5)], 2: [((S - 1) // pt, st.num_pages + 9)]}
    tab = st.table.clone()
    for b, ents in off.items():
        for page, val in ents:
            tab[b, page] = val
    q = torch.randn(B, H * G, 1, d, generator=gen, device=DEV, dtype=torch.bfloat16)
    L = N.lib()
    splits = n_splits or L.qkv_attention_splits(B, H * G, H, 1, d, S)
    ws_bytes = L.qkv_attention_workspace_bytes(B, H * G, H, 1, d, splits)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    out = torch.empty(B, H * G, 1, d, device=DEV)
    kc = N.HostFloats(kq.mse_quantizer.codebook.centroids_host)
    vc = N.HostFloats(e.value_quantizer.codebook.centroids_host)
    N.check(L.qkv_paged_decode_attention(
        q.data_ptr(), N.QKV_BF16, st.kpool.data_ptr(), st.knorm.data_ptr(), st.vpool.data_ptr(),
        st.vnorm.data_ptr(), tab.data_ptr(), per, pt, st.num_pages, S, B, H * G, H, 1, d, 2, 3,
        kq.mse_quantizer.Pi.data_ptr(), kc.ptr, vc.ptr, kq.S.data_ptr(), float(kq.qjl_scale),
        1.0 / math.sqrt(d), 0, out.data_ptr(), N.QKV_F32, ws.data_ptr(), ws_bytes, splits,
        N.stream(dev)))
    torch.cuda.synchronize()
    cs = e._store                       # the tokens gathered into a contiguous store
    kcd, kbt, vcd = (x.cpu() for x in cs.read_codes(0, S))
    kn, vn = (x[:, :, :S].cpu() for x in (cs.knorm, cs.vnorm))
    vq = e.value_quantizer
    for b in range(B):
        keep = torch.ones(S, dtype=torch.bool)
        for page, _ in off[b]:
            keep[page * pt:(page + 1) * pt] = False
        sel = lambda t: t[b:b + 1, :, keep].repeat_interleave(G, dim=1)
        blk = dict(kcodes=sel(kcd), kbits=sel(kbt), knorm=sel(kn), vcodes=sel(vcd),
                   vnorm=sel(vn))
        ref = R.attention_naive(q[b:b + 1].float().cpu(), [blk], kq.mse_quantizer.Pi.cpu(),
                                kq.mse_quantizer.codebook.centroids.cpu(),
                                vq.codebook.centroids.cpu(), kq.S.cpu(), kq.qjl_scale,
                                scale=1.0 / math.sqrt(d))
        _close(out[b:b + 1], ref)


@pytest.mark.parametrize("d", [128, 96, 64])
@pytest.mark.parametrize("shape", ["few", "many"])
def test_paged_kv_append_skips_pages_off_the_pool(d, shape):
    """qkv_paged_store_append_kv never writes through page-table entries
    outside the pool (-1 or >= num_pages): with such entries in the table,
    every pool page that no valid entry names keeps its bytes, keys and values
    and both norms, in the wave-per-block (few tiles) and wave-per-tile (many
    tiles) modes; the pages the valid entries name are written."""
    (B, H), sizes = ((2, 3), (1, 5, 37, 64, 1)) if shape == "few" else ((8, 8), (160, 7))
    dev = torch.device(DEV)
    kq = Q.InnerProductQuantizer(d, 3, seed=7, device=DEV)
    vq = Q.MSEQuantizer(d, 3, seed=8, device=DEV)
    mq = kq.mse_quantizer
    kc = N.HostFloats(mq.codebook.centroids_host)
    kb = N.HostFloats(mq.codebook.boundaries_host)
    vb = N.HostFloats(vq.codebook.boundaries_host)
    total = sum(sizes)
    st = PagedKVStore(B, H, d, 2, 3, B * 8 + 5, dev, 64)
    st.ensure(total)
    g = torch.Generator().manual_seed(12)
    per = st.table.shape[1]
    tab = torch.randperm(st.num_pages, generator=g)[:B * per].view(B, per).to(torch.int32)
    tab[0, 1] = -1                      # off the pool, both ways
    tab[1, 0] = st.num_pages
    tab[B - 1, per - 1] = st.num_pages + 7
    st.table = tab.to(dev)
    for t in (st.kpool, st.vpool):      # sentinel contents
        t.copy_(torch.randint(0, 255, t.shape, generator=g, dtype=torch.int32).to(t.dtype).to(dev))
    for t in (st.knorm, st.vnorm):
        t.copy_(torch.randn(t.shape, generator=g).to(dev))
    before = [t.clone() for t in (st.kpool, st.knorm, st.vpool, st.vnorm)]
    L = N.lib()
    stream = N.stream(dev)
    t0 = 0
    for S in sizes:
        k = torch.randn(B, H, S, d, generator=g).to(torch.bfloat16).to(DEV)
        v = torch.randn(B, H, S, d, generator=g).to(torch.bfloat16).to(DEV)
        N.check(L.qkv_paged_store_append_kv(
            N.QKV_BF16, k.data_ptr(), v.data_ptr(), B, H, S, d, 2, 3, mq.Pi.data_ptr(),
            kq.S.data_ptr(), vq.Pi.data_ptr(), kc.ptr, kb.ptr, vb.ptr, st.kpool.data_ptr(),
            st.knorm.data_ptr(), st.vpool.data_ptr(), st.vnorm.data_ptr(), st.table.data_ptr(),
            per, st.pt, st.num_pages, t0, stream))
        t0 += S
    torch.cuda.synchronize()
    used = sorted({int(p) for p in tab.flatten() if 0 <= int(p) < st.num_pages})
    untouched = [p for p in range(st.num_pages) if p not in used]
    assert untouched and used
    for a, b0 in zip((st.kpool, st.knorm, st.vpool, st.vnorm), before):
        assert torch.equal(a[untouched], b0[untouched])
    # the first token's page of sequence 0 (a valid entry) was written
    p0 = int(tab[0, 0])
    assert not torch.equal(st.knorm[p0], before[1][p0])
