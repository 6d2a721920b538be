"""GPU test of qkv_decode_attention_noalloc (the decode step with its
workspace in the library's static per-device scratch array): called through
the C ABI, its outputs equal qkv_decode_attention's (same kernels, caller
workspace) bit for bit on two calls in a row, the second with a smaller
input, and a call whose workspace exceeds the array is rejected."""

import math

import pytest
import torch

import quashkv_amd as Q
from quashkv_amd import _native as N

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(autouse=True, scope="module")
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")
    N.lib()


def _engine(B, Hkv, T, d, seed):
    gen = torch.Generator().manual_seed(seed)
    eng = Q.QuashKVEngine(head_dim=d, seed=42, device=DEV)
    k = torch.randn(B, Hkv, T, d, generator=gen).to(DEV, torch.bfloat16)
    v = torch.randn(B, Hkv, T, d, generator=gen).to(DEV, torch.bfloat16)
    eng.append(k, v)
    return eng


def _args(eng, q, out):
    """qkv_decode_attention's arguments up to the output dtype, for eng's store."""
    st, kq, vq = eng._store, eng.key_quantizer, eng.value_quantizer
    mq = kq.mse_quantizer
    B, Hq, Qn, d = q.shape
    kc = N.HostFloats(mq.codebook.centroids_host)
    vc = N.HostFloats(vq.codebook.centroids_host)
    args = (q.data_ptr(), N.dtype_code(q.dtype), st.kst.data_ptr(), st.knorm.data_ptr(),
            st.vst.data_ptr(), st.vnorm.data_ptr(), st.capacity, eng.total_tokens, B, Hq, st.H,
            Qn, d, st.mbits, st.vbits, mq.Pi.data_ptr(), kc.ptr, vc.ptr, kq.S.data_ptr(),
            float(kq.qjl_scale), 1.0 / math.sqrt(d), 0, out.data_ptr(), N.QKV_F32)
    return args, (kc, vc)


def _both(eng, q):
    """(workspace entry point output, no-alloc entry point output)."""
    L = N.lib()
    B, Hq, Qn, d = q.shape
    st = eng._store
    ns = L.qkv_attention_splits(B, Hq, st.H, Qn, d, eng.total_tokens)
    need = L.qkv_attention_workspace_bytes(B, Hq, st.H, Qn, d, ns)
    assert 0 < need <= N.NOALLOC_SCRATCH_BYTES
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    ref = torch.empty(B, Hq, Qn, d, dtype=torch.float32, device=DEV)
    got = torch.full_like(ref, float("nan"))
    stream = N.stream(q.device)
    a_ref, keep1 = _args(eng, q, ref)
    N.check(L.qkv_decode_attention(*a_ref, ws.data_ptr(), ws.numel(), ns, stream))
    a_got, keep2 = _args(eng, q, got)
    N.check(L.qkv_decode_attention_noalloc(*a_got, ns, stream))
    torch.cuda.synchronize()
    return ref.cpu(), got.cpu()


def test_noalloc_matches_workspace_entry_point_twice():
    gen = torch.Generator().manual_seed(11)
    # first call: cfg3-like GQA 4:1 at d = 128 over 3000 tokens
    big = _engine(4, 8, 3000, 128, seed=1)
    q1 = torch.randn(4, 32, 1, 128, generator=gen).to(DEV, torch.bfloat16)
    ref1, got1 = _both(big, q1)
    assert torch.isfinite(got1).all()
    assert torch.equal(ref1, got1)
    # second call, smaller input: fewer sequences, heads and tokens, d = 64
    small = _engine(2, 2, 200, 64, seed=2)
    q2 = torch.randn(2, 14, 1, 64, generator=gen).to(DEV, torch.bfloat16)
    ref2, got2 = _both(small, q2)
    assert torch.isfinite(got2).all()
    assert torch.equal(ref2, got2)
    # and the first shape again after the smaller one (the array keeps stale data)
    ref3, got3 = _both(big, q1)
    assert torch.equal(ref3, got3) and torch.equal(got3, got1)


def test_noalloc_rejects_oversized_workspace():
    L = N.lib()
    eng = _engine(1, 1, 64, 128, seed=3)
    q = torch.randn(1, 1, 1, 128).to(DEV, torch.bfloat16)
    out = torch.empty(1, 1, 1, 128, device=DEV)
    args, keep = _args(eng, q, out)
    # a batch and split count whose workspace exceeds the array: rejected on the
    # host before any launch
    args = list(args)
    args[8], args[9], args[10] = 4096, 32, 8          # B, Hq, Hkv (shape fields only)
    need = L.qkv_attention_workspace_bytes(4096, 32, 8, 1, 128, 64)
    assert need > N.NOALLOC_SCRATCH_BYTES
    st = L.qkv_decode_attention_noalloc(*args, 64, N.stream(q.device))
    assert st == N.QKV_E_INVALID
    assert "scratch array" in L.qkv_last_error().decode()
