"""The fused decode attention behind a HuggingFace model (transformers'
attention interface, quashkv_amd.integrations.hf_attention): a small
Qwen2-shaped model (cfg2's head layout: 14 query heads, 2 kv heads,
head_dim 64; seeded random weights, bf16) runs prefill and decode steps with
every layer's K/V compressed in a QuashKVHFCache.

Bars: each attention call inside the model against the oracle's engine
attention (quashkv/engine.py:204-299 restated, causal over the cache for the
prefill) on the cache's own codes, rel-err <= 1e-2 and cosine >= 0.9999 (bf16
queries and outputs); greedy generate() runs and leaves the cache at the
expected length; the model's first-token logits stay close to the same
model's uncompressed eager attention (cosine >= 0.98 with 4-bit K/V)."""

import pytest
import torch

from quashkv_amd import _native as N
from oracle import ref_math as R

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(autouse=True, scope="module")
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")
    N.lib()


def _model(attn):
    from transformers import AutoModelForCausalLM, Qwen2Config
    cfg = Qwen2Config(vocab_size=512, hidden_size=14 * 64, intermediate_size=512,
                      num_hidden_layers=2, num_attention_heads=14, num_key_value_heads=2,
                      max_position_embeddings=256, tie_word_embeddings=False)
    torch.manual_seed(0)
    model = AutoModelForCausalLM.from_config(cfg, attn_implementation=attn,
                                             dtype=torch.bfloat16)
    return model.to(DEV).eval()


def _oracle(q, eng):
    """Engine attention of (B, Hq, Q, d) queries on the engine's codes, causal
    over the cache when Q > 1, kv heads shared by groups of Hq / Hkv."""
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
                             scale=1.0 / 8.0, causal=q.shape[2] > 1, total_tokens=T)


def test_hf_attention_calls_match_oracle():
    from transformers import AttentionInterface
    from transformers.masking_utils import AttentionMaskInterface
    from quashkv_amd.integrations import hf_attention as HA

    calls = []

    def spy(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kw):
        out, w = HA.quashkv_attention(module, query, key, value, attention_mask,
                                      scaling=scaling, dropout=dropout, **kw)
        ref = _oracle(query, key._quashkv_layer.engine)
        calls.append((out.transpose(1, 2).float().cpu(), ref))
        return out, w

    AttentionInterface.register("quashkv_spy", spy)
    AttentionMaskInterface.register("quashkv_spy", lambda *a, **k: None)
    model = _model("quashkv_spy")
    cache = HA.QuashKVHFCache.from_model(model)
    g = torch.Generator().manual_seed(3)
    ids = torch.randint(0, 512, (2, 24), generator=g).to(DEV)
    with torch.no_grad():
        out = model(input_ids=ids, past_key_values=cache, use_cache=True)
        for _ in range(3):
            nxt = out.logits[:, -1:].argmax(-1)
            out = model(input_ids=nxt, past_key_values=cache, use_cache=True)
    assert len(calls) == 2 * 4 and cache.get_seq_length() == 27
    for got, ref in calls:
        err = float((got.double() - ref.double()).norm() / ref.double().norm())
        cos = float((got.flatten().double() @ ref.flatten().double())
                    / (got.double().norm() * ref.double().norm()))
        assert err <= 1e-2 and cos >= 0.9999, (err, cos)


def test_hf_generate_with_compressed_cache():
    from quashkv_amd.integrations import hf_attention as HA
    from quashkv_amd.integrations.hf_cache import QuashKVCacheConfig

    g = torch.Generator().manual_seed(4)
    ids = torch.randint(0, 512, (2, 12), generator=g).to(DEV)
    model = _model(HA.ATTN_IMPLEMENTATION)
    cache = HA.QuashKVHFCache.from_model(model, QuashKVCacheConfig(key_bits=4, value_bits=4))
    with torch.no_grad():
        seq = model.generate(ids, max_new_tokens=6, do_sample=False, past_key_values=cache)
    assert seq.shape == (2, 18) and torch.equal(seq[:, :12], ids)
    assert cache.get_seq_length() == 17
    # prefill logits against the same weights with uncompressed eager attention
    ref_model = _model("eager")
    with torch.no_grad():
        ref = ref_model(input_ids=ids).logits[:, -1].float()
        cache2 = HA.QuashKVHFCache.from_model(model, QuashKVCacheConfig(key_bits=4, value_bits=4))
        got = model(input_ids=ids, past_key_values=cache2, use_cache=True).logits[:, -1].float()
    # 4-bit K/V quantisation noise leaves the logits at cosine ~0.99; a wrong
    # position, head mapping or mask would drop it far below
    cos = float(torch.nn.functional.cosine_similarity(got, ref, dim=-1).min())
    assert cos >= 0.98, cos
