"""Benchmark the TurboQuant hot path on one MI355X.

Headline ("cfg3"): Llama-3-8B-shaped single-layer
decode attention over a 3-bit compressed KV cache -- B=32, 32 query heads over
8 kv heads (GQA 4:1), head_dim 128, context 8192; keys 3-bit IP (2-bit MSE +
1-bit QJL), values 3-bit MSE; bf16 queries; keys N(0,1) with 4 outlier
channels x10.  The packed cache is prebuilt by the HIP compress kernel, then
decode steps are timed.  A step = one qkv_decode_attention call over the whole
cache; at this shape that is ONE launch of decode_fused (query rotation and
integer operands, scores, online softmax, value accumulation and the value
un-rotation in one kernel).  Several distinct caches are rotated between steps
so the 256 MB MALL cannot serve a repeat.  Compress (bf16 K and V -> packed
cache) is timed separately and reported in Gvec/s.

The default line also carries one sub-object per other BASELINE config:
cfg1 (README quickstart), cfg2_layers (Qwen2.5-0.5B-shaped decode over 24
layers), cfg4 (long-context mixed precision), cfg5 (MIPS index) -- each with
its time in us, its fraction of the peak that bounds it and a CPU baseline
from the oracle on the same inputs.  `--workload cfgN` prints one of them as
its own line.

`value` is packed-byte throughput of the decode step (GB/s, inputs resident in
HBM); `roofline` covers decode_fused, timed with HIP events on its launch
stream, with `traffic` from the rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes
recorded in profiles/decode_fused_cfg3_decode.md (`--pmc-summary` turns the
four rocprofv3 output directories into that record).
"""

from __future__ import annotations

import argparse
import csv
import glob
import json
import math
import os
import re
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
PEAK_INT8_TOPS = 5000.0
METRIC = "decode attn over 3-bit KV: µs/step, HBM GB/s % of peak; compress Gvec/s"
DTYPE = ("fp8 x fp4 MFMA scores (query weights as 4 fp8 digits, ~16 bits), i8 MFMA values "
         "(softmax weights as 29-bit fixed point); f32 softmax")
TRAFFIC_RECORD = os.path.join(ROOT, "profiles", "decode_fused_cfg3_decode.md")

B, HQ, HKV, D, T = 32, 32, 8, 128, 8192
KEY_BITS, VAL_BITS = 3, 3
OUTLIERS = (11, 47, 83, 119)


def kv_bytes_per_token_head(d: int) -> int:
    # packed K: 2-bit MSE (d/4) + 1-bit QJL (d/8) + fp32 norm; V: 3-bit (3 ceil(d/8)) + norm
    return (2 * d) // 8 + d // 8 + 4 + 3 * ((d + 7) // 8) + 4


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def host_cores() -> int:
    """CPUs this process may run on: its affinity set, capped by a cgroup CPU
    quota where one is set."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if quota != "max":
            n = min(n, max(1, int(int(quota) // int(period))))
    except (OSError, ValueError):
        pass
    return max(1, n)


def cpu_threads() -> int:
    """torch CPU threads for the baselines: every core the process has."""
    import torch
    torch.set_num_threads(host_cores())
    return torch.get_num_threads()


def median_s(fn, reps: int) -> float:
    """Median wall time of fn() over reps runs after one untimed run."""
    fn()
    ts = []
    for _ in range(max(reps, 1)):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def event_ms(fn, reps: int, stream, flush=None) -> list:
    """Per-call device time (ms) of fn() bracketed by HIP events on ``stream``;
    with ``flush`` the MALL is overwritten before every call."""
    import torch
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(reps)]
    for i, (a, b) in enumerate(evs):
        if flush is not None:
            flush.fill_(float(i))
        a.record(stream)
        fn()
        b.record(stream)
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in evs]


# ------------------------------------------------------------------ PMC traffic

def copy_calibration() -> None:
    """A plain device copy of known size: what rocprofv3's FETCH_SIZE / WRITE_SIZE
    read for it scales the counters of the kernels measured against it."""
    import torch
    n = 256 * 1024 * 1024 // 4
    a = torch.empty(n, device="cuda").uniform_()
    b = torch.empty_like(a)
    flush = torch.empty(512 * 1024 * 1024 // 4, device="cuda")  # evicts the MALL between copies
    for i in range(3):
        flush.fill_(float(i))
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_per_copy": n * 4, "copies": 3}))


def _pmc_mean(run_dir: str, counter: str, kernel_re: str) -> tuple:
    """Mean per-dispatch value of ``counter`` over the dispatches whose kernel
    name matches ``kernel_re`` in a rocprofv3 --pmc csv output directory
    (rows of one dispatch -- one per hardware instance -- are summed)."""
    per = {}
    files = glob.glob(os.path.join(run_dir, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no *counter_collection.csv under {run_dir}")
    rx = re.compile(kernel_re)
    for f in files:
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                if r["Counter_Name"] != counter or not rx.search(r["Kernel_Name"]):
                    continue
                key = (f, r["Dispatch_Id"])
                per[key] = per.get(key, 0.0) + float(r["Counter_Value"])
    if not per:
        raise SystemExit(f"no {counter} rows for /{kernel_re}/ under {run_dir}")
    return sum(per.values()) / len(per), len(per)


def pmc_summary(dirs: list, kernel_re: str) -> None:
    """Prints the traffic record of one kernel from four rocprofv3 --pmc runs:
    the kernel's FETCH_SIZE and WRITE_SIZE passes and the same two counters
    over `bench.py --copy-calibration` (a 256 MiB device copy)."""
    kf, kw, cf, cw = dirs
    fetch, nf = _pmc_mean(kf, "FETCH_SIZE", kernel_re)
    write, nw = _pmc_mean(kw, "WRITE_SIZE", kernel_re)
    copy_re = r"copyBuffer|[Cc]opy"
    cfetch, _ = _pmc_mean(cf, "FETCH_SIZE", copy_re)
    cwrite, _ = _pmc_mean(cw, "WRITE_SIZE", copy_re)
    print(f"pmc-traffic: kernel=/{kernel_re}/ fetch_kib={fetch:.1f} write_kib={write:.1f} "
          f"dispatches={nf},{nw} copy_bytes={256 << 20} copy_fetch_kib={cfetch:.1f} "
          f"copy_write_kib={cwrite:.1f}")


def pmc_traffic(path: str = TRAFFIC_RECORD):
    """HBM bytes per launch from the `pmc-traffic:` record of a profile summary:
    FETCH_SIZE and WRITE_SIZE (KiB per dispatch), each scaled by copy bytes /
    what the same counter reads for the calibration copy.  None if absent."""
    try:
        text = open(path).read()
    except OSError:
        return None
    m = re.search(r"pmc-traffic:.*", text)
    if not m:
        return None
    kv = dict(re.findall(r"(\w+)=([^\s]+)", m.group(0)))
    copy = float(kv["copy_bytes"])
    f = float(kv["fetch_kib"]) * 1024 * copy / (float(kv["copy_fetch_kib"]) * 1024)
    w = float(kv["write_kib"]) * 1024 * copy / (float(kv["copy_write_kib"]) * 1024)
    return {"bytes": int(round(f + w)), "fetch_factor": round(copy / (float(kv["copy_fetch_kib"])
                                                                      * 1024), 3),
            "write_factor": round(copy / (float(kv["copy_write_kib"]) * 1024), 3),
            "source": os.path.relpath(path, ROOT)}


# ------------------------------------------------------------------ cfg3 pieces

def make_inputs(seed: int, dev, gen_dtype):
    import torch
    g = torch.Generator(device=dev).manual_seed(seed)
    k = torch.randn(B, HKV, T, D, device=dev, generator=g, dtype=torch.float32)
    k[..., list(OUTLIERS)] *= 10.0
    v = torch.randn(B, HKV, T, D, device=dev, generator=g, dtype=torch.float32)
    return k.to(gen_dtype), v.to(gen_dtype)


def compress_fp32(args, dev, stream) -> dict:
    """The compress paths on fp32 rows at the cfg3 shape (2^21 K and 2^21 V
    token-heads): the engine append (fused, fp32 rows split hi + lo for the
    fp16 MFMA) into the packed store, and the reference's quantizer operators
    InnerProductQuantizer.compress (keys) + MSEQuantizer.compress (values),
    which return one uint8 code (and QJL bit) per coordinate
    (qkv_compress_mfma).  Rooflines: the bytes each moves at 8 TB/s."""
    import torch
    import quashkv_amd as Q

    k, v = make_inputs(11, dev, torch.float32)
    eng = Q.QuashKVEngine(head_dim=D, key_bits=KEY_BITS, value_bits=VAL_BITS, seed=42,
                          device=dev, capacity=T)

    def append():
        eng.clear()
        eng.append(k, v)

    for _ in range(5):
        append()
    app_ms = statistics.median(event_ms(append, args.compress_reps, stream))
    kq, vq = eng.key_quantizer, eng.value_quantizer
    api = lambda: (kq.compress(k), vq.compress(v))
    for _ in range(3):
        api()
    api_ms = statistics.median(event_ms(api, args.compress_reps, stream))
    n_th = B * HKV * T
    n_vec = 2 * n_th
    app_bytes = n_vec * D * 4 + n_th * kv_bytes_per_token_head(D)
    api_bytes = n_vec * (D * 4 + 4) + n_th * (2 * D + D)   # codes (+ QJL bits) one byte each
    del k, v, eng
    return {
        "what": "cfg3-shaped fp32 K/V (2^21 token-heads each): the engine append into the "
                "packed store, and InnerProductQuantizer.compress + MSEQuantizer.compress "
                "(unpacked uint8 codes) on the MFMA compress",
        "append_gvec_s": round(n_vec / (app_ms * 1e-3) / 1e9, 4),
        "append_pct_of_hbm_roofline": round(100 * app_bytes / (app_ms * 1e-3) / 1e9
                                            / PEAK_HBM_GBS, 2),
        "append_roofline_gvec_s": round(n_vec * PEAK_HBM_GBS * 1e9 / app_bytes / 1e9, 2),
        "quantizer_api_gvec_s": round(n_vec / (api_ms * 1e-3) / 1e9, 4),
        "quantizer_api_pct_of_hbm_roofline": round(100 * api_bytes / (api_ms * 1e-3) / 1e9
                                                   / PEAK_HBM_GBS, 2),
    }


def cpu_baseline(eng, q, n_batch: int, reps: int):
    """Oracle online-softmax decode on the first n_batch sequences of the cache;
    also returns the GPU output's relative error against it."""
    import torch
    from oracle import ref_math as R

    thr = cpu_threads()
    st = eng._store
    kq, vq = eng.key_quantizer, eng.value_quantizer
    kc, kb, vc = (t[:n_batch].cpu() for t in st.read_codes(0, T))
    blk = dict(kcodes=kc, kbits=kb, knorm=st.knorm[:n_batch, :, :T].cpu(), vcodes=vc,
               vnorm=st.vnorm[:n_batch, :, :T].cpu())
    qs = q[:n_batch].float().cpu().reshape(n_batch, HKV, HQ // HKV, D)
    args = (kq.mse_quantizer.Pi.cpu(), kq.mse_quantizer.codebook.centroids.cpu(),
            vq.codebook.centroids.cpu(), kq.S.cpu(), kq.qjl_scale)
    med = median_s(lambda: R.attention_online(qs, [blk], *args), reps)
    ref = R.attention_online(qs, [blk], *args).reshape(n_batch, HQ, 1, D).double()
    got = eng.attention(q).cpu()[:n_batch].double()
    rel = float((got - ref).norm() / ref.norm())
    nbytes = n_batch * HKV * T * kv_bytes_per_token_head(D)
    return nbytes / med / 1e9, med, thr, rel


def cpu_compress_decompress(eng, n_batch: int, reps: int):
    """Oracle compress (keys IP, values MSE; quashkv/triton_kernels/compress.py:34-97
    restated) and decompress (decompress.py:32-55 restated: keys MSE-only and
    values, as QuashKVCache reconstructs) on the host, for n_batch sequences'
    worth of rows.  Returns (compress Gvec/s, decompress GB/s, rows, threads)."""
    import torch
    from oracle import ref_math as R

    thr = cpu_threads()
    kq, vq = eng.key_quantizer, eng.value_quantizer
    mq = kq.mse_quantizer
    n = n_batch * HKV * T
    g = torch.Generator().manual_seed(5)
    k = torch.randn(n, D, generator=g)
    k[:, list(OUTLIERS)] *= 10.0
    k = k.to(torch.bfloat16).float()
    v = torch.randn(n, D, generator=g).to(torch.bfloat16).float()
    kpi, kb, ks, kc = (mq.Pi.cpu(), mq.codebook.boundaries.cpu(), kq.S.cpu(),
                       mq.codebook.centroids.cpu())
    vpi, vb, vc = vq.Pi.cpu(), vq.codebook.boundaries.cpu(), vq.codebook.centroids.cpu()
    t_c = median_s(lambda: (R.compress_ip(k, kpi, kb, ks, kc), R.compress_mse(v, vpi, vb)),
                   reps)
    st = eng._store
    kcodes, _, vcodes = (t[:n_batch].cpu().reshape(n, D) for t in st.read_codes(0, T))
    kn = st.knorm[:n_batch, :, :T].cpu().reshape(n)
    vn = st.vnorm[:n_batch, :, :T].cpu().reshape(n)
    t_d = median_s(lambda: (R.decompress_mse(kcodes, kn, kpi, kc),
                            R.decompress_mse(vcodes, vn, vpi, vc)), reps)
    dec_bytes = n * ((KEY_BITS - 1) * D // 8 + VAL_BITS * D // 8 + 2 * 4 + 2 * D * 4)
    return 2 * n / t_c / 1e9, dec_bytes / t_d / 1e9, n, thr, t_c, t_d


def hbm_read_ceiling(dev, stream) -> float:
    """Read-only HBM ceiling (GB/s): qkv_hbm_read_probe over 4 GiB, non-temporal
    16-byte loads, two 256-thread workgroups per CU, 4 loads in flight per
    thread; best of 5."""
    import torch
    from quashkv_amd import _native as N
    lib = N.lib()
    nbytes = 4 << 30
    buf = torch.empty(nbytes // 4, device=dev, dtype=torch.int32).random_(0, 1 << 20)
    sink = torch.zeros(1024, device=dev, dtype=torch.int32)
    grid = 2 * torch.cuda.get_device_properties(dev).multi_processor_count
    call = lambda: N.check(lib.qkv_hbm_read_probe(buf.data_ptr(), nbytes, sink.data_ptr(), grid,
                                                  4, 1, stream.cuda_stream))
    call()
    ms = min(event_ms(call, 5, stream))
    del buf
    return nbytes / (ms * 1e-3) / 1e9


def paged_decode(args, dev, lib, sptr, stream, engines, queries, kc_h, vc_h, kv_bytes):
    """cfg3 over the paged store (quashkv_amd.paged: pages handed out in
    shuffled order, a device page table per sequence): the same K/V as the
    contiguous caches, appended with qkv_paged_store_append and decoded with
    qkv_paged_decode_attention (the same fused kernel reading through the
    page table)."""
    import random
    import torch
    from quashkv_amd import _native as N
    from quashkv_amd.paged import PagedKVStore, PagedQuashKVEngine

    pengs, app_ms = [], []
    for c in range(args.copies):
        k, v = make_inputs(2 + 1000 * c, dev, torch.bfloat16)
        pe = PagedQuashKVEngine(head_dim=D, key_bits=KEY_BITS, value_bits=VAL_BITS, seed=42,
                                device=dev)
        pe._paged = PagedKVStore(B, HKV, D, KEY_BITS - 1, VAL_BITS, B * T // pe.page_tokens, dev,
                                 pe.page_tokens)
        random.Random(c).shuffle(pe._paged.free)
        pe.append(k, v)
        if c == 0:
            # the append kernels into the allocated pages (as the contiguous
            # measurement re-appends into its allocated store)
            for _ in range(3):
                pe._append_paged(k, v, 0)
            for _ in range(3):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for _ in range(args.compress_reps):
                    pe._append_paged(k, v, 0)
                e1.record(stream)
                torch.cuda.synchronize()
                app_ms.append(e0.elapsed_time(e1) / args.compress_reps)
        pengs.append(pe)
        del k, v
    same = all(torch.equal(pe.attention(q), e.attention(q))
               for pe, e, q in zip(pengs, engines, queries))
    splits = lib.qkv_attention_splits(B, HQ, HKV, 1, D, T)
    ws_bytes = lib.qkv_attention_workspace_bytes(B, HQ, HKV, 1, D, splits)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    out = torch.empty(B, HQ, 1, D, dtype=torch.float32, device=dev)
    scale = 1.0 / math.sqrt(D)

    def step(i):
        pe, q = pengs[i % args.copies], queries[i % args.copies]
        st, kq = pe.paged_store, pe.key_quantizer
        mq = kq.mse_quantizer
        N.check(lib.qkv_paged_decode_attention(
            q.data_ptr(), N.QKV_BF16, st.kpool.data_ptr(), st.knorm.data_ptr(),
            st.vpool.data_ptr(), st.vnorm.data_ptr(), st.table.data_ptr(), st.pages_per_seq,
            st.pt, st.num_pages, T, B, HQ, HKV, 1, D, KEY_BITS - 1, VAL_BITS, mq.Pi.data_ptr(),
            kc_h.ptr, vc_h.ptr,
            kq.S.data_ptr(), kq.qjl_scale, scale, 0, out.data_ptr(), N.QKV_F32, ws.data_ptr(),
            ws_bytes, splits, sptr))

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for i in range(args.steps):
        step(args.warmup + i)
    t1.record(stream)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    io_bytes = B * HQ * D * (2 + 4)
    gbs = (kv_bytes + io_bytes) / (ms * 1e-3) / 1e9
    n_vec = 2 * B * HKV * T
    a_ms = statistics.median(app_ms)
    return {"what": f"cfg3 decode + append over {pengs[0].page_tokens}-token pages "
                    "(shuffled page order, one page table per sequence)",
            "page_tokens": pengs[0].page_tokens,
            "decode_us_per_step": round(ms * 1e3, 2), "GB_s": round(gbs, 1),
            "pct_of_hbm_peak": round(100 * gbs / PEAK_HBM_GBS, 2),
            "append_gvec_s": round(n_vec / (a_ms * 1e-3) / 1e9, 4),
            "output_identical_to_contiguous": same}


def hf_decode_step(args, dev, stream):
    """cfg2's decode step (24 layers, batch 16, 14 query / 2 kv heads, head_dim
    64, 2048 cached tokens) two ways:

    * per-layer attention work: the fused path's calls as the registered HF
      attention function makes them (engine.append of the new token, then
      engine.attention over the compressed cache, per layer) against the
      reference's QuashKVCache path (append, reconstruct the whole K^ / V^ of
      the layer, quashkv/integrations/hf_cache.py:123-152, then torch SDPA);
    * a whole-model decode step of a Qwen2.5-0.5B-shaped model (24 layers,
      hidden 896, MLP 4864; seeded random bf16 weights, 1024-token vocabulary)
      through transformers' forward: attn_implementation="quashkv" with a
      QuashKVHFCache (quashkv_amd.integrations.hf_attention), against the same
      model with its own SDPA attention over an uncompressed bf16 DynamicCache
      of the same length."""
    import torch
    import torch.nn.functional as F
    from quashkv_amd.integrations import hf_attention as HA
    from quashkv_amd.integrations.hf_cache import QuashKVCache

    NL, B2, HQ2, HKV2, D2, T2 = 24, 16, 14, 2, 64, 2048
    steps = max(4, args.steps // 3)
    cap = T2 + 4 * (args.warmup + steps) + 64
    g = torch.Generator(device=dev).manual_seed(5)
    fused = HA.QuashKVHFCache(NL, D2, device=dev)
    recon = QuashKVCache(NL, D2, device=dev)
    kvs = []
    for l in range(NL):
        k = torch.randn(B2, HKV2, T2, D2, generator=g, device=dev).to(torch.bfloat16)
        v = torch.randn(B2, HKV2, T2, D2, generator=g, device=dev).to(torch.bfloat16)
        kvs.append((k, v))
        for e in (fused.engines[l], recon.engines[l]):
            e.initial_capacity = cap
            e.append(k, v)
    q = torch.randn(B2, HQ2, 1, D2, generator=g, device=dev).to(torch.bfloat16)
    kn = torch.randn(B2, HKV2, 1, D2, generator=g, device=dev).to(torch.bfloat16)
    vn = torch.randn(B2, HKV2, 1, D2, generator=g, device=dev).to(torch.bfloat16)

    def step_fused():
        for l in range(NL):
            e = fused.engines[l]
            e.append(kn, vn)
            e.attention(q, out_dtype=torch.bfloat16)

    def step_recon():
        for l in range(NL):
            kh, vh = recon.update(kn, vn, l)
            F.scaled_dot_product_attention(q.float(), kh, vh, enable_gqa=True)

    def timed(fn, n):
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(n):
            fn()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / n * 1e3

    res = {"fused": timed(step_fused, steps), "reconstruct": timed(step_recon, steps)}
    del recon

    # whole-model decode steps through transformers
    from transformers import AutoModelForCausalLM, DynamicCache, Qwen2Config
    HA.register()
    mcfg = Qwen2Config(vocab_size=1024, hidden_size=HQ2 * D2, intermediate_size=4864,
                       num_hidden_layers=NL, num_attention_heads=HQ2, num_key_value_heads=HKV2,
                       max_position_embeddings=T2 + 1024, tie_word_embeddings=True)
    torch.manual_seed(0)
    models = {}
    for attn in (HA.ATTN_IMPLEMENTATION, "sdpa"):
        models[attn] = AutoModelForCausalLM.from_config(
            mcfg, attn_implementation=attn, dtype=torch.bfloat16).to(dev).eval()
    models["sdpa"].load_state_dict(models[HA.ATTN_IMPLEMENTATION].state_dict())
    dyn = DynamicCache()
    for l, (k, v) in enumerate(kvs):
        dyn.update(k, v, l)
    caches = {HA.ATTN_IMPLEMENTATION: fused, "sdpa": dyn}
    ids = torch.randint(0, 1024, (B2, 1), generator=g, device=dev)

    def model_step(attn):
        cache = caches[attn]
        pos = torch.full((B2, 1), cache.get_seq_length(), device=dev, dtype=torch.long)
        with torch.no_grad():
            models[attn](input_ids=ids, past_key_values=cache, position_ids=pos, use_cache=True)

    res["model_quashkv"] = timed(lambda: model_step(HA.ATTN_IMPLEMENTATION), steps)
    res["model_sdpa"] = timed(lambda: model_step("sdpa"), steps)
    del models, caches, dyn
    return {"what": "cfg2 decode step, 24 layers (B 16, 14/2 heads, d 64, ~2048 cached tokens)",
            "attention_calls_us_per_step": round(res["fused"], 1),
            "attention_calls_what": "engine.append + engine.attention per layer (the registered "
                                    "attention function's work), bf16",
            "reconstruct_us_per_step": round(res["reconstruct"], 1),
            "reconstruct_what": "reference path: QuashKVCache.update (append + reconstruct K^/V^) "
                                "+ torch SDPA per layer",
            "fused_speedup_vs_reconstruct": round(res["reconstruct"] / res["fused"], 2),
            "model_step_quashkv_us": round(res["model_quashkv"], 1),
            "model_step_sdpa_uncompressed_us": round(res["model_sdpa"], 1),
            "model_what": "transformers forward of one decode token, Qwen2.5-0.5B-shaped random "
                          "bf16 model: attn_implementation='quashkv' + QuashKVHFCache vs "
                          "'sdpa' + uncompressed bf16 DynamicCache"}


# ------------------------------------------------------------------ other configs

def sub_cfg1(args, dev, stream) -> dict:
    """BASELINE configs[0] (cfg1, the README quickstart): QuashKVEngine(128,
    key_bits=3, value_bits=3, seed=42); fp32 N(0,1) K, V (1, 8, 512, 128)
    appended once; one fp32 N(0,1) query (1, 8, 1, 128); data seed 0.
    Per-stage device times (append = compress K and V into the packed store;
    attention = one decode call), compression ratio, and the output against
    the oracle (compress_ip / compress_mse, attention_online) on the same
    inputs."""
    import torch
    import quashkv_amd as Q
    from oracle import ref_math as R

    g = torch.Generator().manual_seed(0)
    k = torch.randn(1, 8, 512, 128, generator=g)
    v = torch.randn(1, 8, 512, 128, generator=g)
    q = torch.randn(1, 8, 1, 128, generator=g)
    kd, vd, qd = k.to(dev), v.to(dev), q.to(dev)
    eng = Q.QuashKVEngine(head_dim=128, key_bits=3, value_bits=3, seed=42, device=dev)

    def append():
        eng.clear()
        eng.append(kd, vd)

    for _ in range(3):
        append()
    app_ms = statistics.median(event_ms(append, 20, stream))
    att = lambda: eng.attention(qd)
    for _ in range(3):
        att()
    att_ms = statistics.median(event_ms(att, 20, stream))
    out = eng.attention(qd).cpu().double()
    kq, vq = eng.key_quantizer, eng.value_quantizer
    mq = kq.mse_quantizer
    tabs = (mq.Pi.cpu(), mq.codebook.boundaries.cpu(), kq.S.cpu(), mq.codebook.centroids.cpu())

    def oracle():
        kc, kb, kn = R.compress_ip(k, *tabs)
        vc, vn = R.compress_mse(v, vq.Pi.cpu(), vq.codebook.boundaries.cpu())
        blk = dict(kcodes=kc, kbits=kb, knorm=kn, vcodes=vc, vnorm=vn)
        return R.attention_online(q, [blk], mq.Pi.cpu(), mq.codebook.centroids.cpu(),
                                  vq.codebook.centroids.cpu(), kq.S.cpu(), kq.qjl_scale)

    thr = cpu_threads()
    ref = oracle().double()
    rel = float((out - ref).norm() / ref.norm())
    cos = float((out.flatten() @ ref.flatten()) / (out.norm() * ref.norm()))
    kv_bytes = 8 * 512 * kv_bytes_per_token_head(128)
    res = {
        "what": "README quickstart: QuashKVEngine(128, 3, 3); fp32 K/V (1, 8, 512, 128) "
                "appended once, one fp32 query",
        "us": round((app_ms + att_ms) * 1e3, 2),
        "append_us": round(app_ms * 1e3, 2),
        "attention_us": round(att_ms * 1e3, 2),
        "attention_pct_of_hbm_peak": round(100 * kv_bytes / (att_ms * 1e-3) / 1e9
                                           / PEAK_HBM_GBS, 3),
        "compression_ratio": round(eng.compression_ratio(), 4),
        "output_shape": list(out.shape),
        "oracle_rel_err": rel, "oracle_cosine": cos,
    }
    if not args.no_cpu:
        s = median_s(oracle, max(args.cpu_reps, 3))
        res["cpu_baseline"] = {"value": round(s * 1e6, 1), "unit": "us", "cores": thr,
                               "kind": "port",
                               "sample": "the whole workload: oracle compress_ip + compress_mse "
                                         "+ attention_online (fp32 torch CPU), median of "
                                         f"{max(args.cpu_reps, 3)}"}
    return res


def sub_cfg2(args, dev, stream) -> dict:
    """BASELINE configs[1] (cfg2): Qwen2.5-0.5B-shaped decode over all 24 layers.
    Engine seeds 42 + l; B=16, Hq=14, Hkv=2 (GQA 7:1), d=64, context 2048;
    K 3-bit IP, V 3-bit MSE; per token-head K, V = fp16(z / |z| r) with
    z ~ N(0, I_64), r ~ LogNormal(0, 0.5); queries fp16 N(0, 1); data seed 1.
    A step = decode attention of one query per sequence in every layer, as one
    layer-batched call (qkv_decode_attention_layers); the MALL is flushed
    before every timed step.  Also timed: the same step as 24 engine calls, and
    a step with the one-token append per layer."""
    import torch
    import quashkv_amd as Q
    from quashkv_amd import _native as N
    from quashkv_amd import kernels as K

    NL, B2, HQ2, HKV2, D2, T2 = 24, 16, 14, 2, 64, 2048
    g = torch.Generator(device=dev).manual_seed(1)

    def kv():
        z = torch.randn(B2, HKV2, T2, D2, device=dev, generator=g)
        r = torch.exp(0.5 * torch.randn(B2, HKV2, T2, 1, device=dev, generator=g))
        return (z / z.norm(dim=-1, keepdim=True) * r).half()

    engines = []
    for l in range(NL):
        e = Q.QuashKVEngine(head_dim=D2, key_bits=3, value_bits=3, seed=42 + l, device=dev,
                            capacity=T2 + 64)
        e.append(kv(), kv())
        engines.append(e)
    qs = [torch.randn(B2, HQ2, 1, D2, device=dev, generator=g).half() for _ in range(NL)]
    torch.cuda.synchronize()
    lib = N.lib()
    splits = lib.qkv_attention_splits(B2 * NL, HQ2, HKV2, 1, D2, T2)
    flush = torch.empty(512 * 1024 * 1024 // 4, device=dev)
    batch = K.LayerBatch(engines)
    step = lambda: batch(qs, n_splits=splits)
    event_ms(step, args.warmup, stream, flush)
    ms = statistics.median(event_ms(step, args.steps, stream, flush))
    outs = step()
    per_layer = lambda: [e.attention(q) for e, q in zip(engines, qs)]
    event_ms(per_layer, 2, stream, flush)
    ms_pl = statistics.median(event_ms(per_layer, 5, stream, flush))
    ref = per_layer()
    torch.cuda.synchronize()
    agree = max(float((a - b).norm() / b.norm()) for a, b in zip(outs, ref))
    k1 = [kv()[:, :, :1].contiguous() for _ in range(2)]

    def with_append():   # the step's appends of every layer in one K and one V launch
        batch.append([k1[0]] * NL, [k1[1]] * NL)
        return batch(qs, n_splits=splits)

    def with_engine_appends():   # the same through each layer's engine
        for e in engines:
            e.append(k1[0], k1[1])
        return batch(qs, n_splits=splits)

    ms_app = statistics.median(event_ms(with_append, 5, stream, flush))
    ms_app_pl = statistics.median(event_ms(with_engine_appends, 5, stream, flush))
    alg = NL * B2 * HKV2 * T2 * 56
    gbs = alg / (ms * 1e-3) / 1e9
    res = {
        "what": "Qwen2.5-0.5B-shaped decode, 24 layers (B 16, 14/2 heads, d 64, ctx 2048, "
                "3-bit K IP / 3-bit V): one layer-batched call",
        "us": round(ms * 1e3, 2), "GB_s": round(gbs, 1),
        "pct_of_hbm_peak": round(100 * gbs / PEAK_HBM_GBS, 2),
        "n_splits": splits, "tokens_per_s": round(B2 / (ms * 1e-3), 1),
        "per_layer_calls_us": round(ms_pl * 1e3, 2),
        "layer_batched_vs_per_layer_rel_diff": agree,
        "step_with_one_token_append_us": round(ms_app * 1e3, 2),
        "step_with_per_engine_appends_us": round(ms_app_pl * 1e3, 2),
        "algorithmic_bytes": alg,
    }
    if not args.no_cpu:
        from oracle import ref_math as R
        thr = cpu_threads()
        e = engines[0]
        st, kq, vq = e._store, e.key_quantizer, e.value_quantizer
        Tn = e.total_tokens
        kc, kb, vc = st.read_codes(0, Tn)
        blocks = [dict(kcodes=kc.cpu(), kbits=kb.cpu(), knorm=st.knorm[:, :, :Tn].cpu(),
                       vcodes=vc.cpu(), vnorm=st.vnorm[:, :, :Tn].cpu())]
        cargs = (kq.mse_quantizer.Pi.cpu(), kq.mse_quantizer.codebook.centroids.cpu(),
                 vq.codebook.centroids.cpu(), kq.S.cpu(), kq.qjl_scale)
        qc = qs[0].float().cpu().reshape(B2, HKV2, HQ2 // HKV2, D2)
        cpu_s = median_s(lambda: R.attention_online(qc, blocks, *cargs), args.cpu_reps)
        res["cpu_baseline"] = {"value": round(cpu_s * NL * 1e6, 1), "unit": "us",
                               "cores": thr, "kind": "port",
                               "sample": f"oracle attention_online on layer 0 of {NL} (all 16 "
                                         f"sequences, {cpu_s:.3f} s, median of "
                                         f"{max(args.cpu_reps, 1)}), scaled x{NL}"}
    return res


def sub_cfg4(args, dev, stream) -> dict:
    """BASELINE configs[3] (cfg4): long-context mixed precision.  B=1, 32 query
    heads over 8 kv heads, d=128; 131072 tokens appended in 64 chunks of 2048;
    K MixedPrecisionMSEQuantizer(128, 3, 2, 32) calibrated on 65536 keys whose
    32 channels 0, 4, ..., 124 have sigma 8 (the rest 1); V 4-bit MSE; bf16
    K, V and query.  Times the 64 chunked appends and one decode query (one
    qkv_decode_attention_kmixed call; the MALL is flushed before every timed
    decode)."""
    import torch
    import quashkv_amd as Q
    from quashkv_amd import _native as N

    lib = N.lib()
    sptr = stream.cuda_stream
    B4, HQ4, HKV4, TT, CH = 1, 32, 8, 131072, 2048
    out_ch = list(range(0, 128, 4))
    g = torch.Generator(device=dev).manual_seed(3)
    cal = torch.randn(65536, D, device=dev, generator=g)
    cal[:, out_ch] *= 8.0
    kq = Q.MixedPrecisionMSEQuantizer(D, outlier_bits=3, regular_bits=2, n_outliers=32,
                                      seed=42, device=dev)
    kq.calibrate(cal)
    k = torch.randn(B4, HKV4, TT, D, device=dev, generator=g)
    k[..., out_ch] *= 8.0
    k = k.to(torch.bfloat16)
    v = torch.randn(B4, HKV4, TT, D, device=dev, generator=g).to(torch.bfloat16)
    q = torch.randn(B4, HQ4, 1, D, device=dev, generator=g).to(torch.bfloat16)
    eng = Q.QuashKVEngine(head_dim=D, value_bits=4, seed=42, device=dev, key_quantizer=kq,
                          capacity=TT)
    chunks = [(k[:, :, a:a + CH].contiguous(), v[:, :, a:a + CH].contiguous())
              for a in range(0, TT, CH)]

    def append_all():
        eng.clear()
        for kc, vc in chunks:
            eng.append(kc, vc)

    for _ in range(2):
        append_all()
    append_ms = statistics.median(event_ms(append_all, 3, stream))

    st = eng._store
    _, pi_perm, n_out, (oc_h, rc_h, _, _, _) = eng._kmix_setup()
    vq = eng.value_quantizer
    vc_h = N.HostFloats(vq.codebook.centroids_host)
    splits = lib.qkv_attention_splits(B4, HQ4, HKV4, 1, D, TT)
    ws_bytes = lib.qkv_attention_workspace_bytes(B4, HQ4, HKV4, 1, D, splits)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    out = torch.empty(B4, HQ4, 1, D, dtype=torch.float32, device=dev)
    scale = 1.0 / math.sqrt(D)
    flush = torch.empty(512 * 1024 * 1024 // 4, device=dev)

    def decode():
        N.check(lib.qkv_decode_attention_kmixed(
            q.data_ptr(), N.QKV_BF16, st.kst.data_ptr(), st.knorm.data_ptr(), st.vst.data_ptr(),
            st.vnorm.data_ptr(), st.capacity, TT, B4, HQ4, HKV4, 1, D, 4, pi_perm.data_ptr(),
            n_out, oc_h.ptr, rc_h.ptr, vq.Pi.data_ptr(), vc_h.ptr, scale, 0, out.data_ptr(),
            N.QKV_F32, ws.data_ptr(), ws_bytes, splits, sptr))

    event_ms(decode, args.warmup, stream, flush)
    dec_ms = statistics.median(event_ms(decode, args.steps, stream, flush))
    same = bool(torch.equal(eng.attention(q), out))

    n_th = B4 * HKV4 * TT
    alg_bytes = n_th * (36 + 4 + 64 + 4)       # 2.25-bit K packed tight + 4-bit V + norms
    read_bytes = n_th * (st.krb + 4 + 64 + 4)  # what the store holds (40-byte kmixed rows)
    gbs = alg_bytes / (dec_ms * 1e-3) / 1e9
    res = {
        "what": "long-context mixed precision: B 1, 32/8 heads, d 128, 131072 bf16 tokens in "
                "2048-token chunks, K MixedPrecisionMSE 3/2 bits (32 outliers), V 4-bit",
        "us": round(dec_ms * 1e3, 2), "GB_s": round(gbs, 1),
        "pct_of_hbm_peak": round(100 * gbs / PEAK_HBM_GBS, 2),
        "n_splits": splits,
        "algorithmic_bytes": alg_bytes, "store_bytes": read_bytes,
        "store_pct_of_hbm_peak": round(100 * read_bytes / (dec_ms * 1e-3) / 1e9
                                       / PEAK_HBM_GBS, 2),
        "engine_output_identical": same,
        "append_ms_total": round(append_ms, 3),
        "append_gvec_s": round(2 * n_th / (append_ms * 1e-3) / 1e9, 4),
    }
    if not args.no_cpu:
        from oracle import ref_math as R
        thr = cpu_threads()
        kc, _, vc = st.read_codes(0, TT)
        cargs = (kc.cpu(), st.knorm[:, :, :TT].cpu(), vc.cpu(), st.vnorm[:, :, :TT].cpu(),
                 kq.Pi.cpu(), kq._outlier_indices.cpu(), kq.outlier_codebook.centroids.cpu(),
                 kq.regular_codebook.centroids.cpu(), vq.Pi.cpu(), vq.codebook.centroids.cpu())
        qs = q.float().cpu()
        reps = max(args.cpu_reps, 1)
        cpu_s = median_s(lambda: R.attention_mixed_keys(qs, *cargs), reps)
        ro = R.attention_mixed_keys(qs, *cargs).double()
        res["oracle_rel_err"] = float((out.cpu().double() - ro).norm() / ro.norm())
        res["cpu_baseline"] = {"value": round(cpu_s * 1e6, 1), "unit": "us", "cores": thr,
                               "kind": "port",
                               "sample": "oracle attention_mixed_keys (fp32 torch CPU) over the "
                                         f"whole cache, median of {reps}"}
    return res


def sub_cfg5(args, dev, stream) -> dict:
    """BASELINE configs[4] (cfg5): QuashIndex(128, bits=3, seed=42) over 10^6
    L2-normalised N(0,1) vectors, 10^4 queries, top-10.  Search time, recall@10
    against exact fp32 search, and index agreement with the CPU oracle's
    search on identical codes for a sample of queries."""
    import torch
    from quashkv_amd.nn_search import QuashIndex

    NV, M, DD, K = 1_000_000, 10_000, 128, 10
    g = torch.Generator(device=dev).manual_seed(4)
    db = torch.randn(NV, DD, device=dev, generator=g)
    db /= db.norm(dim=1, keepdim=True)
    qs = torch.randn(M, DD, device=dev, generator=g)
    qs /= qs.norm(dim=1, keepdim=True)
    # a throwaway index takes the first call's one-time costs (kernel loads)
    QuashIndex(DD, bits=3, seed=42, device=dev).add(db[:4096])
    idx = QuashIndex(DD, bits=3, seed=42, device=dev)
    add_ms = event_ms(lambda: idx.add(db), 1, stream)[0]
    res_box = {}

    def search():
        res_box["r"] = idx.search(qs, K)

    event_ms(search, max(args.warmup // 2, 1), stream)
    ms = statistics.median(event_ms(search, max(args.steps // 6, 3), stream))
    sc, ix = res_box["r"]
    hits = 0
    for c in range(0, M, 1000):
        ex = torch.topk(qs[c:c + 1000] @ db.T, K, dim=1).indices
        hits += int((ix[c:c + 1000].unsqueeze(2) == ex.unsqueeze(1)).any(dim=2).sum())
    ops = 2.0 * M * NV * 384 * 4      # int8 MACs of the bit-plane dot products, x2
    res = {
        "what": "QuashIndex MIPS: 10^6 x 128 L2-normalised vectors, 3-bit (2-bit MSE + QJL), "
                "10^4 queries, exhaustive top-10",
        "us": round(ms * 1e3, 1), "queries_per_s": round(M / (ms * 1e-3), 1),
        "bound": "int8 MFMA", "executed_int8_tops": round(ops / (ms * 1e-3) / 1e12, 1),
        "pct_of_int8_mfma_peak": round(100 * ops / (ms * 1e-3) / 1e12 / PEAK_INT8_TOPS, 2),
        "add_ms": round(add_ms, 2), "recall_at_10": round(hits / (M * K), 4),
    }
    if not args.no_cpu:
        from oracle import ref_math as R
        thr = cpu_threads()
        mse, qjl = idx._get_unpacked()
        mq = idx.quantizer.mse_quantizer
        nq = 8
        cargs = (mse.cpu(), qjl.cpu(), idx._norms[:NV].cpu(), mq.Pi.cpu(),
                 mq.codebook.centroids.cpu(), idx.quantizer.S.cpu(), idx.quantizer.qjl_scale)
        t0 = time.perf_counter()
        rs, ri = R.index_search(qs[:nq].cpu(), *cargs, K, chunk=nq)
        cpu_s = time.perf_counter() - t0
        res["oracle_index_agreement"] = float((ri == ix[:nq].cpu()).double().mean())
        res["oracle_max_score_diff"] = float((rs - sc[:nq].cpu()).abs().max())
        res["cpu_baseline"] = {"value": round(cpu_s / nq * M * 1e6, 1), "unit": "us",
                               "cores": thr, "kind": "port",
                               "sample": f"oracle index_search on {nq} of {M} queries "
                                         f"({cpu_s:.2f} s), scaled to {M}"}
    return res


SUBS = {"cfg1": sub_cfg1, "cfg2": sub_cfg2, "cfg4": sub_cfg4, "cfg5": sub_cfg5}
# arithmetic of each workload's dominant kernel (d = 64 decodes and MIPS score on int8 MFMA)
SUB_DTYPE = {"cfg1": DTYPE, "cfg2": ("i8 MFMA scores and values (30-bit fixed-point query "
                                    "weights, 29-bit softmax weights); f32 softmax"),
             "cfg4": DTYPE, "cfg5": "i8 MFMA scores (30-bit fixed-point query weights)"}
SUB_KEYS = {"cfg1": "cfg1", "cfg2": "cfg2_layers", "cfg4": "cfg4", "cfg5": "cfg5"}


def standalone(args, name: str) -> None:
    """One configuration as its own JSON line."""
    import torch
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    sub = SUBS[name](args, dev, torch.cuda.current_stream(dev))
    line = {"metric": f"{name}: us per step", "value": sub["us"], "unit": "us", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": sub["us"] / 1e3,
            "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
            "dtype": SUB_DTYPE[name], "data": "synthetic (seeded)", "config": {"workload": name}}
    line.update(sub)
    print(json.dumps(line), flush=True)


# ------------------------------------------------------------------ main

def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--copies", type=int, default=3, help="distinct caches rotated per step")
    ap.add_argument("--compress-reps", type=int, default=5)
    ap.add_argument("--cpu-batch", type=int, default=4, help="sequences in the CPU sample")
    ap.add_argument("--cpu-reps", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="cfg3 decode and compress only (no other configs, paged, HF, "
                         "decompress or ceilings): the profiling passes")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only copy 256 MiB three times (calibrates FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--pmc-summary", nargs=4, metavar=("KFETCH", "KWRITE", "CFETCH", "CWRITE"),
                    help="print the traffic record from four rocprofv3 --pmc output dirs")
    ap.add_argument("--kernel", default=r"decode_fused",
                    help="kernel-name regex for --pmc-summary")
    ap.add_argument("--decompress-reps", type=int, default=10,
                    help="timed full-cache reconstructions (cfg3)")
    ap.add_argument("--workload", choices=("cfg1", "cfg2", "cfg3", "cfg4", "cfg5"),
                    default="cfg3",
                    help="cfg3: the headline line (with every other config as a sub-object); "
                         "cfgN: that config alone")
    args = ap.parse_args()

    if args.pmc_summary:
        pmc_summary(args.pmc_summary, args.kernel)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 "
                                   "(how the path shards is described in DESIGN.md)"}))
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration()
        return
    if args.workload != "cfg3":
        standalone(args, args.workload)
        return

    import torch
    import quashkv_amd as Q
    from quashkv_amd import _native as N

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib = N.lib()
    stream = torch.cuda.current_stream(dev)
    sptr = stream.cuda_stream

    # ---------------------------------------------------------- build caches
    engines = []
    compress_ms = []
    for c in range(args.copies):
        k, v = make_inputs(2 + 1000 * c, dev, torch.bfloat16)
        eng = Q.QuashKVEngine(head_dim=D, key_bits=KEY_BITS, value_bits=VAL_BITS, seed=42,
                              device=dev, pack_storage=True, capacity=T)
        eng.append(k, v)
        engines.append(eng)
        if c == 0:
            # time the append path: compress K (IP) + V (MSE) of all 2^21 token-heads
            # into the packed store; appends are queued back to back so host-side
            # launch work overlaps the device; untimed appends first bring the
            # clocks up
            for _ in range(10):
                eng.clear()
                eng.append(k, v)
            for _ in range(3):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(args.compress_reps):
                    eng.clear()
                    eng.append(k, v)
                e1.record()
                torch.cuda.synchronize()
                compress_ms.append(e0.elapsed_time(e1) / args.compress_reps)
        del k, v
    torch.cuda.synchronize()

    gq = torch.Generator(device=dev).manual_seed(7)
    queries = [torch.randn(B, HQ, 1, D, device=dev, generator=gq).to(torch.bfloat16)
               for _ in range(args.copies)]
    splits = lib.qkv_attention_splits(B, HQ, HKV, 1, D, T)
    ws_bytes = lib.qkv_attention_workspace_bytes(B, HQ, HKV, 1, D, splits)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    out = torch.empty(B, HQ, 1, D, dtype=torch.float32, device=dev)
    scale = 1.0 / math.sqrt(D)
    eng0 = engines[0]
    kq0, vq0 = eng0.key_quantizer, eng0.value_quantizer
    kc_h = N.HostFloats(kq0.mse_quantizer.codebook.centroids_host)
    vc_h = N.HostFloats(vq0.codebook.centroids_host)
    path = lib.qkv_attention_path(D, KEY_BITS - 1, VAL_BITS, kc_h.ptr, vc_h.ptr,
                                  eng0._store.capacity, T, splits)

    def decode(i):
        # the whole step as one call of the product entry point
        eng = engines[i % args.copies]
        q = queries[i % args.copies]
        st = eng._store
        kq = eng.key_quantizer
        mq = kq.mse_quantizer
        N.check(lib.qkv_decode_attention(
            q.data_ptr(), N.QKV_BF16, st.kst.data_ptr(), st.knorm.data_ptr(), st.vst.data_ptr(),
            st.vnorm.data_ptr(), st.capacity, T, B, HQ, HKV, 1, D, KEY_BITS - 1, VAL_BITS,
            mq.Pi.data_ptr(), kc_h.ptr, vc_h.ptr, kq.S.data_ptr(), kq.qjl_scale, scale, 0,
            out.data_ptr(), N.QKV_F32, ws.data_ptr(), ws_bytes, splits, sptr))

    for i in range(args.warmup):
        decode(i)
    torch.cuda.synchronize()
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    t_start.record(stream)
    for i in range(args.steps):
        decode(args.warmup + i)
    t_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    step_ms = t_start.elapsed_time(t_end) / args.steps
    # the fused kernel's average launch duration: at this shape a step is one
    # launch, so the timed region above (HIP events on the launch stream
    # around back-to-back steps) is that average.  The kernel trace of the
    # same loop shows no gaps between the launches; events between single
    # launches are not used, as they slow each launch (~60 -> ~72 us in the
    # trace).
    launch_ms = step_ms

    kv_bytes = B * HKV * T * kv_bytes_per_token_head(D)
    io_bytes = B * HQ * D * (2 + 4)  # bf16 q in, fp32 out
    step_gbs = (kv_bytes + io_bytes) / (step_ms * 1e-3) / 1e9
    launch_gbs = kv_bytes / (launch_ms * 1e-3) / 1e9
    n_vec = 2 * B * HKV * T
    comp_ms = statistics.median(compress_ms)
    comp_gvec = n_vec / (comp_ms * 1e-3) / 1e9
    comp_bytes = n_vec * (D * 2) + B * HKV * T * kv_bytes_per_token_head(D)
    traffic = pmc_traffic() if splits == 1 else None

    line = {
        "metric": METRIC,
        "value": round(step_gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DTYPE,
        "data": "synthetic (seeded N(0,1) K/V/q; keys with 4 outlier channels x10)",
        "config": {
            "workload": "cfg3 Llama-3-8B-shaped decode attention over packed 3-bit KV",
            "batch": B, "q_heads": HQ, "kv_heads": HKV, "head_dim": D, "context": T,
            "key_bits": KEY_BITS, "value_bits": VAL_BITS, "query_dtype": "bf16",
            "cache_copies_rotated": args.copies, "n_splits": splits,
            "kernel_path": "fused (MFMA)" if path == 1 else "valu",
        },
        "decode_us_per_step": round(step_ms * 1e3, 2),
        "decode_pct_of_hbm_peak": round(100 * step_gbs / PEAK_HBM_GBS, 2),
        "compress_gvec_s": round(comp_gvec, 4),
        "compress_pct_of_hbm_roofline": round(100 * comp_bytes / (comp_ms * 1e-3) / 1e9
                                              / PEAK_HBM_GBS, 2),
        "compress_mfma": {
            "what": "rotation GEMM of the append (2 d^2 flops per vector; executed as "
                    "two bf16 passes, Pi split into high and low parts)",
            "algorithmic_tflops": round(n_vec * 2 * D * D / (comp_ms * 1e-3) / 1e12, 1),
            "executed_tflops": round(2 * n_vec * 2 * D * D / (comp_ms * 1e-3) / 1e12, 1),
            "peak_tflops": 2500.0,
            "executed_frac": round(2 * n_vec * 2 * D * D / (comp_ms * 1e-3) / 2.5e15, 4),
        },
        "roofline": {
            "kernel": ("decode_fused<12, 3, false, 128> (qkv_decode_attention, one launch)"
                       if splits == 1 else "qkv_decode_attention (decode_fused + combine)"),
            "bound": "hbm",
            "achieved": round(launch_gbs, 2),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(launch_gbs / PEAK_HBM_GBS, 4),
            "traffic": traffic["bytes"] if traffic else None,
            "traffic_source": traffic,
            "algorithmic_bytes_per_launch": kv_bytes,
            "avg_kernel_us": round(launch_ms * 1e3, 2),
        },
        "wall_s_timed": round(wall, 3),
    }

    if not args.no_extra:
        # full-cache reconstruction (QuashKVCache.update's decompress of every
        # K and V row, quashkv/integrations/hf_cache.py:96-121) of cache 0
        from quashkv_amd.quantizer import decompress_from
        st0 = eng0._store
        n_rows = B * HKV * T
        mq0 = kq0.mse_quantizer

        def reconstruct():
            kh = decompress_from(N.QKV_MODE_MSE, st0.kst, None, st0.knorm, n_rows, mq0.Pi,
                                 mq0.codebook.centroids, KEY_BITS - 1, None, 0.0,
                                 N.QKV_FMT_KPLANES, in_seq=T, in_group_stride=st0.capacity)
            vh = decompress_from(N.QKV_MODE_MSE, st0.vst, None, st0.vnorm, n_rows, vq0.Pi,
                                 vq0.codebook.centroids, VAL_BITS, None, 0.0, N.QKV_FMT_VTILES,
                                 in_seq=T, in_group_stride=st0.capacity // 32)
            return kh, vh

        for _ in range(3):
            reconstruct()
        torch.cuda.synchronize()
        dec_ms = statistics.mean(event_ms(reconstruct, args.decompress_reps, stream))
        dec_bytes = n_rows * ((KEY_BITS - 1) * D // 8 + VAL_BITS * D // 8 + 2 * 4 + 2 * D * 4)
        dec_gbs = dec_bytes / (dec_ms * 1e-3) / 1e9
        line["decompress"] = {
            "what": "full K (2-bit MSE planes) + V (3-bit tiles) reconstruction to fp32, "
                    f"{n_rows} rows each",
            "us": round(dec_ms * 1e3, 1), "GB_s": round(dec_gbs, 1),
            "pct_of_hbm_peak": round(100 * dec_gbs / PEAK_HBM_GBS, 2), "bytes": dec_bytes,
        }
        line["compress_fp32"] = compress_fp32(args, dev, stream)
        line["paged"] = paged_decode(args, dev, lib, sptr, stream, engines, queries, kc_h, vc_h,
                                     kv_bytes)
        line["hf_attention_cfg2"] = hf_decode_step(args, dev, stream)
        # measured HBM ceilings on this device
        read_gbs = hbm_read_ceiling(dev, stream)
        big = torch.empty(1 << 28, device=dev).uniform_()
        dst = torch.empty_like(big)
        dst.copy_(big)
        copy_ms = statistics.mean(event_ms(lambda: dst.copy_(big), 5, stream))
        copy_gbs = 2 * big.numel() * 4 / (copy_ms * 1e-3) / 1e9
        del big, dst
        line["hbm_ceiling_measured"] = {
            "read_only_GB_s": round(read_gbs, 1),
            "read_only_what": "qkv_hbm_read_probe: 4 GiB, non-temporal 16-byte loads, "
                              "2 workgroups of 256 threads per CU, 4 loads in flight",
            "copy_GB_s": round(copy_gbs, 1),
            "decode_kernel_pct_of_read_ceiling": round(100 * launch_gbs / read_gbs, 2),
            "decode_step_pct_of_read_ceiling": round(100 * step_gbs / read_gbs, 2),
            "decompress_pct_of_copy": round(100 * dec_gbs / copy_gbs, 2),
        }
        for name in ("cfg1", "cfg2", "cfg4", "cfg5"):
            torch.cuda.synchronize()
            line[SUB_KEYS[name]] = SUBS[name](args, dev, stream)

    if not args.no_cpu:
        cg, dg, nrow, thr, tc, td = cpu_compress_decompress(engines[0], 4, args.cpu_reps)
        line["cpu_baseline_compress"] = {
            "value": round(cg, 5), "unit": "Gvec/s", "cores": thr, "kind": "port",
            "sample": (f"oracle compress_ip (keys) + compress_mse (values), fp32 torch CPU, "
                       f"{nrow} rows each (4 sequences, 8 kv heads); median of "
                       f"{args.cpu_reps} = {tc:.3f} s")}
        line["cpu_baseline_decompress"] = {
            "value": round(dg, 3), "unit": "GB/s", "cores": thr, "kind": "port",
            "sample": (f"oracle decompress_mse of the store's K and V codes to fp32, "
                       f"{nrow} rows each; median of {args.cpu_reps} = {td:.3f} s")}
        gbs, med, threads, rel = cpu_baseline(engines[0], queries[0], args.cpu_batch,
                                              args.cpu_reps)
        line["oracle_rel_err"] = rel
        line["cpu_baseline"] = {
            "value": round(gbs, 4), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": (f"oracle online-softmax decode (oracle/ref_math.attention_online, "
                       f"fp32 torch CPU) on {args.cpu_batch} of {B} sequences, all 8 kv "
                       f"heads, T={T}; median of {args.cpu_reps} reps = {med:.3f} s; "
                       f"host {cpu_model()}; torch threads = the {host_cores()} CPUs this "
                       f"process may use (os.cpu_count() = {os.cpu_count()})")}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
