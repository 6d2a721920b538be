"""Write the golden vectors that pin the CPU oracle to the reference.

This script runs ONLY in the build container, where the reference package is
mounted read-only (default ``/root/reference``).  It imports the reference,
feeds it small seeded inputs and stores inputs + outputs as ``.npz`` data
files next to this script.  Nothing on the GPU box runs it; the tests there
read the committed ``.npz`` files.

It covers exactly the functions whose outputs no closed form or invariant
pins bit-for-bit:

* ``LloydMaxCodebook`` fp32 centroids/boundaries (scipy-quad iteration,
  ``quashkv/codebook.py:63-139,198-207``),
* ``_random_orthogonal`` / ``_random_signs`` (LAPACK QR + torch RNG,
  ``quashkv/quantizer.py:32-59``),
* compress / decompress / attention / index outputs on seeded inputs
  (``quashkv/quantizer.py:113-279``, ``quashkv/triton_kernels/*.py`` PyTorch
  fallbacks, ``quashkv/engine.py:204-299``, ``quashkv/nn_search/index.py``),
* ``pack_bits`` bytes (``quashkv/packing.py:22-94``) on random codes,
* mixed-precision calibration (``quashkv/mixed_precision.py:92-187``),
* ``QuashKVCache.update`` reconstructions (``quashkv/integrations/hf_cache.py``).

Usage:  python tests/golden/make_golden.py [--ref /root/reference]
"""

from __future__ import annotations

import argparse
import os
import sys
import zlib

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def _np(t):
    return t.detach().cpu().numpy()


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    args = ap.parse_args()

    sys.dont_write_bytecode = True
    sys.path.insert(0, args.ref)
    import torch  # noqa: E402

    torch.set_num_threads(4)
    import quashkv

    # the reference, not this repository's quashkv layout over quashkv_amd
    assert os.path.abspath(quashkv.__file__).startswith(os.path.abspath(args.ref)), quashkv.__file__
    from quashkv.codebook import LloydMaxCodebook, solve_lloyd_max
    from quashkv.quantizer import (
        MSEQuantizer,
        InnerProductQuantizer,
        _random_orthogonal,
        _random_signs,
    )
    from quashkv.packing import pack_bits, packed_size
    from quashkv.engine import QuashKVEngine
    from quashkv.triton_kernels.compress import (
        _compress_mse_pytorch,
        _compress_ip_pytorch,
    )
    from quashkv.triton_kernels.decompress import (
        _decompress_mse_pytorch,
        _decompress_ip_pytorch,
    )
    from quashkv.triton_kernels.attention import (
        _fused_attention_pytorch,
        CompressedBlock,
    )
    from quashkv.mixed_precision import MixedPrecisionMSEQuantizer
    from quashkv.nn_search.index import QuashIndex
    from quashkv.integrations.hf_cache import QuashKVCache

    # ------------------------------------------------------------------
    # 1. codebooks
    # ------------------------------------------------------------------
    cb = {}
    for d in (64, 96, 128):
        for bits in (1, 2, 3, 4):
            c = LloydMaxCodebook(d, bits)
            cb[f"c_d{d}_b{bits}"] = _np(c.centroids)
            cb[f"t_d{d}_b{bits}"] = _np(c.boundaries)
            cents64, bnds64 = solve_lloyd_max(d, bits)
            cb[f"c64_d{d}_b{bits}"] = np.array(cents64, dtype=np.float64)
            cb[f"t64_d{d}_b{bits}"] = np.array(bnds64, dtype=np.float64)
    for d, bits in ((64, 2), (64, 3), (128, 2)):
        c = LloydMaxCodebook(d, bits, use_exact_pdf=True)
        cb[f"ce_d{d}_b{bits}"] = _np(c.centroids)
        cb[f"te_d{d}_b{bits}"] = _np(c.boundaries)
    np.savez_compressed(os.path.join(HERE, "codebooks.npz"), **cb)
    print("codebooks done")

    # ------------------------------------------------------------------
    # 2. rotation matrices and sign vectors
    # ------------------------------------------------------------------
    rot = {}
    for d, seed in ((64, 42), (64, 43), (64, 65), (96, 42), (128, 42), (128, 43), (128, 7)):
        rot[f"Pi_d{d}_s{seed}"] = _np(_random_orthogonal(d, seed, torch.device("cpu")))
        rot[f"S_d{d}_s{seed}"] = _np(_random_signs(d, seed, torch.device("cpu")))
    np.savez_compressed(os.path.join(HERE, "rotations.npz"), **rot)
    print("rotations done")

    # ------------------------------------------------------------------
    # 3. pack_bits bytes
    # ------------------------------------------------------------------
    pk = {}
    g = torch.Generator().manual_seed(1234)
    for d in (8, 63, 64, 65, 100, 128):
        for bits in (1, 2, 3, 4):
            codes = torch.randint(0, 1 << bits, (5, d), generator=g, dtype=torch.uint8)
            pk[f"codes_d{d}_b{bits}"] = _np(codes)
            pk[f"packed_d{d}_b{bits}"] = _np(pack_bits(codes, bits))
            pk[f"psize_d{d}_b{bits}"] = np.array(packed_size(d, bits))
    np.savez_compressed(os.path.join(HERE, "packing.npz"), **pk)
    print("packing done")

    # ------------------------------------------------------------------
    # 4/5. compress + decompress (quantizer classes and fused fallbacks)
    # ------------------------------------------------------------------
    cq = {}
    for d in (64, 128):
        g = torch.Generator().manual_seed(100 + d)
        x = torch.randn(2, 2, 8, d, generator=g)
        x[0, 0, 0] = 0.0                      # zero vector (norm clamp path)
        x[0, 0, 1] = x[0, 0, 1] * 1e-6       # tiny norm
        x[0, 0, 2] = x[0, 0, 2] * 1e4        # large norm
        cq[f"x_d{d}"] = _np(x)
        for bits in (1, 2, 3, 4):
            q = MSEQuantizer(d, bits=bits, seed=42)
            nrm = x.norm(dim=-1, keepdim=True).clamp(min=1e-8)
            y = q.rotate(x / nrm)
            idx, norms = q.compress(x)
            cq[f"mse_y_d{d}_b{bits}"] = _np(y)
            cq[f"mse_idx_d{d}_b{bits}"] = _np(idx)
            cq[f"mse_norm_d{d}_b{bits}"] = _np(norms)
            cq[f"mse_qb_d{d}_b{bits}"] = _np(q.codebook.quantize_boundary(y))
            idx_f, n_f = _compress_mse_pytorch(x, q.Pi, q.codebook.boundaries)
            cq[f"fmse_idx_d{d}_b{bits}"] = _np(idx_f)
            cq[f"fmse_norm_d{d}_b{bits}"] = _np(n_f)
            cq[f"mse_xhat_d{d}_b{bits}"] = _np(q.decompress(idx, norms))
            cq[f"fmse_xhat_d{d}_b{bits}"] = _np(
                _decompress_mse_pytorch(idx, norms, q.Pi, q.codebook.centroids))
        for tb in (2, 3, 4):
            q = InnerProductQuantizer(d, total_bits=tb, seed=42)
            mi, qj, nr = q.compress(x)
            cq[f"ip_mse_d{d}_b{tb}"] = _np(mi)
            cq[f"ip_qjl_d{d}_b{tb}"] = _np(qj)
            cq[f"ip_norm_d{d}_b{tb}"] = _np(nr)
            mq = q.mse_quantizer
            mi_f, qj_f, nr_f = _compress_ip_pytorch(
                x, mq.Pi, mq.codebook.boundaries, q.S, mq.codebook.centroids)
            cq[f"fip_mse_d{d}_b{tb}"] = _np(mi_f)
            cq[f"fip_qjl_d{d}_b{tb}"] = _np(qj_f)
            cq[f"fip_norm_d{d}_b{tb}"] = _np(nr_f)
            cq[f"fip_xhat_d{d}_b{tb}"] = _np(_decompress_ip_pytorch(
                mi, qj, nr, mq.Pi, mq.codebook.centroids, q.S, q.qjl_scale))
            # decompress_for_dot against a fixed query
            gq = torch.Generator().manual_seed(7)
            qv = torch.randn(d, generator=gq)
            q_rot = mq.rotate(qv.unsqueeze(0)).expand(*x.shape[:-1], d)
            cq[f"ip_q_d{d}_b{tb}"] = _np(qv)
            cq[f"ip_dot_d{d}_b{tb}"] = _np(q.decompress_for_dot(mi, qj, nr, q_rot))
    # boundary ties: y exactly at boundaries / zero / huge
    for d, bits in ((128, 2), (128, 3), (64, 4), (128, 1)):
        c = LloydMaxCodebook(d, bits)
        t = c.boundaries
        ys = torch.cat([
            t, torch.nextafter(t, torch.full_like(t, 1.0)),
            torch.nextafter(t, torch.full_like(t, -1.0)),
            torch.tensor([0.0, -0.0, 1.0, -1.0, 1e30, -1e30, 1e-30, -1e-30]),
        ])
        cq[f"tie_y_d{d}_b{bits}"] = _np(ys)
        cq[f"tie_code_d{d}_b{bits}"] = _np(c.quantize_boundary(ys))
        cq[f"tie_bucket_d{d}_b{bits}"] = _np(torch.bucketize(ys, t).to(torch.uint8))
    np.savez_compressed(os.path.join(HERE, "compress.npz"), **cq)
    print("compress done")

    # ------------------------------------------------------------------
    # 6. engine attention + online-softmax fallback
    # ------------------------------------------------------------------
    at = {}
    cases = [
        # name, d, H, blocks(seq lens), Q, kb, vb, packed
        ("single64", 64, 2, (32,), 4, 3, 3, False),
        ("multi64", 64, 2, (16, 8), 4, 3, 3, False),
        ("single128q1", 128, 2, (32,), 1, 3, 3, False),
        ("multi128", 128, 2, (20, 7, 5), 1, 3, 3, True),
        ("bits44_d96", 96, 2, (24,), 2, 4, 4, True),
        ("bits23_d64", 64, 3, (40,), 1, 2, 3, True),
        ("bits34_d128", 128, 1, (33,), 3, 3, 4, False),
    ]
    for name, d, H, seqs, Q, kb, vb, packed in cases:
        g = torch.Generator().manual_seed(zlib.crc32(name.encode()) % 10007)
        eng = QuashKVEngine(head_dim=d, key_bits=kb, value_bits=vb, seed=42,
                            pack_storage=packed)
        ks, vs = [], []
        for s in seqs:
            k = torch.randn(1, H, s, d, generator=g)
            v = torch.randn(1, H, s, d, generator=g)
            eng.append(k, v)
            ks.append(k)
            vs.append(v)
        q = torch.randn(1, H, Q, d, generator=g)
        out = eng.attention(q)
        at[f"{name}_k"] = _np(torch.cat(ks, dim=2))
        at[f"{name}_v"] = _np(torch.cat(vs, dim=2))
        at[f"{name}_q"] = _np(q)
        at[f"{name}_seqs"] = np.array(seqs)
        at[f"{name}_cfg"] = np.array([d, H, Q, kb, vb, int(packed)])
        at[f"{name}_out"] = _np(out)
        # causal variant through the engine
        at[f"{name}_out_causal"] = _np(eng.attention(q, causal=True))
        # online-softmax fallback over unpacked blocks
        blocks = []
        for blk in eng._cache:
            mi, qj, vi = eng._unpack_block(blk)
            blocks.append(CompressedBlock(mi, qj, blk.key_norms, vi, blk.val_norms, blk.seq_len))
        kq = eng.key_quantizer
        fo = _fused_attention_pytorch(
            q, blocks, kq.mse_quantizer.Pi, kq.mse_quantizer.codebook.centroids,
            eng.value_quantizer.codebook.centroids, kq.S, kq.qjl_scale,
            1.0 / (d ** 0.5), False, eng.total_tokens)
        at[f"{name}_fused_out"] = _np(fo)
        at[f"{name}_ratio"] = np.array(eng.compression_ratio())
        at[f"{name}_membytes"] = np.array(eng.actual_memory_bytes())
    # GQA: 8 query heads over 2 KV heads by reshaping q to (B, Hkv, G*Q, d)
    g = torch.Generator().manual_seed(4242)
    d, Hkv, G, T = 128, 2, 4, 48
    eng = QuashKVEngine(head_dim=d, seed=42, pack_storage=True)
    k = torch.randn(2, Hkv, T, d, generator=g)
    v = torch.randn(2, Hkv, T, d, generator=g)
    eng.append(k, v)
    qg = torch.randn(2, Hkv * G, 1, d, generator=g)
    out = eng.attention(qg.reshape(2, Hkv, G, d)).reshape(2, Hkv * G, 1, d)
    at.update(gqa_k=_np(k), gqa_v=_np(v), gqa_q=_np(qg), gqa_out=_np(out))
    np.savez_compressed(os.path.join(HERE, "attention.npz"), **at)
    print("attention done")

    # ------------------------------------------------------------------
    # 7. mixed precision
    # ------------------------------------------------------------------
    mp = {}
    g = torch.Generator().manual_seed(31)
    d = 128
    calib = torch.randn(1024, d, generator=g)
    qm = MixedPrecisionMSEQuantizer(d, outlier_bits=3, regular_bits=2, n_outliers=32, seed=42)
    qm.calibrate(calib)
    x = torch.randn(3, 2, 8, d, generator=g)
    mi, nr = qm.compress(x)
    mp.update(calib=_np(calib), x=_np(x), outliers=_np(qm._outlier_indices),
              idx=_np(mi), norm=_np(nr), xhat=_np(qm.decompress(mi, nr)))
    qm2 = MixedPrecisionMSEQuantizer(64, outlier_bits=4, regular_bits=2, n_outliers=8, seed=43)
    x2 = torch.randn(10, 64, generator=g)
    mi2, nr2 = qm2.compress(x2)         # uncalibrated -> regular codebook everywhere
    mp.update(x2=_np(x2), idx2=_np(mi2), norm2=_np(nr2), xhat2=_np(qm2.decompress(mi2, nr2)))
    np.savez_compressed(os.path.join(HERE, "mixed.npz"), **mp)
    print("mixed done")

    # ------------------------------------------------------------------
    # 8. QuashIndex search
    # ------------------------------------------------------------------
    ix = {}
    g = torch.Generator().manual_seed(55)
    for d, bits in ((64, 3), (128, 3), (128, 4)):
        db = torch.randn(1000, d, generator=g)
        qs = torch.randn(24, d, generator=g)
        idx = QuashIndex(d, bits=bits, seed=42)
        idx.add(db[:600])
        idx.add(db[600:])
        sc, ii = idx.search(qs, k=10)
        ix[f"db_d{d}_b{bits}"] = _np(db)
        ix[f"q_d{d}_b{bits}"] = _np(qs)
        ix[f"scores_d{d}_b{bits}"] = _np(sc)
        ix[f"ids_d{d}_b{bits}"] = _np(ii)
        ix[f"recall_d{d}_b{bits}"] = np.array(idx.recall_at_k(qs, db, k=10))
        ix[f"mem_d{d}_b{bits}"] = np.array(idx.memory_bytes())
    np.savez_compressed(os.path.join(HERE, "index.npz"), **ix)
    print("index done")

    # ------------------------------------------------------------------
    # 9. HF cache reconstructions
    # ------------------------------------------------------------------
    hf = {}
    g = torch.Generator().manual_seed(77)
    cache = QuashKVCache(num_layers=2, head_dim=64)
    k0 = torch.randn(1, 2, 12, 64, generator=g)
    v0 = torch.randn(1, 2, 12, 64, generator=g)
    k1 = torch.randn(1, 2, 1, 64, generator=g)
    v1 = torch.randn(1, 2, 1, 64, generator=g)
    cache.update(k0, v0, layer_idx=1)
    fk, fv = cache.update(k1, v1, layer_idx=1)
    hf.update(k0=_np(k0), v0=_np(v0), k1=_np(k1), v1=_np(v1), fk=_np(fk), fv=_np(fv))
    hf["stats_ratio"] = np.array(cache.compression_stats()["overall_compression_ratio"])
    np.savez_compressed(os.path.join(HERE, "hf_cache.npz"), **hf)
    print("hf_cache done")


if __name__ == "__main__":
    main()
