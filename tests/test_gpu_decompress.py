"""GPU parity of the MFMA decompress kernels (d = 64, 96 and 128) against the CPU
oracle: every code format (unpacked bytes, pack_bits rows, the store's K rows
and V tiles), MSE and IP modes, all bit widths, grouped-row layouts with a
partial last group, fp32 / fp16 / bf16 outputs and the mixed-precision
codebook selector; at the cfg3 size (2^21 vectors) against a float64 torch
GEMM of the same codes.

Bars: fp32 output within 3e-6 relative (Frobenius) of the oracle and within
1e-5 relative per element of its largest magnitude (the reference's own
fused-vs-quantizer check is atol 1e-5, quashkv tests/test_triton_kernels.py:
99-114); 16-bit outputs within one unit in the last place of the oracle's
value rounded to that type (plus that absolute term)."""

import numpy as np
import pytest
import torch

import quashkv_amd as Q
from quashkv_amd import _native as N
from quashkv_amd.quantizer import decompress_from
from oracle import ref_math as R

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(autouse=True, scope="module")
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")
    N.lib()


def kplanes_rows(codes, qjl, mbits):
    """K store rows (numpy): mbits code planes then the QJL plane, LSB-first."""
    planes = [(codes >> r) & 1 for r in range(mbits)] + [qjl & 1]
    return np.concatenate([R.pack_bits(p.astype(np.uint8), 1) for p in planes], axis=-1)


def vtile_words(codes, vbits):
    """V store words (S/32, vbits, d) uint32 for codes (S, d), S % 32 == 0."""
    S, d = codes.shape
    c = codes.astype(np.uint64).reshape(S // 32, 32, d)
    out = np.zeros((S // 32, vbits, d), dtype=np.uint64)
    for k in range(vbits):
        out[:, k, :] = (((c >> k) & 1) << np.arange(32, dtype=np.uint64)[None, :, None]).sum(axis=1)
    return out.astype(np.uint32)


def layout(fmt, codes, qb, norms, bits, d, seq, gstride):
    """Device buffers of n = codes.shape[0] vectors in groups of `seq` rows spaced
    `gstride` rows (V tiles: gstride tiles) apart; returns (codes, qjl, norms)."""
    n = codes.shape[0]
    G = (n + seq - 1) // seq
    if fmt == N.QKV_FMT_VTILES:
        tiles = np.zeros((G, gstride, bits, d), np.uint32)
        nrm = np.zeros((G, gstride * 32), np.float32)
        for g in range(G):
            c = codes[g * seq:(g + 1) * seq]
            pad = np.zeros((-(-c.shape[0] // 32) * 32, d), np.uint8)
            pad[:c.shape[0]] = c
            tiles[g, :pad.shape[0] // 32] = vtile_words(pad, bits)
            nrm[g, :c.shape[0]] = norms[g * seq:(g + 1) * seq]
        return (torch.from_numpy(tiles.view(np.int32)).to(DEV), None,
                torch.from_numpy(nrm).to(DEV))
    if fmt == N.QKV_FMT_UNPACKED:
        rows, qrows = codes, qb
    elif fmt == N.QKV_FMT_PACKED:
        rows, qrows = R.pack_bits(codes, bits), R.pack_bits(qb, 1)
    else:
        rows, qrows = kplanes_rows(codes, qb, bits), None
    buf = np.zeros((G * gstride, rows.shape[1]), np.uint8)
    qbuf = np.zeros((G * gstride, qrows.shape[1]), np.uint8) if qrows is not None else None
    nrm = np.zeros(G * gstride, np.float32)
    for g in range(G):
        a, b = g * seq, min((g + 1) * seq, n)
        buf[g * gstride:g * gstride + b - a] = rows[a:b]
        if qbuf is not None:
            qbuf[g * gstride:g * gstride + b - a] = qrows[a:b]
        nrm[g * gstride:g * gstride + b - a] = norms[a:b]
    return (torch.from_numpy(buf).to(DEV),
            torch.from_numpy(qbuf).to(DEV) if qbuf is not None else None,
            torch.from_numpy(nrm).to(DEV))


def check_fp32(out, ref):
    out, ref = out.double().cpu(), ref.double().cpu()
    rel = float((out - ref).norm() / ref.norm())
    worst = float((out - ref).abs().max() / ref.abs().max())
    assert rel <= 3e-6 and worst <= 1e-5, (rel, worst)


FMTS = {"unpacked": N.QKV_FMT_UNPACKED, "packed": N.QKV_FMT_PACKED,
        "kplanes": N.QKV_FMT_KPLANES, "vtiles": N.QKV_FMT_VTILES}


@pytest.mark.parametrize("d", [64, 96, 128])
@pytest.mark.parametrize("fmt", list(FMTS))
@pytest.mark.parametrize("mode,bits", [("mse", 1), ("mse", 2), ("mse", 3), ("mse", 4),
                                       ("ip", 1), ("ip", 2), ("ip", 3)])
def test_decompress_formats_vs_oracle(d, fmt, mode, bits):
    if mode == "ip" and fmt == "vtiles":
        pytest.skip("V tiles carry no QJL plane")
    gen = torch.Generator().manual_seed(1000 * d + 10 * bits + len(fmt))
    seq, n = 75, 3 * 75 - 11                  # partial last group
    gstride = 3 if fmt == "vtiles" else 90    # tiles / rows between groups
    codes = torch.randint(0, 1 << bits, (n, d), generator=gen, dtype=torch.uint8).numpy()
    qb = torch.randint(0, 2, (n, d), generator=gen, dtype=torch.uint8).numpy()
    norms = (torch.rand(n, generator=gen) * 3 + 0.1).numpy()
    pi = R.random_orthogonal(d, 11 + d)
    s = R.random_signs(d, 11 + d)
    cents = Q.LloydMaxCodebook(d, bits).centroids
    alpha = R.QJL_COEFF / d
    ct, nt = torch.from_numpy(codes), torch.from_numpy(norms)
    if mode == "mse":
        ref = R.decompress_mse(ct, nt, pi, cents)
    else:
        ref = R.decompress_ip(ct, torch.from_numpy(qb), nt, pi, cents, s, alpha)
    c_d, q_d, n_d = layout(FMTS[fmt], codes, qb, norms, bits, d, seq, gstride)
    m = N.QKV_MODE_MSE if mode == "mse" else N.QKV_MODE_IP
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        out = decompress_from(m, c_d, q_d, n_d, n, pi.to(DEV), cents.to(DEV), bits, s.to(DEV),
                              alpha, FMTS[fmt], in_seq=seq, in_group_stride=gstride,
                              out_dtype=dt)
        if dt == torch.float32:
            check_fp32(out, ref)
        else:
            # within one ulp of the oracle rounded to the output type, plus the
            # fp32 bar's absolute term (values near 0 have tiny ulps)
            r16 = ref.to(dt).float()
            _, e = torch.frexp(r16)                 # |x| in [2^(e-1), 2^e)
            ulp = torch.ldexp(torch.ones_like(r16), e - (8 if dt == torch.bfloat16 else 11))
            tol = ulp + 1e-5 * ref.abs().max()
            diff = (out.cpu().float() - r16).abs()
            assert bool((diff <= tol).all()), float((diff / tol).max())
            assert float((diff > 0).double().mean()) <= 0.01


@pytest.mark.parametrize("d", [64, 96, 128])
def test_decompress_mixed_selector(d):
    """Mixed-precision codes (two codebooks selected per coordinate, unpacked)
    against the oracle's mixed_decompress (quashkv/mixed_precision.py:172-187)."""
    gen = torch.Generator().manual_seed(d + 3)
    n, n_out = 333, 16 if d == 64 else 32
    out_idx = torch.randperm(d, generator=gen)[:n_out].sort().values
    codes = torch.randint(0, 4, (n, d), generator=gen, dtype=torch.uint8)
    codes[:, out_idx] = torch.randint(0, 8, (n, n_out), generator=gen, dtype=torch.uint8)
    norms = torch.rand(n, generator=gen) + 0.5
    qm = Q.MixedPrecisionMSEQuantizer(d, outlier_bits=3, regular_bits=2, n_outliers=n_out,
                                      seed=4, device=DEV)
    qm.set_outlier_channels(out_idx.to(DEV))
    out = qm.decompress(codes.to(DEV), norms.to(DEV))
    ref = R.mixed_decompress(codes, norms, qm.Pi.cpu(), out_idx,
                             qm.outlier_codebook.centroids.cpu(),
                             qm.regular_codebook.centroids.cpu())
    check_fp32(out, ref)


def test_decompress_unaligned_rows_take_generic_kernel():
    """An unaligned code pointer routes to the generic kernel; both kernels
    agree with each other and with the oracle."""
    gen = torch.Generator().manual_seed(5)
    n, d, bits = 200, 128, 3
    codes = torch.randint(0, 8, (n, d), generator=gen, dtype=torch.uint8)
    norms = torch.rand(n, generator=gen) + 0.5
    pi = R.random_orthogonal(d, 2)
    cents = Q.LloydMaxCodebook(d, bits).centroids
    ref = R.decompress_mse(codes, norms, pi, cents)
    raw = torch.zeros(n * d + 1, dtype=torch.uint8, device=DEV)
    raw[1:] = codes.reshape(-1).to(DEV)
    shifted = raw[1:].view(n, d)               # data_ptr odd: generic kernel
    a = decompress_from(N.QKV_MODE_MSE, shifted, None, norms.to(DEV), n, pi.to(DEV),
                        cents.to(DEV), bits, None, 0.0, N.QKV_FMT_UNPACKED)
    b = decompress_from(N.QKV_MODE_MSE, codes.to(DEV), None, norms.to(DEV), n, pi.to(DEV),
                        cents.to(DEV), bits, None, 0.0, N.QKV_FMT_UNPACKED)
    check_fp32(a, ref)
    check_fp32(b, ref)


def test_decompress_cfg3_size_vs_float64_gemm():
    """2^21 vectors of d = 128, 3-bit (the cfg3 value cache), unpacked and as V
    tiles (packed on the GPU by qkv_vtiles_pack), against (c[code] Pi) n in
    float64 on the GPU."""
    torch.manual_seed(0)
    d, bits, B, H, T = 128, 3, 32, 8, 8192
    n = B * H * T
    codes = torch.randint(0, 8, (B * H, T, d), dtype=torch.uint8, device=DEV)
    norms = torch.rand(B * H, T, device=DEV) * 2 + 0.1
    pi = R.random_orthogonal(d, 42).to(DEV)
    cents = Q.LloydMaxCodebook(d, bits).centroids.to(DEV)
    out = decompress_from(N.QKV_MODE_MSE, codes.view(n, d), None, norms.view(n), n, pi, cents,
                          bits, None, 0.0, N.QKV_FMT_UNPACKED)
    tiles = torch.zeros(B * H, T // 32, bits, d, dtype=torch.int32, device=DEV)
    N.check(N.lib().qkv_vtiles_pack(codes.data_ptr(), B * H, T, d, bits, tiles.data_ptr(),
                                    T // 32, 0, N.stream(tiles.device)))
    out_v = decompress_from(N.QKV_MODE_MSE, tiles, None, norms.view(n), n, pi, cents, bits, None,
                            0.0, N.QKV_FMT_VTILES, in_seq=T, in_group_stride=T // 32)
    worst, rel_num, rel_den = 0.0, 0.0, 0.0
    for c0 in range(0, n, 1 << 19):            # float64 reference in chunks
        sl = slice(c0, c0 + (1 << 19))
        ref = (cents.double()[codes.view(n, d)[sl].long()] @ pi.double()) * \
            norms.view(n)[sl].double()[:, None]
        for o in (out[sl], out_v[sl]):
            diff = o.double() - ref
            worst = max(worst, float(diff.abs().max() / ref.abs().max()))
            rel_num += float((diff * diff).sum())
            rel_den += float((ref * ref).sum())
    rel = (rel_num / rel_den) ** 0.5
    assert rel <= 3e-6 and worst <= 1e-5, (rel, worst)
