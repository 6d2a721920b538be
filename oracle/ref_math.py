"""CPU restatement of the reference TurboQuant math -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
may use this module; the product (``quashkv_amd``) never does.

Floating-point work is done with torch on the CPU in fp32, in the same order
of operations as the reference's PyTorch paths, so that results match the
committed golden vectors; byte/integer work (packing) is done with numpy.
Every function cites the reference lines (paths relative to the reference
package root) whose behaviour it restates.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import numpy as np
import torch

QJL_COEFF = math.sqrt(math.pi / 2)  # quashkv/constants.py:21


# ---------------------------------------------------------------------------
# Parameters
# ---------------------------------------------------------------------------

def random_orthogonal(d: int, seed: int) -> torch.Tensor:
    """Pi = Q diag(sign(diag R)), QR of a seeded N(0,1) matrix.

    Follows quashkv/quantizer.py:32-44.
    """
    gen = torch.Generator(device="cpu").manual_seed(seed)
    a = torch.randn(d, d, generator=gen, dtype=torch.float32)
    q, r = torch.linalg.qr(a)
    return q * torch.sign(torch.diag(r)).unsqueeze(0)


def random_signs(d: int, seed: int) -> torch.Tensor:
    """S in {-1,+1}^d from randint with seed + 1_000_000 (quantizer.py:51-59)."""
    gen = torch.Generator(device="cpu").manual_seed(seed + 1_000_000)
    s = torch.randint(0, 2, (d,), generator=gen, dtype=torch.float32)
    return s * 2 - 1


# ---------------------------------------------------------------------------
# Codebook primitives
# ---------------------------------------------------------------------------

def quantize_boundary(y: torch.Tensor, boundaries: torch.Tensor) -> torch.Tensor:
    """code = #{i : t_i < y}; ties go to the lower code.

    Follows quashkv/codebook.py:239-259 (== torch.bucketize right=False,
    quashkv/triton_kernels/compress.py:57).
    """
    idx = torch.zeros_like(y, dtype=torch.int32)
    for i in range(boundaries.numel()):
        idx = idx + (y > boundaries[i]).int()
    return idx.to(torch.uint8)


def quantize_argmin(y: torch.Tensor, centroids: torch.Tensor) -> torch.Tensor:
    """Nearest-centroid index (quashkv/codebook.py:209-224)."""
    return (y.unsqueeze(-1) - centroids).abs().argmin(dim=-1).to(torch.uint8)


def dequantize(codes: torch.Tensor, centroids: torch.Tensor) -> torch.Tensor:
    """c[code] (quashkv/codebook.py:226-237)."""
    return centroids[codes.long()]


# ---------------------------------------------------------------------------
# Compress / decompress
# ---------------------------------------------------------------------------

def _norms(x: torch.Tensor) -> torch.Tensor:
    # quashkv/quantizer.py:127 / compress.py:55: clamp form, not sqrt(sum+eps)
    return x.norm(dim=-1, keepdim=True).clamp(min=1e-8)


def rotate(x_unit: torch.Tensor, pi: torch.Tensor) -> torch.Tensor:
    """y = u Pi^T (quashkv/quantizer.py:105-107)."""
    return x_unit @ pi.T


def compress_mse(x: torch.Tensor, pi: torch.Tensor, boundaries: torch.Tensor):
    """(codes uint8, norms fp32); quashkv/triton_kernels/compress.py:34-58,
    quashkv/quantizer.py:113-131."""
    x = x.float()
    n = _norms(x)
    y = (x / n) @ pi.T
    return quantize_boundary(y, boundaries), n.squeeze(-1)


def compress_ip(x: torch.Tensor, pi: torch.Tensor, boundaries: torch.Tensor,
                s: torch.Tensor, centroids: torch.Tensor):
    """(mse codes, qjl bits, norms); quashkv/triton_kernels/compress.py:61-97,
    quashkv/quantizer.py:211-242.  bit_j = [(y_j - c[code_j]) * S_j >= 0]."""
    x = x.float()
    n = _norms(x)
    y = (x / n) @ pi.T
    codes = quantize_boundary(y, boundaries)
    r = y - centroids[codes.long()]
    bits = ((r * s) >= 0).to(torch.uint8)
    return codes, bits, n.squeeze(-1)


def compress_ip_from_y(y: torch.Tensor, boundaries: torch.Tensor,
                       s: torch.Tensor, centroids: torch.Tensor):
    """The code/bit stage of compress_ip applied to a given rotated y."""
    codes = quantize_boundary(y, boundaries)
    r = y - centroids[codes.long()]
    return codes, ((r * s) >= 0).to(torch.uint8)


def decompress_mse(codes: torch.Tensor, norms: torch.Tensor, pi: torch.Tensor,
                   centroids: torch.Tensor) -> torch.Tensor:
    """(c[code] Pi) * n; quashkv/triton_kernels/decompress.py:32-55,
    quashkv/quantizer.py:133-147."""
    return (centroids[codes.long()] @ pi) * norms.unsqueeze(-1)


def decompress_ip(codes: torch.Tensor, bits: torch.Tensor, norms: torch.Tensor,
                  pi: torch.Tensor, centroids: torch.Tensor, s: torch.Tensor,
                  qjl_scale: float) -> torch.Tensor:
    """((c[code] Pi) + (alpha S (2b-1)) Pi) * n;
    quashkv/triton_kernels/decompress.py:58-96 (two separate products, summed)."""
    mse_unrot = centroids[codes.long()] @ pi
    sign_vals = bits.float() * 2.0 - 1.0
    qjl_unrot = (qjl_scale * (s * sign_vals)) @ pi
    return (mse_unrot + qjl_unrot) * norms.unsqueeze(-1)


def decompress_for_dot(codes, bits, norms, q_rot, centroids, s, qjl_scale):
    """n (<q~, c[code]> + alpha sum |q~| (2b-1) S); quashkv/quantizer.py:244-279."""
    k_rot_hat = centroids[codes.long()]
    mse_dot = (q_rot * k_rot_hat).sum(dim=-1)
    sign_vals = bits.float() * 2.0 - 1.0
    corr = qjl_scale * (q_rot.abs() * sign_vals * s).sum(dim=-1)
    return norms * (mse_dot + corr)


# ---------------------------------------------------------------------------
# Packing (numpy, byte-exact)
# ---------------------------------------------------------------------------

def packed_size(d: int, bits: int) -> int:
    """ceil(d*bits/8) -- the reference's helper (quashkv/packing.py:162-165).

    NOTE: for bits=3 the actual packed row is 3*ceil(d/8) bytes
    (quashkv/packing.py:61-81); see ``packed_row_bytes``.
    """
    return (d * bits + 7) // 8


def packed_row_bytes(d: int, bits: int) -> int:
    """Bytes per row that pack_bits actually produces (packing.py:43-89)."""
    if bits == 8:
        return d
    if bits == 3:
        return 3 * ((d + 7) // 8)
    if bits == 1:
        return (d + 7) // 8
    if bits == 2:
        return (d + 3) // 4
    if bits == 4:
        return (d + 1) // 2
    raise ValueError(f"Unsupported bits: {bits}")


def pack_bits(codes: np.ndarray, bits: int) -> np.ndarray:
    """LSB-first packing along the last axis (quashkv/packing.py:22-94).

    1/2/4-bit: value i of a byte group sits at bit offset i*bits; 3-bit: 8
    values form a little-endian 24-bit word split into 3 bytes.  Rows are
    zero-padded to a whole group.
    """
    codes = np.asarray(codes, dtype=np.uint8)
    if bits == 8:
        return codes.copy()
    *lead, d = codes.shape
    flat = codes.reshape(-1, d).astype(np.uint32)
    per = {1: 8, 2: 4, 3: 8, 4: 2}[bits]
    pad = (-d) % per
    if pad:
        flat = np.pad(flat, ((0, 0), (0, pad)))
    g = flat.reshape(flat.shape[0], -1, per)
    shifts = (np.arange(per, dtype=np.uint32) * bits)
    word = (g << shifts).sum(axis=-1, dtype=np.uint32)
    if bits == 3:
        out = np.stack([(word >> (8 * k)) & 0xFF for k in range(3)], axis=-1)
        out = out.reshape(flat.shape[0], -1)
    else:
        out = word
    return out.astype(np.uint8).reshape(*lead, -1)


def unpack_bits(packed: np.ndarray, bits: int, d: int) -> np.ndarray:
    """Inverse of pack_bits, truncating to d values (quashkv/packing.py:97-159)."""
    packed = np.asarray(packed, dtype=np.uint8)
    if bits == 8:
        return packed.copy()
    *lead, p = packed.shape
    flat = packed.reshape(-1, p).astype(np.uint32)
    mask = (1 << bits) - 1
    if bits == 3:
        g = flat[:, : (p // 3) * 3].reshape(flat.shape[0], -1, 3)
        word = g[..., 0] | (g[..., 1] << 8) | (g[..., 2] << 16)
        vals = np.stack([(word >> (3 * i)) & mask for i in range(8)], axis=-1)
    else:
        per = 8 // bits
        vals = np.stack([(flat >> (bits * i)) & mask for i in range(per)], axis=-1)
    vals = vals.reshape(flat.shape[0], -1)[:, :d]
    return vals.astype(np.uint8).reshape(*lead, d)


# ---------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------

def _block_scores(q_rot, kcodes, kbits, knorm, kcent, s, qjl_scale, scale):
    # quashkv/engine.py:250-271 (== attention.py:104-113 up to summation order)
    k_hat = kcent[kcodes.long()]
    mse_dot = torch.einsum("bhqd,bhkd->bhqk", q_rot, k_hat)
    sign_vals = kbits.float() * 2.0 - 1.0
    corr = qjl_scale * torch.einsum("bhqd,bhkd->bhqk", q_rot.abs() * s, sign_vals)
    return knorm.unsqueeze(2) * (mse_dot + corr) * scale


def attention_naive(q, blocks: Sequence[dict], pi, kcent, vcent, s, qjl_scale,
                    scale: Optional[float] = None, causal: bool = False,
                    total_tokens: Optional[int] = None) -> torch.Tensor:
    """Softmax attention over compressed blocks, naive form.

    Follows quashkv/engine.py:204-299.  Each block is a dict with unpacked
    uint8 ``kcodes``, ``kbits``, ``vcodes`` (B,H,S,d) and fp32 ``knorm``,
    ``vnorm`` (B,H,S).
    """
    if not blocks:
        raise ValueError("No compressed KV blocks in cache. Call append() first.")
    q = q.float()
    B, H, Q, d = q.shape
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    if total_tokens is None:
        total_tokens = sum(b["kcodes"].shape[2] for b in blocks)
    q_rot = q @ pi.T
    scores, values = [], []
    off = 0
    for b in blocks:
        kv = b["kcodes"].shape[2]
        sc = _block_scores(q_rot, b["kcodes"], b["kbits"], b["knorm"], kcent, s,
                           qjl_scale, scale)
        if causal:
            qp = torch.arange(Q) + total_tokens - Q
            kp = torch.arange(kv) + off
            sc = sc.masked_fill((kp.unsqueeze(0) > qp.unsqueeze(1))[None, None],
                                float("-inf"))
        scores.append(sc)
        v = (vcent[b["vcodes"].long()] @ pi) * b["vnorm"].unsqueeze(-1)
        values.append(v)
        off += kv
    w = torch.softmax(torch.cat(scores, dim=-1), dim=-1)
    return torch.einsum("bhqk,bhkd->bhqd", w, torch.cat(values, dim=2))


def attention_online(q, blocks: Sequence[dict], pi, kcent, vcent, s, qjl_scale,
                     scale: Optional[float] = None) -> torch.Tensor:
    """Online-softmax (m, l, O) streaming over blocks, non-causal.

    Follows quashkv/triton_kernels/attention.py:55-149 (the reference's CPU
    path of fused_quantized_attention); final O / max(l, 1e-8).
    """
    q = q.float()
    B, H, Q, d = q.shape
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    q_rot = q @ pi.T
    m = torch.full((B, H, Q), float("-inf"))
    l = torch.zeros(B, H, Q)
    o = torch.zeros(B, H, Q, d)
    for b in blocks:
        sc = _block_scores(q_rot, b["kcodes"], b["kbits"], b["knorm"], kcent, s,
                           qjl_scale, scale)
        m_new = torch.maximum(m, sc.max(dim=-1).values)
        alpha = torch.exp(m - m_new)
        l = l * alpha
        o = o * alpha.unsqueeze(-1)
        p = torch.exp(sc - m_new.unsqueeze(-1))
        l = l + p.sum(dim=-1)
        v = (vcent[b["vcodes"].long()] @ pi) * b["vnorm"].unsqueeze(-1)
        o = o + torch.einsum("bhqk,bhkd->bhqd", p, v)
        m = m_new
    return o / l.unsqueeze(-1).clamp(min=1e-8)


def attention_gqa(q, blocks, pi, kcent, vcent, s, qjl_scale, scale=None,
                  online: bool = True):
    """GQA by query reshape: q (B, Hq, Q, d) with Hq = G*Hkv maps q-head h to
    kv-head h // G (HF repeat_kv convention).  Non-causal only."""
    B, Hq, Q, d = q.shape
    Hkv = blocks[0]["kcodes"].shape[1]
    G = Hq // Hkv
    qr = q.reshape(B, Hkv, G * Q, d)
    fn = attention_online if online else attention_naive
    out = fn(qr, blocks, pi, kcent, vcent, s, qjl_scale, scale)
    return out.reshape(B, Hq, Q, d)


def attention_bruteforce(q, kcodes, kbits, knorm, vcodes, vnorm, pi, kcent,
                         vcent, s, qjl_scale, scale=None):
    """Scalar-loop attention for tiny inputs (fp64), from the formula
    score = n_k (sum_j q~_j c[code_j] + alpha sum_j |q~_j| (2b_j-1) S_j) scale,
    out = sum_t softmax(score)_t n_v,t (c_v[vcode_t] Pi).  q: (Q, d)."""
    q = q.double()
    pi = pi.double()
    Q, d = q.shape
    T = kcodes.shape[0]
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    out = torch.zeros(Q, d, dtype=torch.float64)
    for i in range(Q):
        qr = [sum(float(q[i, k]) * float(pi[j, k]) for k in range(d)) for j in range(d)]
        sc = []
        for t in range(T):
            a = sum(qr[j] * float(kcent[int(kcodes[t, j])]) for j in range(d))
            b = sum(abs(qr[j]) * (2 * int(kbits[t, j]) - 1) * float(s[j]) for j in range(d))
            sc.append(float(knorm[t]) * (a + qjl_scale * b) * scale)
        mx = max(sc)
        e = [math.exp(x - mx) for x in sc]
        z = sum(e)
        for t in range(T):
            vr = torch.tensor([float(vcent[int(vcodes[t, j])]) for j in range(d)],
                              dtype=torch.float64)
            out[i] += (e[t] / z) * float(vnorm[t]) * (vr @ pi)
    return out


def compression_ratio(d: int, key_bits: int, value_bits: int,
                      orig_bits: int = 16) -> float:
    """2 d orig / ((kb + vb) d + 64)  (quashkv/engine.py:305-326)."""
    return (2 * d * orig_bits) / (key_bits * d + 32 + value_bits * d + 32)


# ---------------------------------------------------------------------------
# Mixed precision (quashkv/mixed_precision.py:92-322)
# ---------------------------------------------------------------------------

def mixed_calibrate(data: torch.Tensor, pi: torch.Tensor, n_outliers: int) -> torch.Tensor:
    """Sorted indices of the n_outliers highest-variance rotated channels
    (mixed_precision.py:106-115)."""
    n = data.norm(dim=-1, keepdim=True).clamp(min=1e-8)
    xr = (data / n) @ pi.T
    _, top = xr.var(dim=0).topk(n_outliers)
    return top.sort().values


def mixed_compress(x, pi, outlier_idx, t_out, t_reg):
    """Per-channel boundary quantisation (mixed_precision.py:132-158)."""
    n = x.norm(dim=-1, keepdim=True).clamp(min=1e-8)
    xr = (x / n) @ pi.T
    d = x.shape[-1]
    if outlier_idx is None:
        return quantize_boundary(xr, t_reg), n.squeeze(-1)
    mask = torch.zeros(d, dtype=torch.bool)
    mask[outlier_idx] = True
    idx = torch.empty_like(xr, dtype=torch.uint8)
    idx[..., mask] = quantize_boundary(xr[..., mask], t_out)
    idx[..., ~mask] = quantize_boundary(xr[..., ~mask], t_reg)
    return idx, n.squeeze(-1)


def mixed_decompress(codes, norms, pi, outlier_idx, c_out, c_reg):
    """mixed_precision.py:160-187."""
    d = codes.shape[-1]
    if outlier_idx is None:
        xr = c_reg[codes.long()]
    else:
        mask = torch.zeros(d, dtype=torch.bool)
        mask[outlier_idx] = True
        xr = torch.empty(*codes.shape, dtype=torch.float32)
        xr[..., mask] = c_out[codes[..., mask].long()]
        xr[..., ~mask] = c_reg[codes[..., ~mask].long()]
    return (xr @ pi) * norms.unsqueeze(-1)


def attention_mixed_keys(q, kcodes, knorm, vcodes, vnorm, pi_k, outlier_idx, c_out, c_reg,
                         pi_v, vcent, scale: Optional[float] = None) -> torch.Tensor:
    """Decode attention over mixed-precision keys, decompress-then-attend:
    K^ = mixed_decompress (mixed_precision.py:160-187), V^ = c_v[code] Pi_v n
    (quantizer.py:133-152), softmax(q K^T scale) V^ (engine.py:245-297 with
    K^ in place of the IP key estimate).  q (B, Hq, Q, d) with Hq a multiple of
    the cache's heads (head h reads kv head h // G); codes (B, H, T, d)."""
    q = q.float()
    B, Hq, Q, d = q.shape
    H = kcodes.shape[1]
    G = Hq // H
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    k = mixed_decompress(kcodes, knorm, pi_k, outlier_idx, c_out, c_reg)   # (B, H, T, d)
    v = (vcent[vcodes.long()] @ pi_v) * vnorm.unsqueeze(-1)
    qg = q.reshape(B, H, G * Q, d)
    w = torch.softmax((qg @ k.transpose(-1, -2)) * scale, dim=-1)
    return (w @ v).reshape(B, Hq, Q, d)


def _mixed_mask(d, outlier_idx):
    mask = torch.zeros(d, dtype=torch.bool)
    if outlier_idx is not None:
        mask[outlier_idx] = True
    return mask


def mixed_ip_compress_from_y(y, outlier_idx, c_out, t_out, c_reg, t_reg, s):
    """MixedPrecisionIPQuantizer's code stage on rotated unit vectors y
    (mixed_precision.py:283-297): per-channel boundary codes, x_rot_hat from
    each channel's centroids, QJL bit [(y - x_rot_hat) S >= 0]."""
    mask = _mixed_mask(y.shape[-1], outlier_idx)
    codes = torch.empty_like(y, dtype=torch.uint8)
    codes[..., mask] = quantize_boundary(y[..., mask], t_out)
    codes[..., ~mask] = quantize_boundary(y[..., ~mask], t_reg)
    yhat = torch.empty_like(y)
    yhat[..., mask] = c_out[codes[..., mask].long()]
    yhat[..., ~mask] = c_reg[codes[..., ~mask].long()]
    bits = (((y - yhat) * s) >= 0).to(torch.uint8)
    return codes, bits


def mixed_ip_compress(x, pi, outlier_idx, c_out, t_out, c_reg, t_reg, s):
    """(mse codes, qjl bits, norms) of MixedPrecisionIPQuantizer.compress
    (mixed_precision.py:271-297): norms clamped at 1e-8, y = (x / n) Pi^T."""
    x = x.float()
    n = x.norm(dim=-1, keepdim=True).clamp(min=1e-8)
    y = (x / n) @ pi.T
    codes, bits = mixed_ip_compress_from_y(y, outlier_idx, c_out, t_out, c_reg, t_reg, s)
    return codes, bits, n.squeeze(-1)


def attention_mixed_ip_keys(q, kcodes, kbits, knorm, vcodes, vnorm, pi_k, outlier_idx, c_out,
                            c_reg, s, qjl_scale, pi_v, vcent, scale: Optional[float] = None,
                            causal: bool = False) -> torch.Tensor:
    """Decode attention over mixed-precision IP keys: scores as
    decompress_for_dot (quantizer.py:244-279) with each channel's MSE
    centroid, n_k (<q~, c_ch[code]> + qjl_scale sum |q~| (2b - 1) S) scale,
    softmax, V^ = c_v[code] Pi_v n (engine.py:245-297); causal masks key t
    for query row i when t > T - Q + i.  q (B, Hq, Q, d), Hq a multiple of the
    cache's heads (head h reads kv head h // G); codes (B, H, T, d)."""
    q = q.float()
    B, Hq, Q, d = q.shape
    H, T = kcodes.shape[1], kcodes.shape[2]
    G = Hq // H
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    mask = _mixed_mask(d, outlier_idx)
    k_hat = torch.empty(*kcodes.shape, dtype=torch.float32)
    k_hat[..., mask] = c_out[kcodes[..., mask].long()]
    k_hat[..., ~mask] = c_reg[kcodes[..., ~mask].long()]
    q_rot = (q @ pi_k.T).reshape(B, H, G * Q, d)
    sv = kbits.float() * 2.0 - 1.0
    sc = q_rot @ k_hat.transpose(-1, -2) + qjl_scale * ((q_rot.abs() * s) @ sv.transpose(-1, -2))
    sc = knorm.unsqueeze(2) * sc * scale
    if causal:
        qi = torch.arange(G * Q) % Q
        sc = sc.masked_fill(torch.arange(T)[None, :] > (T - Q + qi)[:, None], float("-inf"))
    w = torch.softmax(sc, dim=-1)
    v = (vcent[vcodes.long()] @ pi_v) * vnorm.unsqueeze(-1)
    return (w @ v).reshape(B, Hq, Q, d)


# ---------------------------------------------------------------------------
# MIPS index search (quashkv/nn_search/index.py:121-163)
# ---------------------------------------------------------------------------

def index_scores(queries, codes, bits, norms, pi, centroids, s, qjl_scale):
    """(M, N) scores n_i (<q~, c[code_i]> + alpha (|q~| S) . (2b_i - 1)), no 1/sqrt(d)."""
    q_rot = queries.float() @ pi.T
    cent = centroids[codes.long()]
    mse = q_rot @ cent.T
    sv = bits.float() * 2.0 - 1.0
    corr = qjl_scale * ((q_rot.abs() * s) @ sv.T)
    return norms.unsqueeze(0) * (mse + corr)


def index_search(queries, codes, bits, norms, pi, centroids, s, qjl_scale, k,
                 chunk: int = 256):
    """torch.topk over index_scores, queries processed in chunks."""
    k = min(k, codes.shape[0])
    outs_s, outs_i = [], []
    for i in range(0, queries.shape[0], chunk):
        sc = index_scores(queries[i:i + chunk], codes, bits, norms, pi, centroids,
                          s, qjl_scale)
        v, ix = torch.topk(sc, k, dim=1)
        outs_s.append(v)
        outs_i.append(ix)
    return torch.cat(outs_s), torch.cat(outs_i)
