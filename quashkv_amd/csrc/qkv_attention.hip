// Split-K decode attention over the compressed cache store.
//
// score(q, t) = n_k,t * (sum_j q~_j c_k[code_tj] + alpha sum_j |q~_j| S_j (2b_tj - 1)) * scale
// out         = (sum_t softmax(score)_t n_v,t c_v[vcode_t]) Pi,      q~ = q Pi^T
// Reference: quashkv/engine.py:204-299 (naive) and
// quashkv/triton_kernels/attention.py:55-149 (online softmax).  Unlike the
// reference, values are accumulated in the ROTATED domain and un-rotated once
// per query row in the combine kernel (linearity of x -> x Pi).
// GQA: query head h reads kv head h / G; the G*Q query rows of one kv head
// ("rows") share every K/V byte a workgroup streams.
//
// Cache store (see qkv_store.hip): K rows are bit-plane major
// [MSE plane 0..mbits-1][QJL plane]; V is in 32-token bit-plane tiles.
//
// Two partial-softmax kernels write the same (m, l, O~) split partials, and
// one combine kernel merges them:
//
//   split_mfma   (d = 128, MSE key bits 1-2, value bits 1-4, symmetric
//                 codebooks).  Integer MFMA on bit planes:
//     * a symmetric codebook is a sum of odd Walsh functions of the code bits,
//       c[code] = sum_S g_S prod_{k in S} (2 b_k - 1), so every score and every
//       value coordinate is a weighted sum of 0/1 bit planes;
//     * a 0/1 plane becomes int8 MFMA operands with ONE v_and per 4 bytes:
//       word & (0x01010101 << i) leaves bit i of each byte in place, i.e. the
//       byte value is b * 2^i (b * -128 for i = 7);
//     * the other operand carries the real weights as 30-bit fixed point split
//       into four signed base-256 int8 digits, pre-divided by the byte's 2^i,
//       so the i32 accumulators are exact; digit rows are recombined after.
//     Scores: C[4 rows x 4 digits][16 tokens] += A(query weights)[16][64] x
//     B(K planes)[64][16].  Values: C[16 coords][4 rows x 4 digits] +=
//     A(V planes)[16][64 tokens] x B(p * n_v digits)[64 tokens][16].
//     Scores of a split (<= 2048 tokens) are kept in LDS, so the softmax max is
//     known before the value pass and the integer accumulators never rescale.
//   split_generic (any supported shape): VALU, one token per thread.
#include <math.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <mutex>

#include "qkv_attn_dev.h"


namespace {

using namespace qkv_attn;

// ------------------------------------------------------------ parameters


// ------------------------------------------------------------ workspace

constexpr int kRowsG = 32;       // query rows per workgroup on the generic path
constexpr int kTileG = 256;      // tokens per tile == threads on the generic path

struct WsLayout {
  int64_t qw, aq, rowc, po, pml, total;  // byte offsets
};

inline WsLayout ws_layout(int B, int Hkv, int R, int D, int S) {
  WsLayout w;
  const int64_t bhk = int64_t(B) * Hkv;
  const int64_t chunks = (R + kRowsM - 1) / kRowsM;
  int64_t off = 0;
  w.qw = off;   off += bhk * R * 2 * D * 4;                     // generic: q~, w
  w.aq = off;   off += bhk * chunks * kNUMax * 64 * 16;        // MFMA: query operands
  w.rowc = off; off += bhk * chunks * kRowsM * 2 * 4;          // MFMA: row constants
  w.po = off;   off += int64_t(S) * bhk * R * D * 4;           // split partial O~
  w.pml = off;  off += int64_t(S) * bhk * R * 2 * 4;           // split partial (m, l)
  w.total = off;
  return w;
}

template <typename T>
T* at(void* base, int64_t off) {
  return reinterpret_cast<T*>(static_cast<char*>(base) + off);
}

// ------------------------------------------------------------ store access

template <int D>
__device__ __forceinline__ uint32_t k_code(const uint8_t* __restrict__ row, int j, int mbits) {
  uint32_t c = 0;
  for (int p = 0; p < mbits; ++p) c |= ((row[p * (D / 8) + (j >> 3)] >> (j & 7)) & 1u) << p;
  return c;
}
template <int D>
__device__ __forceinline__ uint32_t k_qjl(const uint8_t* __restrict__ row, int j, int mbits) {
  return (row[mbits * (D / 8) + (j >> 3)] >> (j & 7)) & 1u;
}
// words: the vbits plane words of token t's tile at coordinate j (stride D)
__device__ __forceinline__ uint32_t v_code(const uint32_t* __restrict__ w, int64_t stride,
                                           int t, int vbits) {
  uint32_t c = 0;
  for (int k = 0; k < vbits; ++k) c |= ((w[k * stride] >> (t & 31)) & 1u) << k;
  return c;
}

// ------------------------------------------------------------ generic path

// q~ = q Pi^T and w = alpha |q~| S per query row, into qw[b][hkv][r][2][D].
template <int D>
__global__ __launch_bounds__(128) void qrot_kernel(const void* __restrict__ q, int q_dtype,
                                                   const float* __restrict__ pi,
                                                   const float* __restrict__ signs, float alpha,
                                                   int Hq, int Hkv, int Q,
                                                   float* __restrict__ qw) {
  __shared__ float qs[D];
  const int row = blockIdx.x;  // (b, h, qi) flattened
  const int tid = threadIdx.x;
  if (tid < D) qs[tid] = qkv_load(q, int64_t(row) * D + tid, q_dtype);
  __syncthreads();
  if (tid >= D) return;
  const int qi = row % Q;
  const int h = (row / Q) % Hq;
  const int b = row / (Q * Hq);
  const int G = Hq / Hkv;
  const int hkv = h / G, g = h - hkv * G;
  const int R = G * Q;
  const int r = g * Q + qi;
  float acc = 0.f;
  const float* prow = pi + int64_t(tid) * D;
  for (int k = 0; k < D; ++k) acc = fmaf(qs[k], prow[k], acc);
  float* dst = qw + ((int64_t(b) * Hkv + hkv) * R + r) * 2 * D;
  dst[tid] = acc;
  dst[D + tid] = alpha * fabsf(acc) * signs[tid];
}

template <int D>
__global__ __launch_bounds__(kTileG) void split_generic(
    const float* __restrict__ qw, const uint8_t* __restrict__ kst,
    const float* __restrict__ knorm, const uint32_t* __restrict__ vst,
    const float* __restrict__ vnorm, int64_t t_stride, int64_t T, int Hkv, int R, int Q,
    int row_chunks, int mbits, int vbits, Tables tb, float scale, int causal,
    int64_t split_len, const int32_t* __restrict__ klo, const int32_t* __restrict__ khi,
    int64_t cbase, float* __restrict__ part_o, float* __restrict__ part_ml) {
  __shared__ float qs[kRowsG][D];
  __shared__ float ws[kRowsG][D];
  __shared__ float ps[kRowsG][kTileG];  // scores, then probabilities; reused at the end
  __shared__ float vn[kTileG];
  __shared__ float red[kRowsG][4];
  __shared__ float ms[kRowsG], ls[kRowsG], al[kRowsG];
  __shared__ float kc[16], vc[16];

  const int split = blockIdx.x;
  const int hkv = blockIdx.y / row_chunks;
  const int chunk = blockIdx.y - hkv * row_chunks;
  const int b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r_begin = chunk * kRowsG;
  const int nr = min(kRowsG, R - r_begin);

  const int64_t krb = int64_t(mbits + 1) * D / 8;
  const int64_t bh = int64_t(b) * Hkv + hkv;
  const uint8_t* kbase = kst + bh * t_stride * krb;
  const uint32_t* vbase = vst + bh * (t_stride / 32) * vbits * D;
  const float* knb = knorm + bh * t_stride;
  const float* vnb = vnorm + bh * t_stride;

  const float* qsrc = qw + (bh * R + r_begin) * 2 * D;
  for (int i = tid; i < nr * D; i += kTileG) {
    const int r = i / D, j = i - r * D;
    qs[r][j] = qsrc[r * 2 * D + j];
    ws[r][j] = qsrc[r * 2 * D + D + j];
  }
  if (tid < 16) {
    kc[tid] = tb.kc[tid];
    vc[tid] = tb.vc[tid];
  }
  if (tid < kRowsG) {
    ms[tid] = -INFINITY;
    ls[tid] = 0.f;
  }

  const int64_t t_begin = int64_t(split) * split_len;
  const int64_t t_end = min<int64_t>(T, t_begin + split_len);
  // this sequence's attended keys [k_lo, k_hi) and causal position
  const int64_t k_lo = klo ? max<int64_t>(0, klo[b]) : 0;
  const int64_t k_hi = khi ? min<int64_t>(T, khi[b]) : T;
  const int64_t cpos = cbase > 0 ? cbase : k_hi;

  const int pj = tid & 127, hf = tid >> 7;  // PV layout: coordinate, token half
  float acc[kRowsG];
#pragma unroll
  for (int r = 0; r < kRowsG; ++r) acc[r] = 0.f;
  __syncthreads();

  for (int64_t t0 = t_begin; t0 < t_end; t0 += kTileG) {
    const int64_t t = t0 + tid;
    const bool valid = t < t_end;
    const int64_t tc = valid ? t : t_begin;
    const uint8_t* krow = kbase + tc * krb;
    const float kn = valid ? knb[tc] * scale : 0.f;
    for (int rb = 0; rb < nr; rb += 8) {
      float s[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) s[i] = 0.f;
      for (int j = 0; j < D; ++j) {
        const float c = kc[k_code<D>(krow, j, mbits) & 15u];
        const float z = k_qjl<D>(krow, j, mbits) ? 1.f : -1.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int r = min(rb + i, kRowsG - 1);
          s[i] = fmaf(qs[r][j], c, s[i]);
          s[i] = fmaf(ws[r][j], z, s[i]);
        }
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = rb + i;
        if (r < nr) {
          float v = kn * s[i];
          if (!valid || t < k_lo || t >= k_hi) v = -INFINITY;
          if (causal) {
            const int qi = (r_begin + r) % Q;
            if (t > cpos - Q + qi) v = -INFINITY;
          }
          ps[r][tid] = v;
        }
      }
    }
    vn[tid] = valid && t >= k_lo && t < k_hi ? vnb[tc] : 0.f;
    __syncthreads();

    for (int r = 0; r < nr; ++r) {
      const float m = qkv_wave_max(ps[r][tid]);
      if (lane == 0) red[r][wave] = m;
    }
    __syncthreads();
    if (tid < nr) {
      const float tm = fmaxf(fmaxf(red[tid][0], red[tid][1]), fmaxf(red[tid][2], red[tid][3]));
      const float mo = ms[tid];
      const float mn = fmaxf(mo, tm);
      al[tid] = (mn == -INFINITY) ? 1.f : expf(mo - mn);
      ms[tid] = mn;
    }
    __syncthreads();
    for (int r = 0; r < nr; ++r) {
      const float mn = ms[r];
      const float p = (mn == -INFINITY) ? 0.f : expf(ps[r][tid] - mn);
      ps[r][tid] = p;
      const float sum = qkv_wave_sum(p);
      if (lane == 0) red[r][wave] = sum;
    }
    __syncthreads();
    if (tid < nr) ls[tid] = ls[tid] * al[tid] + (red[tid][0] + red[tid][1]) + (red[tid][2] + red[tid][3]);

#pragma unroll
    for (int r = 0; r < kRowsG; ++r) acc[r] *= (r < nr) ? al[r] : 1.f;
    if (pj < D) {
      const int tt0 = hf * (kTileG / 2);
      for (int tt = tt0; tt < tt0 + kTileG / 2; ++tt) {
        const int64_t tk = t0 + tt;
        if (tk >= t_end) break;
        const uint32_t* w = vbase + (tk >> 5) * vbits * D + pj;
        const float v = vc[v_code(w, D, static_cast<int>(tk & 31), vbits) & 15u] * vn[tt];
#pragma unroll
        for (int r = 0; r < kRowsG; ++r)
          if (r < nr) acc[r] = fmaf(ps[r][tt], v, acc[r]);
      }
    }
    __syncthreads();
  }

  float* red_o = &ps[0][0];  // kRowsG x 128 floats
  if (hf == 1 && pj < D) {
#pragma unroll
    for (int r = 0; r < kRowsG; ++r)
      if (r < nr) red_o[r * 128 + pj] = acc[r];
  }
  __syncthreads();
  const int64_t base = ((int64_t(split) * gridDim.z + b) * Hkv + hkv) * R + r_begin;
  if (hf == 0 && pj < D) {
#pragma unroll
    for (int r = 0; r < kRowsG; ++r)
      if (r < nr) part_o[(base + r) * D + pj] = acc[r] + red_o[r * 128 + pj];
  }
  if (tid < nr) {
    part_ml[(base + tid) * 2 + 0] = ms[tid];
    part_ml[(base + tid) * 2 + 1] = ls[tid];
  }
}

// ------------------------------------------------------------ MFMA path

// Query operands for the score MFMA.  One workgroup per (b, kv head, chunk of
// 4 rows).  Row bit p of a K row (plane-major, D bits per plane) has weight W_p:
//   MSE plane r, coordinate j:  2 kg[r] q~_j
//   QJL plane,   coordinate j:  2 alpha |q~_j| S_j
// (mixed-precision rows: per-slot coefficients, see Tables).  The operand
// holds Z_p = round(W_p 2^Fq / 2^i), negated for i = 7 (a set bit masks to
// the byte value -128), where i = p % 8 is the bit's place in its byte, as
// signed base-256 digits; |Z| < 2^30.  Fq comes from the bound
// max |W| <= 2 max(kg, alpha) ||q|| (Pi is orthogonal), so no reduction over
// the rotated row stands between the rotation and the digits.
// Operand register layout: aq[(bhc * NU + u) * 64 + lane] (4 dwords), lane
// (m = 4 row + digit, g = lane / 16); byte beta of dword e <-> row bit
//   D = 128:  32 (g DPL + u / 2) + 8 beta + 4 (u % 2) + e   (NU = 2 DPL)
//   D = 64:   32 (2 u + g / 2) + 8 beta + 4 (g % 2) + e      (NU = NPL)
// i.e. the score kernel's lane group g reads row dwords g DPL .. (D = 128) or
// 2 u + g / 2 (D = 64) and masks nibble half u % 2 (D = 128) or g % 2.
// NPL planes per row: NPL - 1 MSE planes (odd bit subsets s, weight
// 2 kg[s] q~_j), then the QJL plane.  The decode rows have NPL = mbits + 1
// (mbits <= 2: the subsets are the single bits); the search index also uses
// NPL = 5 for 3-bit MSE codes (three bits and their parity).
// Thread (j, part) rotates coordinate j of all rows over one of 256 / D parts
// of k, then turns coordinate j of rows part, part + 256 / D, ... into digit
// bytes, scattered into an LDS image of the operands that is copied out whole.
template <int D, int NPL, bool FP4>
__global__ __launch_bounds__(256) void prepare_mfma(QLayers ql, int Bl, int q_dtype,
                                                    float alpha, int Hq, int Hkv, int Q, int R,
                                                    int chunks, Tables tb,
                                                    qkv_v4i* __restrict__ aq,
                                                    float* __restrict__ rowc,
                                                    float* __restrict__ qw) {
  constexpr int MB = NPL - 1;  // weighted MSE planes
  constexpr int KRB = NPL * D / 8;
  constexpr int DPL = KRB / 16;
  constexpr int NU = KRB / 8;        // score MFMAs per 16 tokens
  constexpr int NW = NU * 64 * 4;    // operand dwords per chunk
  constexpr int NPART = 256 / D;     // threads per coordinate
  constexpr int KP = D / NPART;      // k per thread in the rotation
  constexpr int RPT = kRowsM / NPART;  // rows per thread in the digit phase
  constexpr int WPP = D / 64;        // waves per part
  static_assert(D == 128 || D == 64, "64- or 128-dim rows");
  static_assert(D == 64 || KRB % 16 == 0, "128-dim rows split into 4 lane groups");
  static_assert(kRowsM == 4, "rows per chunk");
  static_assert(!FP4 || (D == 128 && NPL <= 3), "fp4 operands: the fused d = 128 decode");
  __shared__ float qs[kRowsM][D];
  __shared__ float part[NPART][kRowsM][D];
  __shared__ float nqs[kRowsM];
  __shared__ uint32_t stage[NW];
  __shared__ float red[4][RPT][3];  // [wave][row slot][sq, sw, fp4 halves]

  const int tid = threadIdx.x;
  const int G = Hq / Hkv;
  const int bhc = blockIdx.x;  // over the batch of all layers
  const int chunk = bhc % chunks;
  const int bh = bhc / chunks;
  const int hkv = bh % Hkv, bz = bh / Hkv;
  const int layer = bz / Bl, b = bz - layer * Bl;
  const void* __restrict__ q = ql.q[layer];
  const float* __restrict__ pi = ql.pi[layer];
  const float* __restrict__ signs = ql.signs[layer];
  const int r0 = chunk * kRowsM;
  const int nr = min(kRowsM, R - r0);
  // Pi staged in LDS by coalesced loads (rows padded by 4 floats: the
  // threads of a wave then read 16 rows' float4s conflict-free), then this
  // thread's part of row j from there
  extern __shared__ __align__(16) float4 pis[];  // [D][(D + 4) / 4]
  constexpr int PR4 = (D + 4) / 4;
  {
    const float4* src = reinterpret_cast<const float4*>(pi);
#pragma unroll
    for (int x = 0; x < D * D / 4 / 256; ++x) {
      const int i = tid + 256 * x, row = i / (D / 4), c4 = i - row * (D / 4);
      pis[row * PR4 + c4] = src[i];
    }
  }
  const int j = tid % D, half = tid / D;
  float qv[kRowsM * D / 256];
#pragma unroll
  for (int x = 0; x < kRowsM * D / 256; ++x) {
    const int i = tid + 256 * x;
    const int r = i / D, jj = i - r * D;
    float v = 0.f;
    if (r < nr) {
      const int row = r0 + r;
      const int g = row / Q, qi = row - g * Q;
      const int h = hkv * G + g;
      v = qkv_load(q, ((int64_t(b) * Hq + h) * Q + qi) * D + jj, q_dtype);
    }
    qv[x] = v;
  }
  const float sgn = signs[j];
#pragma unroll
  for (int x = 0; x < kRowsM * D / 256; ++x) {
    const int i = tid + 256 * x;
    qs[i / D][i % D] = qv[x];
  }
  __syncthreads();
  float4 prow[KP / 4];
#pragma unroll
  for (int k4 = 0; k4 < KP / 4; ++k4) prow[k4] = pis[j * PR4 + half * (KP / 4) + k4];
  {  // ||q_r||^2: wave w sums row w
    const int wave = tid >> 6, lane = tid & 63;
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < D / 64; ++c) {
      const float a = qs[wave][lane + 64 * c];
      ss = fmaf(a, a, ss);
    }
    ss = wave_sum_dpp(ss);
    if (lane == 0) nqs[wave] = ss;
  }
  {  // q~_j = sum_k q_k Pi[j][k], this thread's part of k for all rows
    float acc[kRowsM] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k4 = 0; k4 < KP / 4; ++k4) {
      const int k = half * KP + 4 * k4;
#pragma unroll
      for (int r = 0; r < kRowsM; ++r) {
        acc[r] = fmaf(qs[r][k], prow[k4].x, acc[r]);
        acc[r] = fmaf(qs[r][k + 1], prow[k4].y, acc[r]);
        acc[r] = fmaf(qs[r][k + 2], prow[k4].z, acc[r]);
        acc[r] = fmaf(qs[r][k + 3], prow[k4].w, acc[r]);
      }
    }
#pragma unroll
    for (int r = 0; r < kRowsM; ++r) part[half][r][j] = acc[r];
  }
  float kgmax = alpha;
#pragma unroll
  for (int r = 0; r < MB; ++r) kgmax = fmaxf(kgmax, fabsf(tb.kg[r]));
  __syncthreads();

  uint8_t* sb = reinterpret_cast<uint8_t*>(stage);
  // digit bytes of weight W at row bit p of row r
  auto put8 = [&](int p, float W, int fq, int r) {
    const int i = p & 7;
    int Z = static_cast<int>(rintf(ldexpf(W, fq - i)));
    if (i == 7) Z = -Z;
    const uint32_t dg = (static_cast<uint32_t>(Z) + 0x808080u) ^ 0x808080u;
    const int w32 = p >> 5, e = i & 3, beta = (p >> 3) & 3;
    int g, u;
    if constexpr (D == 128) {
      g = w32 / DPL;
      u = 2 * (w32 - g * DPL) + (i >> 2);
    } else {
      g = 2 * (w32 & 1) + (i >> 2);
      u = w32 >> 1;
    }
    const int base = ((u * 64 + 16 * g + 4 * r) * 4 + e) * 4 + beta;
#pragma unroll
    for (int v = 0; v < 4; ++v) sb[base + 16 * v] = static_cast<uint8_t>(dg >> (8 * v));
  };
  float csq[RPT], csw[RPT], chf[RPT];
#pragma unroll
  for (int rr = 0; rr < RPT; ++rr) {
    const int r = half + NPART * rr;
    float hf = 0.f;
    float v = 0.f;
#pragma unroll
    for (int pp = 0; pp < NPART; ++pp) v += part[pp][r][j];
    const float w = alpha * fabsf(v) * sgn;
    if (qw != nullptr && r < nr) {  // q~ and w for the VALU kernel, qw[b][hkv][row][2][D]
      float* dst = qw + (int64_t(bh) * R + r0 + r) * 2 * D;
      dst[j] = v;
      dst[D + j] = w;
    }
    const float wmax = 2.f * kgmax * sqrtf(nqs[r]);
    int ex = 0;
    if (wmax > 0.f) frexpf(wmax, &ex);  // wmax = f 2^ex, f in [0.5, 1)
    // int8 digits: the fixed-point exponent (|Z| < 2^30); fp4: the row's sigma
    const int fq = FP4 ? kf4_sigma(wmax) : wmax > 0.f ? 30 - ex : 0;
    // IP keys (the mixed-key formats run on decode_fused's own prologue)
    if constexpr (FP4) {
      csq[rr] = key_weights<MB>(tb, j, v, w, [&](int pb, float W) {
        hf += kf4_put<DPL, 4 * DPL, false>(sb, pb, W, fq, r);
      });
    } else {
      csq[rr] = v;
#pragma unroll
      for (int pl = 0; pl < MB; ++pl) put8(pl * D + j, 2.f * tb.kg[pl] * v, fq, r);
      put8(MB * D + j, 2.f * w, fq, r);
    }
    csw[rr] = w;
    chf[rr] = hf;
  }
  {  // row constants: sums over j (a wave holds 64 j of one part)
    const int wave = tid >> 6, lane = tid & 63;
#pragma unroll
    for (int rr = 0; rr < RPT; ++rr) {
      const float a = wave_sum_dpp(csq[rr]);
      const float c = wave_sum_dpp(csw[rr]);
      const float h = FP4 ? wave_sum_dpp(chf[rr]) : 0.f;
      if (lane == 0) {
        red[wave][rr][0] = a;
        red[wave][rr][1] = c;
        red[wave][rr][2] = h;
      }
    }
  }
  __syncthreads();
  uint32_t* aqw = reinterpret_cast<uint32_t*>(aq) + int64_t(bhc) * NW;
#pragma unroll
  for (int x = 0; x < NW / 256; ++x) aqw[tid + 256 * x] = stage[tid + 256 * x];
  if (tid < kRowsM) {  // row r = tid: part r % NPART (waves WPP h ..), slot r / NPART
    const int r = tid, h = r % NPART, rr = r / NPART;
    float sq = 0.f, sw = 0.f, sh = 0.f;
#pragma unroll
    for (int w = 0; w < WPP; ++w) {
      sq += red[WPP * h + w][rr][0];
      sw += red[WPP * h + w][rr][1];
      sh += red[WPP * h + w][rr][2];
    }
    const float wmax = 2.f * kgmax * sqrtf(nqs[r]);
    int ex = 0;
    if (wmax > 0.f) frexpf(wmax, &ex);
    const int fq = wmax > 0.f ? 30 - ex : 0;
    rowc[(int64_t(bhc) * kRowsM + r) * 2 + 0] = tb.kconst * sq - sw + sh;
    // fp4: the row's sigma (an integer, as a float); int8: 2^-Fq
    rowc[(int64_t(bhc) * kRowsM + r) * 2 + 1] =
        FP4 ? static_cast<float>(kf4_sigma(wmax)) : ldexpf(1.f, -fq);
  }
}

// Dynamic LDS of prepare_mfma<D, NPL> (the padded Pi), raising the kernel's
// limit past 64 KiB once where needed.
template <int D, int NPL, bool FP4>
uint32_t prep_lds() {
  constexpr uint32_t bytes = D * (D + 4) * 4;
  if constexpr (bytes > 65536) {
    static const bool raised = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&prepare_mfma<D, NPL, FP4>),
        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes)) == hipSuccess;
    (void)raised;
  }
  return bytes;
}

// Four waves per SIMD (at most 128 VGPRs): with 4 workgroups per CU the split
// count fills the chip in whole rounds and hides the K/V load latency.
// RC row chunks (of 4 query rows) per workgroup: with RC = 2 (GQA groups of
// 5..8 rows at d = 64) each K/V operand expanded from the store feeds two
// MFMAs, and the split's K/V bytes are read once for 8 rows.
template <int D, int MB, int VB, int RC, bool RANGES>
__global__ __launch_bounds__(256, 4) void split_mfma(
    const qkv_v4i* __restrict__ aq, const float* __restrict__ rowc, KVLayers kv, int Bl,
    int64_t t_stride, int64_t T, int Hkv, int R, int Q, int chunks, float scale, int causal,
    int64_t split_len, Tables tb, float* __restrict__ part_o, float* __restrict__ part_ml) {
  constexpr int KRB = (MB + 1) * D / 8;  // K row bytes
  constexpr int DPL = KRB / 16;          // row dwords per lane group (D = 128)
  constexpr int NU = KRB / 8;            // score MFMAs per 16 tokens
  // row dwords each lane loads per token: its group's DPL (D = 128), or
  // dword 2 u + g / 2 for each MFMA u (D = 64; nibble half g % 2)
  constexpr int NLD = D == 128 ? DPL : NU;
  constexpr int NP = n_odd_subsets(VB);  // value planes
  constexpr int MTW = D / 64;            // 16-coordinate tiles per wave
  constexpr int RW = kRowsM * RC;        // query rows per workgroup
  static_assert(D == 128 || D == 64, "64- or 128-dim rows");
  static_assert(D == 64 || KRB % 16 == 0, "K rows must split into 4 lane groups of whole dwords");
  static_assert(D % 64 == 0, "value tiles split over 4 waves");
  static_assert(RC == 1 || RC == 2, "one or two row chunks");

  // dynamic LDS, sized by the host to this launch's split length:
  // [ntile_cap][RW rows][64] scores, rewritten in place as value-MFMA digits
  // [ntile_cap][RC][col = 4 row + digit][64 K positions] (RC KB per tile
  // either way), then [ntile_cap * 64] value norms
  extern __shared__ __align__(16) float smem[];
  const int ntile_cap = static_cast<int>((split_len + 63) >> 6);
  float(*sbuf)[RW][64] = reinterpret_cast<float(*)[RW][64]>(smem);
  float* vn = smem + ntile_cap * RW * 64;
  __shared__ float red_m[4][RW];
  __shared__ float red_v[4];
  __shared__ float lsum_s[RW];
  __shared__ long long usum_s[RW];  // sum_t Z_t s_t per row, exact

  const int split = blockIdx.x;
  const int cgroups = (chunks + RC - 1) / RC;
  const int hkv = blockIdx.y / cgroups, cgi = blockIdx.y - hkv * cgroups;
  const int b = blockIdx.z;  // over the batch of all layers
  const int layer = b / Bl;
  const uint8_t* __restrict__ kst = kv.kst[layer];
  const float* __restrict__ knorm = kv.knorm[layer];
  const uint32_t* __restrict__ vst = kv.vst[layer];
  const float* __restrict__ vnorm = kv.vnorm[layer];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ln = lane & 15, lg = lane >> 4;
  const int r0 = cgi * RW;
  const int nr = min(RW, R - r0);  // valid rows of the workgroup
  const int64_t bseq = b - layer * Bl;                       // sequence in the layer
  const int64_t bh = bseq * Hkv + hkv;                        // in the layer's store
  const int64_t ts = int64_t(split) * split_len;
  const int64_t te = min<int64_t>(T, ts + split_len);
  const int ntok = te > ts ? static_cast<int>(te - ts) : 0;
  // the sequence's attended keys, split-relative: [slo, shi) (RANGES: the
  // store has per-sequence key ranges)
  const SeqRange sr = seq_range(kv, bseq, T);
  const int slo = RANGES ? static_cast<int>(min<int64_t>(ntok, max<int64_t>(0, sr.lo - ts))) : 0;
  const int shi = RANGES ? static_cast<int>(min<int64_t>(ntok, max<int64_t>(0, sr.hi - ts))) : ntok;

  // ---------------- phase 1: scores of every token of the split -> LDS
  qkv_v4i a[RC][NU];
  float cr[RC], fq[RC];
  bool row_ok[RC];
  int clim[RC];
  const float scale2 = scale * 1.4426950408889634f;  // scores in log2 units on this path
#pragma unroll
  for (int c = 0; c < RC; ++c) {
    const int chunk = cgi * RC + c;
    const bool cv = chunk < chunks;
    const int64_t bhc = (int64_t(b) * Hkv + hkv) * chunks + (cv ? chunk : 0);  // workspace
#pragma unroll
    for (int u = 0; u < NU; ++u)
      a[c][u] = cv ? aq[(bhc * NU + u) * 64 + lane] : qkv_v4i{0, 0, 0, 0};
    cr[c] = cv ? rowc[(bhc * kRowsM + lg) * 2 + 0] : 0.f;
    fq[c] = cv ? rowc[(bhc * kRowsM + lg) * 2 + 1] : 0.f;
    row_ok[c] = kRowsM * c + lg < nr;
    // causal: token tl (split-relative) is visible to this lane's row iff
    // ts + tl <= cpos - Q + qi
    const int qi = (r0 + kRowsM * c + lg) % Q;
    const int64_t climit = causal ? (sr.cpos - Q + qi - ts) : int64_t(kSplitMax);
    clim[c] = static_cast<int>(max<int64_t>(-1, min<int64_t>(climit, kSplitMax)));
  }

  // Each wave scores 64-token tiles w, w + 4, ... as four 16-token MFMA
  // groups.  K rows, key norms and value norms of the next PD1 tiles are in
  // flight in a register ring while the current tile is scored.
  float mloc[RC], vmax = 0.f;
#pragma unroll
  for (int c = 0; c < RC; ++c) mloc[c] = -INFINITY;
  const int ntile1 = (ntok + 63) >> 6;
  // First store row of the split's 64-token tile `tile`: linear in the tile
  // for a contiguous store, the tile's page for a paged one.
  // (paged: lane l holds the page of the split's tile l, read once; a split
  // has at most kSplitMax / 64 <= 64 tiles)
  const int32_t* __restrict__ ptab = kv.ptab;
  int tile_page = 0;
  const int tsh = kv.plg - 6;  // log2 of the 64-token tiles per page
  if (ptab != nullptr && lane < ntile1) {
    tile_page = ptab[bseq * kv.pmax + ((static_cast<int>(ts >> 6) + lane) >> tsh)];
    if (tile_page < 0 || tile_page >= kv.npages) tile_page = -1;  // outside the pool
  }
  // lanes' bit: the split's tile of that lane lies on a page of the pool
  const uint64_t page_okm = ptab != nullptr ? __ballot(tile_page >= 0) : ~uint64_t(0);
  if (tile_page < 0) tile_page = 0;
  auto tile_row = [&](int tile) -> int64_t {
    if (ptab)
      return ((int64_t(__builtin_amdgcn_readlane(tile_page, tile)) * Hkv + hkv) << kv.plg) +
             (((static_cast<int>(ts >> 6) + tile) & ((1 << tsh) - 1)) << 6);
    return bh * t_stride + ts + int64_t(tile) * 64;
  };
  constexpr int PD1 = RC == 2 ? 1 : 2;  // (registers: two chunks' accumulators)
  uint32_t kd[PD1][4][NLD];
  float kn[PD1][4], vv[PD1][4];
  // Tokens past the split end are read too (masked when scored): the store
  // capacity (a contiguous stream's, or a page) is a multiple of 64 and >= T,
  // so whole 64-token tiles of the split stay inside it.
  const int lsh = 4 * (lg & 1);  // D = 64: this lane group's nibble half
  auto load1 = [&](int slot, int tile) {
    const int64_t rb = tile_row(tile);
    const uint32_t* krow0 = reinterpret_cast<const uint32_t*>(kst + (rb + ln) * KRB) +
                            (D == 128 ? lg * DPL : (lg >> 1));
    const float* knt = knorm + rb;
    const float* vnt = vnorm + rb;
#pragma unroll
    for (int sub = 0; sub < 4; ++sub) {
      const uint32_t* krow = krow0 + sub * 16 * (KRB / 4);
#pragma unroll
      for (int x = 0; x < NLD; ++x) kd[slot][sub][x] = krow[D == 128 ? x : 2 * x];
      kn[slot][sub] = knt[sub * 16 + ln];
      vv[slot][sub] = vnt[sub * 16 + ln];
    }
  };
  auto score1 = [&](int slot, int tile) {
    // four independent 16-token chains per chunk interleaved, one settle for all
    qkv_v4i acc[RC][4];
#pragma unroll
    for (int c = 0; c < RC; ++c)
#pragma unroll
      for (int sub = 0; sub < 4; ++sub) acc[c][sub] = qkv_v4i{0, 0, 0, 0};
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int sh = D == 128 ? 4 * (u & 1) : lsh;
#pragma unroll
      for (int sub = 0; sub < 4; ++sub) {
        const uint32_t x = kd[slot][sub][D == 128 ? u >> 1 : u];
        qkv_v4i bo;
        bo[0] = static_cast<int>(x & (0x01010101u << sh));
        bo[1] = static_cast<int>(x & (0x02020202u << sh));
        bo[2] = static_cast<int>(x & (0x04040404u << sh));
        bo[3] = static_cast<int>(x & (0x08080808u << sh));
#pragma unroll
        for (int c = 0; c < RC; ++c) acc[c][sub] = mfma_i8(a[c][u], bo, acc[c][sub]);
      }
    }
    mfma_settle();
#pragma unroll
    for (int sub = 0; sub < 4; ++sub) {
      const int tl = tile * 64 + sub * 16 + ln;
      // (without ranges the bound is the split's length alone: the register
      // allocation of this loop has no room for the lower bound)
      const bool in = (RANGES ? tl >= slo && tl < shi : tl < ntok) && ((page_okm >> tile) & 1u);
#pragma unroll
      for (int c = 0; c < RC; ++c) {
        const float z = static_cast<float>(acc[c][sub][0]) +
                        256.f * static_cast<float>(acc[c][sub][1]) +
                        65536.f * static_cast<float>(acc[c][sub][2]) +
                        16777216.f * static_cast<float>(acc[c][sub][3]);
        const float sc0 = kn[slot][sub] * scale2 * fmaf(z, fq[c], cr[c]);
        const float sc = (in & row_ok[c] & (tl <= clim[c])) ? sc0 : -INFINITY;
        sbuf[tile][kRowsM * c + lg][sub * 16 + ln] = sc;
        mloc[c] = fmaxf(mloc[c], sc);
      }
      const float vz = in ? vv[slot][sub] : 0.f;
      vn[tl] = vz;  // the four lane groups store the same value
      vmax = fmaxf(vmax, vz);
    }
  };
#pragma unroll
  for (int d = 0; d < PD1; ++d)
    if (wave + 4 * d < ntile1) load1(d, wave + 4 * d);
  for (int tile0 = wave; tile0 < ntile1; tile0 += 4 * PD1) {
#pragma unroll
    for (int d = 0; d < PD1; ++d) {
      const int tile = tile0 + 4 * d;
      if (tile < ntile1) {
        score1(d, tile);
        if (tile + 4 * PD1 < ntile1) load1(d, tile + 4 * PD1);
      }
    }
  }
#pragma unroll
  for (int c = 0; c < RC; ++c) {
    mloc[c] = row_max_last(mloc[c]);  // the 16 lanes of a row group: max in lane 15
    if (ln == 15) red_m[wave][kRowsM * c + lg] = mloc[c];
  }
  vmax = wave_max_dpp(vmax);
  if (lane == 0) red_v[wave] = vmax;
  __syncthreads();

  // ---------------- phase 1.5: p = 2^(s - m), value digits (wave w <-> rows w, w + 4)
  const float vmx = fmaxf(fmaxf(red_v[0], red_v[1]), fmaxf(red_v[2], red_v[3]));
  int ev = 0;
  if (vmx > 0.f) frexpf(vmx, &ev);
  const int Fv = vmx > 0.f ? 30 - ev : 0;  // vmx 2^Fv < 2^30
  const int ntiles = (ntok + 63) >> 6;
  uint8_t* pbase = reinterpret_cast<uint8_t*>(&sbuf[0][0][0]);

  qkv_v4i acc2[RC][MTW][NP];
#pragma unroll
  for (int c = 0; c < RC; ++c)
#pragma unroll
    for (int mi = 0; mi < MTW; ++mi)
#pragma unroll
      for (int s = 0; s < NP; ++s) acc2[c][mi][s] = qkv_v4i{0, 0, 0, 0};
  // V plane words of the next PD2 tiles are in flight in a register ring.
  const int blk = lg >> 1, hsh = 4 * (lg & 1);
  constexpr int PD2 = MTW * VB * RC > 6 ? 4 : 6;
  uint32_t vw[PD2][MTW][VB];
  auto load2 = [&](int slot, int tt) {
    const int64_t vt = (tile_row(tt) >> 5) + blk;  // 32-token V tile
#pragma unroll
    for (int mi = 0; mi < MTW; ++mi) {
      const int j = 16 * (wave * MTW + mi) + ln;
#pragma unroll
      for (int k = 0; k < VB; ++k) vw[slot][mi][k] = vst[(vt * VB + k) * D + j];
    }
  };
  auto pv2 = [&](int slot, int tt) {
    qkv_v4i bq[RC];
#pragma unroll
    for (int c = 0; c < RC; ++c)
      bq[c] = *reinterpret_cast<const qkv_v4i*>(pbase + (tt * RC + c) * 1024 + ln * 64 + lg * 16);
#pragma unroll
    for (int mi = 0; mi < MTW; ++mi) {
#pragma unroll
      for (int s = 0; s < NP; ++s) {
        const uint32_t sub = odd_subset(VB, s);
        uint32_t pw = 0;
#pragma unroll
        for (int k = 0; k < VB; ++k)
          if (sub & (1u << k)) pw ^= vw[slot][mi][k];
        qkv_v4i av;
        av[0] = static_cast<int>(pw & (0x01010101u << hsh));
        av[1] = static_cast<int>(pw & (0x02020202u << hsh));
        av[2] = static_cast<int>(pw & (0x04040404u << hsh));
        av[3] = static_cast<int>(pw & (0x08080808u << hsh));
#pragma unroll
        for (int c = 0; c < RC; ++c)  // C[row x digit][coordinate]
          acc2[c][mi][s] = mfma_i8(bq[c], av, acc2[c][mi][s]);
      }
    }
  };
  // the first value tiles are in flight during phase 1.5
#pragma unroll
  for (int d = 0; d < PD2; ++d)
    if (d < ntiles) load2(d, d);

  // Row w's digits of tile tt occupy exactly the 256 bytes that held row w's
  // scores of that tile, and one wave's LDS operations execute in order, so
  // each wave converts its rows in place without a barrier.  Tokens past the
  // split end hold -inf scores and zero norms (phase 1 writes whole tiles).
  // token (lane) of a 64-token tile -> K position of the value MFMA:
  // lane = 32 blk + 8 beta + i, K = 16 (2 blk + i / 4) + 4 (i % 4) + beta
  const int ii = lane & 7;
  const int kpos = 16 * (2 * (lane >> 5) + (ii >> 2)) + 4 * (ii & 3) + ((lane & 31) >> 3);
  const float zscale = ldexpf(1.f, Fv - ii);  // Z_t s_t = X 2^i, X = round(p' 2^(Fv - i))
#pragma unroll
  for (int c = 0; c < RC; ++c) {
    const int row = kRowsM * c + wave;
    const float m_q = fmaxf(fmaxf(red_m[0][row], red_m[1][row]),
                            fmaxf(red_m[2][row], red_m[3][row]));
    const bool live = row < nr && m_q > -INFINITY;
    const float m_use = live ? m_q : INFINITY;  // absent row: every p = 0
    float lsum = 0.f;
    int64_t xsum = 0;
    for (int tt = 0; tt < ntiles; ++tt) {
      const float p = __builtin_amdgcn_exp2f(sbuf[tt][row][lane] - m_use);
      lsum += p;
      const float pv = p * vn[tt * 64 + lane];
      const int X = static_cast<int>(fmaf(pv, zscale, 0.5f));
      xsum += X;
      const int Z = ii == 7 ? -X : X;
      // signed base-256 digits: byte v of (Z + 0x808080) ^ 0x808080
      const uint32_t dg = (static_cast<uint32_t>(Z) + 0x808080u) ^ 0x808080u;
      uint8_t* dst = pbase + (tt * RC + c) * 1024 + (4 * wave) * 64 + kpos;
      dst[0] = static_cast<uint8_t>(dg);
      dst[64] = static_cast<uint8_t>(dg >> 8);
      dst[128] = static_cast<uint8_t>(dg >> 16);
      dst[192] = static_cast<uint8_t>(dg >> 24);
    }
    lsum = wave_sum_dpp(lsum);
    // sum_t Z_t s_t: what an all-ones plane would accumulate (this lane's
    // tokens all share i = lane % 8)
    const int64_t usum = wave_sum_i64(xsum << ii);
    if (lane == 0) {
      lsum_s[row] = lsum;
      usum_s[row] = usum;
    }
  }
  __syncthreads();

  for (int tt0 = 0; tt0 < ntiles; tt0 += PD2) {
#pragma unroll
    for (int d = 0; d < PD2; ++d) {
      const int tt = tt0 + d;
      if (tt < ntiles) {
        pv2(d, tt);
        if (tt + PD2 < ntiles) load2(d, tt + PD2);
      }
    }
  }

  // ---------------- epilogue: digits + planes -> fp32, write the partials
  // Lane (g = lane / 16, c = lane % 16) holds, per chunk, 16-coordinate tile
  // and plane S, the four digit accumulators of row g at coordinate c.
  // Y_S = sum_v 2^(8v) acc_S[v] = sum_t Z_t s_t phi_S,t exactly (int64), and
  // sum_t p'_t (2 phi_S,t - 1) = 2^-Fv (2 Y_S - U) is formed in integers
  // before the only rounding: O = 2^-Fv sum_S g_S (2 Y_S - U).
  mfma_settle();
  const float oscale = ldexpf(1.f, -Fv);
  const int64_t base = ((int64_t(split) * gridDim.z + b) * Hkv + hkv) * R + r0;
#pragma unroll
  for (int c = 0; c < RC; ++c) {
    const int row = kRowsM * c + lg;
    const int64_t urow = usum_s[row];
#pragma unroll
    for (int mi = 0; mi < MTW; ++mi) {
      float val = 0.f;
#pragma unroll
      for (int s = 0; s < NP; ++s) {
        const int64_t y = static_cast<int64_t>(acc2[c][mi][s][0]) +
                          (static_cast<int64_t>(acc2[c][mi][s][1]) << 8) +
                          (static_cast<int64_t>(acc2[c][mi][s][2]) << 16) +
                          (static_cast<int64_t>(acc2[c][mi][s][3]) << 24);
        val = fmaf(tb.vg[s], static_cast<float>(2 * y - urow), val);
      }
      if (row < nr) part_o[(base + row) * D + 16 * (wave * MTW + mi) + ln] = val * oscale;
    }
  }
  if (tid < nr) {
    const float mq = fmaxf(fmaxf(red_m[0][tid], red_m[1][tid]), fmaxf(red_m[2][tid], red_m[3][tid]));
    part_ml[(base + tid) * 2 + 0] = mq * 0.6931471805599453f;  // log2 -> natural units
    part_ml[(base + tid) * 2 + 1] = lsum_s[tid];
  }
}

// ------------------------------------------------------------ fused decode, d = 128 / 96
//
// The whole decode step at head_dim 128 or 96 (IP keys of MSE bits 1-3, the
// two mixed-precision key formats, value bits 1-4, symmetric codebooks) in
// one kernel.  A workgroup of 16 waves takes one (sequence, kv head, chunk of
// 4 query rows) over a range of tokens (a split) and streams it in chunks of
// kChunkF tokens through a two-stage pipeline:
//   key waves (0-7) score chunk c -- one 64-token tile each, the fp8 x fp4
//     scaled MFMA on the K bit planes (operands described above) -- into
//     LDS, and once the chunk's row maxima are known turn those scores into
//     the int8 digit operands of the value product, in place;
//   value waves (8-15) meanwhile accumulate chunk c - 1's value product for 16
//     coordinates each (integer MFMA on the V bit planes, plus one product
//     with an all-ones plane for the constant term) and merge it into a
//     running fp32 (m, l, O~) per row: exact integers within a chunk, online
//     softmax across chunks.
// Each stage keeps its next chunk's K rows / V plane words in flight in
// registers (nontemporal loads), so both HBM streams run while the other
// stage computes; two workgroup barriers per chunk hand the LDS buffers over.
// The query rotation and digit operands (prepare_mfma's work) run in the
// prologue while the first chunk's loads are in flight.  With one split per
// row group the epilogue divides by max(l, 1e-8) and un-rotates by Pi
// (combine_kernel's work), so a decode step is a single launch; otherwise
// the workgroup writes split partials for combine_kernel.
constexpr int kChunkF = 512;              // tokens per pipeline chunk
constexpr int kTilesF = kChunkF / 64;     // 64-token tiles per chunk (one per key wave)
constexpr int kWavesKF = kTilesF;         // key waves
constexpr int kThreadsF = 64 * 2 * kWavesKF;  // key waves + as many value waves
constexpr int kVSplitF = 6;               // value tiles before the mid-chunk barrier

struct ChunkStats {
  float pmax[kWavesKF][4];   // [key wave][row] score maxima (log2 units)
  float pvmax[kWavesKF];     // [key wave] value norm maxima
  float scale[4];            // [row] 2^(m_prev - m_new): the running sums' rescale
  int fv;                    // the value digits' fixed-point exponent
  int pad[3];
};

// Dynamic LDS of decode_fused (byte offsets).  The prologue's and the
// epilogue's scratch rows overlay the chunk buffers.
struct FusedLds {
  static constexpr int PR4 = (128 + 4) / 4;             // padded Pi row, float4
  static constexpr int PI = 0;                          // Pi [128][PR4]
  static constexpr int STAGE = PI + 128 * PR4 * 16;     // query operand image
  static constexpr int STAGE_BYTES = 10 * 1024;         // up to five fp4 MFMAs per 16 tokens
  static constexpr int BUF = STAGE + STAGE_BYTES;       // [2][kTilesF][1 KiB] scores / digits
  static constexpr int STATS = BUF + 2 * kTilesF * 1024;
  static constexpr int ROWC = STATS + 2 * int(sizeof(ChunkStats));  // [4][2] row constants
  static constexpr int RED = ROWC + 32;                 // [8] norms, [8][2] row sums
  static constexpr int LRED = RED + 128;                // [8 key waves][4 rows] sums of p
  static constexpr int TOTAL = LRED + 128;
  static_assert(BUF % 16 == 0 && STATS % 16 == 0, "alignment");
};

// aq_ws == nullptr: the prologue computes the query operands (Tables tb,
// ql); else they come from prepare_mfma's workspace (aq_ws, rowc_ws).
// final_out != 0 and one split: write the attention output through ol;
// else split partials (part_o, part_ml) for combine_kernel.
// PAGED: the store is a page pool addressed through kv.ptab.
template <int RDW, int VB, bool PAGED, int DS>
__global__ __launch_bounds__(kThreadsF, 1) void decode_fused(
    QLayers ql, KVLayers kv, OutLayers ol, int Bl, int q_dtype, float alpha, int Hq, int Hkv,
    int Q, int R, int chunks, Tables tb, int64_t t_stride, int64_t T, float scale, int causal,
    int64_t split_len, int final_out, int out_dtype, const qkv_v4i* __restrict__ aq_ws,
    const float* __restrict__ rowc_ws, float* __restrict__ part_o, float* __restrict__ part_ml) {
  // DS: the stored head dim, 128, 96 or 64; the operands are 128 wide, the
  // coordinates past DS zero (query, Pi and S padded in the prologue)
  constexpr int D = 128;
  static_assert(DS == 128 || DS == 96 || DS == 64, "stored head dim");
  constexpr int PD = DS / 32;  // dwords per stored plane
  // K rows of RDW dwords: IP keys PD (mbits + 1) (MSE planes + QJL plane), at
  // d = 128 also the mixed-key formats of 9, 10 or 12 dwords (the Tables
  // comment).  Plane-major (PMAJ) rows: 3 MSE bits (weighing four virtual MSE
  // planes b0, b1, b2, b0^b1^b2) or d = 96.
  constexpr bool PMAJ = DS != 128 || RDW == 16;
  constexpr int NPS = PMAJ ? RDW / PD : 0;    // stored planes of a plane-major row
  constexpr bool PAR = PMAJ && NPS == 4;      // 3 MSE bits: the parity plane is computed
  constexpr int MB = PMAJ ? (PAR ? 4 : NPS - 1) : RDW / 4 - 1;  // IP keys: weighted MSE planes
  constexpr int KRB = 4 * RDW;                 // K row bytes
  // fp4 MFMAs per 16 tokens = (virtual) row dwords per lane group
  constexpr int DPL = PMAJ ? MB + 1 : (RDW + 3) / 4;
  constexpr int NLD = PMAJ ? NPS : DPL;        // row dwords a lane loads per token
  static_assert(!PMAJ || NPS * PD == RDW, "whole planes");
  constexpr int NU = 2 * DPL;                  // operand image: NU x 256 dwords
  constexpr int NP = n_odd_subsets(VB);  // value planes
  constexpr int PR4 = FusedLds::PR4;
  constexpr int NT = kThreadsF;
  static_assert(NU * 1024 <= FusedLds::STAGE_BYTES, "operand image");
  static_assert(NT == 1024 && kWavesKF == 8, "layout below assumes 8 + 8 waves");

  extern __shared__ __align__(16) uint8_t lds[];
  float4* pis = reinterpret_cast<float4*>(lds + FusedLds::PI);
  uint32_t* stage = reinterpret_cast<uint32_t*>(lds + FusedLds::STAGE);
  uint8_t* bufs = lds + FusedLds::BUF;
  ChunkStats* stats = reinterpret_cast<ChunkStats*>(lds + FusedLds::STATS);
  float* rowcs = reinterpret_cast<float*>(lds + FusedLds::ROWC);
  float* red = reinterpret_cast<float*>(lds + FusedLds::RED);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 15, lg = lane >> 4;
  const int G = Hq / Hkv;
  const int split = blockIdx.x;
  const int hkv = blockIdx.y / chunks, cki = blockIdx.y - hkv * chunks;
  const int bz = blockIdx.z;  // over the batch of all layers
  const int layer = bz / Bl, b = bz - layer * Bl;
  const int r0 = cki * kRowsM;
  const int nr = min(kRowsM, R - r0);
  const int64_t bh = int64_t(b) * Hkv + hkv;  // in the layer's store
  const int64_t ts = int64_t(split) * split_len;
  const int64_t te = min<int64_t>(T, ts + split_len);
  const int ntok = te > ts ? static_cast<int>(te - ts) : 0;
  const int ntiles = (ntok + 63) >> 6;
  const int nch = (ntiles + kTilesF - 1) / kTilesF;
  const uint8_t* __restrict__ kst = kv.kst[layer];
  const float* __restrict__ knorm = kv.knorm[layer];
  const uint32_t* __restrict__ vst = kv.vst[layer];
  const float* __restrict__ vnorm = kv.vnorm[layer];
  const bool keyw = wave < kWavesKF;
  const int wi = wave & (kWavesKF - 1);  // index within the key or value waves

  // First store row of the split's 64-token tile (contiguous stream, or the
  // tile's page).  Whole tiles stay inside the capacity / page.  Every ring
  // load is issued unconditionally -- a tile past the split's last re-reads
  // the last one (an empty split reads its stream's first tile) and its data
  // goes unused -- so each step issues a fixed number of loads and the
  // in-order load counter waits only for the slot being consumed.
  const int64_t lts = ntiles > 0 ? ts : 0;
  const int64_t srow0 = bh * t_stride + lts;  // contiguous: the split's first row
  // PAGED: the page entries of a chunk's kTilesF tiles come from one vector
  // load per wave (lane l: the entry of tile l % kTilesF of chunk ch), a
  // chunk ahead of their use (chunks 0 and 1 before the prologue), and a tile
  // takes its entry with a lane read: no scalar load, whose wait would also
  // drain the wave's LDS reads in flight, sits in the kernel.  Tiles past the
  // split's last take the last tile's page (they are masked).
  auto chunk_pages = [&](int ch) -> int32_t {
    if constexpr (PAGED) {
      const int t = ntiles > 0 ? min(ch * kTilesF + (lane & (kTilesF - 1)), ntiles - 1) : 0;
      const int gt = static_cast<int>(lts >> 6) + t;
      return kv.ptab[int64_t(b) * kv.pmax + (gt >> (kv.plg - 6))];
    } else {
      return 0;
    }
  };
  // the value waves' per-lane form: lane l's word offset of the V tiles of
  // tile l % kTilesF of chunk ch (entries pe), taken per tile with two lane
  // reads
  auto chunk_voffs = [&](int32_t pe, int ch) -> int64_t {
    const int t = ntiles > 0 ? min(ch * kTilesF + (lane & (kTilesF - 1)), ntiles - 1) : 0;
    const int tsh = kv.plg - 6;
    const int gt = static_cast<int>(lts >> 6) + t;
    const int pg = pe >= 0 && pe < kv.npages ? pe : 0;  // outside the pool: page 0
    const int64_t row = ((int64_t(pg) * Hkv + hkv) << kv.plg) + ((gt & ((1 << tsh) - 1)) << 6);
    return (row >> 5) * (VB * DS);
  };
  // first store row of tile `tile` of the chunk whose entries chunk_pages
  // gave (pe); ok: the tile lies on a page of the pool
  auto tile_row_pe = [&](int32_t pe, int tile, bool& ok) -> int64_t {
    const int tc = ntiles > 0 ? min(tile, ntiles - 1) : 0;
    const int tsh = kv.plg - 6;
    const int gt = static_cast<int>(lts >> 6) + tc;
    int pg = __builtin_amdgcn_readlane(pe, tile & (kTilesF - 1));
    ok = pg >= 0 && pg < kv.npages;
    if (!ok) pg = 0;  // outside the pool: read page 0, masked
    return ((int64_t(pg) * Hkv + hkv) << kv.plg) + ((gt & ((1 << tsh) - 1)) << 6);
  };

  const int32_t pe0 = chunk_pages(0);  // (PAGED) chunk 0's entries
  int32_t pe1 = chunk_pages(1);        // (PAGED) chunk 1's

  // ---- prologue loads (land in LDS before the first chunk's loads are issued)
  const bool pro = aq_ws == nullptr;
  const int pj = tid & (D - 1), ppart = tid >> 7;  // coordinate, part 0..7
  float* qs = reinterpret_cast<float*>(bufs);              // [4][D] query rows
  float* partb = reinterpret_cast<float*>(bufs + 2048);    // [2 k halves][4 rows][D]
  float* sgns = reinterpret_cast<float*>(bufs + 6144);     // [D] QJL signs
  if (pro) {
    // Pi comes from L2 (every workgroup reads it)
    const float4* src = reinterpret_cast<const float4*>(ql.pi[layer]);
    float4 pst[4];
#pragma unroll
    for (int x = 0; x < 4; ++x) pst[x] = pi_f4<DS>(src, tid + NT * x);
    float qv = 0.f;
    if (ppart < nr && pj < DS) {
      const int row = r0 + ppart;
      const int g = row / Q, qi = row - g * Q;
      const int h = hkv * G + g;
      qv = qkv_load(ql.q[layer], ((int64_t(b) * Hq + h) * Q + qi) * DS + pj, q_dtype);
    }
    const float sgn = pj < DS ? ql.signs[layer][pj] : 0.f;
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      const int i = tid + NT * x, row = i >> 5, c4 = i & 31;
      pis[row * PR4 + c4] = pst[x];
    }
    if (ppart < kRowsM) qs[ppart * D + pj] = qv;
    if (ppart == 0) sgns[pj] = sgn;
    if constexpr (!PMAJ && RDW % 4 != 0) {  // operand bytes no row dword feeds stay zero
#pragma unroll
      for (int x = 0; x < (NU * 256 + NT - 1) / NT; ++x)
        if (tid + NT * x < NU * 256) stage[tid + NT * x] = 0u;
    }
  } else {
    // operands and row constants from prepare_mfma's workspace
    const int64_t bhc = (int64_t(bz) * Hkv + hkv) * chunks + cki;
    const uint32_t* src = reinterpret_cast<const uint32_t*>(aq_ws) + bhc * NU * 256;
    uint32_t w[(NU * 256 + NT - 1) / NT];
#pragma unroll
    for (int x = 0; x < (NU * 256 + NT - 1) / NT; ++x)
      if (tid + NT * x < NU * 256) w[x] = src[tid + NT * x];
    const float rc = tid < 2 * kRowsM ? rowc_ws[bhc * kRowsM * 2 + tid] : 0.f;
#pragma unroll
    for (int x = 0; x < (NU * 256 + NT - 1) / NT; ++x)
      if (tid + NT * x < NU * 256) stage[tid + NT * x] = w[x];
    if (tid < 2 * kRowsM) rowcs[tid] = rc;
  }

  // ---- first chunk's loads (registers)
  uint32_t kd[4][NLD];
  float kn[4], vnr = 0.f;
  uint32_t vw[kTilesF][VB];
  const int blk = lg >> 1, hsh = 4 * (lg & 1);
  const int vj = 16 * wi + ln;  // value wave: coordinate of this lane
  // per-tile bases are wave-uniform; lanes add fixed 32-bit offsets
  // bytes into a tile's K rows (PMAJ: dword lg of each plane; lane group 3 of
  // a 96-dim row re-reads group 2's, under zero operand bytes)
  const uint32_t koff = ln * KRB + (PMAJ ? min(lg, PD - 1) : krow_base<DPL, RDW>(lg)) * 4;
  // words into a tile's V planes (coordinates past DS read coordinate DS - 1
  // and give zero)
  const uint32_t voff = blk * VB * DS + min(vj, DS - 1);
  // contiguous store: the split's bases, a tile as a 32-bit row offset from them
  const uint8_t* kbase = kst + srow0 * KRB;
  const float* knbase = knorm + srow0;
  const float* vnbase = vnorm + srow0;
  const uint32_t* vbase = vst + (srow0 >> 5) * (VB * DS);  // srow0 is a multiple of 64
  auto trow = [&](int tile) -> uint32_t {
    return ntiles > 0 ? static_cast<uint32_t>(min(tile, ntiles - 1)) * 64u : 0u;
  };
  // (PAGED: prb is the tile's first store row)
  auto loadK = [&](int tile, int64_t prb) {
    const uint8_t* kb;
    const float* knb;
    const float* vnb;
    if constexpr (PAGED) {
      const int64_t rb = prb;
      kb = kst + rb * KRB;
      knb = knorm + rb;
      vnb = vnorm + rb;
    } else {
      const uint32_t r = trow(tile);
      kb = kbase + r * KRB;
      knb = knbase + r;
      vnb = vnbase + r;
    }
#pragma unroll
    for (int sub = 0; sub < 4; ++sub) {
      const uint32_t* krow = reinterpret_cast<const uint32_t*>(kb + koff + sub * 16 * KRB);
#pragma unroll
      for (int x = 0; x < NLD; ++x) kd[sub][x] = ldnt(krow + (PMAJ ? PD * x : x));
      kn[sub] = ldnt(knb + sub * 16 + ln);
    }
    vnr = ldnt(vnb + lane);
  };
  // (PAGED: pvo is the word offset of the tile's first V tile)
  auto loadV = [&](int slot, int tile, int64_t pvo) {
    const uint32_t* vb;  // the tile's first V tile
    if constexpr (PAGED)
      vb = vst + pvo;
    else
      vb = vbase + (trow(tile) >> 5) * (VB * DS);
#pragma unroll
    for (int k = 0; k < VB; ++k) vw[slot][k] = ldnt(vb + voff + k * DS);
  };
  bool pok0 = true;  // (key waves) tile wi lies on a page of the pool
  if (keyw) {
    loadK(wi, PAGED ? tile_row_pe(pe0, wi, pok0) : 0);
  } else {
    const int64_t vof = PAGED ? chunk_voffs(pe0, 0) : 0;
#pragma unroll
    for (int t = 0; t < kTilesF; ++t) loadV(t, t, PAGED ? readlane_i64(vof, t) : 0);
  }

  // ---- prologue math: q~ = q Pi^T, operand digits (prepare_mfma on 1024 threads)
  if (pro) {
    lds_sync();
    if (ppart < kRowsM) {  // ||q_r||^2: row r = waves 2r, 2r + 1
      const float qv = qs[ppart * D + pj];
      const float ss = wave_sum_dpp(qv * qv);
      if (lane == 0) red[wave] = ss;
    }
    {  // thread (j, r, k half): row r's partial dot product over k in [64 kh, 64 kh + 64)
      const int r = ppart & 3, kh = ppart >> 2;
      float acc = 0.f;
#pragma unroll
      for (int k4 = 0; k4 < 16; ++k4) {
        const float4 p4 = pis[pj * PR4 + 16 * kh + k4];
        const float4 q4 = reinterpret_cast<const float4*>(qs + r * D)[16 * kh + k4];
        acc = fmaf(q4.x, p4.x, acc);
        acc = fmaf(q4.y, p4.y, acc);
        acc = fmaf(q4.z, p4.z, acc);
        acc = fmaf(q4.w, p4.w, acc);
      }
      partb[(kh * kRowsM + r) * D + pj] = acc;
    }
    float kgmax = alpha;
    if (tb.kmix) {
#pragma unroll
      for (int r = 0; r < 4; ++r) kgmax = fmaxf(kgmax, fabsf(tb.kgo[r]));
      kgmax = fmaxf(kgmax, fmaxf(fabsf(tb.kgr[0]), fabsf(tb.kgr[1])));
    } else {  // IP keys
#pragma unroll
      for (int r = 0; r < MB; ++r) kgmax = fmaxf(kgmax, fabsf(tb.kg[r]));
    }
    lds_sync();
    if (ppart < kRowsM) {  // thread (j, r): coordinate j of row r into digit bytes
      const int r = ppart;
      const float v = partb[(0 * kRowsM + r) * D + pj] + partb[(1 * kRowsM + r) * D + pj];
      const float w = alpha * fabsf(v) * sgns[pj];
      const float wmax = 2.f * kgmax * sqrtf(red[2 * r] + red[2 * r + 1]);
      const int sig = kf4_sigma(wmax);
      uint8_t* sb = reinterpret_cast<uint8_t*>(stage);
      float hf = 0.f;  // this coordinate's share of the row constant (bit class 3)
      const float csq = key_weights<MB>(tb, pj, v, w, [&](int p, float W) {
        hf += kf4_put<DPL, RDW, PMAJ>(sb, p, W, sig, r);
      });
      // row constants: sums over j (row r = waves 2r, 2r + 1) into red[8 ..]
      const float a = wave_sum_dpp(csq);
      const float c = wave_sum_dpp(w);
      const float h = wave_sum_dpp(hf);
      if (lane == 0) {
        red[8 + 2 * wave] = a;
        red[8 + 2 * wave + 1] = c;
        red[24 + wave] = h;
      }
    }
    lds_sync();
    if (tid < kRowsM) {  // row tid: score = kn (z + const) in log2 units
      const int rr = tid;
      const float sq = red[8 + 4 * rr] + red[8 + 4 * rr + 2];
      const float sw = red[8 + 4 * rr + 1] + red[8 + 4 * rr + 3];
      const float sh = red[24 + 2 * rr] + red[24 + 2 * rr + 1];
      const float wm = 2.f * kgmax * sqrtf(red[2 * rr] + red[2 * rr + 1]);
      rowcs[2 * rr + 0] = (tb.kmix ? sq - sw : tb.kconst * sq - sw) + sh;
      rowcs[2 * rr + 1] = static_cast<float>(kf4_sigma(wm));  // the row's sigma
    }
  }
  lds_sync();

  const float scale2 = scale * 1.4426950408889634f;  // scores in log2 units
  float* lred = reinterpret_cast<float*>(lds + FusedLds::LRED);  // [key wave][row] sums of p
  float orun = 0.f;  // value waves: row lg, coordinate vj, relative to the running maximum

  if (keyw) {
    // ------------------------------------------------ key waves: tile wi of each chunk
    const uint32_t k88 = vgpr_u32(0x88888888u), k11 = vgpr_u32(0x11111111u);
    // fp8 digit operands of the score MFMAs, one per K-row dword of a lane group
    qkv_v8i a[DPL];
#pragma unroll
    for (int u = 0; u < DPL; ++u) a[u] = *reinterpret_cast<const qkv_v8i*>(stage + (u * 64 + lane) * 8);
    const float cr2 = rowcs[2 * lg] * scale2;
    // E8M0 scale of this lane's operand row ln = 4 r + d: 2^(sigma_r - 4 d)
    const int asc = 127 + static_cast<int>(rowcs[2 * (ln >> 2) + 1]) - 4 * (ln & 3);
    const bool row_ok = lg < nr;
    // the sequence's attended keys, split-relative: [slo, shi)
    const SeqRange sr = seq_range(kv, b, T);
    const int slo = static_cast<int>(min<int64_t>(ntok, max<int64_t>(0, sr.lo - ts)));
    const int shi = static_cast<int>(min<int64_t>(ntok, max<int64_t>(0, sr.hi - ts)));
    // causal: split-relative token tl is visible to row lg iff tl <= clim
    const int qi = (r0 + lg) % Q;
    const int64_t climit = causal ? (sr.cpos - Q + qi - ts) : int64_t(INT_MAX);
    const int clim = static_cast<int>(max<int64_t>(-1, min<int64_t>(climit, INT_MAX)));
    int cmin = INT_MAX;  // the smallest limit over the valid rows (wave-uniform)
    if (causal) {
#pragma unroll
      for (int r = 0; r < kRowsM; ++r) {
        if (r < nr) {
          const int q2 = (r0 + r) % Q;
          cmin = static_cast<int>(min<int64_t>(cmin, max<int64_t>(-1, sr.cpos - Q + q2 - ts)));
        }
      }
    }
    const int ii = lane & 7;
    // token (lane) of a 64-token tile -> K position of the value MFMA:
    // lane = 32 blk + 8 beta + i, K = 16 (2 blk + i / 4) + 4 (i % 4) + beta
    const int kpos = 16 * (2 * (lane >> 5) + (ii >> 2)) + 4 * (ii & 3) + ((lane & 31) >> 3);
    // Z_t s_t = X 2^i with X = round(p' 2^(Fv - i)); the byte of bit 7 is -128,
    // so those lanes store -X: sign and rounding offset fold into constants
    const float sgn7 = ii == 7 ? -1.f : 1.f;
    // the chunk's maxima, one per lane: (key wave l & 7, row l >> 3) for lanes
    // 0..31, the value-norm maximum of key wave l & 7 for lanes 32..
    const int sidx = lane < 32 ? (lane & 7) * kRowsM + (lane >> 3) : kWavesKF * kRowsM + (lane & 7);
    // running row maxima (log2 units, floored so that a row without a visible
    // token yet gives p = 0 rather than NaN) and this lane's running sums of p
    float mk[kRowsM], lacc[kRowsM];
#pragma unroll
    for (int r = 0; r < kRowsM; ++r) {
      mk[r] = kMFloor;
      lacc[r] = 0.f;
    }
    bool pok = pok0;  // tile wi of chunk c lies on a page of the pool
    for (int c = 0; c < nch; ++c) {
      uint8_t* cbuf = bufs + (c & 1) * kTilesF * 1024;
      ChunkStats& cs = stats[c & 1];
      const int tile = c * kTilesF + wi;
      const int32_t pe2 = chunk_pages(c + 2);
      // ---- stage 1: scores of tile wi of chunk c.  A tile past the split's
      // last (only in the last chunk) runs on the re-read last tile and is
      // masked out whole: its scores are -inf, so its p and value digits are 0.
      qkv_v4f acc[4];
#pragma unroll
      for (int u = 0; u < DPL; ++u) {
#pragma unroll
        for (int sub = 0; sub < 4; ++sub) {
          // PAR: planes b0, b1, b2, their parity, QJL
          const uint32_t x = !PAR ? kd[sub][u < NLD ? u : 0]
                             : u < 3   ? kd[sub][u]
                             : u == 3  ? kd[sub][0] ^ kd[sub][1] ^ kd[sub][2]
                                       : kd[sub][3];
          qkv_v8i bo;  // 32 fp4 elements (4 dwords) by bit class
          bo[0] = static_cast<int>(x & 0x11111111u);
          bo[1] = static_cast<int>(x & 0x22222222u);
          bo[2] = static_cast<int>(x & 0x44444444u);
          bo[3] = static_cast<int>((x & k88) | k11);
          bo[4] = bo[5] = bo[6] = bo[7] = 0;
          acc[sub] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              a[u], bo, u == 0 ? qkv_v4f{0.f, 0.f, 0.f, 0.f} : acc[sub], 0, 4, 0, asc, 0, 127);
        }
      }
      float knt[4];
#pragma unroll
      for (int sub = 0; sub < 4; ++sub) knt[sub] = kn[sub];
      float vz = vnr;
      bool pokn = true;
      const int64_t rbn = PAGED ? tile_row_pe(pe1, tile + kTilesF, pokn) : 0;
      loadK(tile + kTilesF, rbn);  // the slot is free: refill it
      mfma_settle();
      const int tbase = tile * 64;
      const bool full = pok && tbase >= slo && tbase + 64 <= shi && nr == kRowsM &&
                        tbase + 63 <= cmin;
      float* srow = reinterpret_cast<float*>(cbuf + wi * 1024 + lg * 256);
      float mloc = -INFINITY;
#pragma unroll
      for (int sub = 0; sub < 4; ++sub) {
        // the four digit rows of row lg, already scaled: z = sum of them
        const float z = (acc[sub][0] + acc[sub][1]) + (acc[sub][2] + acc[sub][3]);
        float sc = knt[sub] * fmaf(z, scale2, cr2);
        if (!full) {
          const int tl = tbase + sub * 16 + ln;
          sc = (pok && tl >= slo && tl < shi && row_ok && tl <= clim) ? sc : -INFINITY;
        }
        srow[sub * 16 + ln] = sc;
        mloc = fmaxf(mloc, sc);
      }
      if (!full) vz = (pok && tbase + lane >= slo && tbase + lane < shi) ? vz : 0.f;
      mloc = row_max_last(mloc);  // the 16 lanes of row lg: max in lane 15
      const float vloc = wave_max_dpp(vz);
      if (ln == 15) cs.pmax[wi][lg] = mloc;
      if (lane == 0) cs.pvmax[wi] = vloc;
      lds_sync();
      // ---- stage 2: new running maxima; p = 2^(s - m), value digits in place
      const float t = max8_dpp(reinterpret_cast<const float*>(&cs)[sidx]);
      float mrow[kRowsM];
#pragma unroll
      for (int r = 0; r < kRowsM; ++r) {
        const float Mc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t), 8 * r));
        mrow[r] = fmaxf(mk[r], Mc);
        const float rs = __builtin_amdgcn_exp2f(mk[r] - mrow[r]);  // 2^(m_prev - m_new)
        lacc[r] *= rs;
        mk[r] = mrow[r];
        if (wi == 0 && lane == 0) cs.scale[r] = rs;
      }
      const float vmx = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t), 32));
      int ev = 0;
      if (vmx > 0.f) frexpf(vmx, &ev);
      const int Fv = vmx > 0.f ? 29 - ev : 0;  // vmx 2^Fv < 2^29
      if (wi == 0 && lane == 0) cs.fv = Fv;
      const float vzs = vz * ldexpf(sgn7, Fv - ii);
      const float hz = 0.5f * sgn7;
      uint8_t* tb8 = cbuf + wi * 1024;
#pragma unroll
      for (int r = 0; r < kRowsM; ++r) {
        const float s = reinterpret_cast<const float*>(tb8 + r * 256)[lane];
        const float p = __builtin_amdgcn_exp2f(s - mrow[r]);
        lacc[r] += p;
        const int Z = static_cast<int>(fmaf(p, vzs, hz));
        // signed base-256 digits: byte v of (Z + 0x808080) ^ 0x808080
        const uint32_t dg = (static_cast<uint32_t>(Z) + 0x808080u) ^ 0x808080u;
        const uint32_t dg8 = dg >> 8;
        uint8_t* dst = tb8 + (4 * r) * 64 + kpos;
        dst[0] = static_cast<uint8_t>(dg);
        dst[64] = static_cast<uint8_t>(dg8);
        dst[128] = static_cast<uint8_t>(dg >> 16);
        dst[192] = static_cast<uint8_t>(dg8 >> 16);
      }
      pok = pokn;
      pe1 = pe2;
      lds_sync();
    }
    // the step in which the value waves take the last chunk
    lds_sync();
    lds_sync();
    // the key waves' sums of p meet in LDS (read after the next barrier)
#pragma unroll
    for (int r = 0; r < kRowsM; ++r) {
      const float l = wave_sum_dpp(lacc[r]);
      if (lane == 0) lred[wi * kRowsM + r] = l;
    }
    if (!(final_out && gridDim.x == 1)) {
      lds_sync();
      if (wi == 0 && lane < nr) {  // split partials: (m, l) of row `lane`
        float l = lred[lane];
#pragma unroll
        for (int w = 1; w < kWavesKF; ++w) l += lred[w * kRowsM + lane];
        const float m = lane == 0 ? mk[0] : lane == 1 ? mk[1] : lane == 2 ? mk[2] : mk[3];
        const int64_t base = ((int64_t(split) * gridDim.z + bz) * Hkv + hkv) * R + r0;
        part_ml[(base + lane) * 2 + 0] = m * 0.6931471805599453f;  // log2 -> natural units
        part_ml[(base + lane) * 2 + 1] = l;
      }
    }
  } else {
    // ------------------------------------------------ value waves: coordinates 16 wi ..
    qkv_v4i acc[NP], accU;
    qkv_v4i ones;  // an all-ones plane as the operand's bytes (b * 2^i, i = bit in byte)
#pragma unroll
    for (int e = 0; e < 4; ++e) ones[e] = static_cast<int>(0x01010101u << (e + hsh));
    // the digit operand of tile t of a chunk buffer
    auto ldbq = [&](const uint8_t* vbuf, int t) {
      return *reinterpret_cast<const qkv_v4i*>(vbuf + t * 1024 + ln * 64 + lg * 16);
    };
    // the first tile of a chunk starts the accumulators from zero
    auto pv = [&](int slot, qkv_v4i bq, bool first) {
      const qkv_v4i zero = qkv_v4i{0, 0, 0, 0};
#pragma unroll
      for (int s = 0; s < NP; ++s) {
        const uint32_t sub = odd_subset(VB, s);
        uint32_t pw = 0;
#pragma unroll
        for (int k = 0; k < VB; ++k)
          if (sub & (1u << k)) pw ^= vw[slot][k];
        qkv_v4i av;
        av[0] = static_cast<int>(pw & (0x01010101u << hsh));
        av[1] = static_cast<int>(pw & (0x02020202u << hsh));
        av[2] = static_cast<int>(pw & (0x04040404u << hsh));
        av[3] = static_cast<int>(pw & (0x08080808u << hsh));
        acc[s] = mfma_i8(bq, av, first ? zero : acc[s]);  // C[row x digit][coordinate]
      }
      accU = mfma_i8(bq, ones, first ? zero : accU);
    };
    // step 0: the ring holds chunk 0; nothing to accumulate yet
    lds_sync();
    lds_sync();
    for (int c = 1; c <= nch; ++c) {
      const int cv = c - 1;  // the chunk this stage accumulates
      const int32_t pe2 = chunk_pages(c + 1);
      const int64_t vof = PAGED ? chunk_voffs(pe1, c) : 0;  // the tiles loaded below
      const uint8_t* vbuf = bufs + (cv & 1) * kTilesF * 1024;
      // slot t is refilled with tile t of the next chunk once consumed; tiles
      // past the split's last are zero digits over re-read planes.  The digit
      // operands are read one tile ahead (the buffer was completed in the
      // previous step).
      qkv_v4i bqn = ldbq(vbuf, 0);
#pragma unroll
      for (int t = 0; t < kVSplitF; ++t) {
        // one tile at a time: operations of later tiles hoisted above would wait
        // on the in-order load counter for every load in flight
        __builtin_amdgcn_sched_barrier(0);
        const qkv_v4i bq = bqn;
        bqn = ldbq(vbuf, t + 1);
        pv(t, bq, t == 0);
        loadV(t, c * kTilesF + t, PAGED ? readlane_i64(vof, t) : 0);
      }
      lds_sync();
#pragma unroll
      for (int t = kVSplitF; t < kTilesF; ++t) {
        __builtin_amdgcn_sched_barrier(0);
        const qkv_v4i bq = bqn;
        if (t + 1 < kTilesF) bqn = ldbq(vbuf, t + 1);
        pv(t, bq, false);
        loadV(t, c * kTilesF + t, PAGED ? readlane_i64(vof, t) : 0);
      }
      pe1 = pe2;
      {
        // chunk cv into the running O~: sum_t p'_t (2 phi_S,t - 1) = 2^-Fv (2 Y_S - U)
        // per digit half in exact int32 (|acc| < 2^21 for a 512-token chunk),
        // then fp32; O~ = O~ 2^(m_prev - m_new) + sum_S g_S (...)
        mfma_settle();
        const ChunkStats& cs = stats[cv & 1];
        const float rs = cs.scale[lg];
        const int Fv = cs.fv;
        const int nulo = -(__mul24(accU[1], 256) + accU[0]);
        const int nuhi = -(__mul24(accU[3], 256) + accU[2]);
        float val = 0.f;
#pragma unroll
        for (int s = 0; s < NP; ++s) {
          const int lo = 2 * (__mul24(acc[s][1], 256) + acc[s][0]) + nulo;
          const int hi = 2 * (__mul24(acc[s][3], 256) + acc[s][2]) + nuhi;
          const float y = fmaf(static_cast<float>(hi), 65536.f, static_cast<float>(lo));
          val = fmaf(tb.vg[s], y, val);
        }
        orun = fmaf(orun, rs, ldexpf(val, -Fv));
      }
      lds_sync();
    }
    if (!(final_out && gridDim.x == 1)) {
      lds_sync();
      const int64_t base = ((int64_t(split) * gridDim.z + bz) * Hkv + hkv) * R + r0;
      if (lg < nr && vj < DS) part_o[(base + lg) * DS + vj] = orun;
    }
  }

  // ---------------------------------------------------------------- epilogue
  if (final_out && gridDim.x == 1) {
    // out = (O~ / max(l, 1e-8)) Pi_v, rows r0 .. r0 + nr - 1
    float* obuf = reinterpret_cast<float*>(bufs);            // [4][D]
    float* opart = reinterpret_cast<float*>(bufs + 2048);    // [4 k parts][4 rows][D]
    lds_sync();  // the key waves' sums of p
    if (!keyw) {
      float l = lred[lg];
#pragma unroll
      for (int w = 1; w < kWavesKF; ++w) l += lred[w * kRowsM + lg];
      obuf[lg * D + vj] = lg < nr && vj < DS ? orun / fmaxf(l, 1e-8f) : 0.f;
    }
    const float* piv = ol.pi[layer];
    if (!pro || piv != ql.pi[layer]) {  // values un-rotate by their own Pi
      const float4* src = reinterpret_cast<const float4*>(piv);
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        const int i = tid + NT * x, row = i >> 5, c4 = i & 31;
        pis[row * PR4 + c4] = pi_f4<DS>(src, i);
      }
    }
    lds_sync();
    if (tid < 512) {  // thread (j4, r, kp): columns 4 j4 .. + 3 of row r, k in [32 kp, 32 kp + 32)
      const int j4 = tid & 31, r = (tid >> 5) & 3, kp = tid >> 7;
      float4 o4 = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 8
      for (int k = 32 * kp; k < 32 * kp + 32; ++k) {
        const float o = obuf[r * D + k];
        const float4 p4 = pis[k * PR4 + j4];
        o4.x = fmaf(o, p4.x, o4.x);
        o4.y = fmaf(o, p4.y, o4.y);
        o4.z = fmaf(o, p4.z, o4.z);
        o4.w = fmaf(o, p4.w, o4.w);
      }
      reinterpret_cast<float4*>(opart)[(kp * kRowsM + r) * (D / 4) + j4] = o4;
    }
    lds_sync();
    if (tid < 512) {
      const int r = tid >> 7, j = tid & (D - 1);
      if (r < nr && j < DS) {
        const float o = (opart[(0 * kRowsM + r) * D + j] + opart[(1 * kRowsM + r) * D + j]) +
                        (opart[(2 * kRowsM + r) * D + j] + opart[(3 * kRowsM + r) * D + j]);
        const int row = r0 + r;
        const int g = row / Q, qi = row - g * Q;
        const int h = hkv * G + g;
        qkv_store(ol.out[layer], ((int64_t(b) * Hq + h) * Q + qi) * DS + j, o, out_dtype);
      }
    }
  }
}

// ------------------------------------------------------------ small decode, d = 64
//
// The decode step at head_dim 64 (IP keys of 1-2 MSE bits, value bits 1-4,
// symmetric codebooks) over many short sequences -- a model's layers in one
// call -- as one launch.  A workgroup of 4 waves takes one (sequence, kv
// head, RC chunks of 4 query rows) over a split of its tokens:
//   prologue: q~ = q Pi^T and the int8 digit operands of the scores
//     (prepare_mfma's work, the same operand layout) for its 4 RC rows;
//   then chunks of 256 tokens, two workgroup barriers each:
//     A  wave w scores tile w of the chunk on the integer MFMA (split_mfma's
//        plane operands) into LDS, with the tile's row and value-norm maxima;
//     B  the running row maxima; wave w turns rows w, w + 4 of the chunk's
//        scores into p = 2^(s - m) and the value product's int8 digits (a
//        per-chunk fixed point), in place;
//     C  wave w accumulates the chunk's value product for coordinates
//        16 w .. 16 w + 15 (exact integers) and merges it into its running
//        fp32 O~: online softmax across chunks;
//   the next chunk's K rows load during A..C and its V planes during C, the
//   scores alternate between two LDS buffers;
//   epilogue: with one split, O~ / max(l, 1e-8) un-rotated by Pi into the
//   output; otherwise split partials for combine_kernel.
// With one split per (sequence, kv head) a 24-layer cfg2 batch is one round
// of workgroups (three per CU), each streaming its 2,048 tokens.
constexpr int kChunkS = 256;  // tokens per chunk: one 64-token tile per wave

template <int MB, int VB, int RC, bool PAGED>
__global__ __launch_bounds__(256, 3) void decode_small(
    QLayers ql, KVLayers kv, OutLayers ol, int Bl, int q_dtype, float alpha, int Hq, int Hkv,
    int Q, int R, int cgroups, Tables tb, int64_t t_stride, int64_t T, float scale, int causal,
    int64_t split_len, int final_out, int out_dtype, float* __restrict__ part_o,
    float* __restrict__ part_ml) {
  constexpr int D = 64;
  constexpr int NPL = MB + 1;            // K-row planes: MSE bits, QJL
  constexpr int KRB = NPL * D / 8;       // K row bytes
  constexpr int NU = NPL;                // score MFMAs per 16 tokens
  constexpr int NP = n_odd_subsets(VB);  // value planes
  constexpr int RW = kRowsM * RC;        // query rows per workgroup
  constexpr int PR = D + 4;              // padded Pi row (floats)
  static_assert(MB == 1 || MB == 2, "key MSE bits");
  static_assert(RC == 1 || RC == 2, "row chunks");

  __shared__ __align__(16) float pis[D * PR];          // Pi rows (query side, then values')
  __shared__ __align__(16) float qs[RW][D];            // query rows; O~ / l in the epilogue
  __shared__ __align__(16) uint32_t stage[RC * NU * 256];  // score operand image
  __shared__ __align__(16) float sbuf[2][4][RW][64];   // scores -> value digits, per chunk
  __shared__ float vns[2][kChunkS];                     // value norms of the chunk's tokens
  __shared__ float red_m[4][RW];
  __shared__ float red_v[4];
  __shared__ float rowcs[RW][2];                        // score row constants
  __shared__ float rsc[RW], mls[RW][2];
  __shared__ int fvs;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 15, lg = lane >> 4;
  const int G = Hq / Hkv;
  const int split = blockIdx.x;
  const int hkv = blockIdx.y / cgroups, cgi = blockIdx.y - hkv * cgroups;
  const int bz = blockIdx.z;  // over the batch of all layers
  const int layer = bz / Bl, b = bz - layer * Bl;
  const int r0 = cgi * RW;
  const int nr = min(RW, R - r0);
  const int64_t bh = int64_t(b) * Hkv + hkv;  // in the layer's store
  const int64_t ts = int64_t(split) * split_len;
  const int64_t te = min<int64_t>(T, ts + split_len);
  const int ntok = te > ts ? static_cast<int>(te - ts) : 0;
  const int ntile = (ntok + 63) >> 6;
  const int nch = (ntok + kChunkS - 1) / kChunkS;
  const uint8_t* __restrict__ kst = kv.kst[layer];
  const float* __restrict__ knorm = kv.knorm[layer];
  const uint32_t* __restrict__ vst = kv.vst[layer];
  const float* __restrict__ vnorm = kv.vnorm[layer];

  // ---- prologue: Pi and the query rows into LDS
  {
    const float4* src = reinterpret_cast<const float4*>(ql.pi[layer]);
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      const int i = tid + 256 * x, row = i >> 4, c4 = i & 15;
      reinterpret_cast<float4*>(pis + row * PR)[c4] = src[i];
    }
#pragma unroll
    for (int x = 0; x < RC; ++x) {
      const int i = tid + 256 * x, r = i >> 6, j = i & 63;
      float v = 0.f;
      if (r < nr) {
        const int row = r0 + r;
        const int g = row / Q, qi = row - g * Q;
        v = qkv_load(ql.q[layer], ((int64_t(b) * Hq + hkv * G + g) * Q + qi) * D + j, q_dtype);
      }
      qs[r][j] = v;
    }
  }
  // the first chunk's loads fly during the prologue's arithmetic
  typedef const __attribute__((address_space(4))) int32_t* ctab_t;
  auto tile_row = [&](int tile) -> int64_t {  // first store row of the split's tile
    const int tc = ntile > 0 ? min(tile, ntile - 1) : 0;
    if constexpr (PAGED) {
      const ctab_t ptab = (ctab_t)kv.ptab;
      const int tsh = kv.plg - 6;
      const int gt = static_cast<int>(ts >> 6) + tc;
      int pg = ptab[int64_t(b) * kv.pmax + (gt >> tsh)];
      if (pg < 0 || pg >= kv.npages) pg = 0;  // outside the pool: read page 0, masked
      return ((int64_t(pg) * Hkv + hkv) << kv.plg) + ((gt & ((1 << tsh) - 1)) << 6);
    } else {
      return bh * t_stride + ts + int64_t(tc) * 64;
    }
  };
  auto page_ok = [&](int tile) -> bool {
    if constexpr (PAGED) {
      const ctab_t ptab = (ctab_t)kv.ptab;
      const int gt = static_cast<int>(ts >> 6) + tile;
      const int pg = ptab[int64_t(b) * kv.pmax + (gt >> (kv.plg - 6))];
      return pg >= 0 && pg < kv.npages;
    } else {
      return true;
    }
  };
  // per-tile bases are wave-uniform; lanes add fixed 32-bit offsets
  uint32_t kd[4][NU];
  float kn[4], vv[4];
  const uint32_t koff = ln * (KRB / 4) + (lg >> 1);  // dwords into a tile's K rows
  auto loadK = [&](int tile) {
    const int64_t rb = tile_row(tile);
    const uint32_t* kb = reinterpret_cast<const uint32_t*>(kst + rb * KRB);
    const float* knb = knorm + rb;
    const float* vnb = vnorm + rb;
#pragma unroll
    for (int sub = 0; sub < 4; ++sub) {
#pragma unroll
      for (int u = 0; u < NU; ++u) kd[sub][u] = ldnt(kb + koff + sub * 16 * (KRB / 4) + 2 * u);
      kn[sub] = ldnt(knb + sub * 16 + ln);
      vv[sub] = ldnt(vnb + sub * 16 + ln);
    }
  };
  const int blk = lg >> 1, hsh = 4 * (lg & 1);
  const int vj = 16 * wave + ln;  // this lane's value coordinate
  const uint32_t voff = blk * VB * D + vj;  // words into a tile's V planes
  uint32_t vw[4][VB];
  auto loadV = [&](int slot, int tile) {
    const uint32_t* vb = vst + (tile_row(tile) >> 5) * (VB * D);  // the tile's first V tile
#pragma unroll
    for (int k = 0; k < VB; ++k) vw[slot][k] = ldnt(vb + voff + k * D);
  };
  if (nch > 0) {
    loadK(wave);
#pragma unroll
    for (int t = 0; t < 4; ++t) loadV(t, t);
  }
  __syncthreads();

  // ---- prologue math: q~, the digit operands and row constants (wave w: rows w, w + 4)
  float kgmax = alpha;
#pragma unroll
  for (int r = 0; r < MB; ++r) kgmax = fmaxf(kgmax, fabsf(tb.kg[r]));
  const float sgn = ql.signs[layer][lane];
  uint8_t* sb = reinterpret_cast<uint8_t*>(stage);
#pragma unroll
  for (int c = 0; c < RC; ++c) {
    const int r = kRowsM * c + wave;
    const float qj = qs[r][lane];
    const float nq = wave_sum_dpp(qj * qj);
    float v = 0.f;  // q~_j = sum_k q_k Pi[j][k], j = lane
    const float4* prow = reinterpret_cast<const float4*>(pis + lane * PR);
#pragma unroll
    for (int k4 = 0; k4 < D / 4; ++k4) {
      const float4 p4 = prow[k4];
      const float4 q4 = reinterpret_cast<const float4*>(qs[r])[k4];
      v = fmaf(q4.x, p4.x, v);
      v = fmaf(q4.y, p4.y, v);
      v = fmaf(q4.z, p4.z, v);
      v = fmaf(q4.w, p4.w, v);
    }
    const float w = alpha * fabsf(v) * sgn;
    const float wmax = 2.f * kgmax * sqrtf(nq);
    int ex = 0;
    if (wmax > 0.f) frexpf(wmax, &ex);
    const int fq = wmax > 0.f ? 30 - ex : 0;  // |Z| < 2^30
    // digit bytes of weight W at row bit p (the operand layout of prepare_mfma, D = 64)
    auto put8 = [&](int p, float W) {
      const int i = p & 7;
      int Z = static_cast<int>(rintf(ldexpf(W, fq - i)));
      if (i == 7) Z = -Z;
      const uint32_t dg = (static_cast<uint32_t>(Z) + 0x808080u) ^ 0x808080u;
      const int w32 = p >> 5, e = i & 3, beta = (p >> 3) & 3;
      const int g = 2 * (w32 & 1) + (i >> 2), u = w32 >> 1;
      const int base = c * NU * 1024 + ((u * 64 + 16 * g + 4 * wave) * 4 + e) * 4 + beta;
#pragma unroll
      for (int dv = 0; dv < 4; ++dv) sb[base + 16 * dv] = static_cast<uint8_t>(dg >> (8 * dv));
    };
#pragma unroll
    for (int pl = 0; pl < MB; ++pl) put8(pl * D + lane, 2.f * tb.kg[pl] * v);
    put8(MB * D + lane, 2.f * w);
    const float sq = wave_sum_dpp(v);
    const float sw = wave_sum_dpp(w);
    if (lane == 0) {
      rowcs[r][0] = tb.kconst * sq - sw;
      rowcs[r][1] = ldexpf(1.f, -fq);
    }
  }
  __syncthreads();
  // the score operands stay in LDS (read back each chunk: registers)
  const qkv_v4i* aop = reinterpret_cast<const qkv_v4i*>(stage) + lane;
  float cr[RC], fqs[RC], mrun[RC], lrun[RC], orun[RC];
  bool row_ok[RC];
  int clim[RC];
#pragma unroll
  for (int c = 0; c < RC; ++c) {
    const int rl = kRowsM * c + lg;  // this lane's row in the score phase
    cr[c] = rowcs[rl][0];
    fqs[c] = rowcs[rl][1];
    row_ok[c] = rl < nr;
    const int qi = (r0 + rl) % Q;
    const int64_t climit = causal ? (T - Q + qi - ts) : int64_t(INT_MAX);
    clim[c] = static_cast<int>(max<int64_t>(-1, min<int64_t>(climit, INT_MAX)));
    mrun[c] = kMFloor;  // phase B: rows wave + 4 c
    lrun[c] = 0.f;
    orun[c] = 0.f;      // phase C: rows lg + 4 c, coordinate vj
  }
  const float scale2 = scale * 1.4426950408889634f;  // scores in log2 units
  const int ii = lane & 7;
  // token (lane) of a 64-token tile -> K position of the value MFMA:
  // lane = 32 blk + 8 beta + i, K = 16 (2 blk + i / 4) + 4 (i % 4) + beta
  const int kpos = 16 * (2 * (lane >> 5) + (ii >> 2)) + 4 * (ii & 3) + ((lane & 31) >> 3);

  for (int ch = 0; ch < nch; ++ch) {
    const int buf = ch & 1;
    // ---- A: scores of tile `wave` of the chunk
    const int tile = ch * 4 + wave;
    {
      qkv_v4i acc[RC][4];
#pragma unroll
      for (int c = 0; c < RC; ++c)
#pragma unroll
        for (int sub = 0; sub < 4; ++sub) acc[c][sub] = qkv_v4i{0, 0, 0, 0};
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        qkv_v4i au[RC];
#pragma unroll
        for (int c = 0; c < RC; ++c) au[c] = aop[(c * NU + u) * 64];
#pragma unroll
        for (int sub = 0; sub < 4; ++sub) {
          const uint32_t x = kd[sub][u];
          qkv_v4i bo;
          bo[0] = static_cast<int>(x & (0x01010101u << hsh));
          bo[1] = static_cast<int>(x & (0x02020202u << hsh));
          bo[2] = static_cast<int>(x & (0x04040404u << hsh));
          bo[3] = static_cast<int>(x & (0x08080808u << hsh));
#pragma unroll
          for (int c = 0; c < RC; ++c) acc[c][sub] = mfma_i8(au[c], bo, acc[c][sub]);
        }
      }
      float knt[4], vvt[4];
#pragma unroll
      for (int sub = 0; sub < 4; ++sub) {
        knt[sub] = kn[sub];
        vvt[sub] = vv[sub];
      }
      if (ch + 1 < nch) loadK(tile + 4);  // the slot is free: the next chunk's tile
      mfma_settle();
      const bool pin = tile < ntile && page_ok(ntile > 0 ? min(tile, ntile - 1) : 0);
      float mloc[RC], vmax = 0.f;
#pragma unroll
      for (int c = 0; c < RC; ++c) mloc[c] = -INFINITY;
#pragma unroll
      for (int sub = 0; sub < 4; ++sub) {
        const int tl = tile * 64 + sub * 16 + ln;
        const bool in = pin && tl < ntok;
#pragma unroll
        for (int c = 0; c < RC; ++c) {
          // digits in two exact int32 halves (|acc| < 2^21), one rounding each
          const int zlo = __mul24(acc[c][sub][1], 256) + acc[c][sub][0];
          const int zhi = __mul24(acc[c][sub][3], 256) + acc[c][sub][2];
          const float z = fmaf(static_cast<float>(zhi), 65536.f, static_cast<float>(zlo));
          const float sc0 = knt[sub] * scale2 * fmaf(z, fqs[c], cr[c]);
          const float sc = (in & row_ok[c] & (tl <= clim[c])) ? sc0 : -INFINITY;
          sbuf[buf][wave][kRowsM * c + lg][sub * 16 + ln] = sc;
          mloc[c] = fmaxf(mloc[c], sc);
        }
        const float vz = in ? vvt[sub] : 0.f;
        vns[buf][wave * 64 + sub * 16 + ln] = vz;  // the four lane groups store the same value
        vmax = fmaxf(vmax, vz);
      }
#pragma unroll
      for (int c = 0; c < RC; ++c) {
        mloc[c] = row_max_last(mloc[c]);  // the 16 lanes of a row: max in lane 15
        if (ln == 15) red_m[wave][kRowsM * c + lg] = mloc[c];
      }
      vmax = wave_max_dpp(vmax);
      if (lane == 0) red_v[wave] = vmax;
    }
    __syncthreads();
    // ---- B: running maxima, p = 2^(s - m) and value digits of rows wave + 4 c
    {
      const float vmx = fmaxf(fmaxf(red_v[0], red_v[1]), fmaxf(red_v[2], red_v[3]));
      int ev = 0;
      if (vmx > 0.f) frexpf(vmx, &ev);
      const int Fv = vmx > 0.f ? 29 - ev : 0;  // vmx 2^Fv < 2^29
      const float zscale = ldexpf(1.f, Fv - ii);  // Z_t s_t = X 2^i, X = round(p' 2^(Fv - i))
      uint8_t* pbase = reinterpret_cast<uint8_t*>(&sbuf[buf][0][0][0]);
#pragma unroll
      for (int c = 0; c < RC; ++c) {
        const int row = kRowsM * c + wave;
        const float mc = fmaxf(fmaxf(red_m[0][row], red_m[1][row]),
                               fmaxf(red_m[2][row], red_m[3][row]));
        const float mnew = fmaxf(mrun[c], mc);
        const float rs = __builtin_amdgcn_exp2f(mrun[c] - mnew);
        mrun[c] = mnew;
        float lsum = 0.f;
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
          const float p = __builtin_amdgcn_exp2f(sbuf[buf][tt][row][lane] - mnew);
          lsum += p;
          const int X = static_cast<int>(fmaf(p * vns[buf][tt * 64 + lane], zscale, 0.5f));
          const int Z = ii == 7 ? -X : X;
          // signed base-256 digits: byte v of (Z + 0x808080) ^ 0x808080
          const uint32_t dg = (static_cast<uint32_t>(Z) + 0x808080u) ^ 0x808080u;
          uint8_t* dst = pbase + (tt * RC + c) * 1024 + (4 * wave) * 64 + kpos;
          dst[0] = static_cast<uint8_t>(dg);
          dst[64] = static_cast<uint8_t>(dg >> 8);
          dst[128] = static_cast<uint8_t>(dg >> 16);
          dst[192] = static_cast<uint8_t>(dg >> 24);
        }
        lsum = wave_sum_dpp(lsum);
        lrun[c] = fmaf(lrun[c], rs, lsum);
        if (lane == 0) rsc[row] = rs;
      }
      if (tid == 0) fvs = Fv;
    }
    __syncthreads();
    // ---- C: the chunk's value product for coordinate vj, merged into O~
    {
      const uint8_t* pbase = reinterpret_cast<const uint8_t*>(&sbuf[buf][0][0][0]);
      qkv_v4i ones;  // an all-ones plane as the operand's bytes (b * 2^i, i = bit in byte)
#pragma unroll
      for (int e = 0; e < 4; ++e) ones[e] = static_cast<int>(0x01010101u << (e + hsh));
      qkv_v4i acc2[RC][NP], accU[RC];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        qkv_v4i bq[RC];
#pragma unroll
        for (int c = 0; c < RC; ++c)
          bq[c] = *reinterpret_cast<const qkv_v4i*>(pbase + (tt * RC + c) * 1024 + ln * 64 + lg * 16);
#pragma unroll
        for (int s = 0; s < NP; ++s) {
          const uint32_t subs = odd_subset(VB, s);
          uint32_t pw = 0;
#pragma unroll
          for (int k = 0; k < VB; ++k)
            if (subs & (1u << k)) pw ^= vw[tt][k];
          qkv_v4i av;
          av[0] = static_cast<int>(pw & (0x01010101u << hsh));
          av[1] = static_cast<int>(pw & (0x02020202u << hsh));
          av[2] = static_cast<int>(pw & (0x04040404u << hsh));
          av[3] = static_cast<int>(pw & (0x08080808u << hsh));
#pragma unroll
          for (int c = 0; c < RC; ++c)  // C[row x digit][coordinate]
            acc2[c][s] = mfma_i8(bq[c], av, tt == 0 ? qkv_v4i{0, 0, 0, 0} : acc2[c][s]);
        }
#pragma unroll
        for (int c = 0; c < RC; ++c)
          accU[c] = mfma_i8(bq[c], ones, tt == 0 ? qkv_v4i{0, 0, 0, 0} : accU[c]);
        if (ch + 1 < nch) loadV(tt, (ch + 1) * 4 + tt);
      }
      // sum_t p'_t (2 phi_S,t - 1) = 2^-Fv (2 Y_S - U) per digit half in exact
      // int32 (|acc| < 2^20 for a 256-token chunk), then fp32
      mfma_settle();
      const float oscale = ldexpf(1.f, -fvs);
#pragma unroll
      for (int c = 0; c < RC; ++c) {
        const int row = kRowsM * c + lg;
        const int nulo = -(__mul24(accU[c][1], 256) + accU[c][0]);
        const int nuhi = -(__mul24(accU[c][3], 256) + accU[c][2]);
        float val = 0.f;
#pragma unroll
        for (int s = 0; s < NP; ++s) {
          const int lo = 2 * (__mul24(acc2[c][s][1], 256) + acc2[c][s][0]) + nulo;
          const int hi = 2 * (__mul24(acc2[c][s][3], 256) + acc2[c][s][2]) + nuhi;
          val = fmaf(tb.vg[s], fmaf(static_cast<float>(hi), 65536.f, static_cast<float>(lo)), val);
        }
        orun[c] = fmaf(orun[c], rsc[row], val * oscale);
      }
    }
  }

  // ---- epilogue: (m, l) of rows wave + 4 c to LDS, then output or partials
#pragma unroll
  for (int c = 0; c < RC; ++c) {
    if (lane == 0) {
      mls[kRowsM * c + wave][0] = mrun[c];
      mls[kRowsM * c + wave][1] = lrun[c];
    }
  }
  __syncthreads();
  if (final_out && gridDim.x == 1) {
    // out = (O~ / max(l, 1e-8)) Pi_v
#pragma unroll
    for (int c = 0; c < RC; ++c) {
      const int row = kRowsM * c + lg;
      qs[row][vj] = row < nr ? orun[c] / fmaxf(mls[row][1], 1e-8f) : 0.f;
    }
    const float* piv = ol.pi[layer];
    if (piv != ql.pi[layer]) {
      const float4* src = reinterpret_cast<const float4*>(piv);
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        const int i = tid + 256 * x, row = i >> 4, c4 = i & 15;
        reinterpret_cast<float4*>(pis + row * PR)[c4] = src[i];
      }
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < RC; ++c) {
      const int r = kRowsM * c + wave;
      if (r < nr) {
        float o = 0.f;
#pragma unroll 16
        for (int k = 0; k < D; ++k) o = fmaf(qs[r][k], pis[k * PR + lane], o);
        const int row = r0 + r;
        const int g = row / Q, qi = row - g * Q;
        qkv_store(ol.out[layer], ((int64_t(b) * Hq + hkv * G + g) * Q + qi) * D + lane, o,
                  out_dtype);
      }
    }
  } else {
    const int64_t base = ((int64_t(split) * gridDim.z + bz) * Hkv + hkv) * R + r0;
#pragma unroll
    for (int c = 0; c < RC; ++c) {
      const int row = kRowsM * c + lg;
      if (row < nr) part_o[(base + row) * D + vj] = orun[c];
    }
    if (tid < nr) {
      part_ml[(base + tid) * 2 + 0] = mls[tid][0] * 0.6931471805599453f;  // log2 -> natural units
      part_ml[(base + tid) * 2 + 1] = mls[tid][1];
    }
  }
}

// ------------------------------------------------------------ combine

constexpr int kRowsC = 4;       // query rows merged per block (many rows)

// Merge the split partials of RPB consecutive query rows (of the B*Hkv*R
// rows): log-sum-exp over splits, / max(l, 1e-8), un-rotate with Pi, store
// with the GQA mapping (query head h = hkv * G + r / Q).  2*D threads as
// (j4, sp): coordinates 4 j4 .. 4 j4 + 3 and split lane sp of 8.
//   1. lane sp merges splits sp, sp + 8, ... of every row (float4 partial
//      loads, BATCH splits per row in flight);
//   2. the 8 lane results meet in LDS: thread (j, half) finishes coordinate j
//      of rows half, half + 2, ...;
//   3. thread (j4, kr) applies Pi rows [kr D/8, (kr+1) D/8) to output columns
//      4 j4 .. 4 j4 + 3 from float4 loads issued at kernel entry; the eight
//      k-range sums meet in LDS.
// RPB = 4 shares each Pi load among 4 rows; RPB = 1 spreads few rows with
// many splits over more workgroups.
template <int D, int RPB>
__global__ __launch_bounds__(2 * D) void combine_kernel(const float* __restrict__ part_o,
                                                        const float* __restrict__ part_ml,
                                                        OutLayers ol, int n_splits, int Bl,
                                                        int Hkv, int R, int Q, int Hq,
                                                        int out_dtype) {
  constexpr int JG = D / 4, KPER = D / 8, NSP = 8;
  constexpr int BATCH = RPB == 1 ? 8 : 2;  // splits per row per load round
  __shared__ float o[RPB][D];
  __shared__ float4 red[NSP][RPB][JG];
  __shared__ float2 mls[NSP][RPB];
  const int tid = threadIdx.x;
  const int layer = blockIdx.y;
  const float* __restrict__ pi = ol.pi[layer];
  void* __restrict__ out = ol.out[layer];
  const int64_t nrl = int64_t(Bl) * Hkv * R;           // rows of one layer
  const int64_t nrows = nrl * gridDim.y;               // rows of the partials
  const int64_t row0 = int64_t(blockIdx.x) * RPB;      // in the layer
  const int64_t grow0 = int64_t(layer) * nrl + row0;   // in the partials
  const int nr = static_cast<int>(min<int64_t>(RPB, nrl - row0));

  const int j4 = tid % JG, kr = tid / JG;  // kr doubles as the split lane
  float4 pv[KPER];
  const float4* pk = reinterpret_cast<const float4*>(pi + int64_t(kr) * KPER * D) + j4;
#pragma unroll
  for (int i = 0; i < KPER; ++i) pv[i] = pk[i * JG];

  {  // 1. per-lane merge
    float M[RPB], L[RPB];
    float4 a[RPB];
#pragma unroll
    for (int r = 0; r < RPB; ++r) {
      M[r] = -INFINITY;
      L[r] = 0.f;
      a[r] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const float2* ml2 = reinterpret_cast<const float2*>(part_ml);
    const float4* o4 = reinterpret_cast<const float4*>(part_o);
    for (int s0 = kr; s0 < n_splits; s0 += NSP * BATCH) {
      float2 mlb[BATCH][RPB];
      float4 ob[BATCH][RPB];
#pragma unroll
      for (int x = 0; x < BATCH; ++x) {
        const int sidx = s0 + NSP * x;
#pragma unroll
        for (int r = 0; r < RPB; ++r) {
          const bool ok = sidx < n_splits && r < nr;
          const int64_t base = int64_t(ok ? sidx : 0) * nrows + (ok ? grow0 + r : 0);
          mlb[x][r] = ok ? ml2[base] : make_float2(-INFINITY, 0.f);
          ob[x][r] = ok ? o4[base * JG + j4] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
#pragma unroll
      for (int r = 0; r < RPB; ++r) {
        float bm = M[r];
#pragma unroll
        for (int x = 0; x < BATCH; ++x) bm = fmaxf(bm, mlb[x][r].x);
        if (bm != -INFINITY) {
          const float c = (M[r] == -INFINITY) ? 0.f : expf(M[r] - bm);
          L[r] *= c;
          a[r].x *= c;
          a[r].y *= c;
          a[r].z *= c;
          a[r].w *= c;
#pragma unroll
          for (int x = 0; x < BATCH; ++x) {
            if (mlb[x][r].x != -INFINITY) {
              const float w = expf(mlb[x][r].x - bm);
              L[r] = fmaf(w, mlb[x][r].y, L[r]);
              a[r].x = fmaf(w, ob[x][r].x, a[r].x);
              a[r].y = fmaf(w, ob[x][r].y, a[r].y);
              a[r].z = fmaf(w, ob[x][r].z, a[r].z);
              a[r].w = fmaf(w, ob[x][r].w, a[r].w);
            }
          }
          M[r] = bm;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < RPB; ++r) {
      red[kr][r][j4] = a[r];
      if (j4 == 0) mls[kr][r] = make_float2(M[r], L[r]);
    }
  }
  __syncthreads();
  const int j = tid % D, half = tid / D;
  {  // 2. merge the lanes
#pragma unroll
    for (int rr = 0; rr < (RPB + 1) / 2; ++rr) {
      const int r = half + 2 * rr;
      if (r < RPB) {
        float mx = -INFINITY;
#pragma unroll
        for (int k = 0; k < NSP; ++k) mx = fmaxf(mx, mls[k][r].x);
        float L = 0.f, a = 0.f;
        if (mx != -INFINITY) {
          const float* redf = reinterpret_cast<const float*>(&red[0][r][0]);
#pragma unroll
          for (int k = 0; k < NSP; ++k) {
            const float w = mls[k][r].x == -INFINITY ? 0.f : expf(mls[k][r].x - mx);
            L = fmaf(w, mls[k][r].y, L);
            a = fmaf(w, redf[k * RPB * D + j], a);
          }
        }
        o[r][j] = r < nr ? a / fmaxf(L, 1e-8f) : 0.f;
      }
    }
  }
  __syncthreads();
  {  // 3. un-rotate
    float4 acc[RPB];
#pragma unroll
    for (int r = 0; r < RPB; ++r) acc[r] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < KPER; ++i) {
#pragma unroll
      for (int r = 0; r < RPB; ++r) {
        const float ov = o[r][kr * KPER + i];
        acc[r].x = fmaf(ov, pv[i].x, acc[r].x);
        acc[r].y = fmaf(ov, pv[i].y, acc[r].y);
        acc[r].z = fmaf(ov, pv[i].z, acc[r].z);
        acc[r].w = fmaf(ov, pv[i].w, acc[r].w);
      }
    }
#pragma unroll
    for (int r = 0; r < RPB; ++r) red[kr][r][j4] = acc[r];
  }
  __syncthreads();
  const int G = Hq / Hkv;
  const float* redf = reinterpret_cast<const float*>(&red[0][0][0]);
#pragma unroll
  for (int rr = 0; rr < (RPB + 1) / 2; ++rr) {
    const int r = half + 2 * rr;
    if (r < nr) {
      float v = 0.f;
#pragma unroll
      for (int k = 0; k < NSP; ++k) v += redf[(k * RPB + r) * D + j];
      const int64_t row = row0 + r;  // in the layer: ((b * Hkv) + hkv) * R + r
      const int rq = static_cast<int>(row % R);
      const int hkv = static_cast<int>((row / R) % Hkv);
      const int b = static_cast<int>(row / (int64_t(R) * Hkv));
      const int g = rq / Q, qi = rq - g * Q;
      qkv_store(out, ((int64_t(b) * Hq + hkv * G + g) * Q + qi) * D + j, v, out_dtype);
    }
  }
}

// ------------------------------------------------------------ MIPS search

// QuashIndex.search (quashkv/nn_search/index.py:121-163): for each query q and
// database vector x (K row + norm), score = n_x (<q~, c[code]> + alpha
// sum_j |q~_j| S_j (2 b_j - 1)), no 1/sqrt(d); then the k largest scores per
// query (descending; equal scores: lower index first).
//
// The scores are the decode kernel's integer MFMA dot products (same query
// operands from prepare_mfma), with the database row bits as the B operand.
// A workgroup (4 waves) takes 16 QC queries (QC chunks of 4 per wave) and a
// range of vectors; the 128 rows of each step are staged once in LDS and every
// wave expands them against its own query operands, held in registers.  Each
// wave keeps a sorted top-k list per query in LDS; a score enters only if it
// beats the list's k-th (a ballot finds the rare candidates).  Lists go to the
// workspace per (query, vector split) and mips_merge picks the final k.
constexpr int kMipsStep = 128;  // vectors staged per workgroup step (13.2 ms at cfg5; 64: 14.1)
constexpr int kMipsKMax = 256;

// Order-preserving float <-> uint32 map, for a device-wide running maximum
// (atomicMax on the image) of each query's k-th best score.
__device__ __forceinline__ uint32_t fkey(float f) {
  const uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b ^ 0x80000000u);
}
__device__ __forceinline__ float fkey_inv(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k ^ 0x80000000u) : ~k);
}

template <int MB, int PDW>
struct MipsCfg {
  static constexpr int NS = n_odd_subsets(MB);  // MSE planes of the virtual row
  static constexpr int NPL = NS + 1;            // + QJL plane
  static constexpr int RAWD = (MB + 1) * PDW;   // stored row dwords (PDW = d / 32)
  static constexpr int DPL = NPL;               // virtual dwords per lane group
  static constexpr int NU = 2 * DPL;            // MFMAs per 16 vectors and chunk
  static constexpr int QC = MB <= 2 ? 4 : 2;    // query chunks (of 4) per wave
};

// Rows of d < 128 (PDW = d / 32 dwords per plane) run as 128-wide rows whose
// missing plane words are zero, against queries padded with zeros.  Two
// workgroups per CU: the query operands (QC x NU x 4 registers), two groups'
// accumulators and the pipelined expansion need more than a third of the
// register file without spills.
template <int MB, int PDW>
__global__ __launch_bounds__(256, 2) void mips_scan(const qkv_v4i* __restrict__ aq,
                                                 const float* __restrict__ rowc, int M,
                                                 const uint8_t* __restrict__ kst,
                                                 const float* __restrict__ norms, int64_t N,
                                                 int nvc, int64_t vlen, int64_t n_items, int k,
                                                 float* __restrict__ cand_s,
                                                 int* __restrict__ cand_i,
                                                 uint32_t* __restrict__ gth) {
  using C = MipsCfg<MB, PDW>;
  constexpr int NU = C::NU, QC = C::QC, RAWD = C::RAWD;
  constexpr int QW = 4 * QC;                      // queries per wave
  constexpr int SD = kMipsStep * RAWD;            // row dwords per step
  constexpr int LPT = (SD + 255) / 256;           // row dwords each thread stages
  extern __shared__ __align__(16) float smem_ms[];
  uint32_t* rows = reinterpret_cast<uint32_t*>(smem_ms);           // [2][64][RAWD]
  float* nrm_s = smem_ms + 2 * kMipsStep * RAWD;                    // [2][kMipsStep]
  float* ls = nrm_s + 2 * kMipsStep;                                // [4][QW][k] scores
  int* li = reinterpret_cast<int*>(ls + 4 * QW * k);                // [4][QW][k] indices

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ln = lane & 15, lg = lane >> 4;
  const int nchunks = (M + 3) / 4;
  float* wls = ls + wave * QW * k;
  int* wli = li + wave * QW * k;
  const uint32_t* kw = reinterpret_cast<const uint32_t*>(kst);
  // this lane's virtual row dwords lg*DPL + x: up to three stored dwords
  // (offsets within a row) XORed, a zero mask where the plane word is absent
  // (d < 128) -- precomputed so the row loop has no divergent branches
  constexpr int NT = MB >= 3 ? 3 : 1;
  int voff[C::DPL][NT];
  uint32_t vmask[C::DPL][NT];
#pragma unroll
  for (int x = 0; x < C::DPL; ++x) {
    const int vv = lg * C::DPL + x, pv = vv >> 2, w = vv & 3;
    int t = 0;
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      voff[x][j] = 0;
      vmask[x][j] = 0u;
    }
    if (w < PDW) {
      if (pv < C::NS) {
        const uint32_t sub = odd_subset(MB, pv);
        for (int r = 0; r < MB; ++r)
          if (((sub >> r) & 1u) && t < NT) {
            voff[x][t] = PDW * r + w;
            vmask[x][t] = 0xffffffffu;
            ++t;
          }
      } else {
        voff[x][0] = PDW * MB + w;
        vmask[x][0] = 0xffffffffu;
      }
    }
  }

  // items (query tile, vector chunk), vector-chunk major, so that a query's
  // later chunks start from the k-th best score its earlier chunks published
  // (gth); a workgroup takes items blockIdx.x, blockIdx.x + gridDim.x, ...
  const int qtiles = static_cast<int>(n_items / nvc);
  for (int64_t item = blockIdx.x; item < n_items; item += gridDim.x) {
    const int vc = static_cast<int>(item / qtiles), qt = static_cast<int>(item % qtiles);
    const int chunk0 = (qt * 4 + wave) * QC;  // first query chunk of this wave
    const int64_t v0 = int64_t(vc) * vlen;
    const int64_t v1 = min<int64_t>(N, v0 + vlen);

    qkv_v4i a[QC][NU];
    // theta: this chunk list's k-th score (a candidate must beat it);
    // tg: the query's device-wide bound (a candidate must reach it);
    // thr = max(the float above theta, tg): a candidate is a score >= thr
    float fq[QC], cr[QC], theta[QC], tg[QC], thr[QC];
#pragma unroll
    for (int c = 0; c < QC; ++c) {
      const int ch = min(chunk0 + c, nchunks - 1);
#pragma unroll
      for (int u = 0; u < NU; ++u) a[c][u] = aq[(int64_t(ch) * NU + u) * 64 + lane];
      cr[c] = rowc[(int64_t(ch) * kRowsM + lg) * 2 + 0];
      fq[c] = rowc[(int64_t(ch) * kRowsM + lg) * 2 + 1];
      theta[c] = -INFINITY;
      const int qg = (chunk0 + c) * 4 + lg;
      tg[c] = qg < M ? fkey_inv(__hip_atomic_load(&gth[qg], __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT))
                     : INFINITY;
      thr[c] = fmaxf(-__FLT_MAX__, tg[c]);
    }
    for (int i = lane; i < QW * k; i += 64) {
      wls[i] = -INFINITY;
      wli[i] = -1;
    }

    // rows of step s0 staged through registers: loaded one step ahead
    uint32_t pre[LPT];
    float pn = 0.f;
    auto fetch = [&](int64_t s0) {
#pragma unroll
      for (int x = 0; x < LPT; ++x) {
        const int i = tid + 256 * x;
        const int64_t v = s0 + i / RAWD;
        pre[x] = (i < SD && v < v1) ? kw[v * RAWD + i % RAWD] : 0u;
      }
      // rows past the range score NaN, which no threshold test admits
      if (tid < kMipsStep) pn = s0 + tid < v1 ? norms[s0 + tid] : __builtin_nanf("");
    };
    auto stash = [&](int buf) {
#pragma unroll
      for (int x = 0; x < LPT; ++x)
        if (tid + 256 * x < SD) rows[buf * SD + tid + 256 * x] = pre[x];
      if (tid < kMipsStep) nrm_s[buf * kMipsStep + tid] = pn;
    };
    __syncthreads();  // the previous item's buffers are consumed
    fetch(v0);
    stash(0);
    __syncthreads();
    int buf = 0;
    for (int64_t s0 = v0; s0 < v1; s0 += kMipsStep) {
      const bool more = s0 + kMipsStep < v1;
      if (more) fetch(s0 + kMipsStep);  // in flight during this step
      const uint32_t* rb = rows + buf * kMipsStep * RAWD;
      const float* nb = nrm_s + buf * kMipsStep;
      // 16-vector groups, software-pipelined: group g + 1's row words are
      // expanded and its MFMAs issued before group g's scores and candidates,
      // so that the score arithmetic overlaps the matrix cores' work
      constexpr int NG = kMipsStep / 16;
      auto expand_mfma = [&](int g, qkv_v4i* acc) {
        // virtual row dwords lg*DPL .. : plane p < NS is the parity of the
        // code bits in odd subset p, plane NS the QJL plane
        uint32_t vd[C::DPL];
        const uint32_t* rv = rb + (g * 16 + ln) * RAWD;
#pragma unroll
        for (int x = 0; x < C::DPL; ++x) {
          uint32_t val = rv[voff[x][0]] & vmask[x][0];
#pragma unroll
          for (int j = 1; j < NT; ++j) val ^= rv[voff[x][j]] & vmask[x][j];
          vd[x] = val;
        }
#pragma unroll
        for (int u = 0; u < NU; ++u) {
          const uint32_t x = vd[u >> 1];
          const int sh = 4 * (u & 1);
          qkv_v4i bo;
          bo[0] = static_cast<int>(x & (0x01010101u << sh));
          bo[1] = static_cast<int>(x & (0x02020202u << sh));
          bo[2] = static_cast<int>(x & (0x04040404u << sh));
          bo[3] = static_cast<int>(x & (0x08080808u << sh));
#pragma unroll
          for (int c = 0; c < QC; ++c)
            acc[c] = mfma_i8(a[c][u], bo, u == 0 ? qkv_v4i{0, 0, 0, 0} : acc[c]);
        }
      };
      qkv_v4i accs[2][QC];
      expand_mfma(0, accs[0]);
      // (a group's accumulators are read after the next group's MFMAs and a
      // branch; the first and the last group take the explicit pad)
      mfma_settle();
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        if (g + 1 < NG) expand_mfma(g + 1, accs[(g + 1) & 1]);
        if (g + 1 == NG) mfma_settle();
        const qkv_v4i* acc = accs[g & 1];
        const float nv = nb[g * 16 + ln];  // NaN past the range
        float sc[QC];
#pragma unroll
        for (int c = 0; c < QC; ++c) {
          if constexpr (NU * (1 << 20) < (1 << 23)) {
            // |digit sums| < NU 2^20 < 2^23: two exact int32 halves
            // (base 256), one rounding each
            const int zlo = acc[c][0] + acc[c][1] * 256;
            const int zhi = acc[c][2] + acc[c][3] * 256;
            sc[c] = nv * fmaf(static_cast<float>(zhi), 65536.f * fq[c],
                              fmaf(static_cast<float>(zlo), fq[c], cr[c]));
          } else {
            const float z = static_cast<float>(acc[c][0]) +
                            256.f * static_cast<float>(acc[c][1]) +
                            65536.f * static_cast<float>(acc[c][2]) +
                            16777216.f * static_cast<float>(acc[c][3]);
            sc[c] = nv * fmaf(z, fq[c], cr[c]);
          }
        }
#pragma unroll
        for (int c = 0; c < QC; ++c) {
          uint64_t cand = __builtin_amdgcn_ballot_w64(sc[c] >= thr[c]);
          while (cand) {  // rare: insert in ascending lane (= index) order
            const int L = __builtin_ctzll(cand);
            cand &= cand - 1;
            const float s_new = __shfl(sc[c], L, 64);
            const int q = c * 4 + (L >> 4);  // wave-local query
            float* qs = wls + q * k;
            int* qi = wli + q * k;
            if (s_new > qs[k - 1]) {
              // position = number of entries >= s_new (they hold lower indices)
              int ge = 0;
              for (int j = lane; j < k; j += 64) ge += qs[j] >= s_new ? 1 : 0;
              ge = qkv_wave_sum(ge);
              // shift [ge, k - 1) up by one, 64-entry blocks from the top down
              // (a block reads its entries before the block below is written)
              for (int t = (k - 1) >> 6; t >= 0; --t) {
                const int j = lane + 64 * t;
                const bool mv = j > ge && j < k;
                const float sv = mv ? qs[j - 1] : 0.f;
                const int iv = mv ? qi[j - 1] : 0;
                if (mv) {
                  qs[j] = sv;
                  qi[j] = iv;
                }
              }
              if (lane == 0) {
                qs[ge] = s_new;
                qi[ge] = static_cast<int>(s0 + g * 16 + (L & 15));
              }
              const float th = qs[k - 1];
              if (lg == (L >> 4)) {
                theta[c] = th;
                thr[c] = fmaxf(nextafterf(th, INFINITY), tg[c]);
              }
            }
          }
        }
      }
      if (more) stash(buf ^ 1);
      __syncthreads();
      buf ^= 1;
    }
    // this wave's lists -> candidates [query][vector chunk][k]; a full list's
    // k-th score raises the query's device-wide bound
    for (int q = 0; q < QW; ++q) {
      const int qg = (chunk0 + q / 4) * 4 + (q % 4);
      if (qg >= M) break;
      const int64_t base = (int64_t(qg) * nvc + vc) * k;
      for (int j = lane; j < k; j += 64) {
        cand_s[base + j] = wls[q * k + j];
        cand_i[base + j] = wli[q * k + j];
      }
      if (lane == 0 && wli[q * k + k - 1] >= 0)
        atomicMax(&gth[qg], fkey(wls[q * k + k - 1]));
    }
  }
}

// Final top-k per query over its (vector split) candidate lists: k rounds of a
// wave-wide arg-max (score descending, index ascending).
__global__ __launch_bounds__(64) void mips_merge(const float* __restrict__ cand_s,
                                                 const int* __restrict__ cand_i, int nsplit,
                                                 int k, float* __restrict__ out_s,
                                                 int64_t* __restrict__ out_i) {
  extern __shared__ __align__(16) float smem_mm[];
  const int q = blockIdx.x, lane = threadIdx.x;
  const int n = nsplit * k;
  float* cs = smem_mm;
  int* ci = reinterpret_cast<int*>(smem_mm + n);
  for (int i = lane; i < n; i += 64) {
    cs[i] = cand_s[int64_t(q) * n + i];
    ci[i] = cand_i[int64_t(q) * n + i];
  }
  __syncthreads();
  for (int r = 0; r < k; ++r) {
    float bs = -INFINITY;
    int bi = INT_MAX, bp = -1;
    for (int i = lane; i < n; i += 64) {
      const float s = cs[i];
      const int id = ci[i];
      if (id >= 0 && (s > bs || (s == bs && id < bi))) {
        bs = s;
        bi = id;
        bp = i;
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float os = __shfl_xor(bs, o, 64);
      const int oi = __shfl_xor(bi, o, 64), op = __shfl_xor(bp, o, 64);
      if (op >= 0 && (bp < 0 || os > bs || (os == bs && oi < bi))) {
        bs = os;
        bi = oi;
        bp = op;
      }
    }
    if (lane == 0) {
      out_s[int64_t(q) * k + r] = bs;
      out_i[int64_t(q) * k + r] = bi;
      if (bp >= 0) ci[bp] = -1;
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------ host helpers

// Walsh coefficients of a codebook: c[code] = g_empty + sum_S g_S chi_S(code),
// chi_S(code) = prod_{k in S} (2 bit_k(code) - 1).  The plane decomposition
// used by the MFMA path needs a symmetric codebook (c[~code] == -c[code]),
// for which every even-size subset (g_empty included) has g_S = 0.
bool walsh_odd(const float* cent, int bits, float* g, float* gconst) {
  const int n = 1 << bits;
  for (int c = 0; c < n; ++c)
    if (cent[(n - 1) ^ c] != -cent[c]) return false;
  const int ns = n_odd_subsets(bits);
  double sum = 0.0;
  for (int s = 0; s < ns; ++s) {
    const uint32_t sub = odd_subset(bits, s);
    double acc = 0.0;
    for (int c = 0; c < n / 2; ++c) {  // pair code c with ~c: chi flips sign for odd S
      int par = 0;
      for (int k = 0; k < bits; ++k)
        if ((sub >> k) & 1u) par += ((c >> k) & 1) ? 0 : 1;  // count of (-1) factors
      const double chi = (par & 1) ? -1.0 : 1.0;
      acc += 2.0 * static_cast<double>(cent[c]) * chi;
    }
    g[s] = static_cast<float>(acc / n);
    sum += acc / n;
  }
  // reconstruction check
  for (int c = 0; c < n; ++c) {
    double v = 0.0;
    for (int s = 0; s < ns; ++s) {
      const uint32_t sub = odd_subset(bits, s);
      double chi = 1.0;
      for (int k = 0; k < bits; ++k)
        if ((sub >> k) & 1u) chi *= ((c >> k) & 1) ? 1.0 : -1.0;
      v += static_cast<double>(g[s]) * chi;
    }
    if (fabs(v - cent[c]) > 1e-6 * (fabs(static_cast<double>(cent[c])) + 1e-6)) return false;
  }
  *gconst = static_cast<float>(-sum);
  return true;
}

Tables make_tables(const float* kc, int mbits, const float* vc, int vbits) {
  Tables t{};
  for (int i = 0; i < 16; ++i) {
    t.kc[i] = i < (1 << mbits) ? kc[i] : 0.f;
    t.vc[i] = i < (1 << vbits) ? vc[i] : 0.f;
  }
  bool ok = mbits >= 1 && mbits <= 3 && vbits >= 1 && vbits <= 4;
  if (ok) ok = walsh_odd(kc, mbits, t.kg, &t.kconst);
  if (ok) ok = walsh_odd(vc, vbits, t.vg, &t.vconst);
  t.fused_ok = ok ? 1 : 0;
  t.mfma_ok = ok && mbits <= 2 ? 1 : 0;
  return t;
}

// Mixed-precision key coefficients into tb: kind 1, MSE keys with 3-bit
// outlier / 2-bit regular codebooks; kind 2, IP keys whose MSE stage has
// 2-bit outlier / 1-bit regular codebooks.
bool add_kmix(Tables& tb, int kind, const float* out_cent, const float* reg_cent, int n_out) {
  const int ob = kind == 1 ? 3 : 2, rb = ob - 1;
  float go[4] = {0.f, 0.f, 0.f, 0.f}, gr[4] = {0.f, 0.f, 0.f, 0.f};
  float kconst_o = 0.f, kconst_r = 0.f;
  if (!walsh_odd(out_cent, ob, go, &kconst_o) || !walsh_odd(reg_cent, rb, gr, &kconst_r))
    return false;
  for (int i = 0; i < 4; ++i) tb.kgo[i] = go[i];
  tb.kgr[0] = gr[0];
  tb.kgr[1] = gr[1];
  tb.kco = kconst_o;
  tb.kcr = kconst_r;
  tb.kmix = kind;
  tb.n_out = n_out;
  return true;
}

// K row dwords of a mixed-key format (the Tables comment).
int kmixed_rdw(int kind, int n_out) { return kind == 1 ? 8 + n_out / 16 : 8 + n_out / 32; }

int64_t mfma_split_len(int64_t T, int n_splits) {
  return ((T + n_splits - 1) / n_splits + 63) / 64 * 64;
}

// d = 128 runs on decode_fused (any split length), d = 64 on split_mfma
// (splits of at most kSplitMax tokens, scores held in LDS).
bool use_mfma(const Tables& tb, int d, int64_t t_stride, int64_t T, int n_splits) {
  return tb.mfma_ok && t_stride % 64 == 0 &&
         (d == 128 || (d == 64 && mfma_split_len(T, n_splits) <= kSplitMax));
}

int validate_common(int32_t B, int32_t Hq, int32_t Hkv, int32_t Q, int32_t d, int32_t n_splits,
                    const void* workspace, int64_t ws_bytes) {
  if (!qkv_d_ok(d)) {
    qkv_set_error("head_dim %d unsupported (64, 96 or 128)", d);
    return QKV_E_UNSUPPORTED;
  }
  QKV_REQUIRE(B > 0 && Hq > 0 && Hkv > 0 && Q > 0, "invalid shape");
  QKV_REQUIRE(Hq % Hkv == 0, "query heads (%d) must be a multiple of kv heads (%d)", Hq, Hkv);
  QKV_REQUIRE(B <= 65535, "batch too large");
  QKV_REQUIRE(n_splits >= 1 && n_splits <= 1024, "n_splits %d out of range", n_splits);
  const int R = (Hq / Hkv) * Q;
  QKV_REQUIRE(int64_t(Hkv) * ((R + kRowsM - 1) / kRowsM) <= 65535, "too many kv heads x rows");
  QKV_REQUIRE(workspace != nullptr, "null workspace");
  QKV_REQUIRE(qkv_aligned(workspace, 256), "workspace must be 256-byte aligned");
  const int64_t need = ws_layout(B, Hkv, R, d, n_splits).total;
  QKV_REQUIRE(ws_bytes >= need, "workspace too small: %lld < %lld", (long long)ws_bytes,
              (long long)need);
  return QKV_OK;
}

// Row chunks per split_mfma workgroup: two at d = 64 when the GQA group has
// more than 4 rows (the K/V operands then serve 8 rows), else one.
int mfma_rc(int d, int R) { return d == 64 && R > kRowsM ? 2 : 1; }

// Dynamic LDS bytes of split_mfma for a split length (scores + value norms).
int64_t mfma_smem_bytes(int64_t split_len, int rc) {
  const int64_t nt = (split_len + 63) / 64;
  return nt * kRowsM * rc * 64 * 4 + nt * 64 * 4;
}

// Resident split_mfma workgroups per CU for a split length (queried per
// length; the kernel's registers and this LDS size set it).
int mfma_blocks_per_cu(int64_t split_len, int rc) {
  static int cache[2][kSplitMax / 64 + 1] = {};
  const int nt = static_cast<int>((split_len + 63) / 64);
  if (nt < 1 || nt > kSplitMax / 64) return 1;
  int& slot = cache[rc == 2][nt];
  if (slot == 0) {
    int v = 0;
    const size_t smem = static_cast<size_t>(mfma_smem_bytes(nt * 64, rc));
    const hipError_t e =
        rc == 2 ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, split_mfma<64, 2, 3, 2, false>, 256,
                                                               smem)
                : hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, split_mfma<64, 2, 3, 1, false>, 256,
                                                               smem);
    if (e != hipSuccess || v <= 0) v = 1;
    slot = v;
  }
  return slot;
}

// Splits of the fused d = 128 decode: enough workgroups for one per CU when
// the row groups are fewer than the CUs, with at least ~1024 tokens each.
int fused_splits(int64_t groups, int64_t T) {
  const int64_t ncu = qkv_num_cus();
  int64_t s = (ncu + groups - 1) / groups;
  s = std::min<int64_t>(s, std::max<int64_t>(1, (T + 1023) / 1024));
  return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(s, 1024)));
}

bool use_fused(const Tables& tb, int d, int64_t t_stride) {
  return tb.fused_ok && (d == 128 || d == 96 || d == 64) && t_stride % 64 == 0;
}

// The MFMA decode of the layer-batched and paged entries: decode_fused at
// d = 128 and 96, split_mfma at d = 64 (its two row chunks per workgroup read
// a 5-8-row GQA group's K/V once).  Single calls take decode_fused at d = 64
// too (use_fused), with the split count of this model.
bool use_mfma_path(const Tables& tb, int d, int64_t t_stride, int64_t T, int n_splits) {
  return d == 64 ? use_mfma(tb, d, t_stride, T, n_splits) : use_fused(tb, d, t_stride);
}

// Launch decode_small over nl layers (d = 64, key MSE bits 1-2; B sequences
// each; workspace for B * nl): final_out with one split writes the output
// (ol), otherwise split partials for combine_layers.
int launch_small(const QLayers& ql, const KVLayers& kv, const OutLayers& ol, int nl, int B,
                 int q_dtype, float alpha, int Hq, int Hkv, int Q, int mbits, int vbits,
                 const Tables& tb, int64_t t_stride, int64_t T, float scale, int causal,
                 int n_splits, int final_out, int out_dtype, void* workspace, hipStream_t s) {
  const int R = (Hq / Hkv) * Q;
  const int rc = R > kRowsM ? 2 : 1;
  const int cgroups = (R + kRowsM * rc - 1) / (kRowsM * rc);
  const WsLayout L = ws_layout(B * nl, Hkv, R, 64, n_splits);
  const int64_t split_len = ((T + n_splits - 1) / n_splits + 63) / 64 * 64;
  const dim3 grid(n_splits, Hkv * cgroups, B * nl);
  float* po = at<float>(workspace, L.po);
  float* pml = at<float>(workspace, L.pml);
#define QKV_SM(MBV, VBV, RCV)                                                                   \
  do {                                                                                          \
    if (kv.ptab)                                                                                \
      hipLaunchKernelGGL((decode_small<MBV, VBV, RCV, true>), grid, dim3(256), 0, s, ql, kv,   \
                         ol, B, q_dtype, alpha, Hq, Hkv, Q, R, cgroups, tb, t_stride, T, scale, \
                         causal, split_len, final_out, out_dtype, po, pml);                     \
    else                                                                                        \
      hipLaunchKernelGGL((decode_small<MBV, VBV, RCV, false>), grid, dim3(256), 0, s, ql, kv,  \
                         ol, B, q_dtype, alpha, Hq, Hkv, Q, R, cgroups, tb, t_stride, T, scale, \
                         causal, split_len, final_out, out_dtype, po, pml);                     \
  } while (0)
#define QKV_SMV(MBV, RCV)                  \
  switch (vbits) {                         \
    case 1: QKV_SM(MBV, 1, RCV); break;    \
    case 2: QKV_SM(MBV, 2, RCV); break;    \
    case 3: QKV_SM(MBV, 3, RCV); break;    \
    default: QKV_SM(MBV, 4, RCV); break;   \
  }
  if (mbits == 1) {
    if (rc == 2) {
      QKV_SMV(1, 2)
    } else {
      QKV_SMV(1, 1)
    }
  } else {
    if (rc == 2) {
      QKV_SMV(2, 2)
    } else {
      QKV_SMV(2, 1)
    }
  }
#undef QKV_SMV
#undef QKV_SM
  QKV_LAUNCHED();
  return QKV_OK;
}

// Launch decode_fused over nl layers (B sequences each; workspace for B * nl)
// at head dim d (128 or 96) on K rows of rdw dwords: (d / 32) (kbits + 1) for
// IP keys of kbits MSE bits, kmixed_rdw() for the mixed-key formats.  pro: query operands computed in the
// kernel (else prepare_mfma's, from the workspace).  final_out with one split: the kernel writes the output (ol);
// otherwise it writes split partials and the caller runs combine_layers.
int launch_fused(const QLayers& ql, const KVLayers& kv, const OutLayers& ol, int nl, int B,
                 int q_dtype, float alpha, int Hq, int Hkv, int Q, int d, int rdw,
                 int vbits, const Tables& tb, int64_t t_stride, int64_t T, float scale,
                 int causal, int n_splits, int final_out, int out_dtype, void* workspace,
                 bool pro, hipStream_t s) {
  const int R = (Hq / Hkv) * Q;
  const WsLayout L = ws_layout(B * nl, Hkv, R, d, n_splits);
  const int chunks = (R + kRowsM - 1) / kRowsM;
  const int64_t split_len = ((T + n_splits - 1) / n_splits + 63) / 64 * 64;
  const dim3 grid(n_splits, Hkv * chunks, B * nl);
  const qkv_v4i* aq = pro ? nullptr : at<qkv_v4i>(workspace, L.aq);
  const float* rowc = at<float>(workspace, L.rowc);
  float* po = at<float>(workspace, L.po);
  float* pml = at<float>(workspace, L.pml);
  constexpr uint32_t smem = FusedLds::TOTAL;
#define QKV_FU3(RW, VB, PG, DSV)                                                               \
  do {                                                                                         \
    static const hipError_t attr_ = hipFuncSetAttribute(                                       \
        reinterpret_cast<const void*>(&decode_fused<RW, VB, PG, DSV>),                         \
        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem));                   \
    QKV_HIP(attr_);                                                                            \
    hipLaunchKernelGGL((decode_fused<RW, VB, PG, DSV>), grid, dim3(kThreadsF), smem, s, ql,   \
                       kv, ol, B, q_dtype, alpha, Hq, Hkv, Q, R, chunks, tb, t_stride, T,      \
                       scale, causal, split_len, final_out, out_dtype, aq, rowc, po, pml);     \
  } while (0)
#define QKV_FU2(RW, VB, PG) QKV_FU3(RW, VB, PG, 128)
#define QKV_FU(RW, VB)              \
  do {                              \
    if (kv.ptab)                    \
      QKV_FU2(RW, VB, true);        \
    else                            \
      QKV_FU2(RW, VB, false);       \
  } while (0)
  // the mixed-key formats (9 and 10 dwords; 12 shares the IP code) have no
  // paged store
  QKV_REQUIRE((rdw % 4 == 0 && d == 128) || d == 64 || d == 96 || kv.ptab == nullptr,
              "mixed keys are not paged");
#define QKV_FUC(RW, VB)    \
  QKV_FU2(RW, VB, false);  \
  break
#define QKV_FU96(RW, VB)                \
  if (kv.ptab)                          \
    QKV_FU3(RW, VB, true, 96);          \
  else                                  \
    QKV_FU3(RW, VB, false, 96);         \
  break
#define QKV_FU64(RW, VB)                \
  if (kv.ptab)                          \
    QKV_FU3(RW, VB, true, 64);          \
  else                                  \
    QKV_FU3(RW, VB, false, 64);         \
  break
  if (d == 64) {
    switch (rdw * 10 + vbits) {
      case 41: QKV_FU64(4, 1);
      case 42: QKV_FU64(4, 2);
      case 43: QKV_FU64(4, 3);
      case 44: QKV_FU64(4, 4);
      case 61: QKV_FU64(6, 1);
      case 62: QKV_FU64(6, 2);
      case 63: QKV_FU64(6, 3);
      case 64: QKV_FU64(6, 4);
      case 81: QKV_FU64(8, 1);
      case 82: QKV_FU64(8, 2);
      case 83: QKV_FU64(8, 3);
      case 84: QKV_FU64(8, 4);
      default:
        qkv_set_error("fused decode (d = 64): K rows of %d dwords / value bits %d unsupported",
                      rdw, vbits);
        return QKV_E_UNSUPPORTED;
    }
    QKV_LAUNCHED();
    return QKV_OK;
  }
  if (d == 96) {
    switch (rdw * 10 + vbits) {
      case 61: QKV_FU96(6, 1);
      case 62: QKV_FU96(6, 2);
      case 63: QKV_FU96(6, 3);
      case 64: QKV_FU96(6, 4);
      case 91: QKV_FU96(9, 1);
      case 92: QKV_FU96(9, 2);
      case 93: QKV_FU96(9, 3);
      case 94: QKV_FU96(9, 4);
      case 121: QKV_FU96(12, 1);
      case 122: QKV_FU96(12, 2);
      case 123: QKV_FU96(12, 3);
      case 124: QKV_FU96(12, 4);
      default:
        qkv_set_error("fused decode (d = 96): K rows of %d dwords / value bits %d unsupported",
                      rdw, vbits);
        return QKV_E_UNSUPPORTED;
    }
    QKV_LAUNCHED();
    return QKV_OK;
  }
  switch (rdw * 10 + vbits) {
    case 81: QKV_FU(8, 1); break;
    case 82: QKV_FU(8, 2); break;
    case 83: QKV_FU(8, 3); break;
    case 84: QKV_FU(8, 4); break;
    case 121: QKV_FU(12, 1); break;
    case 122: QKV_FU(12, 2); break;
    case 123: QKV_FU(12, 3); break;
    case 124: QKV_FU(12, 4); break;
    case 161: QKV_FU(16, 1); break;
    case 162: QKV_FU(16, 2); break;
    case 163: QKV_FU(16, 3); break;
    case 164: QKV_FU(16, 4); break;
    case 91: QKV_FUC(9, 1);
    case 92: QKV_FUC(9, 2);
    case 93: QKV_FUC(9, 3);
    case 94: QKV_FUC(9, 4);
    case 101: QKV_FUC(10, 1);
    case 102: QKV_FUC(10, 2);
    case 103: QKV_FUC(10, 3);
    case 104: QKV_FUC(10, 4);
    default:
      qkv_set_error("fused decode: K rows of %d dwords / value bits %d unsupported", rdw, vbits);
      return QKV_E_UNSUPPORTED;
  }
#undef QKV_FU96
#undef QKV_FU64
#undef QKV_FUC
#undef QKV_FU
#undef QKV_FU2
#undef QKV_FU3
  QKV_LAUNCHED();
  return QKV_OK;
}

}  // namespace

// ------------------------------------------------------------ C ABI

extern "C" int32_t qkv_attention_splits(int32_t B, int32_t Hq, int32_t Hkv, int32_t Q,
                                        int32_t d, int64_t T) {
  if (B <= 0 || Hkv <= 0 || Hq <= 0 || Q <= 0 || T <= 0) return 1;
  const int R = (Hq / Hkv) * Q;
  if (d == 128 || d == 96)
    return fused_splits(int64_t(B) * Hkv * ((R + kRowsM - 1) / kRowsM), T);
  // d = 64: decode_small (three workgroups per CU, 256-token chunks): enough
  // splits for two workgroups per CU, of at least one chunk each (and at most
  // kSplitMax tokens, the split kernel's LDS bound)
  const int rc = R > kRowsM ? 2 : 1;
  const int64_t groups = int64_t(B) * Hkv * ((R + kRowsM * rc - 1) / (kRowsM * rc));
  const int64_t ncu = qkv_num_cus();
  int64_t sp = std::min<int64_t>((2 * ncu + groups - 1) / groups, (T + kChunkS - 1) / kChunkS);
  sp = std::max<int64_t>(sp, (T + kSplitMax - 1) / kSplitMax);
  return static_cast<int32_t>(std::max<int64_t>(1, std::min<int64_t>(sp, 1024)));
}

extern "C" int64_t qkv_attention_workspace_bytes(int32_t B, int32_t Hq, int32_t Hkv, int32_t Q,
                                                 int32_t d, int32_t n_splits) {
  if (B <= 0 || Hkv <= 0 || Hq <= 0 || Q <= 0 || d <= 0 || n_splits <= 0) return -1;
  return ws_layout(B, Hkv, (Hq / Hkv) * Q, d, n_splits).total;
}

extern "C" int32_t qkv_attention_path(int32_t d, int32_t kbits, int32_t vbits,
                                      const float* kcent_host, const float* vcent_host,
                                      int64_t t_stride, int64_t T, int32_t n_splits) {
  if (!kcent_host || !vcent_host || !qkv_bits_ok(kbits) || !qkv_bits_ok(vbits) || n_splits < 1)
    return -1;
  const Tables tb = make_tables(kcent_host, kbits, vcent_host, vbits);
  return use_fused(tb, d, t_stride) || use_mfma_path(tb, d, t_stride, T, n_splits) ? 1 : 0;
}

// prepare for nl layers (B sequences each; the workspace holds B * nl)
int prepare_layers(const QLayers& ql, int nl, int32_t q_dtype, int32_t B, int32_t Hq,
                   int32_t Hkv, int32_t Q, int32_t d, int32_t kbits, int32_t vbits,
                   const float* kcent_host, const float* vcent_host, float qjl_scale,
                   void* workspace, int64_t ws_bytes, int32_t n_splits, hipStream_t s) {
  QKV_REQUIRE(qkv_dtype_ok(q_dtype), "unsupported query dtype %d", q_dtype);
  QKV_REQUIRE(qkv_bits_ok(kbits) && qkv_bits_ok(vbits), "bits must be in {1, 2, 3, 4}");
  int st = validate_common(B * nl, Hq, Hkv, Q, d, n_splits, workspace, ws_bytes);
  if (st != QKV_OK) return st;
  QKV_REQUIRE(kcent_host && vcent_host, "null pointer");
  for (int l = 0; l < nl; ++l) {
    QKV_REQUIRE(ql.q[l] && ql.pi[l] && ql.signs[l], "null pointer");
    QKV_REQUIRE(qkv_aligned(ql.pi[l], 16), "pi must be 16-byte aligned");
  }
  const int R = (Hq / Hkv) * Q;
  const WsLayout L = ws_layout(B * nl, Hkv, R, d, n_splits);
  const Tables tb = make_tables(kcent_host, kbits, vcent_host, vbits);
  if (tb.mfma_ok && (d == 128 || d == 64)) {
    // MFMA query operands; the same kernel writes q~ and w for the VALU kernel
    const int chunks = (R + kRowsM - 1) / kRowsM;
    const dim3 grid(B * nl * Hkv * chunks);
#define QKV_PREP(DD, NPLV)                                                                   \
  hipLaunchKernelGGL((prepare_mfma<DD, NPLV, DD == 128>), grid, dim3(256),                  \
                     (prep_lds<DD, NPLV, DD == 128>()), s,                                  \
                     ql, B,                                                                 \
                     q_dtype,                                                               \
                     qjl_scale, Hq, Hkv, Q, R, chunks, tb, at<qkv_v4i>(workspace, L.aq),    \
                     at<float>(workspace, L.rowc), at<float>(workspace, L.qw))
    if (d == 128) {
      if (kbits == 2) QKV_PREP(128, 3); else QKV_PREP(128, 2);
    } else {
      if (kbits == 2) QKV_PREP(64, 3); else QKV_PREP(64, 2);
    }
#undef QKV_PREP
    QKV_LAUNCHED();
    return QKV_OK;
  }
  if (nl != 1) {
    qkv_set_error("layer-batched decode runs on the MFMA path (symmetric codebooks, key MSE "
                  "bits <= 2, head_dim 64 or 128)");
    return QKV_E_UNSUPPORTED;
  }
  switch (d) {
#define QKV_CASE(DD)                                                                          \
  case DD:                                                                                    \
    hipLaunchKernelGGL(qrot_kernel<DD>, dim3(B * Hq * Q), dim3(128), 0, s, ql.q[0], q_dtype,  \
                       ql.pi[0], ql.signs[0], qjl_scale, Hq, Hkv, Q,                          \
                       at<float>(workspace, L.qw));                                           \
    break;
    QKV_CASE(64)
    QKV_CASE(96)
    QKV_CASE(128)
#undef QKV_CASE
  }
  QKV_LAUNCHED();
  return QKV_OK;
}

extern "C" int qkv_attention_prepare(const void* q, int32_t q_dtype, int32_t B, int32_t Hq,
                                     int32_t Hkv, int32_t Q, int32_t d, int32_t kbits,
                                     int32_t vbits, const float* pi, const float* kcent_host,
                                     const float* vcent_host, const float* signs,
                                     float qjl_scale, void* workspace, int64_t ws_bytes,
                                     int32_t n_splits, void* stream) {
  QLayers ql{};
  ql.q[0] = q;
  ql.pi[0] = pi;
  ql.signs[0] = signs;
  return prepare_layers(ql, 1, q_dtype, B, Hq, Hkv, Q, d, kbits, vbits, kcent_host, vcent_host,
                        qjl_scale, workspace, ws_bytes, n_splits,
                        static_cast<hipStream_t>(stream));
}

// partial for nl layers (B sequences each)
int partial_layers(const KVLayers& kv, int nl, int64_t t_stride, int64_t T, int32_t B,
                   int32_t Hq, int32_t Hkv, int32_t Q, int32_t d, int32_t kbits, int32_t vbits,
                   const float* kcent_host, const float* vcent_host, float scale,
                   int32_t causal, void* workspace, int64_t ws_bytes, int32_t n_splits,
                   hipStream_t s) {
  QKV_REQUIRE(qkv_bits_ok(kbits) && qkv_bits_ok(vbits), "bits must be in {1, 2, 3, 4}");
  QKV_REQUIRE(T > 0, "No compressed KV blocks in cache. Call append() first.");
  QKV_REQUIRE(t_stride >= T && t_stride % 32 == 0,
              "t_stride %lld must be >= T %lld and a multiple of 32", (long long)t_stride,
              (long long)T);
  int st = validate_common(B * nl, Hq, Hkv, Q, d, n_splits, workspace, ws_bytes);
  if (st != QKV_OK) return st;
  QKV_REQUIRE(kcent_host && vcent_host, "null pointer");
  for (int l = 0; l < nl; ++l) {
    QKV_REQUIRE(kv.kst[l] && kv.knorm[l] && kv.vst[l] && kv.vnorm[l], "null pointer");
    QKV_REQUIRE(qkv_aligned(kv.kst[l], 4) && qkv_aligned(kv.vst[l], 4),
                "store must be 4-byte aligned");
  }
  const int R = (Hq / Hkv) * Q;
  const WsLayout L = ws_layout(B * nl, Hkv, R, d, n_splits);
  const Tables tb = make_tables(kcent_host, kbits, vcent_host, vbits);
  float* po = at<float>(workspace, L.po);
  float* pml = at<float>(workspace, L.pml);
  if (use_mfma(tb, d, t_stride, T, n_splits) && d == 128) {
    // the fused kernel in partial mode: operands from prepare_mfma, split partials out
    return launch_fused(QLayers{}, kv, OutLayers{}, nl, B, QKV_F32, 0.f, Hq, Hkv, Q, d,
                        4 * (kbits + 1),
                        vbits, tb, t_stride, T, scale, causal, n_splits, 0, QKV_F32, workspace,
                        false, s);
  }
  if (use_mfma(tb, d, t_stride, T, n_splits)) {
    const int chunks = (R + kRowsM - 1) / kRowsM;
    const int rc = mfma_rc(d, R);
    const int64_t split_len = mfma_split_len(T, n_splits);
    const int64_t smem = mfma_smem_bytes(split_len, rc);
    const dim3 grid(n_splits, Hkv * ((chunks + rc - 1) / rc), B * nl);
    const qkv_v4i* aq = at<qkv_v4i>(workspace, L.aq);
    const float* rowc = at<float>(workspace, L.rowc);
#define QKV_MF2(DD, MB, VB, RCV, RG)                                                            \
  do {                                                                                          \
    if (smem > 65536)                                                                           \
      QKV_HIP(hipFuncSetAttribute(                                                              \
          reinterpret_cast<const void*>(&split_mfma<DD, MB, VB, RCV, RG>),                      \
          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem)));                  \
    hipLaunchKernelGGL((split_mfma<DD, MB, VB, RCV, RG>), grid, dim3(256),                      \
                       static_cast<uint32_t>(smem), s, aq, rowc, kv, B, t_stride, T, Hkv, R,    \
                       Q, chunks, scale, causal, split_len, tb, po, pml);                       \
  } while (0)
#define QKV_MF(DD, MB, VB, RCV)                  \
  do {                                           \
    if (kv.klo || kv.khi)                        \
      QKV_MF2(DD, MB, VB, RCV, true);            \
    else                                         \
      QKV_MF2(DD, MB, VB, RCV, false);           \
  } while (0)
#define QKV_MFD(DD, RCV)                           \
  switch (kbits * 10 + vbits) {                    \
    case 11: QKV_MF(DD, 1, 1, RCV); break;         \
    case 12: QKV_MF(DD, 1, 2, RCV); break;         \
    case 13: QKV_MF(DD, 1, 3, RCV); break;         \
    case 14: QKV_MF(DD, 1, 4, RCV); break;         \
    case 21: QKV_MF(DD, 2, 1, RCV); break;         \
    case 22: QKV_MF(DD, 2, 2, RCV); break;         \
    case 23: QKV_MF(DD, 2, 3, RCV); break;         \
    case 24: QKV_MF(DD, 2, 4, RCV); break;         \
  }
    if (rc == 2) {
      QKV_MFD(64, 2)
    } else {
      QKV_MFD(64, 1)
    }
#undef QKV_MFD
#undef QKV_MF
#undef QKV_MF2
    QKV_LAUNCHED();
    return QKV_OK;
  }
  if (nl != 1) {
    qkv_set_error("layer-batched decode runs on the MFMA path (store capacity a multiple of "
                  "64, splits of at most %d tokens)", kSplitMax);
    return QKV_E_UNSUPPORTED;
  }
  const int chunks = (R + kRowsG - 1) / kRowsG;
  const int64_t split_len = ((T + n_splits - 1) / n_splits + kTileG - 1) / kTileG * kTileG;
  const float* qw = at<float>(workspace, L.qw);
  switch (d) {
#define QKV_CASE(DD)                                                                           \
  case DD:                                                                                     \
    hipLaunchKernelGGL(split_generic<DD>, dim3(n_splits, Hkv * chunks, B), dim3(kTileG), 0, s, \
                       qw, kv.kst[0], kv.knorm[0], kv.vst[0], kv.vnorm[0], t_stride, T, Hkv,   \
                       R, Q, chunks, kbits, vbits, tb, scale, causal, split_len, kv.klo,       \
                       kv.khi, kv.cbase, po, pml);                                             \
    break;
    QKV_CASE(64)
    QKV_CASE(96)
    QKV_CASE(128)
#undef QKV_CASE
  }
  QKV_LAUNCHED();
  return QKV_OK;
}

extern "C" int qkv_attention_partial(const uint8_t* kstore, const float* knorm,
                                     const uint32_t* vstore, const float* vnorm,
                                     int64_t t_stride, int64_t T, int32_t B, int32_t Hq,
                                     int32_t Hkv, int32_t Q, int32_t d, int32_t kbits,
                                     int32_t vbits, const float* kcent_host,
                                     const float* vcent_host, float scale, int32_t causal,
                                     void* workspace, int64_t ws_bytes, int32_t n_splits,
                                     void* stream) {
  KVLayers kv{};
  kv.kst[0] = kstore;
  kv.knorm[0] = knorm;
  kv.vst[0] = vstore;
  kv.vnorm[0] = vnorm;
  return partial_layers(kv, 1, t_stride, T, B, Hq, Hkv, Q, d, kbits, vbits, kcent_host,
                        vcent_host, scale, causal, workspace, ws_bytes, n_splits,
                        static_cast<hipStream_t>(stream));
}

// combine for nl layers (B sequences each)
int combine_layers(const OutLayers& ol, int nl, int32_t B, int32_t Hq, int32_t Hkv, int32_t Q,
                   int32_t d, int32_t out_dtype, void* workspace, int64_t ws_bytes,
                   int32_t n_splits, hipStream_t s) {
  QKV_REQUIRE(qkv_dtype_ok(out_dtype), "unsupported output dtype %d", out_dtype);
  int st = validate_common(B * nl, Hq, Hkv, Q, d, n_splits, workspace, ws_bytes);
  if (st != QKV_OK) return st;
  for (int l = 0; l < nl; ++l) {
    QKV_REQUIRE(ol.pi[l] && ol.out[l], "null pointer");
    QKV_REQUIRE(qkv_aligned(ol.pi[l], 16), "pi must be 16-byte aligned");
  }
  const int R = (Hq / Hkv) * Q;
  const WsLayout L = ws_layout(B * nl, Hkv, R, d, n_splits);
  const int64_t nrl = int64_t(B) * Hkv * R;  // rows per layer
  // few rows: one per workgroup (more workgroups over the splits); many rows:
  // four per workgroup (each Pi load serves four)
  const bool wide = nrl * nl < int64_t(kRowsC) * qkv_num_cus();
  const dim3 cgrid(static_cast<int>(wide ? nrl : (nrl + kRowsC - 1) / kRowsC), nl);
  const float* po = at<float>(workspace, L.po);
  const float* pml = at<float>(workspace, L.pml);
  switch (d) {
#define QKV_CASE(DD)                                                                          \
  case DD:                                                                                    \
    if (wide)                                                                                 \
      hipLaunchKernelGGL((combine_kernel<DD, 1>), cgrid, dim3(2 * DD), 0, s, po, pml, ol,     \
                         n_splits, B, Hkv, R, Q, Hq, out_dtype);                              \
    else                                                                                      \
      hipLaunchKernelGGL((combine_kernel<DD, kRowsC>), cgrid, dim3(2 * DD), 0, s, po, pml,    \
                         ol, n_splits, B, Hkv, R, Q, Hq, out_dtype);                          \
    break;
    QKV_CASE(64)
    QKV_CASE(96)
    QKV_CASE(128)
#undef QKV_CASE
  }
  QKV_LAUNCHED();
  return QKV_OK;
}

extern "C" int qkv_attention_combine(int32_t B, int32_t Hq, int32_t Hkv, int32_t Q, int32_t d,
                                     const float* pi, void* out, int32_t out_dtype,
                                     void* workspace, int64_t ws_bytes, int32_t n_splits,
                                     void* stream) {
  OutLayers ol{};
  ol.pi[0] = pi;
  ol.out[0] = out;
  return combine_layers(ol, 1, B, Hq, Hkv, Q, d, out_dtype, workspace, ws_bytes, n_splits,
                        static_cast<hipStream_t>(stream));
}

extern "C" int qkv_attention_run(const uint8_t* kstore, const float* knorm,
                                 const uint32_t* vstore, const float* vnorm, int64_t t_stride,
                                 int64_t T, int32_t B, int32_t Hq, int32_t Hkv, int32_t Q,
                                 int32_t d, int32_t kbits, int32_t vbits, const float* pi,
                                 const float* kcent_host, const float* vcent_host, float scale,
                                 int32_t causal, void* out, int32_t out_dtype, void* workspace,
                                 int64_t ws_bytes, int32_t n_splits, void* stream) {
  // validate both halves before the first launch
  QKV_REQUIRE(qkv_dtype_ok(out_dtype), "unsupported output dtype %d", out_dtype);
  QKV_REQUIRE(pi && out, "null pointer");
  QKV_REQUIRE(qkv_aligned(pi, 16), "pi must be 16-byte aligned");
  int st = qkv_attention_partial(kstore, knorm, vstore, vnorm, t_stride, T, B, Hq, Hkv, Q, d,
                                 kbits, vbits, kcent_host, vcent_host, scale, causal, workspace,
                                 ws_bytes, n_splits, stream);
  if (st != QKV_OK) return st;
  return qkv_attention_combine(B, Hq, Hkv, Q, d, pi, out, out_dtype, workspace, ws_bytes,
                               n_splits, stream);
}

namespace {

// qkv_decode_attention over the key ranges of kr (klo / khi / cbase; the
// store pointers of kr are ignored).
int decode_attention_impl(const void* q, int32_t q_dtype, const uint8_t* kstore,
                          const float* knorm, const uint32_t* vstore, const float* vnorm,
                          int64_t t_stride, int64_t T, int32_t B, int32_t Hq, int32_t Hkv,
                          int32_t Q, int32_t d, int32_t kbits, int32_t vbits, const float* pi,
                          const float* kcent_host, const float* vcent_host, const float* signs,
                          float qjl_scale, float scale, int32_t causal, void* out,
                          int32_t out_dtype, void* workspace, int64_t ws_bytes, int32_t n_splits,
                          const KVLayers& kr, void* stream) {
  // validate everything before the first launch
  QKV_REQUIRE(qkv_dtype_ok(q_dtype) && qkv_dtype_ok(out_dtype), "unsupported dtype");
  QKV_REQUIRE(qkv_bits_ok(kbits) && qkv_bits_ok(vbits), "bits must be in {1, 2, 3, 4}");
  QKV_REQUIRE(T > 0, "No compressed KV blocks in cache. Call append() first.");
  QKV_REQUIRE(t_stride >= T && t_stride % 32 == 0,
              "t_stride %lld must be >= T %lld and a multiple of 32", (long long)t_stride,
              (long long)T);
  QKV_REQUIRE(kr.cbase >= 0, "causal position %lld must be >= 0", (long long)kr.cbase);
  int st = validate_common(B, Hq, Hkv, Q, d, n_splits, workspace, ws_bytes);
  if (st != QKV_OK) return st;
  QKV_REQUIRE(q && kstore && knorm && vstore && vnorm && pi && kcent_host && vcent_host &&
                  signs && out,
              "null pointer");
  KVLayers kv{};
  kv.kst[0] = kstore;
  kv.knorm[0] = knorm;
  kv.vst[0] = vstore;
  kv.vnorm[0] = vnorm;
  kv.klo = kr.klo;
  kv.khi = kr.khi;
  kv.cbase = kr.cbase;
  auto s = static_cast<hipStream_t>(stream);
  const Tables tb = make_tables(kcent_host, kbits, vcent_host, vbits);
  if (d == 64 && tb.mfma_ok && t_stride % 64 == 0 && !kr.klo && !kr.khi && kr.cbase == 0) {
    // decode_small: one launch (plus combine_kernel with several splits)
    QKV_REQUIRE(qkv_aligned(pi, 16) && qkv_aligned(kstore, 4) && qkv_aligned(vstore, 4),
                "pi must be 16-byte and the store 4-byte aligned");
    QLayers ql{};
    ql.q[0] = q;
    ql.pi[0] = pi;
    ql.signs[0] = signs;
    OutLayers ol{};
    ol.pi[0] = pi;
    ol.out[0] = out;
    st = launch_small(ql, kv, ol, 1, B, q_dtype, qjl_scale, Hq, Hkv, Q, kbits, vbits, tb, t_stride,
                      T, scale, causal, n_splits, 1, out_dtype, workspace, s);
    if (st != QKV_OK || n_splits == 1) return st;
    return combine_layers(ol, 1, B, Hq, Hkv, Q, d, out_dtype, workspace, ws_bytes, n_splits, s);
  }
  if (use_fused(tb, d, t_stride)) {
    QKV_REQUIRE(qkv_aligned(pi, 16) && qkv_aligned(kstore, 4) && qkv_aligned(vstore, 4),
                "pi must be 16-byte and the store 4-byte aligned");
    QLayers ql{};
    ql.q[0] = q;
    ql.pi[0] = pi;
    ql.signs[0] = signs;
    OutLayers ol{};
    ol.pi[0] = pi;
    ol.out[0] = out;
    st = launch_fused(ql, kv, ol, 1, B, q_dtype, qjl_scale, Hq, Hkv, Q, d,
                      (d / 32) * (kbits + 1), vbits, tb,
                      t_stride, T, scale, causal, n_splits, 1, out_dtype, workspace, true, s);
    if (st != QKV_OK || n_splits == 1) return st;
    return combine_layers(ol, 1, B, Hq, Hkv, Q, d, out_dtype, workspace, ws_bytes, n_splits, s);
  }
  QKV_REQUIRE(qkv_dtype_ok(out_dtype), "unsupported output dtype %d", out_dtype);
  QKV_REQUIRE(qkv_aligned(pi, 16), "pi must be 16-byte aligned");
  st = qkv_attention_prepare(q, q_dtype, B, Hq, Hkv, Q, d, kbits, vbits, pi, kcent_host,
                             vcent_host, signs, qjl_scale, workspace, ws_bytes, n_splits, stream);
  if (st != QKV_OK) return st;
  st = partial_layers(kv, 1, t_stride, T, B, Hq, Hkv, Q, d, kbits, vbits, kcent_host, vcent_host,
                      scale, causal, workspace, ws_bytes, n_splits, s);
  if (st != QKV_OK) return st;
  return qkv_attention_combine(B, Hq, Hkv, Q, d, pi, out, out_dtype, workspace, ws_bytes,
                               n_splits, stream);
}

}  // namespace

extern "C" int qkv_decode_attention(const void* q, int32_t q_dtype, const uint8_t* kstore,
                                    const float* knorm, const uint32_t* vstore,
                                    const float* vnorm, int64_t t_stride, int64_t T, int32_t B,
                                    int32_t Hq, int32_t Hkv, int32_t Q, int32_t d, int32_t kbits,
                                    int32_t vbits, const float* pi, const float* kcent_host,
                                    const float* vcent_host, const float* signs,
                                    float qjl_scale, float scale, int32_t causal, void* out,
                                    int32_t out_dtype, void* workspace, int64_t ws_bytes,
                                    int32_t n_splits, void* stream) {
  return decode_attention_impl(q, q_dtype, kstore, knorm, vstore, vnorm, t_stride, T, B, Hq,
                               Hkv, Q, d, kbits, vbits, pi, kcent_host, vcent_host, signs,
                               qjl_scale, scale, causal, out, out_dtype, workspace, ws_bytes,
                               n_splits, KVLayers{}, stream);
}

extern "C" int qkv_decode_attention_ranges(
    const void* q, int32_t q_dtype, const uint8_t* kstore, const float* knorm,
    const uint32_t* vstore, const float* vnorm, int64_t t_stride, int64_t T,
    const int32_t* kv_start, const int32_t* kv_end, int64_t q_end, int32_t B, int32_t Hq,
    int32_t Hkv, int32_t Q, int32_t d, int32_t kbits, int32_t vbits, const float* pi,
    const float* kcent_host, const float* vcent_host, const float* signs, float qjl_scale,
    float scale, int32_t causal, void* out, int32_t out_dtype, void* workspace, int64_t ws_bytes,
    int32_t n_splits, void* stream) {
  QKV_REQUIRE(kv_start == nullptr || qkv_aligned(kv_start, 4), "kv_start must be 4-byte aligned");
  QKV_REQUIRE(kv_end == nullptr || qkv_aligned(kv_end, 4), "kv_end must be 4-byte aligned");
  KVLayers kr{};
  kr.klo = kv_start;
  kr.khi = kv_end;
  kr.cbase = q_end;
  return decode_attention_impl(q, q_dtype, kstore, knorm, vstore, vnorm, t_stride, T, B, Hq,
                               Hkv, Q, d, kbits, vbits, pi, kcent_host, vcent_host, signs,
                               qjl_scale, scale, causal, out, out_dtype, workspace, ws_bytes,
                               n_splits, kr, stream);
}

// ------------------------------------------------------------ no-allocation variant
//
// qkv_decode_attention with its workspace in a file-scope device array of
// QKV_NOALLOC_SCRATCH_BYTES instead of a caller buffer, for callers that
// cannot allocate.  Each GPU holds its own copy of the array (for the life of
// the process); its address on the current device is looked up once per
// device with hipGetSymbolAddress and only that address is handed to kernels.
// Every kernel of the decode step writes each workspace entry it later reads
// (query operands, row constants, split partials), so nothing has to start at
// zero.  Calls that overlap on one GPU share the array and race.
namespace {

static __device__ __align__(256) uint8_t scratch[QKV_NOALLOC_SCRATCH_BYTES];

constexpr int kScratchDevices = 64;
std::mutex scratch_mu;
void* scratch_dev[kScratchDevices] = {};

// Address of `scratch` on the current device (nullptr + error set on failure).
void* scratch_on_current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kScratchDevices) {
    qkv_set_error("no usable current HIP device for the scratch array");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (scratch_dev[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      qkv_set_error("hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                    hipGetErrorString(e));
      return nullptr;
    }
    scratch_dev[dev] = ptr;
  }
  return scratch_dev[dev];
}

}  // namespace

extern "C" int qkv_decode_attention_noalloc(const void* q, int32_t q_dtype,
                                            const uint8_t* kstore, const float* knorm,
                                            const uint32_t* vstore, const float* vnorm,
                                            int64_t t_stride, int64_t T, int32_t B, int32_t Hq,
                                            int32_t Hkv, int32_t Q, int32_t d, int32_t kbits,
                                            int32_t vbits, const float* pi,
                                            const float* kcent_host, const float* vcent_host,
                                            const float* signs, float qjl_scale, float scale,
                                            int32_t causal, void* out, int32_t out_dtype,
                                            int32_t n_splits, void* stream) {
  QKV_REQUIRE(B > 0 && Hq > 0 && Hkv > 0 && Q > 0 && Hq % Hkv == 0, "invalid shape");
  QKV_REQUIRE(n_splits >= 1 && n_splits <= 1024, "n_splits %d out of range", n_splits);
  const int64_t need = qkv_attention_workspace_bytes(B, Hq, Hkv, Q, d, n_splits);
  QKV_REQUIRE(need > 0, "invalid shape");
  QKV_REQUIRE(need <= int64_t(QKV_NOALLOC_SCRATCH_BYTES),
              "qkv_decode_attention_noalloc: this call needs %lld workspace bytes, more than "
              "the %lld-byte scratch array (use qkv_decode_attention with a workspace)",
              (long long)need, (long long)QKV_NOALLOC_SCRATCH_BYTES);
  void* ws = scratch_on_current_device();
  if (ws == nullptr) return QKV_E_HIP;
  return qkv_decode_attention(q, q_dtype, kstore, knorm, vstore, vnorm, t_stride, T, B, Hq, Hkv,
                              Q, d, kbits, vbits, pi, kcent_host, vcent_host, signs, qjl_scale,
                              scale, causal, out, out_dtype, ws, QKV_NOALLOC_SCRATCH_BYTES,
                              n_splits, stream);
}

// Decode attention over a paged store (pages of 64 tokens holding all Hkv
// heads of one sequence; see QkvPages): the MFMA path only.
extern "C" int qkv_paged_decode_attention(
    const void* q, int32_t q_dtype, const uint8_t* kpool, const float* knorm,
    const uint32_t* vpool, const float* vnorm, const int32_t* page_table, int32_t pages_per_seq,
    int32_t page_tokens, int32_t num_pages, int64_t T, int32_t B, int32_t Hq, int32_t Hkv,
    int32_t Q, int32_t d, int32_t kbits,
    int32_t vbits, const float* pi, const float* kcent_host, const float* vcent_host,
    const float* signs, float qjl_scale, float scale, int32_t causal, void* out,
    int32_t out_dtype, void* workspace, int64_t ws_bytes, int32_t n_splits, void* stream) {
  QKV_REQUIRE(qkv_dtype_ok(q_dtype) && qkv_dtype_ok(out_dtype), "unsupported dtype");
  QKV_REQUIRE(qkv_bits_ok(kbits) && qkv_bits_ok(vbits), "bits must be in {1, 2, 3, 4}");
  QKV_REQUIRE(T > 0, "No compressed KV blocks in cache. Call append() first.");
  QKV_REQUIRE(page_table && pages_per_seq > 0 && qkv_aligned(page_table, 4),
              "page table missing or not 4-byte aligned");
  QKV_REQUIRE(num_pages > 0, "num_pages %d must be positive", num_pages);
  const int plg = qkv_page_lg(page_tokens);
  QKV_REQUIRE(plg > 0, "page_tokens %d must be 64, 128, ..., 2048", page_tokens);
  QKV_REQUIRE(T <= (int64_t(pages_per_seq) << plg),
              "%lld tokens exceed the page table's %d pages of %d", (long long)T, pages_per_seq,
              page_tokens);
  int st = validate_common(B, Hq, Hkv, Q, d, n_splits, workspace, ws_bytes);
  if (st != QKV_OK) return st;
  QKV_REQUIRE(q && kpool && knorm && vpool && vnorm && pi && kcent_host && vcent_host && signs &&
                  out,
              "null pointer");
  const int64_t t_stride = int64_t(pages_per_seq) << plg;
  if (!use_fused(make_tables(kcent_host, kbits, vcent_host, vbits), d, t_stride)) {
    qkv_set_error("paged stores decode on the MFMA path only (symmetric codebooks, key MSE "
                  "bits <= 3)");
    return QKV_E_UNSUPPORTED;
  }
  QKV_REQUIRE(qkv_dtype_ok(out_dtype) && qkv_aligned(pi, 16), "pi must be 16-byte aligned");
  KVLayers kv{};
  kv.kst[0] = kpool;
  kv.knorm[0] = knorm;
  kv.vst[0] = vpool;
  kv.vnorm[0] = vnorm;
  kv.ptab = page_table;
  kv.pmax = pages_per_seq;
  kv.plg = plg;
  kv.npages = num_pages;
  {  // the kernels of the contiguous single call: decode_small at d = 64 with
     // key MSE bits <= 2, decode_fused otherwise
    QLayers ql{};
    ql.q[0] = q;
    ql.pi[0] = pi;
    ql.signs[0] = signs;
    OutLayers ol{};
    ol.pi[0] = pi;
    ol.out[0] = out;
    auto s = static_cast<hipStream_t>(stream);
    const Tables tb = make_tables(kcent_host, kbits, vcent_host, vbits);
    if (d == 64 && tb.mfma_ok) {
      st = launch_small(ql, kv, ol, 1, B, q_dtype, qjl_scale, Hq, Hkv, Q, kbits, vbits, tb,
                        t_stride, T, scale, causal, n_splits, 1, out_dtype, workspace, s);
      if (st != QKV_OK || n_splits == 1) return st;
      return combine_layers(ol, 1, B, Hq, Hkv, Q, d, out_dtype, workspace, ws_bytes, n_splits,
                            s);
    }
    st = launch_fused(ql, kv, ol, 1, B, q_dtype, qjl_scale, Hq, Hkv, Q, d,
                      (d / 32) * (kbits + 1), vbits,
                      make_tables(kcent_host, kbits, vcent_host, vbits), t_stride, T, scale,
                      causal, n_splits, 1, out_dtype, workspace, true, s);
    if (st != QKV_OK || n_splits == 1) return st;
    return combine_layers(ol, 1, B, Hq, Hkv, Q, d, out_dtype, workspace, ws_bytes, n_splits, s);
  }
}

// One decode step over n_layers layers that share shapes, bit widths and
// codebooks (a model's layers), as three launches instead of 3 n_layers.
// Per-layer device pointers come in HOST arrays of n_layers entries; the
// workspace is sized for a batch of B * n_layers sequences.  Only the MFMA
// path takes layers (symmetric codebooks, key MSE bits <= 2, d = 64 or 128,
// store capacity a multiple of 64, splits of at most 2048 tokens).
// The layer-batched decode over contiguous stores (page_table null) or over
// per-layer page pools sharing one page table (pages of 1 << plg tokens).
static int decode_layers(int32_t n_layers, const void* const* q, int32_t q_dtype,
                         const uint8_t* const* kstore, const float* const* knorm,
                         const uint32_t* const* vstore, const float* const* vnorm,
                         int64_t t_stride, int64_t T, int32_t B, int32_t Hq, int32_t Hkv,
                         int32_t Q, int32_t d, int32_t kbits, int32_t vbits,
                         const float* const* pi, const float* kcent_host,
                         const float* vcent_host, const float* const* signs, float qjl_scale,
                         float scale, int32_t causal, void* const* out, int32_t out_dtype,
                         void* workspace, int64_t ws_bytes, int32_t n_splits, void* stream,
                         const int32_t* page_table, int32_t pages_per_seq, int plg,
                         int32_t num_pages) {
  QKV_REQUIRE(n_layers >= 1 && n_layers <= kMaxLayers, "n_layers %d not in 1..%d", n_layers,
              kMaxLayers);
  QKV_REQUIRE(q && kstore && knorm && vstore && vnorm && pi && signs && out && kcent_host &&
                  vcent_host,
              "null pointer");
  QKV_REQUIRE(qkv_dtype_ok(q_dtype) && qkv_dtype_ok(out_dtype), "unsupported dtype");
  QKV_REQUIRE(qkv_bits_ok(kbits) && qkv_bits_ok(vbits), "bits must be in {1, 2, 3, 4}");
  QKV_REQUIRE(T > 0, "No compressed KV blocks in cache. Call append() first.");
  QKV_REQUIRE(t_stride >= T && t_stride % 32 == 0,
              "t_stride %lld must be >= T %lld and a multiple of 32", (long long)t_stride,
              (long long)T);
  int st = validate_common(B * n_layers, Hq, Hkv, Q, d, n_splits, workspace, ws_bytes);
  if (st != QKV_OK) return st;
  const Tables tb = make_tables(kcent_host, kbits, vcent_host, vbits);
  // d = 64 batches run decode_small (its two row chunks per workgroup read a
  // 5-8-row GQA group's K/V once) where it takes the shape (key MSE bits <= 2),
  // decode_fused otherwise, as every other head dim
  const bool split64 = d == 64 && tb.mfma_ok && t_stride % 64 == 0;
  if (!split64 && !use_fused(tb, d, t_stride)) {
    qkv_set_error("layer-batched decode runs on the MFMA path (symmetric codebooks, key MSE "
                  "bits <= 3, capacity a multiple of 64)");
    return QKV_E_UNSUPPORTED;
  }
  QLayers ql{};
  KVLayers kv{};
  OutLayers ol{};
  for (int l = 0; l < n_layers; ++l) {
    ql.q[l] = q[l];
    ql.pi[l] = pi[l];
    ql.signs[l] = signs[l];
    kv.kst[l] = kstore[l];
    kv.knorm[l] = knorm[l];
    kv.vst[l] = vstore[l];
    kv.vnorm[l] = vnorm[l];
    ol.pi[l] = pi[l];
    ol.out[l] = out[l];
  }
  kv.ptab = page_table;
  kv.pmax = pages_per_seq;
  kv.plg = plg;
  kv.npages = num_pages;
  auto s = static_cast<hipStream_t>(stream);
  if (split64) {
    // decode_small: one launch; one split per (sequence, kv head) where that
    // gives at least two workgroups per CU, else the caller's split count
    const int R = (Hq / Hkv) * Q;
    const int rows_wg = R > kRowsM ? 2 * kRowsM : kRowsM;
    const int64_t wgs = int64_t(B) * n_layers * Hkv * ((R + rows_wg - 1) / rows_wg);
    const int ns = wgs >= 2 * int64_t(qkv_num_cus()) ? 1 : n_splits;
    st = launch_small(ql, kv, ol, n_layers, B, q_dtype, qjl_scale, Hq, Hkv, Q, kbits, vbits, tb,
                      t_stride, T, scale, causal, ns, 1, out_dtype, workspace, s);
    if (st != QKV_OK || ns == 1) return st;
    return combine_layers(ol, n_layers, B, Hq, Hkv, Q, d, out_dtype, workspace, ws_bytes, ns,
                          s);
  }
  {
    st = launch_fused(ql, kv, ol, n_layers, B, q_dtype, qjl_scale, Hq, Hkv, Q, d,
                      (d / 32) * (kbits + 1), vbits, tb,
                      t_stride, T, scale, causal, n_splits, 1, out_dtype, workspace, true, s);
    if (st != QKV_OK || n_splits == 1) return st;
    return combine_layers(ol, n_layers, B, Hq, Hkv, Q, d, out_dtype, workspace, ws_bytes,
                          n_splits, s);
  }
}

extern "C" int qkv_decode_attention_layers(
    int32_t n_layers, const void* const* q, int32_t q_dtype, const uint8_t* const* kstore,
    const float* const* knorm, const uint32_t* const* vstore, const float* const* vnorm,
    int64_t t_stride, int64_t T, int32_t B, int32_t Hq, int32_t Hkv, int32_t Q, int32_t d,
    int32_t kbits, int32_t vbits, const float* const* pi, const float* kcent_host,
    const float* vcent_host, const float* const* signs, float qjl_scale, float scale,
    int32_t causal, void* const* out, int32_t out_dtype, void* workspace, int64_t ws_bytes,
    int32_t n_splits, void* stream) {
  return decode_layers(n_layers, q, q_dtype, kstore, knorm, vstore, vnorm, t_stride, T, B, Hq,
                       Hkv, Q, d, kbits, vbits, pi, kcent_host, vcent_host, signs, qjl_scale,
                       scale, causal, out, out_dtype, workspace, ws_bytes, n_splits, stream,
                       nullptr, 0, 0, 0);
}

// One decode step over n_layers layers kept in paged stores: per-layer page
// pools (host arrays of device pointers) and ONE page table shared by every
// layer, as a serving engine's block table is.
extern "C" int qkv_paged_decode_attention_layers(
    int32_t n_layers, const void* const* q, int32_t q_dtype, const uint8_t* const* kpool,
    const float* const* knorm, const uint32_t* const* vpool, const float* const* vnorm,
    const int32_t* page_table, int32_t pages_per_seq, int32_t page_tokens, int32_t num_pages,
    int64_t T, int32_t B, int32_t Hq, int32_t Hkv, int32_t Q, int32_t d, int32_t kbits,
    int32_t vbits, const float* const* pi, const float* kcent_host, const float* vcent_host,
    const float* const* signs, float qjl_scale, float scale, int32_t causal, void* const* out,
    int32_t out_dtype, void* workspace, int64_t ws_bytes, int32_t n_splits, void* stream) {
  QKV_REQUIRE(page_table && pages_per_seq > 0 && qkv_aligned(page_table, 4),
              "page table missing or not 4-byte aligned");
  QKV_REQUIRE(num_pages > 0, "num_pages %d must be positive", num_pages);
  const int plg = qkv_page_lg(page_tokens);
  QKV_REQUIRE(plg > 0, "page_tokens %d must be 64, 128, ..., 2048", page_tokens);
  QKV_REQUIRE(T <= (int64_t(pages_per_seq) << plg),
              "%lld tokens exceed the page table's %d pages of %d", (long long)T, pages_per_seq,
              page_tokens);
  return decode_layers(n_layers, q, q_dtype, kpool, knorm, vpool, vnorm,
                       int64_t(pages_per_seq) << plg, T, B, Hq, Hkv, Q, d, kbits, vbits, pi,
                       kcent_host, vcent_host, signs, qjl_scale, scale, causal, out, out_dtype,
                       workspace, ws_bytes, n_splits, stream, page_table, pages_per_seq, plg,
                       num_pages);
}

namespace {

// Decode attention over mixed-precision K rows (kind 1: MSE keys, kind 2: IP
// keys; signs_perm and qjl_scale for kind 2) and b-bit MSE V tiles.  Only
// decode_fused reads these row formats, so the store and split shape must
// admit it.
int kmixed_decode_impl(int kind, const void* q, int32_t q_dtype, const uint8_t* kstore,
                       const float* knorm, const uint32_t* vstore, const float* vnorm,
                       int64_t t_stride, int64_t T, int32_t B, int32_t Hq, int32_t Hkv,
                       int32_t Q, int32_t d, int32_t vbits, const float* pi_perm,
                       const float* signs_perm, float qjl_scale, int32_t n_out,
                       const float* out_cent_host, const float* reg_cent_host,
                       const float* pi_v, const float* vcent_host, float scale, int32_t causal,
                       void* out, int32_t out_dtype, void* workspace, int64_t ws_bytes,
                       int32_t n_splits, void* stream) {
  QKV_REQUIRE(qkv_dtype_ok(q_dtype) && qkv_dtype_ok(out_dtype), "unsupported dtype");
  QKV_REQUIRE(qkv_bits_ok(vbits), "bits must be in {1, 2, 3, 4}");
  QKV_REQUIRE(T > 0, "No compressed KV blocks in cache. Call append() first.");
  int st = validate_common(B, Hq, Hkv, Q, d, n_splits, workspace, ws_bytes);
  if (st != QKV_OK) return st;
  QKV_REQUIRE(q && kstore && knorm && vstore && vnorm && pi_perm && out_cent_host &&
                  reg_cent_host && pi_v && vcent_host && out && (kind == 1 || signs_perm),
              "null pointer");
  // the value tables (the key entries of make_tables are unused here)
  Tables tb = make_tables(reg_cent_host, kind == 1 ? 2 : 1, vcent_host, vbits);
  if (d != 128 || (n_out != 32 && n_out != 64) || !use_fused(tb, d, t_stride) ||
      !add_kmix(tb, kind, out_cent_host, reg_cent_host, n_out)) {
    qkv_set_error("mixed-precision keys need head_dim 128, 32 or 64 outlier channels, a store "
                  "capacity that is a multiple of 64 and symmetric codebooks");
    return QKV_E_UNSUPPORTED;
  }
  QKV_REQUIRE(qkv_aligned(pi_perm, 16) && qkv_aligned(pi_v, 16), "pi must be 16-byte aligned");
  QKV_REQUIRE(qkv_aligned(kstore, 4), "K rows must be 4-byte aligned");
  QLayers ql{};
  ql.q[0] = q;
  ql.pi[0] = pi_perm;
  // MSE keys: read, weighted by alpha = 0 (no QJL term)
  ql.signs[0] = kind == 1 ? pi_perm : signs_perm;
  KVLayers kv{};
  kv.kst[0] = kstore;
  kv.knorm[0] = knorm;
  kv.vst[0] = vstore;
  kv.vnorm[0] = vnorm;
  OutLayers ol{};
  ol.pi[0] = pi_v;
  ol.out[0] = out;
  auto s = static_cast<hipStream_t>(stream);
  st = launch_fused(ql, kv, ol, 1, B, q_dtype, kind == 1 ? 0.f : qjl_scale, Hq, Hkv, Q, d,
                    kmixed_rdw(kind, n_out), vbits, tb, t_stride, T, scale, causal, n_splits, 1,
                    out_dtype, workspace, true, s);
  if (st != QKV_OK || n_splits == 1) return st;
  return combine_layers(ol, 1, B, Hq, Hkv, Q, d, out_dtype, workspace, ws_bytes, n_splits, s);
}

}  // namespace

extern "C" int qkv_decode_attention_kmixed(
    const void* q, int32_t q_dtype, const uint8_t* kstore, const float* knorm,
    const uint32_t* vstore, const float* vnorm, int64_t t_stride, int64_t T, int32_t B,
    int32_t Hq, int32_t Hkv, int32_t Q, int32_t d, int32_t vbits, const float* pi_perm,
    int32_t n_out, const float* out_cent_host, const float* reg_cent_host, const float* pi_v,
    const float* vcent_host, float scale, int32_t causal, void* out, int32_t out_dtype,
    void* workspace, int64_t ws_bytes, int32_t n_splits, void* stream) {
  return kmixed_decode_impl(1, q, q_dtype, kstore, knorm, vstore, vnorm, t_stride, T, B, Hq, Hkv,
                            Q, d, vbits, pi_perm, nullptr, 0.f, n_out, out_cent_host,
                            reg_cent_host, pi_v, vcent_host, scale, causal, out, out_dtype,
                            workspace, ws_bytes, n_splits, stream);
}

extern "C" int qkv_decode_attention_kipmixed(
    const void* q, int32_t q_dtype, const uint8_t* kstore, const float* knorm,
    const uint32_t* vstore, const float* vnorm, int64_t t_stride, int64_t T, int32_t B,
    int32_t Hq, int32_t Hkv, int32_t Q, int32_t d, int32_t vbits, const float* pi_perm,
    const float* signs_perm, float qjl_scale, int32_t n_out, const float* out_cent_host,
    const float* reg_cent_host, const float* pi_v, const float* vcent_host, float scale,
    int32_t causal, void* out, int32_t out_dtype, void* workspace, int64_t ws_bytes,
    int32_t n_splits, void* stream) {
  return kmixed_decode_impl(2, q, q_dtype, kstore, knorm, vstore, vnorm, t_stride, T, B, Hq, Hkv,
                            Q, d, vbits, pi_perm, signs_perm, qjl_scale, n_out, out_cent_host,
                            reg_cent_host, pi_v, vcent_host, scale, causal, out, out_dtype,
                            workspace, ws_bytes, n_splits, stream);
}

// ------------------------------------------------------------ MIPS search (ABI)

// Device-wide per-query bounds start at -inf.
__global__ __launch_bounds__(256) void mips_init(uint32_t* __restrict__ gth, int M) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < M) gth[i] = 0x007fffffu;  // fkey(-inf)
}

// Queries (fp32), Pi and S of a d < 128 index zero-padded to 128.
__global__ __launch_bounds__(256) void mips_pad(const void* __restrict__ q, int q_dtype, int M,
                                                int d, const float* __restrict__ pi,
                                                const float* __restrict__ signs,
                                                float* __restrict__ qp, float* __restrict__ pip,
                                                float* __restrict__ sp) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  const int64_t nq = int64_t(M) * 128;
  if (i < nq) {
    const int64_t m = i / 128;
    const int j = static_cast<int>(i - m * 128);
    qp[i] = j < d ? qkv_load(q, m * d + j, q_dtype) : 0.f;
  } else if (i < nq + 128 * 128) {
    const int64_t e = i - nq;
    const int r = static_cast<int>(e / 128), c = static_cast<int>(e % 128);
    pip[e] = (r < d && c < d) ? pi[r * d + c] : 0.f;
  } else if (i < nq + 128 * 128 + 128) {
    const int j = static_cast<int>(i - nq - 128 * 128);
    sp[j] = j < d ? signs[j] : 0.f;
  }
}

namespace {

struct MipsLayout {
  int64_t aq, rowc, cs, ci, gth, pad, total;
};

// Vector chunks per query tile: enough (query tile, chunk) items for several
// per workgroup slot (12 per CU: six per workgroup at two per CU; fewer,
// longer chunks fill fewer per-chunk top-k lists -- cfg5 14.0 ms against
// 14.4 at 24 per CU and 15.4 at 48), chunks of at least 16 steps, at most
// 256 chunks.
int mips_splits(int32_t M, int64_t N, int mbits) {
  const int qc = mbits <= 2 ? 4 : 2;
  const int64_t qtiles = (M + 16 * qc - 1) / (16 * qc);
  const int64_t want = (12 * int64_t(qkv_num_cus()) + qtiles - 1) / qtiles;
  const int64_t maxs = std::max<int64_t>(1, (N + 16 * kMipsStep - 1) / (16 * kMipsStep));
  return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>({want, maxs, 256})));
}

MipsLayout mips_layout(int32_t M, int d, int mbits, int k, int nsplit) {
  const int ns = n_odd_subsets(mbits);
  const int64_t nu = 2 * (ns + 1);
  const int64_t chunks = (M + kRowsM - 1) / kRowsM;
  MipsLayout w{};
  int64_t off = 0;
  auto up = [](int64_t x) { return (x + 255) / 256 * 256; };
  w.aq = off;   off += up(chunks * nu * 64 * 16);
  w.rowc = off; off += up(chunks * kRowsM * 2 * 4);
  w.cs = off;   off += up(int64_t(M) * nsplit * k * 4);
  w.ci = off;   off += up(int64_t(M) * nsplit * k * 4);
  w.gth = off;  off += up(int64_t(M) * 4);
  w.pad = off;  // d < 128: padded queries, Pi and S (fp32)
  if (d < 128) off += up((int64_t(M) * 128 + 128 * 128 + 128) * 4);
  w.total = off;
  return w;
}

int64_t mips_scan_smem(int d, int mbits, int k) {
  const int rawd = (mbits + 1) * (d / 32), qw = 4 * (mbits <= 2 ? 4 : 2);
  return 2 * (int64_t(kMipsStep) * rawd * 4 + kMipsStep * 4) + int64_t(4) * qw * k * 8;
}

}  // namespace

extern "C" int64_t qkv_mips_workspace_bytes(int32_t M, int32_t d, int32_t mbits, int32_t k,
                                            int64_t N) {
  if (M <= 0 || !qkv_d_ok(d) || mbits < 1 || mbits > 3 || k <= 0 || N <= 0) return -1;
  const int kk = static_cast<int>(std::min<int64_t>(k, N));
  return mips_layout(M, d, mbits, kk, mips_splits(M, N, mbits)).total;
}

extern "C" int qkv_mips_search(const void* queries, int32_t q_dtype, int32_t M, int32_t d,
                               int32_t mbits, const float* pi, const float* signs,
                               const float* kcent_host, float qjl_scale, const uint8_t* kstore,
                               const float* norms, int64_t N, int32_t k, float* out_scores,
                               int64_t* out_indices, void* workspace, int64_t ws_bytes,
                               void* stream) {
  QKV_REQUIRE(qkv_dtype_ok(q_dtype), "unsupported query dtype %d", q_dtype);
  QKV_REQUIRE(N > 0, "Index is empty. Call add() first.");
  QKV_REQUIRE(N < (int64_t(1) << 31), "index holds at most 2^31 - 1 vectors");
  QKV_REQUIRE(M > 0 && k > 0, "invalid shape");
  if (!qkv_d_ok(d) || mbits < 1 || mbits > 3) {
    qkv_set_error("search runs on dim 64, 96 or 128 with 2..4-bit codes (got dim %d, %d MSE "
                  "bits)", d, mbits);
    return QKV_E_UNSUPPORTED;
  }
  k = static_cast<int32_t>(std::min<int64_t>(k, N));
  if (k > kMipsKMax) {
    qkv_set_error("search returns at most %d neighbours per query (asked %d)", kMipsKMax, k);
    return QKV_E_UNSUPPORTED;
  }
  QKV_REQUIRE(queries && pi && signs && kcent_host && kstore && norms && out_scores &&
                  out_indices && workspace,
              "null pointer");
  QKV_REQUIRE(qkv_aligned(pi, 16) && qkv_aligned(kstore, 4) && qkv_aligned(workspace, 256),
              "pi 16-B, store 4-B and workspace 256-B aligned");
  Tables tb{};
  for (int i = 0; i < (1 << mbits); ++i) tb.kc[i] = kcent_host[i];
  if (!walsh_odd(kcent_host, mbits, tb.kg, &tb.kconst)) {
    qkv_set_error("search needs a symmetric key codebook");
    return QKV_E_UNSUPPORTED;
  }
  tb.mfma_ok = 1;
  const int nsplit = mips_splits(M, N, mbits);
  const MipsLayout L = mips_layout(M, d, mbits, k, nsplit);
  QKV_REQUIRE(ws_bytes >= L.total, "workspace too small: %lld < %lld", (long long)ws_bytes,
              (long long)L.total);
  auto s = static_cast<hipStream_t>(stream);
  const int chunks = (M + kRowsM - 1) / kRowsM;
  qkv_v4i* aq = at<qkv_v4i>(workspace, L.aq);
  float* rowc = at<float>(workspace, L.rowc);
  float* cs = at<float>(workspace, L.cs);
  int* ci = at<int>(workspace, L.ci);
  uint32_t* gth = at<uint32_t>(workspace, L.gth);
  hipLaunchKernelGGL(mips_init, dim3((M + 255) / 256), dim3(256), 0, s, gth, M);
  const void* qsrc = queries;
  int qdt = q_dtype;
  const float* pisrc = pi;
  const float* ssrc = signs;
  if (d < 128) {
    float* qp = at<float>(workspace, L.pad);
    float* pip = qp + int64_t(M) * 128;
    float* sp = pip + 128 * 128;
    const int64_t n = int64_t(M) * 128 + 128 * 128 + 128;
    hipLaunchKernelGGL(mips_pad, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s,
                       queries, q_dtype, M, d, pi, signs, qp, pip, sp);
    QKV_LAUNCHED();
    qsrc = qp;
    qdt = QKV_F32;
    pisrc = pip;
    ssrc = sp;
  }
  // query operands: the decode prepare kernel with one "kv head" of M rows
  QLayers ql{};
  ql.q[0] = qsrc;
  ql.pi[0] = pisrc;
  ql.signs[0] = ssrc;
#define QKV_PREP(NPLV)                                                                        \
  hipLaunchKernelGGL((prepare_mfma<128, NPLV, false>), dim3(chunks), dim3(256),                     \
                     (prep_lds<128, NPLV, false>()), s, ql, 1, qdt,                                \
                     qjl_scale, M, 1, 1, M, chunks, tb, aq, rowc, nullptr)
  if (mbits == 1) QKV_PREP(2);
  else if (mbits == 2) QKV_PREP(3);
  else QKV_PREP(5);
#undef QKV_PREP
  QKV_LAUNCHED();
  const int qc = mbits <= 2 ? 4 : 2;
  const int64_t vlen = ((N + nsplit - 1) / nsplit + kMipsStep - 1) / kMipsStep * kMipsStep;
  const int64_t qtiles = (chunks + 4 * qc - 1) / (4 * qc);
  const int64_t n_items = qtiles * nsplit;
  const int64_t smem = mips_scan_smem(d, mbits, k);
  int per_cu = 0;
  switch (mbits * 10 + d / 32) {
#define QKV_OCC(MBV, PDWV, CASEV)                                                         \
  case CASEV:                                                                             \
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, mips_scan<MBV, PDWV>, 256,  \
                                                     static_cast<size_t>(smem)) != hipSuccess) \
      per_cu = 0;                                                                         \
    break;
    QKV_OCC(1, 2, 12) QKV_OCC(1, 3, 13) QKV_OCC(1, 4, 14)
    QKV_OCC(2, 2, 22) QKV_OCC(2, 3, 23) QKV_OCC(2, 4, 24)
    QKV_OCC(3, 2, 32) QKV_OCC(3, 3, 33) QKV_OCC(3, 4, 34)
#undef QKV_OCC
  }
  per_cu = std::max(per_cu, 1);
  const dim3 grid(static_cast<unsigned>(
      std::min<int64_t>(n_items, int64_t(per_cu) * qkv_num_cus())));
#define QKV_SCAN(MBV, PDWV)                                                                       \
  do {                                                                                            \
    if (smem > 65536)                                                                             \
      QKV_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&mips_scan<MBV, PDWV>),          \
                                  hipFuncAttributeMaxDynamicSharedMemorySize,                     \
                                  static_cast<int>(smem)));                                       \
    hipLaunchKernelGGL((mips_scan<MBV, PDWV>), grid, dim3(256), static_cast<uint32_t>(smem), s,  \
                       aq, rowc, M, kstore, norms, N, nsplit, vlen, n_items, k, cs, ci, gth);     \
  } while (0)
  switch (mbits * 10 + d / 32) {
    case 12: QKV_SCAN(1, 2); break;
    case 13: QKV_SCAN(1, 3); break;
    case 14: QKV_SCAN(1, 4); break;
    case 22: QKV_SCAN(2, 2); break;
    case 23: QKV_SCAN(2, 3); break;
    case 24: QKV_SCAN(2, 4); break;
    case 32: QKV_SCAN(3, 2); break;
    case 33: QKV_SCAN(3, 3); break;
    case 34: QKV_SCAN(3, 4); break;
  }
#undef QKV_SCAN
  QKV_LAUNCHED();
  const int64_t msmem = int64_t(nsplit) * k * 8;
  if (msmem > 65536)
    QKV_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&mips_merge),
                                hipFuncAttributeMaxDynamicSharedMemorySize,
                                static_cast<int>(std::min<int64_t>(msmem, 160 * 1024))));
  QKV_REQUIRE(msmem <= 160 * 1024, "too many candidates per query");
  hipLaunchKernelGGL(mips_merge, dim3(M), dim3(64), static_cast<uint32_t>(msmem), s, cs, ci,
                     nsplit, k, out_scores, out_indices);
  QKV_LAUNCHED();
  return QKV_OK;
}
