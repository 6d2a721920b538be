// Fused decompress on the matrix cores (d = 64 and 128):
//
//   x^ = ((c[code] [+ qjl_scale S (2 bit - 1)]) Pi) * n
//
// Reference: quashkv/triton_kernels/decompress.py:32-96 (PyTorch path) and
// :104-187 (per-vector kernels), quashkv/quantizer.py:133-147; the full-cache
// reconstruction of QuashKVCache (quashkv/integrations/hf_cache.py:96-121)
// reads the engine's K rows and V tiles through the same kernel.
//
// GEMM.  One wave turns a block of 16 R vectors into their outputs with
// 16x16x32 fp16 MFMAs, C = Pi^T V^T: the A operand is a 16-column slice of Pi
// (rows j of Pi^T), the B operand 16 vectors' values v_k = c[code_k]
// (+ qjl term).  A result VGPR quad holds four consecutive output coordinates
// of one vector, so the stores are 16-byte vector writes.
//
// Precision.  Pi and the values are split into fp16 high and low parts
// (p = p_hi + p_lo, v = v_hi + v_lo, each part rounded to nearest) after
// scaling both by powers of two that bring their largest magnitude into
// [1, 2), and three MFMA passes accumulate p_hi v_hi + p_lo v_hi + p_hi v_lo in
// fp32: every product carries ~22 significant bits and the dropped p_lo v_lo
// term is ~2^-22 relative, within a few fp32 rounding steps of the reference's
// fp32 loop.  The scales are undone exactly in the final multiply by n.
//
// k order.  Lane l of a wave (vector l mod 16, k group g = l / 16) owns the d/4
// consecutive coordinates g d/4 .. g d/4 + d/4 - 1 of its vector; k-step ks of
// the MFMA takes its elements 8 ks .. 8 ks + 7.  Pi's fragments in LDS use the
// same coordinate order, so every lane reads its codes as one contiguous run
// of the row (32 bytes unpacked, 12 bytes of a 3-bit row at d = 128).
//
// Values come from a 32-entry LDS table (16 codes x the two codebooks of the
// mixed-precision format), pre-split into fp16 (hi, lo) pairs for MSE codes;
// IP codes add the per-coordinate qjl term in fp32 and split after.
//
// Code formats: unpacked bytes (code & 15), pack_bits rows
// (quashkv/packing.py:22-165), the store's K rows (bit planes of 32
// coordinates per dword, the QJL plane last) and V tiles (one dword per
// coordinate and plane holding 32 tokens' bits; a wave stages a tile in LDS
// and each lane gathers its token's bits).  Rows are addressed in groups of
// in_seq vectors spaced in_group_stride rows apart, as in the generic kernel.

#include <cmath>

#include "qkv_common.h"

namespace {

typedef _Float16 qkv_f16x8 __attribute__((ext_vector_type(8)));
typedef float qkv_f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;

__device__ __forceinline__ qkv_f32x4 mma(uint4 a, uint4 b, qkv_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(qkv_f16x8, a),
                                                __builtin_bit_cast(qkv_f16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t h16(_Float16 h) {
  return __builtin_bit_cast(uint16_t, h);
}

// hi | lo << 16: hi = fp16(v), lo = fp16(v - hi), both round to nearest
__device__ __forceinline__ uint32_t split_pair(float v) {
  const _Float16 h = static_cast<_Float16>(v);
  const _Float16 l = static_cast<_Float16>(v - static_cast<float>(h));
  return h16(h) | (h16(l) << 16);
}

// Power of two s with m s in [1, 2); 1 for m = 0 or a non-finite m.
__device__ __forceinline__ float pow2_scale(float m) {
  if (!(m > 0.f) || !(m <= 3.0e38f)) return 1.f;
  int e;
  frexpf(m, &e);  // m = f 2^e, f in [0.5, 1)
  return ldexpf(1.f, 1 - e);
}

// Output coordinate of C row mm (0..15) in column tile jt: tiles 2p and 2p+1
// interleave in quads so that lane group g holds coordinates 32 p + 8 g + 0..7.
__device__ __forceinline__ int out_col(int jt, int mm) {
  return 32 * (jt >> 1) + 8 * (mm >> 2) + 4 * (jt & 1) + (mm & 3);
}

__device__ __forceinline__ uint32_t bfe(uint32_t w, uint32_t off, uint32_t width) {
  return __builtin_amdgcn_ubfe(w, off, width);
}

// Bits 0..7 of b spread to bit 0 of the eight nibbles of a word.
__device__ __forceinline__ uint32_t spread8(uint32_t b) {
  b = (b | (b << 12)) & 0x000F000Fu;
  b = (b | (b << 6)) & 0x03030303u;
  b = (b | (b << 3)) & 0x11111111u;
  return b;
}

template <int D>
struct Geo {
  static constexpr int NE = D / 4;   // coordinates per lane
  static constexpr int NK = D / 32;  // MFMA k-steps
  static constexpr int NJ = D / 16;  // output column tiles
  static constexpr int NW = NE / 8;  // nibble words per lane
};

// A lane's codes of one vector, as read from the row, and the element access.
//   UNPACKED: NE bytes (SEL: bit 4 of byte = mixed-precision selector)
//   PACKED:   NE * BITS bits of the pack_bits stream
//   nibbles:  NE 4-bit codes, 8 per word (K rows and V tiles are turned into
//             this form from their bit planes)
template <int D, int FMT, int BITS>
struct CodeWords {
  static constexpr int N = FMT == QKV_FMT_UNPACKED ? D / 16
                         : FMT == QKV_FMT_PACKED   ? (D * BITS / 4 + 31) / 32
                                                   : D / 32;
  uint32_t w[N];

  __device__ __forceinline__ uint32_t code(int e) const {
    if constexpr (FMT == QKV_FMT_UNPACKED) {
      return bfe(w[e >> 2], 8 * (e & 3), 5);
    } else if constexpr (FMT == QKV_FMT_PACKED) {
      const int pos = BITS * e, i = pos >> 5, o = pos & 31;
      if (o + BITS <= 32) return bfe(w[i], o, BITS);
      return ((w[i] >> o) | (w[i + 1] << (32 - o))) & ((1u << BITS) - 1u);
    } else {
      return bfe(w[e >> 3], 4 * (e & 7), 4);
    }
  }
};

template <int D, int FMT>
struct QjlWords {
  static constexpr int N = FMT == QKV_FMT_UNPACKED ? D / 16 : 1;
  uint32_t w[N];
  // 1 for a QJL bit of 1 (+1), 0 for -1
  __device__ __forceinline__ bool bit(int e) const {
    if constexpr (FMT == QKV_FMT_UNPACKED) return bfe(w[e >> 2], 8 * (e & 3), 8) != 0u;
    else return ((w[0] >> e) & 1u) != 0u;
  }
};

// Lane's NE bits of a bit plane / 1-bit row starting at byte `p`.
template <int D>
__device__ __forceinline__ uint32_t lane_bits(const uint8_t* p, int g) {
  if constexpr (D == 128) return reinterpret_cast<const uint32_t*>(p)[g];
  else return reinterpret_cast<const uint16_t*>(p)[g];
}

template <int D, int FMT, int BITS, bool IP, bool SEL, int R>
__global__ __launch_bounds__(kThreads, 2) void decompress_mfma(
    const uint8_t* __restrict__ codes, const uint8_t* __restrict__ qjl,
    const float* __restrict__ norms, int64_t n, int bits, const float* __restrict__ pi,
    const float* __restrict__ cents, const float* __restrict__ signs, float qjl_scale,
    int64_t in_seq, int64_t in_gstride, void* __restrict__ out, int out_dtype,
    const uint8_t* __restrict__ sel, const float* __restrict__ alt_cents, int alt_bits) {
  using G = Geo<D>;
  constexpr int NE = G::NE, NK = G::NK, NJ = G::NJ, NW = G::NW;
  constexpr int RB = 16 * R;  // vectors per wave block
  constexpr bool VT = FMT == QKV_FMT_VTILES;
  static_assert(!VT || R % 2 == 0, "V tiles are 32 tokens: R must be even");
  __shared__ uint4 frag[NJ * NK * 2 * 64];  // [jt][ks][hi, lo][lane]
  __shared__ uint32_t tab[32];              // [codebook][code]
  __shared__ float red[kWaves + 1];
  __shared__ uint4 stage[VT ? kWaves * D : 1];  // one V tile (<= 4 planes) per wave

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m = lane & 15, g = lane >> 4;

  // ---- scales: Pi and the values into [1, 2) before the fp16 split
  float pm = 0.f;
  for (int i = tid; i < D * D; i += kThreads) pm = fmaxf(pm, fabsf(pi[i]));
  pm = qkv_wave_max(pm);
  float tv = 0.f;
  if (tid < 32) {
    const int s = tid >> 4, c = tid & 15;
    if (s == 0) tv = c < (1 << bits) ? cents[c] : 0.f;
    else if (SEL) tv = c < (1 << alt_bits) ? alt_cents[c] : 0.f;
  }
  const float vm = qkv_wave_max(fabsf(tv));
  if (lane == 0) red[wave] = pm;
  if (tid == 0) red[kWaves] = vm;
  __syncthreads();
  float pmax = red[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) pmax = fmaxf(pmax, red[w]);
  const float ps = pow2_scale(pmax);
  const float sv = pow2_scale(red[kWaves] + (IP ? fabsf(qjl_scale) : 0.f));
  if (tid < 32) tab[tid] = IP ? __float_as_uint(tv * sv) : split_pair(tv * sv);

  // ---- Pi fragments: lane l of (jt, ks) holds Pi[k][out_col(jt, l % 16)] for
  // the 8 coordinates k = (l / 16) NE + 8 ks + 0..7
  for (int i = tid; i < NJ * NK * 64; i += kThreads) {
    const int l = i & 63, blk = i >> 6;
    const int jt = blk / NK, ks = blk - jt * NK;
    const int col = out_col(jt, l & 15);
    const float* src = pi + int64_t((l >> 4) * NE + 8 * ks) * D + col;
    uint32_t hi[4], lo[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t a = split_pair(src[(2 * q) * D] * ps);
      const uint32_t b = split_pair(src[(2 * q + 1) * D] * ps);
      hi[q] = __builtin_amdgcn_perm(b, a, 0x05040100u);
      lo[q] = __builtin_amdgcn_perm(b, a, 0x07060302u);
    }
    frag[(2 * blk) * 64 + l] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    frag[(2 * blk + 1) * 64 + l] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
  }

  // ---- per-lane constants of its coordinates g NE .. g NE + NE - 1
  uint32_t selw[SEL ? NE / 4 : 1];
  if constexpr (SEL) {
#pragma unroll
    for (int c = 0; c < NE / 4; ++c) {
      uint32_t s = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) s |= (sel[g * NE + 4 * c + b] != 0 ? 0x10u : 0u) << (8 * b);
      selw[c] = s;
    }
  }
  float qs[IP ? NE : 1];
  if constexpr (IP) {
#pragma unroll
    for (int e = 0; e < NE; ++e) qs[e] = qjl_scale * signs[g * NE + e] * sv;
  }
  const float ofac = 1.f / (ps * sv);  // exact: a power of two
  __syncthreads();

  const int64_t groups = (n + in_seq - 1) / in_seq;
  const int64_t bpg = (in_seq + RB - 1) / RB;
  const int64_t nblk = groups * bpg;
  const int64_t pb = FMT == QKV_FMT_PACKED ? qkv_row_bytes(D, BITS)
                   : FMT == QKV_FMT_KPLANES ? int64_t(bits + 1) * (D / 8) : D;
  const int64_t pq = FMT == QKV_FMT_PACKED ? D / 8 : D;
  uint4* stg = &stage[VT ? wave * D : 0];

  for (int64_t blk = int64_t(blockIdx.x) * kWaves + wave; blk < nblk;
       blk += int64_t(gridDim.x) * kWaves) {
    const int64_t grp = blk / bpg;
    const int64_t t0 = (blk - grp * bpg) * RB;
    const int64_t tend = min(in_seq, n - grp * in_seq);  // valid tokens of the group

    uint4 ah[R][NK], al[R][NK];
    float nf[R];
    CodeWords<D, FMT, BITS> cw[R];
    QjlWords<D, FMT> qw[R];

    if constexpr (VT) {
      // tiles of 32 tokens: stage, then gather bit (m + 16 h) of the lane's NE
      // coordinate words of every plane into nibble codes
      const int nd4 = bits * D / 4;  // uint4 per tile
#pragma unroll
      for (int h = 0; h < R / 2; ++h) {
        const int64_t tt = t0 + 32 * h;
#pragma unroll
        for (int r = 2 * h; r < 2 * h + 2; ++r)
#pragma unroll
          for (int i = 0; i < NW; ++i) cw[r].w[i] = 0u;
        if (tt < tend) {
          const uint4* src = reinterpret_cast<const uint4*>(codes) +
                             ((grp * in_gstride + (tt >> 5)) * bits) * (D / 4);
          __builtin_amdgcn_wave_barrier();
          for (int i = lane; i < nd4; i += 64) stg[i] = src[i];
          __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the tile is in LDS
          __builtin_amdgcn_wave_barrier();
          for (int p = 0; p < bits; ++p) {
            const uint4* row = stg + p * (D / 4) + g * (NE / 4);
#pragma unroll
            for (int c = 0; c < NE / 4; ++c) {
              const uint4 v = row[c];
              const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
              for (int u = 0; u < 4; ++u) {
                const int e = 4 * c + u;
                const uint32_t sh = 4 * (e & 7) + p;
                cw[2 * h].w[e >> 3] |= bfe(wv[u], m, 1) << sh;
                cw[2 * h + 1].w[e >> 3] |= bfe(wv[u], m + 16, 1) << sh;
              }
            }
          }
        }
      }
    }

#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t t = t0 + 16 * r + m;
      const bool ok = t < tend;
      const int64_t row = grp * in_gstride + t;
      nf[r] = ok ? norms[VT ? grp * in_gstride * 32 + t : row] * ofac : 0.f;
      if constexpr (!VT) {
#pragma unroll
        for (int i = 0; i < CodeWords<D, FMT, BITS>::N; ++i) cw[r].w[i] = 0u;
#pragma unroll
        for (int i = 0; i < QjlWords<D, FMT>::N; ++i) qw[r].w[i] = 0u;
      }
      if (ok) {
        if constexpr (FMT == QKV_FMT_UNPACKED) {
          const uint4* src = reinterpret_cast<const uint4*>(codes + row * D + g * NE);
#pragma unroll
          for (int i = 0; i < NE / 16; ++i) {
            const uint4 v = src[i];
            cw[r].w[4 * i] = v.x; cw[r].w[4 * i + 1] = v.y;
            cw[r].w[4 * i + 2] = v.z; cw[r].w[4 * i + 3] = v.w;
          }
#pragma unroll
          for (int i = 0; i < NE / 4; ++i) {
            cw[r].w[i] &= 0x0F0F0F0Fu;
            if constexpr (SEL) cw[r].w[i] |= selw[i];
          }
          if constexpr (IP) {
            const uint4* qsrc = reinterpret_cast<const uint4*>(qjl + row * D + g * NE);
#pragma unroll
            for (int i = 0; i < NE / 16; ++i) {
              const uint4 v = qsrc[i];
              qw[r].w[4 * i] = v.x; qw[r].w[4 * i + 1] = v.y;
              qw[r].w[4 * i + 2] = v.z; qw[r].w[4 * i + 3] = v.w;
            }
          }
        } else if constexpr (FMT == QKV_FMT_PACKED) {
          const uint8_t* rp = codes + row * pb;
          if constexpr (D == 128) {
            const uint32_t* src = reinterpret_cast<const uint32_t*>(rp) + BITS * g;
#pragma unroll
            for (int i = 0; i < BITS; ++i) cw[r].w[i] = src[i];
          } else {
            const uint16_t* src = reinterpret_cast<const uint16_t*>(rp) + BITS * g;
#pragma unroll
            for (int i = 0; i < BITS; ++i) cw[r].w[i >> 1] |= uint32_t(src[i]) << (16 * (i & 1));
          }
          if constexpr (IP) qw[r].w[0] = lane_bits<D>(qjl + row * pq, g);
        } else if constexpr (FMT == QKV_FMT_KPLANES) {
          const uint8_t* rp = codes + row * pb;
          for (int p = 0; p < bits; ++p) {
            const uint32_t pw = lane_bits<D>(rp + p * (D / 8), g);
#pragma unroll
            for (int i = 0; i < NW; ++i) cw[r].w[i] |= spread8(bfe(pw, 8 * i, 8)) << p;
          }
          if constexpr (IP) qw[r].w[0] = lane_bits<D>(rp + bits * (D / 8), g);
        }
      }

      // values -> fp16 (hi, lo) fragments
#pragma unroll
      for (int ks = 0; ks < NK; ++ks) {
        uint32_t hv[4], lv[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int e0 = 8 * ks + 2 * q, e1 = e0 + 1;
          const uint32_t i0 = cw[r].code(e0), i1 = cw[r].code(e1);
          if constexpr (IP) {
            const float c0 = __uint_as_float(tab[i0]), c1 = __uint_as_float(tab[i1]);
            const float v0 = c0 + (qw[r].bit(e0) ? qs[e0] : -qs[e0]);
            const float v1 = c1 + (qw[r].bit(e1) ? qs[e1] : -qs[e1]);
            const uint32_t a = split_pair(v0), b = split_pair(v1);
            hv[q] = __builtin_amdgcn_perm(b, a, 0x05040100u);
            lv[q] = __builtin_amdgcn_perm(b, a, 0x07060302u);
          } else {
            const uint32_t a = tab[i0], b = tab[i1];
            hv[q] = __builtin_amdgcn_perm(b, a, 0x05040100u);
            lv[q] = __builtin_amdgcn_perm(b, a, 0x07060302u);
          }
        }
        ah[r][ks] = make_uint4(hv[0], hv[1], hv[2], hv[3]);
        al[r][ks] = make_uint4(lv[0], lv[1], lv[2], lv[3]);
      }
    }

    // ---- C = Pi^T V^T, two column tiles (32 output coordinates) at a time
#pragma unroll
    for (int p = 0; p < NJ / 2; ++p) {
      // one column pair at a time: keeps the scheduler from hoisting every
      // fragment read of the block ahead of the MFMAs
      __builtin_amdgcn_sched_barrier(0);
      qkv_f32x4 acc[2][R];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[hh][r] = qkv_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < NK; ++ks) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int blk2 = 2 * ((2 * p + hh) * NK + ks);
          const uint4 ph = frag[blk2 * 64 + lane];
          const uint4 pl = frag[(blk2 + 1) * 64 + lane];
#pragma unroll
          for (int r = 0; r < R; ++r) acc[hh][r] = mma(ph, ah[r][ks], acc[hh][r]);
#pragma unroll
          for (int r = 0; r < R; ++r) acc[hh][r] = mma(pl, ah[r][ks], acc[hh][r]);
#pragma unroll
          for (int r = 0; r < R; ++r) acc[hh][r] = mma(ph, al[r][ks], acc[hh][r]);
        }
      }
      // lane (m, g) holds coordinates 32 p + 8 g + 0..7 of vector t0 + 16 r + m
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int64_t t = t0 + 16 * r + m;
        if (t >= tend) continue;
        const int64_t o = (grp * in_seq + t) * D + 32 * p + 8 * g;
        const float f = nf[r];
        const float v[8] = {acc[0][r][0] * f, acc[0][r][1] * f, acc[0][r][2] * f,
                            acc[0][r][3] * f, acc[1][r][0] * f, acc[1][r][1] * f,
                            acc[1][r][2] * f, acc[1][r][3] * f};
        if (out_dtype == QKV_F32) {
          float4* dst = reinterpret_cast<float4*>(static_cast<float*>(out) + o);
          dst[0] = make_float4(v[0], v[1], v[2], v[3]);
          dst[1] = make_float4(v[4], v[5], v[6], v[7]);
        } else {
          uint32_t h[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            uint32_t a, b;
            if (out_dtype == QKV_F16) {
              a = h16(static_cast<_Float16>(v[2 * q]));
              b = h16(static_cast<_Float16>(v[2 * q + 1]));
            } else {
              a = qkv_f32_to_bf16(v[2 * q]);
              b = qkv_f32_to_bf16(v[2 * q + 1]);
            }
            h[q] = a | (b << 16);
          }
          *reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + o) =
              make_uint4(h[0], h[1], h[2], h[3]);
        }
      }
    }
  }
}

template <int D, int FMT, int BITS, bool IP, bool SEL, int R>
int launch(const QkvDecompressArgs& a, hipStream_t s) {
  auto k = decompress_mfma<D, FMT, BITS, IP, SEL, R>;
  static int per_cu = 0;
  if (per_cu == 0) {
    int b = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, k, kThreads, 0) != hipSuccess || b < 1)
      b = 1;
    per_cu = b;
  }
  const int64_t in_seq = a.in_seq;
  const int64_t groups = (a.n + in_seq - 1) / in_seq;
  const int64_t nblk = groups * ((in_seq + 16 * R - 1) / (16 * R));
  int64_t grid = (nblk + kWaves - 1) / kWaves;
  const int64_t cap = int64_t(qkv_num_cus()) * per_cu;
  if (grid > cap) grid = cap;
  hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, s, a.codes,
                     a.qjl, a.norms, a.n, a.bits, a.pi, a.cents, a.signs, a.qjl_scale, a.in_seq,
                     a.in_gstride, a.out, a.out_dtype, a.sel, a.alt_cents, a.alt_bits);
  return QKV_OK;
}

template <int D>
int dispatch(const QkvDecompressArgs& a, hipStream_t s) {
  constexpr int R = 2;
  const bool ip = a.mode == QKV_MODE_IP;
  const bool sel = a.sel != nullptr;
  switch (a.fmt) {
    case QKV_FMT_UNPACKED:
      if (ip) return sel ? launch<D, QKV_FMT_UNPACKED, 0, true, true, R>(a, s)
                         : launch<D, QKV_FMT_UNPACKED, 0, true, false, R>(a, s);
      return sel ? launch<D, QKV_FMT_UNPACKED, 0, false, true, R>(a, s)
                 : launch<D, QKV_FMT_UNPACKED, 0, false, false, R>(a, s);
    case QKV_FMT_PACKED:
      switch (a.bits) {
        case 1: return ip ? launch<D, QKV_FMT_PACKED, 1, true, false, R>(a, s)
                          : launch<D, QKV_FMT_PACKED, 1, false, false, R>(a, s);
        case 2: return ip ? launch<D, QKV_FMT_PACKED, 2, true, false, R>(a, s)
                          : launch<D, QKV_FMT_PACKED, 2, false, false, R>(a, s);
        case 3: return ip ? launch<D, QKV_FMT_PACKED, 3, true, false, R>(a, s)
                          : launch<D, QKV_FMT_PACKED, 3, false, false, R>(a, s);
        default: return launch<D, QKV_FMT_PACKED, 4, false, false, R>(a, s);
      }
    case QKV_FMT_KPLANES:
      return ip ? launch<D, QKV_FMT_KPLANES, 0, true, false, R>(a, s)
                : launch<D, QKV_FMT_KPLANES, 0, false, false, R>(a, s);
    default:
      return launch<D, QKV_FMT_VTILES, 0, false, false, R>(a, s);
  }
}

}  // namespace

bool qkv_decompress_mfma_ok(const QkvDecompressArgs& a) {
  if (a.d != 64 && a.d != 128) return false;
  if (a.sel && a.fmt != QKV_FMT_UNPACKED) return false;
  if (a.fmt == QKV_FMT_PACKED && a.mode == QKV_MODE_IP && a.bits == 4) return false;
  // 16-byte unpacked reads, 4-byte (2-byte at d = 64) packed and plane reads
  const int ca = a.fmt == QKV_FMT_UNPACKED || a.fmt == QKV_FMT_VTILES ? 16 : (a.d == 128 ? 4 : 2);
  if (!qkv_aligned(a.codes, ca)) return false;
  if (a.mode == QKV_MODE_IP && a.fmt != QKV_FMT_KPLANES &&
      !qkv_aligned(a.qjl, a.fmt == QKV_FMT_UNPACKED ? 16 : (a.d == 128 ? 4 : 2)))
    return false;
  return qkv_aligned(a.out, 16);  // 16-byte output stores
}

int qkv_decompress_mfma(const QkvDecompressArgs& a, hipStream_t s) {
  return a.d == 128 ? dispatch<128>(a, s) : dispatch<64>(a, s);
}
