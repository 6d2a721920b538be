// Fused decompress on the matrix cores (d = 64, 96 and 128):
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
// of the row (32 bytes unpacked, 12 bytes of a 3-bit row at d = 128).  At
// d = 96 a lane's run (24 coordinates) starts mid-dword in the bit-packed
// formats; it is read as the dwords that hold it and aligned in registers.
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
typedef uint32_t qkv_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t qkv_u32x2 __attribute__((ext_vector_type(2)));

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

// Output coordinate of C row mm (0..15) in column tile jt: lane group g of a
// tile holds coordinates 16 jt + 4 g + 0..3, so one store instruction writes
// 64 contiguous bytes (fp32) of each of its 16 vectors.
__device__ __forceinline__ int out_col(int jt, int mm) { return 16 * jt + mm; }

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

// Bytes off .. off + NB - 1 of a dword-aligned row of row_words dwords, as
// (NB + 3) / 4 words (bytes past NB unspecified): the dwords that hold them,
// clamped to the row, shifted into place.
template <int NB>
__device__ __forceinline__ void lane_span(const uint8_t* row, int row_words, int off,
                                          uint32_t* out) {
  constexpr int NO = (NB + 3) / 4;
  const uint32_t* w = reinterpret_cast<const uint32_t*>(row);
  const int wi = off >> 2, sh = off & 3;
  uint32_t a[NO + 1];
#pragma unroll
  for (int k = 0; k <= NO; ++k) a[k] = w[min(wi + k, row_words - 1)];
#pragma unroll
  for (int k = 0; k < NO; ++k) out[k] = __builtin_amdgcn_alignbyte(a[k + 1], a[k], sh);
}

// Lane's NE bits of a bit plane / 1-bit row starting at byte `p` (at d = 96
// bits 24..31 are unspecified).
template <int D>
__device__ __forceinline__ uint32_t lane_bits(const uint8_t* p, int g) {
  if constexpr (D == 128) {
    return reinterpret_cast<const uint32_t*>(p)[g];
  } else if constexpr (D == 96) {
    uint32_t w;
    lane_span<3>(p, 3, 3 * g, &w);
    return w;
  } else {
    return reinterpret_cast<const uint16_t*>(p)[g];
  }
}

// ------------------------------------------------------------------ shared parts

// Per-workgroup set-up: the power-of-two scales that bring Pi's and the
// values' largest magnitudes into [1, 2), the value table and Pi's fragments
// in LDS.  Returns the value scale sv and the exact output factor 1 / (ps sv).
template <int D, bool IP, bool SEL>
__device__ void setup(int nthreads, float* red, uint32_t* tab, uint4* frag,
                      const float* __restrict__ pi, const float* __restrict__ cents, int bits,
                      const float* __restrict__ alt_cents, int alt_bits, float qjl_scale,
                      float& sv, float& ofac) {
  constexpr int NE = Geo<D>::NE, NK = Geo<D>::NK, NJ = Geo<D>::NJ;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = nthreads / 64;
  float pm = 0.f;
  for (int i = tid; i < D * D; i += nthreads) pm = fmaxf(pm, fabsf(pi[i]));
  pm = qkv_wave_max(pm);
  float tv = 0.f;
  if (tid < 32) {
    const int s = tid >> 4, c = tid & 15;
    if (s == 0) tv = c < (1 << bits) ? cents[c] : 0.f;
    else if (SEL) tv = c < (1 << alt_bits) ? alt_cents[c] : 0.f;
  }
  const float vm = qkv_wave_max(fabsf(tv));
  if (lane == 0) red[wave] = pm;
  if (tid == 0) red[nw] = vm;
  __syncthreads();
  float pmax = red[0];
  for (int w = 1; w < nw; ++w) pmax = fmaxf(pmax, red[w]);
  const float ps = pow2_scale(pmax);
  sv = pow2_scale(red[nw] + (IP ? fabsf(qjl_scale) : 0.f));
  ofac = 1.f / (ps * sv);
  if (tid < 32) tab[tid] = IP ? __float_as_uint(tv * sv) : split_pair(tv * sv);
  // lane l of fragment (jt, ks) holds Pi[k][out_col(jt, l % 16)] for the 8
  // coordinates k = (l / 16) NE + 8 ks + 0..7, fp16 high part then low part
  for (int i = tid; i < NJ * NK * 64; i += nthreads) {
    const int l = i & 63, blk = i >> 6;
    const int jt = blk / NK, ks = blk - jt * NK;
    const float* src = pi + int64_t((l >> 4) * NE + 8 * ks) * D + out_col(jt, l & 15);
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
}

// Per-lane constants of the lane's coordinates g NE .. g NE + NE - 1: the
// mixed-precision selector bits (bit 4 of each code byte) and the scaled
// QJL terms qjl_scale S_k sv.
template <int D, bool IP, bool SEL>
struct LaneConsts {
  static constexpr int NE = Geo<D>::NE;
  uint32_t selw[SEL ? NE / 4 : 1];
  float qs[IP ? NE : 1];
  __device__ __forceinline__ void load(int g, const uint8_t* __restrict__ sel,
                                       const float* __restrict__ signs, float qjl_scale, float sv) {
    if constexpr (SEL) {
#pragma unroll
      for (int c = 0; c < NE / 4; ++c) {
        uint32_t s = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) s |= (sel[g * NE + 4 * c + b] != 0 ? 0x10u : 0u) << (8 * b);
        selw[c] = s;
      }
    }
    if constexpr (IP) {
#pragma unroll
      for (int e = 0; e < NE; ++e) qs[e] = qjl_scale * signs[g * NE + e] * sv;
    }
  }
};

// Raw words of one wave block (R row tiles of 16 vectors) as this lane needs
// them (V tiles are read from a staged tile in LDS instead).
template <int D, int FMT, int BITS, bool IP, int R>
struct Raw {
  static constexpr int CWN = FMT == QKV_FMT_KPLANES ? 4 : CodeWords<D, FMT, BITS>::N;
  static constexpr int QWN = IP ? QjlWords<D, FMT>::N : 1;
  uint32_t c[R][CWN];  // code words (K rows: plane words)
  uint32_t q[R][QWN];  // QJL words
  float n[R];          // norms
};

// Codes -> fp16 (hi, lo) value fragments ah / al of the lane's R vectors.
// `tile`: the block's V tile (32 tokens) staged in LDS, for V tiles.
template <int D, int FMT, int BITS, bool IP, bool SEL, int R>
__device__ __forceinline__ void expand(const Raw<D, FMT, BITS, IP, R>& x, const uint4* tile,
                                       int bits, int lane, const uint32_t* tab,
                                       const LaneConsts<D, IP, SEL>& lc,
                                       uint4 (&ah)[R][Geo<D>::NK], uint4 (&al)[R][Geo<D>::NK]) {
  constexpr int NE = Geo<D>::NE, NK = Geo<D>::NK, NW = Geo<D>::NW;
  const int m = lane & 15, g = lane >> 4;
  CodeWords<D, FMT, BITS> cw[R];
  QjlWords<D, FMT> qw[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if constexpr (FMT == QKV_FMT_UNPACKED) {
#pragma unroll
      for (int i = 0; i < NE / 4; ++i) {
        cw[r].w[i] = x.c[r][i] & 0x0F0F0F0Fu;
        if constexpr (SEL) cw[r].w[i] |= lc.selw[i];
      }
    } else if constexpr (FMT == QKV_FMT_PACKED) {
#pragma unroll
      for (int i = 0; i < CodeWords<D, FMT, BITS>::N; ++i) cw[r].w[i] = x.c[r][i];
    } else if constexpr (FMT == QKV_FMT_KPLANES) {
#pragma unroll
      for (int i = 0; i < NW; ++i) {
        uint32_t v = 0u;
#pragma unroll
        for (int p = 0; p < 4; ++p)
          if (p < bits) v |= spread8(bfe(x.c[r][p], 8 * i, 8)) << p;
        cw[r].w[i] = v;
      }
    }
    if constexpr (IP) {
#pragma unroll
      for (int i = 0; i < QjlWords<D, FMT>::N; ++i) qw[r].w[i] = x.q[r][i];
    }
  }
  if constexpr (FMT == QKV_FMT_VTILES) {
    // gather bit m (row tile 0) and m + 16 (row tile 1) of the lane's NE
    // coordinate words of every plane into nibble codes
    static_assert(R == 2, "one 32-token V tile per block");
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int i = 0; i < NW; ++i) cw[r].w[i] = 0u;
    for (int p = 0; p < bits; ++p) {
      const uint4* row = tile + p * (D / 4) + g * (NE / 4);
#pragma unroll
      for (int c = 0; c < NE / 4; ++c) {
        const uint4 v = row[c];
        const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int e = 4 * c + u;
          const uint32_t sh = 4 * (e & 7) + p;
          cw[0].w[e >> 3] |= bfe(wv[u], m, 1) << sh;
          cw[1].w[e >> 3] |= bfe(wv[u], m + 16, 1) << sh;
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
#pragma unroll
    for (int ks = 0; ks < NK; ++ks) {
      uint32_t hv[4], lv[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int e0 = 8 * ks + 2 * q, e1 = e0 + 1;
        const uint32_t i0 = cw[r].code(e0), i1 = cw[r].code(e1);
        uint32_t a, b;
        if constexpr (IP) {
          const float c0 = __uint_as_float(tab[i0]), c1 = __uint_as_float(tab[i1]);
          a = split_pair(c0 + (qw[r].bit(e0) ? lc.qs[e0] : -lc.qs[e0]));
          b = split_pair(c1 + (qw[r].bit(e1) ? lc.qs[e1] : -lc.qs[e1]));
        } else {
          a = tab[i0];
          b = tab[i1];
        }
        hv[q] = __builtin_amdgcn_perm(b, a, 0x05040100u);
        lv[q] = __builtin_amdgcn_perm(b, a, 0x07060302u);
      }
      ah[r][ks] = make_uint4(hv[0], hv[1], hv[2], hv[3]);
      al[r][ks] = make_uint4(lv[0], lv[1], lv[2], lv[3]);
    }
  }
}

// Orders this wave's LDS accesses across its lanes (LDS executes a wave's
// accesses in order; this keeps the compiler from moving them).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

// C = Pi^T V^T for the lane's R vectors and the stores (rows 16 r + m of the
// buffer `ob`, whose byte range drops rows past the group's end).  Steps
// (p, ks): column tiles 2p, 2p+1 (32 output coordinates), k-step ks; Pi's
// fragments of step s+1 are read from LDS while the MFMAs of step s run (two
// register buffers; the scheduling barriers keep the compiler from sinking
// the reads to their use).
template <int D, int R>
__device__ __forceinline__ void mma_store(const uint4 (&ah)[R][Geo<D>::NK],
                                          const uint4 (&al)[R][Geo<D>::NK], const float (&nf)[R],
                                          const uint4* frag, int lane, uint8_t* ost,
                                          __amdgpu_buffer_rsrc_t ob, int out_dtype) {
  constexpr int NK = Geo<D>::NK, NJ = Geo<D>::NJ;
  constexpr int NSTEP = (NJ / 2) * NK;
  const int m = lane & 15, g = lane >> 4;
  const int obytes = out_dtype == QKV_F32 ? 4 : 2;
  uint4 fh[2][2], fl[2][2];  // [buffer][column tile of the pair]
  auto read_frags = [&](int s, int buf) {
    const int p = s / NK, ks = s - p * NK;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int f = 2 * ((2 * p + hh) * NK + ks);
      fh[buf][hh] = frag[f * 64 + lane];
      fl[buf][hh] = frag[(f + 1) * 64 + lane];
    }
  };
  qkv_f32x4 acc[2][R];
  read_frags(0, 0);
#pragma unroll
  for (int s = 0; s < NSTEP; ++s) {
    const int p = s / NK, ks = s - p * NK, cur = s & 1;
    if (s + 1 < NSTEP) read_frags(s + 1, cur ^ 1);
    __builtin_amdgcn_sched_barrier(0);
    if (ks == 0) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[hh][r] = qkv_f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int r = 0; r < R; ++r) acc[hh][r] = mma(fh[cur][hh], ah[r][ks], acc[hh][r]);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int r = 0; r < R; ++r) acc[hh][r] = mma(fl[cur][hh], ah[r][ks], acc[hh][r]);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int r = 0; r < R; ++r) acc[hh][r] = mma(fh[cur][hh], al[r][ks], acc[hh][r]);
    __builtin_amdgcn_sched_barrier(0);
    if (ks != NK - 1) continue;
    // lane (m, g) holds coordinates 16 (2p + hh) + 4 g + 0..3 of row 16 r + m:
    // through the wave's LDS staging rows (32 coordinates, 16 bytes of padding)
    // into stores of whole 128-byte (fp32) / 64-byte (16-bit) row segments
    const int rsb = 32 * obytes + 16;
    wave_lds_sync();
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float f = nf[r];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const float v0 = acc[hh][r][0] * f, v1 = acc[hh][r][1] * f;
        const float v2 = acc[hh][r][2] * f, v3 = acc[hh][r][3] * f;
        uint8_t* dst = ost + (16 * r + m) * rsb + (16 * hh + 4 * g) * obytes;
        if (out_dtype == QKV_F32) {
          *reinterpret_cast<float4*>(dst) = make_float4(v0, v1, v2, v3);
        } else {
          uint32_t w0, w1;
          if (out_dtype == QKV_F16) {
            w0 = h16(static_cast<_Float16>(v0)) | (h16(static_cast<_Float16>(v1)) << 16);
            w1 = h16(static_cast<_Float16>(v2)) | (h16(static_cast<_Float16>(v3)) << 16);
          } else {
            w0 = qkv_f32_to_bf16(v0) | (uint32_t(qkv_f32_to_bf16(v1)) << 16);
            w1 = qkv_f32_to_bf16(v2) | (uint32_t(qkv_f32_to_bf16(v3)) << 16);
          }
          *reinterpret_cast<uint2*>(dst) = make_uint2(w0, w1);
        }
      }
    }
    wave_lds_sync();
    // 16-byte chunks: cpr per row segment, 64 / cpr rows per store
    const int cpr = 2 * obytes, rows = 64 / cpr;
    const int q = lane % cpr;
    for (int v = lane / cpr; v < 16 * R; v += rows) {
      const uint4 w = *reinterpret_cast<const uint4*>(ost + v * rsb + 16 * q);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(qkv_u32x4, w), ob,
                                             (v * D + 32 * p) * obytes + 16 * q, 0, 0);
    }
  }
}

// A block's place: group, first token, end of the group's valid tokens.
struct BlockPos {
  int64_t grp, t0, tend;
  __device__ __forceinline__ BlockPos(int blk, int bpg, int rb, int64_t n, int64_t in_seq) {
    const int gi = blk / bpg;
    grp = gi;
    t0 = int64_t(blk - gi * bpg) * rb;
    tend = min(in_seq, n - grp * in_seq);
  }
};

// Output buffer of a block: rows t0 .. tend - 1 of the group (range-checked
// buffer stores drop the rest).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t out_rsrc(void* out, const BlockPos& b, int rb,
                                                           int d, int obytes, int64_t in_seq) {
  const int64_t nrows = min<int64_t>(rb, b.tend - b.t0);
  return __builtin_amdgcn_make_buffer_rsrc(
      static_cast<char*>(out) + (b.grp * in_seq + b.t0) * d * obytes, 0,
      static_cast<int>(nrows * d * obytes), 0x00020000);
}

// -------------------------------------------- d = 64 and 96: per-wave pipeline

// One wave per block of 32 vectors, each wave fetching its next block (loads
// only) before the current block's MFMAs and stores, then expanding it.
// Rows past a group's end are clamped loads and dropped stores, so no branch
// hides a memory instruction from the compiler's wait counts.
template <int D, int FMT, int BITS, bool IP, bool SEL>
__global__ __launch_bounds__(kThreads, 2) void decompress_waves(
    const uint8_t* __restrict__ codes, const uint8_t* __restrict__ qjl,
    const float* __restrict__ norms, int64_t n, int bits, const float* __restrict__ pi,
    const float* __restrict__ cents, const float* __restrict__ signs, float qjl_scale,
    int64_t in_seq, int64_t in_gstride, void* __restrict__ out, int out_dtype,
    const uint8_t* __restrict__ sel, const float* __restrict__ alt_cents, int alt_bits) {
  using G = Geo<D>;
  constexpr int NE = G::NE, NK = G::NK, R = 2, RB = 32;
  constexpr bool VT = FMT == QKV_FMT_VTILES;
  __shared__ uint4 frag[G::NJ * NK * 2 * 64];  // [jt][ks][hi, lo][lane]
  __shared__ uint32_t tab[32];                 // [codebook][code]
  __shared__ float red[kWaves + 1];
  // per wave: a V tile (<= 4 planes) while expanding, output rows while storing
  __shared__ uint4 stage[kWaves * 288];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m = lane & 15, g = lane >> 4;
  float sv, ofac;
  setup<D, IP, SEL>(kThreads, red, tab, frag, pi, cents, bits, alt_cents, alt_bits, qjl_scale,
                    sv, ofac);
  LaneConsts<D, IP, SEL> lc;
  lc.load(g, sel, signs, qjl_scale, sv);
  __syncthreads();

  // blocks of 32 vectors numbered group by group (below 2^31: host check)
  const int bpg = static_cast<int>((in_seq + RB - 1) / RB);
  const int nblk = static_cast<int>((n + in_seq - 1) / in_seq) * bpg;
  const int64_t pb = FMT == QKV_FMT_PACKED ? qkv_row_bytes(D, BITS)
                   : FMT == QKV_FMT_KPLANES ? int64_t(bits + 1) * (D / 8) : D;
  const int64_t pq = FMT == QKV_FMT_PACKED ? D / 8 : D;
  const int obytes = out_dtype == QKV_F32 ? 4 : 2;
  uint4* stg = &stage[wave * 288];

  Raw<D, FMT, BITS, IP, R> x;
  constexpr int NRT = (D + 63) / 64;
  uint4 rt[VT ? NRT : 1];  // V tiles: this lane's share of the tile's words
  auto fetch = [&](int blk) {
    const BlockPos b(blk, bpg, RB, n, in_seq);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t t = min(b.t0 + 16 * r + m, b.tend - 1);  // clamped: last valid row
      const int64_t row = b.grp * in_gstride + t;
      x.n[r] = norms[VT ? b.grp * in_gstride * 32 + t : row];
#pragma unroll
      for (int i = 0; i < Raw<D, FMT, BITS, IP, R>::CWN; ++i) x.c[r][i] = 0u;
#pragma unroll
      for (int i = 0; i < Raw<D, FMT, BITS, IP, R>::QWN; ++i) x.q[r][i] = 0u;
      if constexpr (FMT == QKV_FMT_UNPACKED) {
        // NE bytes: 16-byte reads, 8-byte reads at d = 96 (NE = 24)
        auto bytes = [&](const uint8_t* p, uint32_t* dst) {
          if constexpr (NE % 16 == 0) {
            const uint4* src = reinterpret_cast<const uint4*>(p);
#pragma unroll
            for (int i = 0; i < NE / 16; ++i) {
              const uint4 v = src[i];
              dst[4 * i] = v.x; dst[4 * i + 1] = v.y; dst[4 * i + 2] = v.z; dst[4 * i + 3] = v.w;
            }
          } else {
            const uint2* src = reinterpret_cast<const uint2*>(p);
#pragma unroll
            for (int i = 0; i < NE / 8; ++i) {
              const uint2 v = src[i];
              dst[2 * i] = v.x; dst[2 * i + 1] = v.y;
            }
          }
        };
        bytes(codes + row * D + g * NE, x.c[r]);
        if constexpr (IP) bytes(qjl + row * D + g * NE, x.q[r]);
      } else if constexpr (FMT == QKV_FMT_PACKED) {
        const uint8_t* rp = codes + row * pb;
        if constexpr (D == 96) {
          // 3 BITS bytes from byte 3 BITS g of a 12 BITS-byte row
          lane_span<3 * BITS>(rp, 3 * BITS, 3 * BITS * g, x.c[r]);
        } else if constexpr (D == 128) {
          const uint32_t* src = reinterpret_cast<const uint32_t*>(rp) + BITS * g;
#pragma unroll
          for (int i = 0; i < BITS; ++i) x.c[r][i] = src[i];
        } else {
          const uint16_t* src = reinterpret_cast<const uint16_t*>(rp) + BITS * g;
#pragma unroll
          for (int i = 0; i < BITS; ++i) x.c[r][i >> 1] |= uint32_t(src[i]) << (16 * (i & 1));
        }
        if constexpr (IP) x.q[r][0] = lane_bits<D>(qjl + row * pq, g);
      } else if constexpr (FMT == QKV_FMT_KPLANES) {
        const uint8_t* rp = codes + row * pb;
#pragma unroll
        for (int p = 0; p < 4; ++p)  // planes past `bits` re-read plane 0 (masked at use)
          x.c[r][p] = lane_bits<D>(rp + (p < bits ? p : 0) * (D / 8), g);
        if constexpr (IP) x.q[r][0] = lane_bits<D>(rp + bits * (D / 8), g);
      }
    }
    if constexpr (VT) {
      const int nd4 = bits * D / 4;  // uint4 per tile
      const uint4* src = reinterpret_cast<const uint4*>(codes) +
                         ((b.grp * in_gstride + (b.t0 >> 5)) * bits) * (D / 4);
#pragma unroll
      for (int u = 0; u < NRT; ++u) {
        const int i = lane + 64 * u;
        rt[u] = src[i < nd4 ? i : nd4 - 1];
      }
    }
  };

  uint4 ah[R][NK], al[R][NK];
  float nf[R];
  auto expand_fetched = [&]() {
    if constexpr (VT) {
      wave_lds_sync();
#pragma unroll
      for (int u = 0; u < NRT; ++u) stg[lane + 64 * u] = rt[u];
      wave_lds_sync();
    }
    expand<D, FMT, BITS, IP, SEL, R>(x, stg, bits, lane, tab, lc, ah, al);
#pragma unroll
    for (int r = 0; r < R; ++r) nf[r] = x.n[r] * ofac;
  };

  const int stride = static_cast<int>(gridDim.x) * kWaves;
  int blk = static_cast<int>(blockIdx.x) * kWaves + __builtin_amdgcn_readfirstlane(wave);
  if (blk >= nblk) return;
  fetch(blk);
  expand_fetched();
  for (;;) {
    const int nb = blk + stride;
    const bool more = nb < nblk;
    fetch(more ? nb : blk);  // unconditional: the last round re-reads its own block
    const BlockPos b(blk, bpg, RB, n, in_seq);
    mma_store<D, R>(ah, al, nf, frag, lane, reinterpret_cast<uint8_t*>(stg),
                    out_rsrc(out, b, RB, D, obytes, in_seq), out_dtype);
    if (!more) break;
    expand_fetched();
    blk = nb;
  }
}

// ------------------------------------- d = 128: loader wave + compute waves

typedef __attribute__((address_space(3))) void* qkv_lds_ptr;
typedef __attribute__((address_space(1))) void* qkv_global_ptr;

// size-byte global -> LDS copy per lane (lane i lands at dst + i * max(size, 4))
template <int SIZE>
__device__ __forceinline__ void to_lds(const void* src, void* dst) {
  static_assert(SIZE == 4 || SIZE == 16, "copy size");
  if constexpr (SIZE == 16)
    __builtin_amdgcn_global_load_lds((qkv_global_ptr)(src), (qkv_lds_ptr)(dst), 16, 0, 0);
  else
    __builtin_amdgcn_global_load_lds((qkv_global_ptr)(src), (qkv_lds_ptr)(dst), 4, 0, 0);
}

// All workgroup waves meet; orders LDS accesses only (a global-memory fence
// would wait for the compute waves' outstanding stores).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Bytes of one compute wave's staging slot (codes, QJL words, norms) at d = 128.
template <int FMT, int BITS, bool IP>
struct Slot {
  static constexpr int CB = FMT == QKV_FMT_UNPACKED ? 4096
                          : FMT == QKV_FMT_PACKED   ? 2 * BITS * 256
                          : FMT == QKV_FMT_KPLANES  ? 2 * 5 * 256
                                                    : 2048;
  static constexpr int QB = !IP ? 0 : FMT == QKV_FMT_UNPACKED ? 4096 : FMT == QKV_FMT_PACKED ? 512 : 0;
  // also the output staging rows of the wave's stores: 32 x 144 bytes
  static constexpr int BYTES = CB + QB + 512 > 4608 ? CB + QB + 512 : 4608;
};

// The loader wave (the last of the workgroup) copies the codes, QJL words and
// norms of the NC compute waves' next blocks into LDS with global->LDS loads,
// laid out in the compute lanes' order; the compute waves read them from LDS
// and so never wait on global loads, which on this architecture would also
// wait for their own outstanding output stores (one in-order counter covers
// both).  Double-buffered slots, one LDS-only barrier per round.
template <int FMT, int BITS, bool IP, bool SEL, int NC>
__global__ __launch_bounds__(64 * (NC + 1), 1) void decompress_staged(
    const uint8_t* __restrict__ codes, const uint8_t* __restrict__ qjl,
    const float* __restrict__ norms, int64_t n, int bits, const float* __restrict__ pi,
    const float* __restrict__ cents, const float* __restrict__ signs, float qjl_scale,
    int64_t in_seq, int64_t in_gstride, void* __restrict__ out, int out_dtype,
    const uint8_t* __restrict__ sel, const float* __restrict__ alt_cents, int alt_bits) {
  constexpr int D = 128, NT = 64 * (NC + 1), R = 2, RB = 32;
  using G = Geo<D>;
  using S = Slot<FMT, BITS, IP>;
  constexpr int NK = G::NK;
  constexpr bool VT = FMT == QKV_FMT_VTILES;
  __shared__ uint4 frag[G::NJ * NK * 2 * 64];
  __shared__ uint32_t tab[32];
  __shared__ float red[NC + 2];
  __shared__ uint4 slots[2 * NC * S::BYTES / 16];  // [buffer][compute wave]

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int m = lane & 15, g = lane >> 4;
  float sv, ofac;
  setup<D, IP, SEL>(NT, red, tab, frag, pi, cents, bits, alt_cents, alt_bits, qjl_scale, sv,
                    ofac);
  __syncthreads();

  const int bpg = static_cast<int>((in_seq + RB - 1) / RB);
  const int nblk = static_cast<int>((n + in_seq - 1) / in_seq) * bpg;
  const int per_round = static_cast<int>(gridDim.x) * NC;
  const int rounds = (nblk + per_round - 1) / per_round;
  const int64_t pb = FMT == QKV_FMT_PACKED ? qkv_row_bytes(D, BITS)
                   : FMT == QKV_FMT_KPLANES ? int64_t(bits + 1) * (D / 8) : D;
  const int64_t pq = D / 8;
  uint8_t* slot0 = reinterpret_cast<uint8_t*>(slots);
  auto slot = [&](int buf, int c) { return slot0 + (buf * NC + c) * S::BYTES; };
  auto block_of = [&](int round, int c) { return (round * static_cast<int>(gridDim.x) + static_cast<int>(blockIdx.x)) * NC + c; };

  if (wave == NC) {
    // ---- loader
    auto load_round = [&](int round, int buf) {
      for (int c = 0; c < NC; ++c) {
        const int blk = block_of(round, c);
        if (blk >= nblk) break;
        const BlockPos b(blk, bpg, RB, n, in_seq);
        uint8_t* sl = slot(buf, c);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int64_t t = min(b.t0 + 16 * r + m, b.tend - 1);  // clamped: last valid row
          const int64_t row = b.grp * in_gstride + t;
          to_lds<4>(norms + (VT ? b.grp * in_gstride * 32 + t : row), sl + S::CB + S::QB + r * 256);
          if constexpr (FMT == QKV_FMT_UNPACKED) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              to_lds<16>(codes + row * D + 32 * g + 16 * h, sl + (2 * r + h) * 1024);
              if constexpr (IP) to_lds<16>(qjl + row * D + 32 * g + 16 * h, sl + S::CB + (2 * r + h) * 1024);
            }
          } else if constexpr (FMT == QKV_FMT_PACKED) {
#pragma unroll
            for (int i = 0; i < BITS; ++i)
              to_lds<4>(codes + row * pb + 4 * (BITS * g + i), sl + (r * BITS + i) * 256);
            if constexpr (IP) to_lds<4>(qjl + row * pq + 4 * g, sl + S::CB + r * 256);
          } else if constexpr (FMT == QKV_FMT_KPLANES) {
            for (int p = 0; p < bits; ++p)
              to_lds<4>(codes + row * pb + 16 * p + 4 * g, sl + (r * 5 + p) * 256);
            if constexpr (IP) to_lds<4>(codes + row * pb + 16 * bits + 4 * g, sl + (r * 5 + 4) * 256);
          }
        }
        if constexpr (VT) {
          const int nd4 = bits * D / 4;  // uint4 per tile
          const uint4* src = reinterpret_cast<const uint4*>(codes) +
                             ((b.grp * in_gstride + (b.t0 >> 5)) * bits) * (D / 4);
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int i = lane + 64 * u;
            to_lds<16>(src + (i < nd4 ? i : nd4 - 1), sl + u * 1024);
          }
        }
      }
    };
    load_round(0, 0);
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the round's copies landed
    lds_barrier();
    for (int round = 0; round < rounds; ++round) {
      if (round + 1 < rounds) load_round(round + 1, (round + 1) & 1);
      __builtin_amdgcn_s_waitcnt(0x0f70);
      lds_barrier();
    }
  } else {
    // ---- compute
    LaneConsts<D, IP, SEL> lc;
    lc.load(g, sel, signs, qjl_scale, sv);
    const int obytes = out_dtype == QKV_F32 ? 4 : 2;
    lds_barrier();
    for (int round = 0; round < rounds; ++round) {
      const int blk = block_of(round, wave);
      if (blk < nblk) {
        const uint8_t* sl = slot(round & 1, wave);
        Raw<D, FMT, BITS, IP, R> x;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          x.n[r] = reinterpret_cast<const float*>(sl + S::CB + S::QB + r * 256)[lane];
#pragma unroll
          for (int i = 0; i < Raw<D, FMT, BITS, IP, R>::CWN; ++i) x.c[r][i] = 0u;
#pragma unroll
          for (int i = 0; i < Raw<D, FMT, BITS, IP, R>::QWN; ++i) x.q[r][i] = 0u;
          if constexpr (FMT == QKV_FMT_UNPACKED) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const uint4 v = reinterpret_cast<const uint4*>(sl + (2 * r + h) * 1024)[lane];
              x.c[r][4 * h] = v.x; x.c[r][4 * h + 1] = v.y; x.c[r][4 * h + 2] = v.z; x.c[r][4 * h + 3] = v.w;
              if constexpr (IP) {
                const uint4 u = reinterpret_cast<const uint4*>(sl + S::CB + (2 * r + h) * 1024)[lane];
                x.q[r][4 * h] = u.x; x.q[r][4 * h + 1] = u.y; x.q[r][4 * h + 2] = u.z; x.q[r][4 * h + 3] = u.w;
              }
            }
          } else if constexpr (FMT == QKV_FMT_PACKED) {
#pragma unroll
            for (int i = 0; i < BITS; ++i)
              x.c[r][i] = reinterpret_cast<const uint32_t*>(sl + (r * BITS + i) * 256)[lane];
            if constexpr (IP) x.q[r][0] = reinterpret_cast<const uint32_t*>(sl + S::CB + r * 256)[lane];
          } else if constexpr (FMT == QKV_FMT_KPLANES) {
#pragma unroll
            for (int p = 0; p < 4; ++p)
              x.c[r][p] = p < bits ? reinterpret_cast<const uint32_t*>(sl + (r * 5 + p) * 256)[lane] : 0u;
            if constexpr (IP) x.q[r][0] = reinterpret_cast<const uint32_t*>(sl + (r * 5 + 4) * 256)[lane];
          }
        }
        uint4 ah[R][NK], al[R][NK];
        expand<D, FMT, BITS, IP, SEL, R>(x, reinterpret_cast<const uint4*>(sl), bits, lane, tab, lc,
                                         ah, al);
        float nf[R];
#pragma unroll
        for (int r = 0; r < R; ++r) nf[r] = x.n[r] * ofac;
        const BlockPos b(blk, bpg, RB, n, in_seq);
        mma_store<D, R>(ah, al, nf, frag, lane, const_cast<uint8_t*>(sl),
                        out_rsrc(out, b, RB, D, obytes, in_seq), out_dtype);
      }
      lds_barrier();
    }
  }
}

// ------------------------------------------------------------------- launch

// resident workgroups per CU from a kernel's LDS (160 KiB per gfx950 CU) and
// VGPRs (512 per SIMD lane, four SIMDs)
template <typename K>
int per_cu(K k, int waves) {
  int b = 1;
  hipFuncAttributes at;
  if (hipFuncGetAttributes(&at, reinterpret_cast<const void*>(k)) == hipSuccess) {
    const int by_lds = 160 * 1024 / static_cast<int>(at.sharedSizeBytes > 0 ? at.sharedSizeBytes : 1);
    const int regs = at.numRegs > 0 ? (at.numRegs + 7) / 8 * 8 : 512;
    const int by_regs = (512 / regs) * 4 / waves;
    b = by_lds < by_regs ? by_lds : by_regs;
  }
  return b < 1 ? 1 : b;
}

int64_t blocks_of(const QkvDecompressArgs& a) {
  return (a.n + a.in_seq - 1) / a.in_seq * ((a.in_seq + 31) / 32);
}

template <int D, int FMT, int BITS, bool IP, bool SEL>
int launch_waves(const QkvDecompressArgs& a, hipStream_t s) {
  auto k = decompress_waves<D, FMT, BITS, IP, SEL>;
  static const int pc = per_cu(k, kWaves);
  int64_t grid = (blocks_of(a) + kWaves - 1) / kWaves;
  const int64_t cap = int64_t(qkv_num_cus()) * pc;
  if (grid > cap) grid = cap;
  hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, s, a.codes, a.qjl,
                     a.norms, a.n, a.bits, a.pi, a.cents, a.signs, a.qjl_scale, a.in_seq,
                     a.in_gstride, a.out, a.out_dtype, a.sel, a.alt_cents, a.alt_bits);
  return QKV_OK;
}

template <int FMT, int BITS, bool IP, bool SEL>
int launch_staged(const QkvDecompressArgs& a, hipStream_t s) {
  constexpr int NC = IP ? 4 : 8;  // compute waves (VGPRs / LDS slots)
  auto k = decompress_staged<FMT, BITS, IP, SEL, NC>;
  static const int pc = per_cu(k, NC + 1);
  int64_t grid = (blocks_of(a) + NC - 1) / NC;
  const int64_t cap = int64_t(qkv_num_cus()) * pc;
  if (grid > cap) grid = cap;
  hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(grid)), dim3(64 * (NC + 1)), 0, s, a.codes,
                     a.qjl, a.norms, a.n, a.bits, a.pi, a.cents, a.signs, a.qjl_scale, a.in_seq,
                     a.in_gstride, a.out, a.out_dtype, a.sel, a.alt_cents, a.alt_bits);
  return QKV_OK;
}

template <int D, int FMT, int BITS, bool IP, bool SEL>
int launch(const QkvDecompressArgs& a, hipStream_t s) {
  if constexpr (D == 128) return launch_staged<FMT, BITS, IP, SEL>(a, s);
  else return launch_waves<D, FMT, BITS, IP, SEL>(a, s);
}

template <int D>
int dispatch(const QkvDecompressArgs& a, hipStream_t s) {
  const bool ip = a.mode == QKV_MODE_IP;
  const bool sel = a.sel != nullptr;
  switch (a.fmt) {
    case QKV_FMT_UNPACKED:
      if (ip) return sel ? launch<D, QKV_FMT_UNPACKED, 0, true, true>(a, s)
                         : launch<D, QKV_FMT_UNPACKED, 0, true, false>(a, s);
      return sel ? launch<D, QKV_FMT_UNPACKED, 0, false, true>(a, s)
                 : launch<D, QKV_FMT_UNPACKED, 0, false, false>(a, s);
    case QKV_FMT_PACKED:
      switch (a.bits) {
        case 1: return ip ? launch<D, QKV_FMT_PACKED, 1, true, false>(a, s)
                          : launch<D, QKV_FMT_PACKED, 1, false, false>(a, s);
        case 2: return ip ? launch<D, QKV_FMT_PACKED, 2, true, false>(a, s)
                          : launch<D, QKV_FMT_PACKED, 2, false, false>(a, s);
        case 3: return ip ? launch<D, QKV_FMT_PACKED, 3, true, false>(a, s)
                          : launch<D, QKV_FMT_PACKED, 3, false, false>(a, s);
        default: return launch<D, QKV_FMT_PACKED, 4, false, false>(a, s);
      }
    case QKV_FMT_KPLANES:
      return ip ? launch<D, QKV_FMT_KPLANES, 0, true, false>(a, s)
                : launch<D, QKV_FMT_KPLANES, 0, false, false>(a, s);
    default:
      return launch<D, QKV_FMT_VTILES, 0, false, false>(a, s);
  }
}

}  // namespace

bool qkv_decompress_mfma_ok(const QkvDecompressArgs& a) {
  if (!qkv_d_ok(a.d)) return false;
  // block numbers (32 vectors per block, per group) are 32-bit
  const int64_t groups = (a.n + a.in_seq - 1) / a.in_seq;
  if (groups * ((a.in_seq + 31) / 32) > int64_t(0x7fffffff) - int64_t(qkv_num_cus()) * 64) return false;
  if (a.sel && a.fmt != QKV_FMT_UNPACKED) return false;
  if (a.fmt == QKV_FMT_PACKED && a.mode == QKV_MODE_IP && a.bits == 4) return false;
  // unpacked reads of 16 bytes (8 at d = 96), V tiles of 16; packed and
  // plane reads of 4 bytes (2 at d = 64)
  const int ua = a.d == 96 ? 8 : 16, ba = a.d == 64 ? 2 : 4;
  const int ca = a.fmt == QKV_FMT_UNPACKED ? ua : a.fmt == QKV_FMT_VTILES ? 16 : ba;
  if (!qkv_aligned(a.codes, ca)) return false;
  if (a.mode == QKV_MODE_IP && a.fmt != QKV_FMT_KPLANES &&
      !qkv_aligned(a.qjl, a.fmt == QKV_FMT_UNPACKED ? ua : ba))
    return false;
  return qkv_aligned(a.out, 16);  // 16-byte output stores
}

int qkv_decompress_mfma(const QkvDecompressArgs& a, hipStream_t s) {
  if (a.d == 128) return dispatch<128>(a, s);
  return a.d == 96 ? dispatch<96>(a, s) : dispatch<64>(a, s);
}
