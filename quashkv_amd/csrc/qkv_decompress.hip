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

  // Blocks of RB vectors, numbered group by group (the host keeps the count
  // below 2^31); block numbers are wave-uniform, so their arithmetic is scalar.
  const int bpg = static_cast<int>((in_seq + RB - 1) / RB);
  const int nblk = static_cast<int>((n + in_seq - 1) / in_seq) * bpg;
  const int64_t pb = FMT == QKV_FMT_PACKED ? qkv_row_bytes(D, BITS)
                   : FMT == QKV_FMT_KPLANES ? int64_t(bits + 1) * (D / 8) : D;
  const int64_t pq = FMT == QKV_FMT_PACKED ? D / 8 : D;
  const int obytes = out_dtype == QKV_F32 ? 4 : 2;
  uint4* stg = &stage[VT ? wave * D : 0];

  // Software pipeline per wave: fetch block b+1 (loads only), MFMAs and stores
  // of block b, then expand block b+1's codes.  The loads are issued before
  // block b's stores, so the wait for them does not wait for those stores
  // (one in-order counter covers both); rows past a group's end are clamped
  // loads and range-checked buffer stores, so no branch hides a memory
  // instruction from that count.
  constexpr int CWN = FMT == QKV_FMT_KPLANES ? 4 : CodeWords<D, FMT, BITS>::N;
  constexpr int QWN = IP ? QjlWords<D, FMT>::N : 1;
  constexpr int TV = VT ? R / 2 : 1, TU = VT ? D / 64 : 1;
  uint32_t rc[R][CWN];  // code words (K rows: plane words)
  uint32_t rq[R][QWN];  // QJL words
  uint4 rt[TV][TU];     // V tiles: this lane's share of each tile's words
  float rn[R];          // norms

  auto fetch = [&](int blk) {
    const int gi = blk / bpg;
    const int64_t grp = gi;
    const int64_t t0 = int64_t(blk - gi * bpg) * RB;
    const int64_t tend = min(in_seq, n - grp * in_seq);  // valid tokens of the group
#pragma unroll
    for (int r = 0; r < R; ++r) {
      // rows past the group's end read its last row; their outputs are dropped
      const int64_t t = min(t0 + 16 * r + m, tend - 1);
      const int64_t row = grp * in_gstride + t;
      rn[r] = norms[VT ? grp * in_gstride * 32 + t : row];
#pragma unroll
      for (int i = 0; i < CWN; ++i) rc[r][i] = 0u;
#pragma unroll
      for (int i = 0; i < QWN; ++i) rq[r][i] = 0u;
      if constexpr (FMT == QKV_FMT_UNPACKED) {
        const uint4* src = reinterpret_cast<const uint4*>(codes + row * D + g * NE);
#pragma unroll
        for (int i = 0; i < NE / 16; ++i) {
          const uint4 v = src[i];
          rc[r][4 * i] = v.x; rc[r][4 * i + 1] = v.y; rc[r][4 * i + 2] = v.z; rc[r][4 * i + 3] = v.w;
        }
        if constexpr (IP) {
          const uint4* qsrc = reinterpret_cast<const uint4*>(qjl + row * D + g * NE);
#pragma unroll
          for (int i = 0; i < NE / 16; ++i) {
            const uint4 v = qsrc[i];
            rq[r][4 * i] = v.x; rq[r][4 * i + 1] = v.y; rq[r][4 * i + 2] = v.z; rq[r][4 * i + 3] = v.w;
          }
        }
      } else if constexpr (FMT == QKV_FMT_PACKED) {
        const uint8_t* rp = codes + row * pb;
        if constexpr (D == 128) {
          const uint32_t* src = reinterpret_cast<const uint32_t*>(rp) + BITS * g;
#pragma unroll
          for (int i = 0; i < BITS; ++i) rc[r][i] = src[i];
        } else {
          const uint16_t* src = reinterpret_cast<const uint16_t*>(rp) + BITS * g;
#pragma unroll
          for (int i = 0; i < BITS; ++i) rc[r][i >> 1] |= uint32_t(src[i]) << (16 * (i & 1));
        }
        if constexpr (IP) rq[r][0] = lane_bits<D>(qjl + row * pq, g);
      } else if constexpr (FMT == QKV_FMT_KPLANES) {
        const uint8_t* rp = codes + row * pb;
#pragma unroll
        for (int p = 0; p < 4; ++p)  // planes past `bits` re-read plane 0 (masked at use)
          rc[r][p] = lane_bits<D>(rp + (p < bits ? p : 0) * (D / 8), g);
        if constexpr (IP) rq[r][0] = lane_bits<D>(rp + bits * (D / 8), g);
      }
    }
    if constexpr (VT) {
      const int nd4 = bits * D / 4;  // uint4 per tile
#pragma unroll
      for (int h = 0; h < TV; ++h) {
        const int64_t tt = min(t0 + 32 * h, tend - 1);  // a tile past the end re-reads the last
        const uint4* src = reinterpret_cast<const uint4*>(codes) +
                           ((grp * in_gstride + (tt >> 5)) * bits) * (D / 4);
#pragma unroll
        for (int u = 0; u < TU; ++u) {
          const int i = lane + 64 * u;
          rt[h][u] = src[i < nd4 ? i : nd4 - 1];
        }
      }
    }
  };

  uint4 ah[R][NK], al[R][NK];
  float nf[R];
  // codes of the fetched block -> fp16 (hi, lo) value fragments and scaled norms
  auto expand = [&]() {
    CodeWords<D, FMT, BITS> cw[R];
    QjlWords<D, FMT> qw[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if constexpr (FMT == QKV_FMT_UNPACKED) {
#pragma unroll
        for (int i = 0; i < NE / 4; ++i) {
          cw[r].w[i] = rc[r][i] & 0x0F0F0F0Fu;
          if constexpr (SEL) cw[r].w[i] |= selw[i];
        }
      } else if constexpr (FMT == QKV_FMT_PACKED) {
#pragma unroll
        for (int i = 0; i < CodeWords<D, FMT, BITS>::N; ++i) cw[r].w[i] = rc[r][i];
      } else if constexpr (FMT == QKV_FMT_KPLANES) {
#pragma unroll
        for (int i = 0; i < NW; ++i) {
          uint32_t v = 0u;
#pragma unroll
          for (int p = 0; p < 4; ++p)
            if (p < bits) v |= spread8(bfe(rc[r][p], 8 * i, 8)) << p;
          cw[r].w[i] = v;
        }
      }
      if constexpr (IP) {
#pragma unroll
        for (int i = 0; i < QjlWords<D, FMT>::N; ++i) qw[r].w[i] = rq[r][i];
      }
    }
    if constexpr (VT) {
      // tiles of 32 tokens: stage in LDS, then gather bit (m + 16 h) of the
      // lane's NE coordinate words of every plane into nibble codes
#pragma unroll
      for (int h = 0; h < TV; ++h) {
#pragma unroll
        for (int r = 2 * h; r < 2 * h + 2; ++r)
#pragma unroll
          for (int i = 0; i < NW; ++i) cw[r].w[i] = 0u;
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int u = 0; u < TU; ++u) stg[lane + 64 * u] = rt[h][u];
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
            a = split_pair(c0 + (qw[r].bit(e0) ? qs[e0] : -qs[e0]));
            b = split_pair(c1 + (qw[r].bit(e1) ? qs[e1] : -qs[e1]));
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
      nf[r] = rn[r] * ofac;
    }
  };

  const int stride = static_cast<int>(gridDim.x) * kWaves;
  int blk = static_cast<int>(blockIdx.x) * kWaves + __builtin_amdgcn_readfirstlane(wave);
  if (blk >= nblk) return;
  fetch(blk);
  expand();
  for (;;) {
    const int nb = blk + stride;
    const bool more = nb < nblk;
    fetch(more ? nb : blk);  // unconditional: the last round re-reads its own block

    const int gi = blk / bpg;
    const int64_t grp = gi;
    const int64_t t0 = int64_t(blk - gi * bpg) * RB;
    const int64_t tend = min(in_seq, n - grp * in_seq);
    // this block's outputs: rows t0 .. tend - 1 of the group, as one buffer
    // whose byte range drops the stores of rows past the end
    const int64_t nrows = min<int64_t>(RB, tend - t0);
    const __amdgpu_buffer_rsrc_t ob = __builtin_amdgcn_make_buffer_rsrc(
        static_cast<char*>(out) + (grp * in_seq + t0) * D * obytes, 0,
        static_cast<int>(nrows * D * obytes), 0x00020000);

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
      // lane (m, g) holds coordinates 32 p + 8 g + 0..7 of row 16 r + m
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int off = ((16 * r + m) * D + 32 * p + 8 * g) * obytes;
        const float f = nf[r];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const float v0 = acc[hh][r][0] * f, v1 = acc[hh][r][1] * f;
          const float v2 = acc[hh][r][2] * f, v3 = acc[hh][r][3] * f;
          if (out_dtype == QKV_F32) {
            __builtin_amdgcn_raw_buffer_store_b128(
                __builtin_bit_cast(qkv_u32x4, make_float4(v0, v1, v2, v3)), ob, off + 16 * hh, 0, 0);
          } else {
            uint32_t w0, w1;
            if (out_dtype == QKV_F16) {
              w0 = h16(static_cast<_Float16>(v0)) | (h16(static_cast<_Float16>(v1)) << 16);
              w1 = h16(static_cast<_Float16>(v2)) | (h16(static_cast<_Float16>(v3)) << 16);
            } else {
              w0 = qkv_f32_to_bf16(v0) | (uint32_t(qkv_f32_to_bf16(v1)) << 16);
              w1 = qkv_f32_to_bf16(v2) | (uint32_t(qkv_f32_to_bf16(v3)) << 16);
            }
            __builtin_amdgcn_raw_buffer_store_b64(qkv_u32x2{w0, w1}, ob, off + 8 * hh, 0, 0);
          }
        }
      }
    }
    if (!more) break;
    expand();
    blk = nb;
  }
}

template <int D, int FMT, int BITS, bool IP, bool SEL, int R>
int launch(const QkvDecompressArgs& a, hipStream_t s) {
  auto k = decompress_mfma<D, FMT, BITS, IP, SEL, R>;
  // resident workgroups per CU from the kernel's LDS (160 KiB per gfx950 CU)
  // and VGPRs (512 per SIMD lane, four SIMDs)
  static int per_cu = 0;
  if (per_cu == 0) {
    int b = 2;
    hipFuncAttributes at;
    if (hipFuncGetAttributes(&at, reinterpret_cast<const void*>(k)) == hipSuccess) {
      const int by_lds = 160 * 1024 / static_cast<int>(at.sharedSizeBytes > 0 ? at.sharedSizeBytes : 1);
      const int regs = at.numRegs > 0 ? (at.numRegs + 7) / 8 * 8 : 512;
      const int by_regs = (512 / regs) * 4 / kWaves;
      b = by_lds < by_regs ? by_lds : by_regs;
    }
    per_cu = b < 1 ? 1 : b;
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
  // block numbers (32 vectors per block, per group) are 32-bit
  const int64_t groups = (a.n + a.in_seq - 1) / a.in_seq;
  if (groups * ((a.in_seq + 31) / 32) > int64_t(0x7fffffff) - int64_t(qkv_num_cus()) * 64) return false;
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
