// Fused compress straight into the cache store, for bf16, fp16 or fp32 K and V
// rows with d = 128, 96 or 64: normalise -> rotate (MFMA) -> Lloyd-Max
// boundary search -> QJL sign -> bit planes, one pass over the inputs.
//
// Reference: QuashKVEngine.append (quashkv/engine.py:145-172) compresses keys
// with InnerProductQuantizer.compress (quashkv/quantizer.py:211-242) and values
// with MSEQuantizer.compress (quashkv/quantizer.py:113-131); the GPU operator
// surface is fused_compress_ip / fused_compress_mse
// (quashkv/triton_kernels/compress.py:210-303).  The codes land in the K-row and
// V-tile store formats that the decode kernel reads.
//
// Rotation.  z = x Pi^T runs on the 32x32x16 bf16 (fp16) MFMA with x as it is
// stored (a bf16 / fp16 value is exact in the operand type) and Pi split into
// a high and a low 16-bit part, Pi ~= Pi_hi + Pi_lo, accumulated in fp32: two
// MFMA passes carry ~16 (bf16) / ~22 (fp16) significant bits of Pi, against
// 24 for the reference's fp32 GEMM, and y = z / |x| (the reference divides
// before the GEMM).  fp32 rows are divided first, as the reference does:
// x 2^8 / |x| is split into fp16 hi + lo and the fp16 MFMA sums hi Pi_hi +
// hi Pi_lo + lo Pi_hi (~22 significant bits).  Codes computed from x may
// therefore differ from the reference's where y lies within ~1e-5 (bf16 /
// fp16 rows) or ~1e-6 (fp32 rows) relative of a boundary.  The same kernels take a given fp32 y instead of x
// (FROM_Y: the *_rotated entry points) and then run the search, QJL and store
// code below on it; from an identical y the codes are the reference's, bit for
// bit, ties included.
//
// Boundary search as lane masks.  For the value y of one coordinate the
// reference's code is #{i : t_i < y} (torch.bucketize, right=False) and the
// QJL bit is [(y - c_code) S_j >= 0].  Keys search the fine list
// c_0 < t_0 < c_1 < ... < c_{2^m-1} (centroids and boundaries interleaved):
// its count f gives code = f >> 1 and, with the centroids counted as
// [c <= y] where S_j > 0 and [c < y] where S_j < 0, the QJL bit = (f & 1)
// xor [S_j < 0] -- exact, r = 0 included.  Lloyd-Max lists are symmetric about
// 0 (t_mid = 0), so the top bit of f is [y > 0] and the rest is a search of
// |y| in the positive half, complemented for y <= 0.  Strictness survives the
// mirror through integer keys: a = rotl(bits(y), 1) = 2 |y|_bits + sign, and
// thresholds 2 |p|_bits, so [a > 2 p] is [|y| > p] for y > 0 and [|y| >= p]
// for y < 0 -- after the complement, a strict count of y on both sides.  The
// centroid level compares a xor [S_j > 0], which flips that strictness for
// S_j > 0.  Values search their boundaries the same way without the centroid
// level.  A binary search decides one code bit per level with one compare,
// whose 64-lane result mask is directly that bit plane for the wave's 64
// values; the next level's threshold is picked per lane with v_cndmask on the
// masks already found (levels of 1, 2, 4, ... candidates).
//
// Lane-local words.  In a 32x32x16 MFMA result, lane l holds C column l & 31
// and, in its 16 registers, rows 8 (v >> 2) + 4 (l >> 5) + (v & 3).  The
// store words are built inside the lanes: the lanes hold the word's owner
// (keys: C = coordinates x tokens, lane = token; values: C = tokens x
// coordinates, lane = coordinate), the rows of the other operand are ordered
// half-major so that register v of lane half h is position 16 h + v, and
// each compare mask is shifted into per-lane 16-bit accumulators through the
// carry-in of v_addc_co_u32 (shift_in); the two lane halves then merge into
// 32-bit words (merge_halves, v_permlane32_swap) and each lane stores its own
// K-row dwords or V-tile words.  The A and B operand layouts are symmetric,
// so the same x and Pi register fragments serve both orders.
//
// This header holds the device side (the kernels and their helpers) of the
// fused store append; qkv_append.hip holds its C ABI and qkv_append_kv.hip
// the one-launch key + value kernels, each translation unit instantiating
// the templates it launches.

#pragma once

#include <cmath>
#include <cstring>
#include <type_traits>
#include <utility>

#include "qkv_common.h"

// Types shared by both translation units of the append (kernel arguments and
// the one-launch key + value launcher's signature).
namespace qkv_app {

// Positive half of a symmetric comparison list as integer keys 2 bits(p),
// ascending (at most 7 entries: 4-bit value boundaries, the 3-bit key MSE
// fine list).
struct Half {
  uint32_t t[7];
};

// Per-layer pointers of a layer-batched append (kernel arguments by value):
// rows, Pi, S (keys), store array and norms of layer l = blockIdx.y.
constexpr int kMaxAppendLayers = 32;
struct AppendLayers {
  const void* x[kMaxAppendLayers];
  const float* pi[kMaxAppendLayers];
  const float* signs[kMaxAppendLayers];
  void* st[kMaxAppendLayers];
  float* nrm[kMaxAppendLayers];
};

// One launch of append_k_run and append_v_run over n_layers contiguous stores
// (grid.y = layer, grid.x = key workgroups then value workgroups), for
// vbits == mbits + 1 (defined in qkv_append_kv.hip); every wave takes one tile
// (nsplit = 1) or one 32-coordinate block of one tile (nsplit = d / 32), and
// the block counts must cover that.  Returns false, launching nothing, for
// the combinations it does not instantiate or grids that do not cover.
bool launch_append_kv(int mbits, int vbits, int xt, int d, const AppendLayers& ak,
                      const AppendLayers& av, int n_layers, int kblocks, int vblocks, int64_t S,
                      int64_t ktpg, int64_t kntiles, int64_t vtpg, int64_t vntiles, Half fine,
                      Half bnd, int64_t t_stride, int64_t t0, int nsplit, hipStream_t s);

// launch_append_kv over one paged store (append_k_run and append_v_run with
// PAGED), keys and values each with their own Pi.
bool launch_append_kv_paged(int mbits, int vbits, int xt, int d, const void* keys,
                            const void* values, int kblocks, int vblocks, int64_t S,
                            int64_t ktpg, int64_t kntiles, int64_t vtpg, int64_t vntiles,
                            const float* kpi, const float* signs, const float* vpi, Half fine,
                            Half bnd, uint8_t* kpool, float* knorm, uint32_t* vpool,
                            float* vnorm, int64_t t_stride, int64_t t0, const QkvPages& pg,
                            int nsplit, hipStream_t s);

// One launch of append_kmix_run (mixed-precision keys, n_out outlier slots,
// IP or MSE) and append_v_run (value bits 2..4) over one contiguous store
// (defined in qkv_append_kv.hip); false, launching nothing, for combinations
// it does not instantiate.
bool launch_append_kmixv(int n_out, bool ipm, int vbits, int xt, const void* keys,
                         const void* values, int kblocks, int vblocks, int64_t S, int64_t ktpg,
                         int64_t kntiles, int64_t vtpg, int64_t vntiles, const float* pi_perm,
                         const float* signs_perm, Half po, Half pr, uint8_t* kst, float* knorm,
                         const float* vpi, Half bnd, uint32_t* vst, float* vnorm,
                         int64_t t_stride, int64_t t0, int nsplit, hipStream_t s);

}  // namespace qkv_app

namespace {

using qkv_app::AppendLayers;
using qkv_app::Half;
using qkv_app::kMaxAppendLayers;

typedef __bf16 qkv_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 qkv_f16x8 __attribute__((ext_vector_type(8)));

constexpr int kD = 128;                 // head dim of the mixed-key path
constexpr int kHalves = 1;              // 32-token MFMA column blocks per wave tile
constexpr int kTok = 32 * kHalves;      // tokens per wave tile
constexpr int kWaves = 8;               // waves per workgroup (two workgroups per CU)
constexpr int kThreads = 64 * kWaves;
// Pi fragments [block of 32 rows][k-step of 16][split][lane]: 64 KiB at d = 128
template <int D>
constexpr int frag_n() { return (D / 32) * (D / 16) * 2 * 64; }
constexpr int kFragN = frag_n<kD>();
constexpr float kPScaleF16 = 256.f;     // keeps the fp16 low part of Pi out of subnormals

typedef float qkv_f32x16 __attribute__((ext_vector_type(16)));

template <bool F16>
__device__ __forceinline__ qkv_f32x16 mma(uint4 a, uint4 b, qkv_f32x16 c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(qkv_f16x8, a),
                                                  __builtin_bit_cast(qkv_f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(qkv_bf16x8, a),
                                                   __builtin_bit_cast(qkv_bf16x8, b), c, 0, 0, 0);
}

// A wave-uniform value held in a VGPR (a v_cndmask may then take two of them
// with its mask without exceeding the one-scalar-operand limit).
__device__ __forceinline__ uint32_t in_vgpr(uint32_t x) {
  uint32_t r;
  asm("v_mov_b32 %0, %1" : "=v"(r) : "s"(x));
  return r;
}

__device__ __forceinline__ uint64_t lanes_where(bool p) { return __builtin_amdgcn_ballot_w64(p); }

// 2 acc + bit `lane` of mask: shifts this lane's bit of a 64-lane compare mask
// into a lane-local word (v_addc_co_u32 with the mask as carry-in, one
// instruction per mask; no clang builtin spells the carry-in operand).
__device__ __forceinline__ uint32_t shift_in(uint32_t acc, uint64_t mask) {
  uint32_t r;
  uint64_t co;
  asm("v_addc_co_u32 %0, %1, %2, %2, %3" : "=v"(r), "=s"(co) : "v"(acc), "s"(mask));
  return r;
}

// Two 16-bit lane-half accumulators into 32-bit words: lanes 0..31 get
// a(l) | a(l + 32) << 16, lanes 32..63 get b(l - 32) | b(l) << 16.
__device__ __forceinline__ uint32_t merge_halves(uint32_t a, uint32_t b) {
  const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
  return r[0] | (r[1] << 16);
}

// Position of C row m (0..31) of a 32x32 MFMA tile within its 32-block when
// the operand rows are ordered so that lane half h's result registers
// v = 0..15 (rows 8 (v >> 2) + 4 h + (v & 3)) hold positions 16 h + v.
__host__ __device__ constexpr int half_major(int m) {
  return 16 * ((m >> 2) & 1) + 4 * (m >> 3) + (m & 3);
}

// f(std::integral_constant<int, 0>), ..., f(<N - 1>): compile-time unrolled
// loops whose index must be a constant (register-array indices, the slot
// blocks' codebooks).
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Binary search of the key a in the ascending key list t[0 .. 2^LM - 2]: bit i
// of #{j : t[j] < a} as the lane mask g[i].  With CLAST the last level (whose
// candidates are the list's even entries) compares ac instead of a.  T: the
// integer keys, or floats for search_sym_scaled.
template <int LM, bool CLAST, typename T>
__device__ __forceinline__ void search_levels(T a, T ac, const T* t, bool (&c)[LM]) {
  static_for<LM>([&](auto kc) {
    constexpr int k = decltype(kc)::value;  // level k decides bit LM - 1 - k
    T cand[1 << k];
#pragma unroll
    for (int p = 0; p < (1 << k); ++p) cand[p] = t[(2 * p + 1) * (1 << (LM - 1 - k)) - 1];
    // prefix bit j (LSB first) is c[LM - k + j]
#pragma unroll
    for (int j = 0; j < k; ++j)
#pragma unroll
      for (int q = 0; q < (1 << (k - 1 - j)); ++q)
        cand[q] = c[LM - k + j] ? cand[2 * q + 1] : cand[2 * q];
    const T av = (CLAST && k == LM - 1) ? ac : a;
    c[LM - 1 - k] = av > cand[0];
  });
}

template <int LM, bool CLAST>
__device__ __forceinline__ void search_keys(uint32_t a, uint32_t ac, const uint32_t* t,
                                            uint64_t (&g)[LM]) {
  bool c[LM];
  search_levels<LM, CLAST>(a, ac, t, c);
#pragma unroll
  for (int i = 0; i < LM; ++i) g[i] = lanes_where(c[i]);
}

// Strict count #{j : F[j] < y} over a list F of 2^L - 1 entries symmetric
// about 0 (F[j] = -F[2^L - 2 - j], middle entry 0), given the integer keys of
// its positive half: bit i as the lane mask m[i].  The top bit is [y > 0]; the
// others search a = rotl(bits(y), 1) in the positive half and are
// complemented for y <= 0.  With CLAST the last level counts an entry equal to
// |y| as below y on the lanes where cx = 1 (see the file comment).
template <int L, bool CLAST>
__device__ __forceinline__ void search_sym(float y, const uint32_t* p, uint32_t cx,
                                           uint64_t (&m)[L]) {
  const uint32_t u = __builtin_bit_cast(uint32_t, y);
  // [y > 0] on the bits (denormals included, whatever the float mode)
  const uint64_t pos = lanes_where(static_cast<int32_t>(u) > 0);
  m[L - 1] = pos;
  if constexpr (L > 1) {
    const uint32_t a = __builtin_amdgcn_alignbit(u, u, 31);
    uint64_t g[L - 1];
    search_keys<L - 1, CLAST>(a, a ^ cx, p, g);
#pragma unroll
    for (int i = 0; i < L - 1; ++i) m[i] = ~(g[i] ^ pos);
  }
}

// search_sym's lane masks for a value z on another scale (z = y s, s > 0):
// [z > 0] for the top bit and a search of |z| in P, the positive half of the
// list times s, for the others.  Where |z| equals an entry of P the count may
// land on either side of it (search_sym decides those exactly, on y).
template <int L>
__device__ __forceinline__ void search_sym_scaled(float z, const float* P, uint64_t (&m)[L]) {
  const uint64_t pos = lanes_where(z > 0.f);
  m[L - 1] = pos;
  if constexpr (L > 1) {
    const float az = fabsf(z);
    bool c[L - 1];
    search_levels<L - 1, false>(az, az, P, c);
#pragma unroll
    for (int i = 0; i < L - 1; ++i) m[i] = ~(lanes_where(c[i]) ^ pos);
  }
}

// search_sym's count for this lane alone (no lane masks).
template <int L, bool CLAST>
__device__ __forceinline__ uint32_t search_sym_count(float y, const uint32_t* p, uint32_t cx) {
  const uint32_t u = __builtin_bit_cast(uint32_t, y);
  const bool pos = static_cast<int32_t>(u) > 0;
  uint32_t f = pos ? 1u << (L - 1) : 0u;
  if constexpr (L > 1) {
    const uint32_t a = __builtin_amdgcn_alignbit(u, u, 31);
    bool c[L - 1];
    search_levels<L - 1, CLAST>(a, a ^ cx, p, c);
#pragma unroll
    for (int i = 0; i < L - 1; ++i) f |= (c[i] == pos ? 1u : 0u) << i;
  }
  return f;
}

typedef __bf16 qkv_bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 qkv_f16x2 __attribute__((ext_vector_type(2)));

// s + sum of squares of the eight 16-bit values in q (v_dot2: exact products,
// fp32 accumulation)
template <bool F16>
__device__ __forceinline__ float sumsq(uint4 q, float s) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (F16)
      s = __builtin_amdgcn_fdot2(__builtin_bit_cast(qkv_f16x2, w[i]),
                                 __builtin_bit_cast(qkv_f16x2, w[i]), s, false);
    else
      s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(qkv_bf16x2, w[i]),
                                          __builtin_bit_cast(qkv_bf16x2, w[i]), s, false);
  }
  return s;
}

template <bool F16>
__device__ __forceinline__ uint16_t to16(float v) {
  if constexpr (F16)
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
  else
    return qkv_f32_to_bf16(v);
}

typedef __bf16 qkv_bf16x2v __attribute__((ext_vector_type(2)));
typedef float qkv_f32x2v __attribute__((ext_vector_type(2)));

// a (low half) and b as bf16, each rounded to nearest even (one
// v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  const qkv_f32x2v v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, qkv_bf16x2v));
}

template <bool F16>
__device__ __forceinline__ float from16(uint16_t h) {
  if constexpr (F16)
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
  else
    return qkv_bf16_to_f32(h);
}

// Stage the rotation operand in LDS.  Entry ((b * NKS + s) * 2 + split) * 64 + l
// holds, for lane l, Pi'[32 b + r(l & 31)][16 s + 8 (l >> 5) + e], e = 0..7, as
// eight 16-bit values: the high part (split 0) or the low part (split 1) of
// Pi' = Pi * pscale; r(m) = m, or half_major(m) with PERM (the A operand of
// the key append, whose result rows are then coordinates in half-major order).
//
// blk >= 0 stages the slots of coordinate block blk only (a workgroup whose
// waves all compute that block), at the same positions.
template <bool F16, int D = kD, bool PERM = false>
__device__ __forceinline__ void stage_pi(uint4* __restrict__ frag, const float* __restrict__ pi,
                                         float pscale, int blk = -1) {
  // kThreads threads (every launch uses that block size); each takes NPT
  // (block, k-step, lane) slots and writes both splits of each, with all of
  // its Pi loads in flight before the first conversion
  constexpr int NKS = D / 16;  // k-steps
  constexpr int NSLOT = frag_n<D>() / 2;
  constexpr int NPT = (NSLOT + kThreads - 1) / kThreads;  // the last may be partial (d = 96)
  constexpr int NS1 = NKS * 64;                           // one block's slots
  static_assert(NS1 <= kThreads, "one block's slots: at most one per thread");
  auto addr = [&](int u) {
    const int ln = u & 63, s = (u >> 6) % NKS, b = (u >> 6) / NKS;
    const int j = 32 * b + (PERM ? half_major(ln & 31) : (ln & 31)), k0 = 16 * s + 8 * (ln >> 5);
    return pi + j * D + k0;
  };
  auto put = [&](int u, float4 p0, float4 p1) {
    const int ln = u & 63, s = (u >> 6) % NKS, b = (u >> 6) / NKS;
    // pscale = 2^k: the scaling is exact
    const float v[8] = {p0.x * pscale, p0.y * pscale, p0.z * pscale, p0.w * pscale,
                        p1.x * pscale, p1.y * pscale, p1.z * pscale, p1.w * pscale};
    uint32_t hw[4], lw[4];  // pairs of 16-bit values, element 2 i low
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (F16) {
        const uint32_t h0 = to16<true>(v[2 * i]), h1 = to16<true>(v[2 * i + 1]);
        hw[i] = h0 | (h1 << 16);
        lw[i] = to16<true>(v[2 * i] - from16<true>(h0)) |
                (static_cast<uint32_t>(to16<true>(v[2 * i + 1] - from16<true>(h1))) << 16);
      } else {
        // v_cvt_pk_bf16_f32: two round-to-nearest-even conversions (the
        // entries are finite)
        hw[i] = pk_bf16(v[2 * i], v[2 * i + 1]);
        lw[i] = pk_bf16(v[2 * i] - __uint_as_float(hw[i] << 16),
                        v[2 * i + 1] - __uint_as_float(hw[i] & 0xffff0000u));
      }
    }
    const int e = ((b * NKS + s) * 2) * 64 + ln;
    frag[e] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    frag[e + 64] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
  };
  if (blk >= 0) {
    if (threadIdx.x < NS1) {
      const int u = blk * NS1 + threadIdx.x;
      const float* a = addr(u);
      put(u, *reinterpret_cast<const float4*>(a), *reinterpret_cast<const float4*>(a + 4));
    }
    return;
  }
  float4 p[NPT][2];
#pragma unroll
  for (int x = 0; x < NPT; ++x) {
    const float* a = addr(min(threadIdx.x + kThreads * x, NSLOT - 1));
    p[x][0] = *reinterpret_cast<const float4*>(a);
    p[x][1] = *reinterpret_cast<const float4*>(a + 4);
  }
#pragma unroll
  for (int x = 0; x < NPT; ++x) {
    const int u = threadIdx.x + kThreads * x;
    if (NSLOT % kThreads != 0 && u >= NSLOT) break;
    put(u, p[x][0], p[x][1]);
  }
}

// Workgroups of a one-tile-per-wave launch (ONE below): nsplit = 1 gives wave
// g = b kWaves + w tile g; nsplit > 1 gives workgroup b coordinate block
// b % nsplit of tiles (b / nsplit) kWaves + w, so that it stages that block of
// Pi only.
__host__ __device__ constexpr int64_t one_blocks(int64_t ntiles, int nsplit) {
  return nsplit * ((ntiles + kWaves - 1) / kWaves);
}

constexpr int kXcds = 8;  // MI355X deals consecutive workgroups to its 8 XCDs in turn

// Coordinate block `blk` and first tile of wave wv of workgroup bid of nb
// (nsplit > 1).  Block-major; when nb is a whole number of rounds of kXcds
// tile groups, the nsplit workgroups of a tile group share bid % kXcds, so
// that they run on one XCD and its L2 fetches their rows once.
__device__ __forceinline__ int64_t one_first(int bid, int nb, int nsplit, int wv, int& blk) {
  int g;
  if (nb % (kXcds * nsplit) == 0) {
    const int r = bid / kXcds;
    blk = r % nsplit;
    g = (r / nsplit) * kXcds + bid % kXcds;
  } else {
    blk = bid % nsplit;
    g = bid / nsplit;
  }
  return int64_t(g) * kWaves + wv;
}

// Group of tile `tile` (tpg tiles per group) in 32-bit arithmetic: the hosts
// keep tile counts below 2^31 (a 64-bit division is ~130 scalar instructions
// ahead of a wave's first load).
__device__ __forceinline__ int64_t tile_group(int64_t tile, int64_t tpg) {
  return static_cast<uint32_t>(tile) / static_cast<uint32_t>(tpg);
}

// x fragments of a wave tile: xf[tt][s], lane l = (row l & 31, half l >> 5)
// holds x[token 32 tt + (l & 31)][16 s + 8 (l >> 5) .. + 7], read from row[tt]
// (this lane's token row of block tt; callers point lanes without a token at a
// valid row, whose results are never stored).
template <int NKS>
__device__ __forceinline__ void load_x(uint4 (&xf)[kHalves][NKS],
                                       const uint16_t* const (&row)[kHalves], int lane) {
#pragma unroll
  for (int tt = 0; tt < kHalves; ++tt)
#pragma unroll
    for (int s = 0; s < NKS; ++s)
      xf[tt][s] = *reinterpret_cast<const uint4*>(row[tt] + 16 * s + 8 * (lane >> 5));
}

// fp32 rows for the fp16 MFMA: x 2^8 / |x| = hi + lo, both fp16, in load_x's
// fragment layout (xh, xl).  The rotation then sums hi Pi_hi + hi Pi_lo +
// lo Pi_hi (Pi' = 2^8 Pi split likewise), ~22 significant bits, and the MFMA
// result is 2^16 y.  |x| (clamped at 1e-8, as the reference clamps) of the
// lane's token row per block in nrm.
template <int NKS>
__device__ __forceinline__ void load_x_f32(uint4 (&xh)[kHalves][NKS], uint4 (&xl)[kHalves][NKS],
                                           float (&nrm)[kHalves],
                                           const float* const (&row)[kHalves], int lane) {
#pragma unroll
  for (int tt = 0; tt < kHalves; ++tt) {
    float4 v[NKS][2];
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
      const float* p = row[tt] + 16 * s + 8 * (lane >> 5);
      v[s][0] = *reinterpret_cast<const float4*>(p);
      v[s][1] = *reinterpret_cast<const float4*>(p + 4);
    }
    float ss = 0.f;
#pragma unroll
    for (int s = 0; s < NKS; ++s)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        ss = fmaf(v[s][h].x, v[s][h].x, ss);
        ss = fmaf(v[s][h].y, v[s][h].y, ss);
        ss = fmaf(v[s][h].z, v[s][h].z, ss);
        ss = fmaf(v[s][h].w, v[s][h].w, ss);
      }
    ss += __shfl_xor(ss, 32, 64);
    const float n = fmaxf(sqrtf(ss), 1e-8f);
    nrm[tt] = n;
    const float sc = 256.f / n;
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
      const float a[8] = {v[s][0].x, v[s][0].y, v[s][0].z, v[s][0].w,
                          v[s][1].x, v[s][1].y, v[s][1].z, v[s][1].w};
      uint32_t hw[4], lw[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float a0 = a[2 * e] * sc, a1 = a[2 * e + 1] * sc;
        const _Float16 h0 = static_cast<_Float16>(a0), h1 = static_cast<_Float16>(a1);
        const _Float16 l0 = static_cast<_Float16>(a0 - static_cast<float>(h0));
        const _Float16 l1 = static_cast<_Float16>(a1 - static_cast<float>(h1));
        hw[e] = __builtin_bit_cast(uint16_t, h0) |
                (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h1)) << 16);
        lw[e] = __builtin_bit_cast(uint16_t, l0) |
                (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, l1)) << 16);
      }
      xh[tt][s] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
      xl[tt][s] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
    }
  }
}

// ------------------------------------------------------------------ keys

// One wave per tile of kTok consecutive tokens of one (b, h) group.  Input rows
// grp * S + s; store rows grp * t_stride + t0 + s ((MB + 1) * D / 8 bytes:
// MB MSE planes, then the QJL plane).  FROM_Y: `xin` holds fp32 rotated unit
// rows y (rows as above) and `nin` their norms; the normalisation and the
// rotation are skipped, and the search is search_sym's exact one on y.
// XT: the input rows' type, 0 bf16, 1 fp16, 2 fp32 (on the fp16 MFMA, split)
//
// Orientation: C = coordinates x tokens (A = Pi's rows in half-major order,
// B = x), so lane l holds token l & 31 and, in register v, coordinate
// 32 n + 16 (l >> 5) + v of block n.  Each compare mask is shifted into the
// lanes' own 16-bit plane accumulators (shift_in), the two lane halves are
// merged into 32-coordinate words (merge_halves), and every lane stores a
// contiguous run of its own token's K row.  From x the search compares the
// raw MFMA result against the list scaled by the lane's token norm.
//
// ONE: small appends, where one wave's chain is the kernel's time.  Each wave
// takes at most one tile (nb * kWaves >= ntiles * nsplit, the host's
// guarantee), or with nsplit = D / 32 one 32-coordinate block of one tile, so
// that the chain is a quarter (d = 128) or a half (d = 64) of a tile's MFMAs
// and searches; a bf16 / fp16 wave's rows are loaded before Pi is staged, so
// that the two global-load latencies overlap.
template <int MB, int XT, int D, bool PAGED, bool FROM_Y, bool ONE = false>
__device__ __forceinline__ void append_k_run(
    const void* __restrict__ xin, const float* __restrict__ nin, int64_t S, int64_t tpg,
    int64_t ntiles, const float* __restrict__ pi, const float* __restrict__ signs, Half fine,
    uint8_t* __restrict__ kst, float* __restrict__ knorm, int64_t t_stride, int64_t t0,
    QkvPages pg, uint4* __restrict__ frag, int bid, int nb, int nsplit = 1) {
  static_assert(kHalves == 1, "one 32-token MFMA column block per wave tile");
  constexpr bool F16 = XT != 0, F32 = XT == 2;  // fp16 MFMA / fp32 rows split for it
  constexpr int L = MB + 1;           // search levels over the fine list
  constexpr int NP = (1 << MB) - 1;   // positive half of the fine list c_0, t_0, ..., c_{2^MB-1}
  constexpr int NBK = D / 32;         // coordinate blocks = dwords per plane
  constexpr int NKS = D / 16;         // k-steps
  constexpr int RD = NBK * L;         // dwords per row
  constexpr int RDH = (RD + 1) / 2;   // dwords per row a lane half stores
  constexpr int LH = (L + 1) / 2;     // split: planes per lane half
  const int lane = threadIdx.x & 63, li = lane & 31, hh = lane >> 5;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // tile math on the SALU
  // ONE with nsplit = NBK: the workgroup's coordinate block and tiles as in
  // one_blocks, each wave computing and storing that block's words only;
  // nsplit = 1: wave g takes tile g whole
  const bool split = ONE && nsplit > 1;
  int myblk = 0;
  const int64_t gw = split ? one_first(bid, nb, NBK, wv, myblk)  // the wave's first tile
                           : int64_t(bid) * kWaves + wv;
  constexpr bool PRE = ONE && !FROM_Y && !F32;  // rows loaded before the Pi staging
  uint4 xpre[1][PRE ? NKS : 1];
  if constexpr (PRE) {
    const int64_t tile = gw;
    if (tile < ntiles) {
      const int64_t grp = tile_group(tile, tpg), s0 = (tile - grp * tpg) * kTok;
      const int nv = static_cast<int>(min<int64_t>(kTok, S - s0));
      const uint16_t* row[1] = {static_cast<const uint16_t*>(xin) +
                                (grp * S + s0 + min(li, nv - 1)) * D};
      load_x<NKS>(xpre, row, lane);
    }
  }
  if constexpr (!FROM_Y) {
    stage_pi<F16, D, true>(frag, pi, F16 ? kPScaleF16 : 1.f, split ? myblk : -1);
    __syncthreads();
  }

  // the positive half of the fine list: integer keys (FROM_Y) or floats
  uint32_t fv[NP];
  float fp[NP];
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    fv[i] = in_vgpr(fine.t[i]);
    fp[i] = __uint_as_float(fine.t[i] >> 1);
  }
  // per block n, bits v of this lane half's coordinates 32 n + 16 h + v:
  // [S < 0] (the QJL plane's flip) and [S >= 0] (the exact search's centroid
  // level counts c <= y there)
  uint32_t qflip[NBK], cxw[NBK];
#pragma unroll
  for (int n = 0; n < NBK; ++n) {
    const uint32_t negw = static_cast<uint32_t>(lanes_where(signs[32 * n + li] < 0.f));
    qflip[n] = (negw >> (16 * hh)) & 0xffffu;
    cxw[n] = qflip[n] ^ 0xffffu;
  }
  const float iscale = F16 ? 1.f / kPScaleF16 : 1.f;
  const int64_t wstep = int64_t(nb) * kWaves;

  for (int64_t tile = gw; tile < ntiles; tile += wstep) {
    const int64_t grp = tile_group(tile, tpg);
    const int64_t s0 = (tile - grp * tpg) * kTok;
    const int nv = static_cast<int>(min<int64_t>(kTok, S - s0));
    const int64_t srow = grp * S + s0 + min(li, nv - 1);  // this lane's token row (clamped)
    QkvSpan sp{};
    if constexpr (PAGED) sp = qkv_span(pg, grp, t_stride, t0 + s0);
    uint4 xf[1][NKS];  // tokens past S read the last row; their results are not stored
    uint4 xl[1][F32 ? NKS : 1];  // fp32 rows: the low fp16 parts
    float thr[NP];               // the list in MFMA-result units of this lane's token
    if constexpr (FROM_Y) {
      if (lane < 32 && li < nv) {
        const int64_t t = t0 + s0 + li;
        const int64_t r = PAGED ? sp.row(t) : grp * t_stride + t;
        if (r >= 0) knorm[r] = nin[srow];
      }
    } else {
      float nrm[1];
      if constexpr (F32) {
        const float* row[1] = {static_cast<const float*>(xin) + srow * D};
        load_x_f32<NKS>(xf, xl, nrm, row, lane);
      } else {
        if constexpr (PRE) {
#pragma unroll
          for (int s = 0; s < NKS; ++s) xf[0][s] = xpre[0][s];
        } else {
          const uint16_t* row[1] = {static_cast<const uint16_t*>(xin) + srow * D};
          load_x<NKS>(xf, row, lane);
        }
        float ss = 0.f;
#pragma unroll
        for (int s = 0; s < NKS; ++s) ss = sumsq<F16>(xf[0][s], ss);
        ss += __shfl_xor(ss, 32, 64);
        nrm[0] = fmaxf(sqrtf(ss), 1e-8f);
      }
      if (lane < 32 && li < nv) {
        const int64_t t = t0 + s0 + li;
        const int64_t r = PAGED ? sp.row(t) : grp * t_stride + t;
        if (r >= 0 && myblk == 0) knorm[r] = nrm[0];
      }
      // the MFMA result is y |x| / iscale (fp32 rows: 2^16 y)
      const float zs = F32 ? 65536.f : nrm[0] / iscale;
#pragma unroll
      for (int i = 0; i < NP; ++i) thr[i] = fp[i] * zs;
    }

    uint32_t kw[RD];  // [plane][block]: this lane half's 16 bits of each row dword
#pragma unroll
    for (int i = 0; i < RD; ++i) kw[i] = 0u;

    static_for<NBK>([&](auto nc) {  // coordinates 32 n .. 32 n + 31: word n of each plane
      constexpr int n = decltype(nc)::value;
      if (split && n != myblk) return;
      // one coordinate block at a time: keeps the scheduler from overlapping
      // blocks (and their accumulators and fragments) beyond the register file
      __builtin_amdgcn_sched_barrier(0);
      float yv[16];  // coordinate 32 n + 16 h + v of this lane's token
      if constexpr (FROM_Y) {
        const float4* y = reinterpret_cast<const float4*>(static_cast<const float*>(xin) +
                                                          srow * D + 32 * n + 16 * hh);
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const float4 q = y[a];
          yv[4 * a] = q.x; yv[4 * a + 1] = q.y; yv[4 * a + 2] = q.z; yv[4 * a + 3] = q.w;
        }
      } else {
        qkv_f32x16 acc = {};
#pragma unroll
        for (int s = 0; s < NKS; ++s)
#pragma unroll
          for (int sp2 = 0; sp2 < 2; ++sp2) {
            const uint4 af = frag[((n * NKS + s) * 2 + sp2) * 64 + lane];
            acc = mma<F16>(af, xf[0][s], acc);
            if (F32 && sp2 == 0) acc = mma<F16>(af, xl[0][F32 ? s : 0], acc);
          }
#pragma unroll
        for (int v = 0; v < 16; ++v) yv[v] = acc[v];
      }
      // registers high to low: bit v of each accumulator is register v
      static_for<16>([&](auto vc) {
        constexpr int v = 15 - decltype(vc)::value;
        uint64_t f[L];
        if constexpr (FROM_Y)
          search_sym<L, true>(yv[v], fv, (cxw[n] >> v) & 1u, f);
        else
          search_sym_scaled<L>(yv[v], thr, f);
        // plane r: MSE bit r (fine-count bit r + 1); plane MB: QJL (bit 0)
#pragma unroll
        for (int r = 0; r < L; ++r) kw[r * NBK + n] = shift_in(kw[r * NBK + n], f[r < MB ? r + 1 : 0]);
      });
      kw[MB * NBK + n] ^= qflip[n];
    });

    // lane half h stores dwords h RDH .. of its token's row (split: planes
    // h LH .. of block myblk)
    const int64_t tk = t0 + s0 + li;
    const int64_t row = li < nv ? (PAGED ? sp.row(tk) : grp * t_stride + tk) : -1;
    uint32_t* dst = reinterpret_cast<uint32_t*>(kst) + row * RD;
    if (split) {
#pragma unroll
      for (int i = 0; i < LH; ++i) {
        const int rb = i + LH < L ? i + LH : i;
        const uint32_t w = merge_halves(kw[i * NBK + myblk], kw[rb * NBK + myblk]);
        const int r = hh ? rb : i;
        if (row >= 0 && (hh == 0 || i + LH < L)) dst[r * NBK + myblk] = w;
      }
    } else {
      uint32_t ow[RDH];
#pragma unroll
      for (int i = 0; i < RDH; ++i) ow[i] = merge_halves(kw[i], kw[i + RDH < RD ? i + RDH : i]);
      if (row >= 0) {
        uint32_t* d = dst + hh * RDH;
        constexpr int VW = (RDH % 4 == 0 && RD % 4 == 0) ? 4 : (RDH % 2 == 0 && RD % 2 == 0) ? 2 : 1;
#pragma unroll
        for (int i = 0; i < RDH; i += VW) {
          if (RD % 2 != 0 && hh == 1 && RDH + i >= RD) continue;
          if constexpr (VW == 4)
            *reinterpret_cast<uint4*>(d + i) = make_uint4(ow[i], ow[i + 1], ow[i + 2], ow[i + 3]);
          else if constexpr (VW == 2)
            *reinterpret_cast<uint2*>(d + i) = make_uint2(ow[i], ow[i + 1]);
          else
            d[i] = ow[i];
        }
      }
    }
    if constexpr (ONE) break;
  }
}

template <int MB, int XT, int D, bool PAGED, bool FROM_Y>
__global__ __launch_bounds__(kThreads, PAGED ? 2 : 4) void append_k_mfma(
    const void* __restrict__ xin, const float* __restrict__ nin, int64_t S, int64_t tpg,
    int64_t ntiles, const float* __restrict__ pi, const float* __restrict__ signs, Half fine,
    uint8_t* __restrict__ kst, float* __restrict__ knorm, int64_t t_stride, int64_t t0,
    QkvPages pg) {
  __shared__ uint4 frag[FROM_Y ? 1 : frag_n<D>()];  // Pi operand fragments
  append_k_run<MB, XT, D, PAGED, FROM_Y>(xin, nin, S, tpg, ntiles, pi, signs, fine, kst, knorm,
                                         t_stride, t0, pg, frag, blockIdx.x, gridDim.x);
}

// append_k_mfma over the contiguous stores of blockIdx.y's layer
template <int MB, int XT, int D>
__global__ __launch_bounds__(kThreads, 4) void append_k_layers(AppendLayers al, int64_t S,
                                                               int64_t tpg, int64_t ntiles,
                                                               Half fine, int64_t t_stride,
                                                               int64_t t0) {
  __shared__ uint4 frag[frag_n<D>()];
  const int l = blockIdx.y;
  append_k_run<MB, XT, D, false, false>(al.x[l], nullptr, S, tpg, ntiles, al.pi[l], al.signs[l],
                                        fine, static_cast<uint8_t*>(al.st[l]), al.nrm[l],
                                        t_stride, t0, QkvPages{}, frag, blockIdx.x, gridDim.x);
}

// ------------------------------------------------- mixed-precision keys

// Mixed-precision keys over permuted coordinates (outliers first; the caller
// passes Pi with its rows permuted and, for IP keys, S in the same slot order)
// into rows of whole dwords:
//  * !IPM, MixedPrecisionMSEQuantizer (quashkv/mixed_precision.py:132-158)
//    with 3-bit outlier and 2-bit regular channels: plane b0 and plane b1 of
//    every slot, then b2 of the NO outlier slots, then their parity
//    b0^b1^b2 -- 32 + NO / 4 bytes;
//  * IPM, MixedPrecisionIPQuantizer (quashkv/mixed_precision.py:283-297) with
//    a 2-bit outlier / 1-bit regular MSE stage: plane b0 of every slot, the
//    QJL plane [(y - c) S >= 0] of every slot, then b1 of the NO outlier
//    slots -- 32 + NO / 8 bytes.
// The outlier slots fill whole 32-slot blocks (NO = 32 or 64), so each block's
// codebook is fixed at compile time.  FROM_Y: `xin` holds fp32 rotated unit
// rows in slot order and `nin` their norms, searched exactly (search_sym, the
// reference's QJL tie rule); from x the search compares the raw MFMA result
// against each codebook's list scaled by the lane's token norm, as
// append_k_run's does.  Orientation, lane-local words, ONE and nsplit as in
// append_k_run (Pi's rows in slot order, half-major within each block).
template <int NO, int XT, bool FROM_Y, bool IPM, bool ONE = false>
__device__ __forceinline__ void append_kmix_run(
    const void* __restrict__ xin, const float* __restrict__ nin, int64_t S, int64_t tpg,
    int64_t ntiles, const float* __restrict__ pi_perm, const float* __restrict__ signs_perm,
    Half po, Half pr, uint8_t* __restrict__ kst, float* __restrict__ knorm, int64_t t_stride,
    int64_t t0, uint4* __restrict__ frag, int bid, int nb, int nsplit = 1) {
  static_assert(kHalves == 1, "one 32-token MFMA column block per wave tile");
  constexpr bool F16 = XT != 0, F32 = XT == 2;        // fp16 MFMA / fp32 rows split for it
  constexpr int NOB = NO / 32;                         // outlier blocks
  constexpr int NBK = kD / 32;                         // slot blocks
  constexpr int NKS = kD / 16;                         // k-steps
  constexpr int RD = IPM ? 8 + NOB : 8 + 2 * NOB;      // dwords per row
  constexpr int RDH = (RD + 1) / 2;                    // dwords per row a lane half stores
  const int lane = threadIdx.x & 63, li = lane & 31, hh = lane >> 5;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool split = ONE && nsplit > 1;
  int myblk = 0;
  const int64_t gw = split ? one_first(bid, nb, NBK, wv, myblk)  // the wave's first tile
                           : int64_t(bid) * kWaves + wv;
  constexpr bool PRE = ONE && !FROM_Y && !F32;
  uint4 xpre[1][PRE ? NKS : 1];
  if constexpr (PRE) {
    if (gw < ntiles) {
      const int64_t grp = tile_group(gw, tpg), s0 = (gw - grp * tpg) * kTok;
      const int nv = static_cast<int>(min<int64_t>(kTok, S - s0));
      const uint16_t* row[1] = {static_cast<const uint16_t*>(xin) +
                                (grp * S + s0 + min(li, nv - 1)) * kD};
      load_x<NKS>(xpre, row, lane);
    }
  }
  if constexpr (!FROM_Y) {
    stage_pi<F16, kD, true>(frag, pi_perm, F16 ? kPScaleF16 : 1.f, split ? myblk : -1);
    __syncthreads();
  }

  // positive halves: outlier and regular boundaries (MSE keys) or fine lists
  // (IP keys), three and one entries either way; integer keys (FROM_Y) or floats
  uint32_t pov[3], prv[1];
  float pof[3], prf[1];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    pov[i] = in_vgpr(po.t[i]);
    pof[i] = __uint_as_float(po.t[i] >> 1);
  }
  prv[0] = in_vgpr(pr.t[0]);
  prf[0] = __uint_as_float(pr.t[0] >> 1);
  // IP keys, per block n, bits v of this lane half's slots 32 n + 16 h + v:
  // [S < 0] (the QJL plane's flip) and [S >= 0] (the exact search's centroid
  // level counts c <= y there)
  uint32_t qflip[NBK], cxw[NBK];
#pragma unroll
  for (int n = 0; n < NBK; ++n) {
    qflip[n] = 0u;
    if constexpr (IPM) {
      const uint32_t negw = static_cast<uint32_t>(lanes_where(signs_perm[32 * n + li] < 0.f));
      qflip[n] = (negw >> (16 * hh)) & 0xffffu;
    }
    cxw[n] = qflip[n] ^ 0xffffu;
  }
  const float iscale = F16 ? 1.f / kPScaleF16 : 1.f;
  const int64_t wstep = int64_t(nb) * kWaves;

  for (int64_t tile = gw; tile < ntiles; tile += wstep) {
    const int64_t grp = tile_group(tile, tpg);
    const int64_t s0 = (tile - grp * tpg) * kTok;
    const int nv = static_cast<int>(min<int64_t>(kTok, S - s0));
    const int64_t srow = grp * S + s0 + min(li, nv - 1);  // this lane's token row (clamped)
    float* nrow = knorm + grp * t_stride + t0 + s0;
    uint4 xf[1][NKS];
    uint4 xl[1][F32 ? NKS : 1];  // fp32 rows: the low fp16 parts
    float tho[3], thr[1];        // the lists in MFMA-result units of this lane's token
    if constexpr (FROM_Y) {
      if (lane < 32 && li < nv) nrow[li] = nin[srow];
    } else {
      float nrm[1];
      if constexpr (F32) {
        const float* row[1] = {static_cast<const float*>(xin) + srow * kD};
        load_x_f32<NKS>(xf, xl, nrm, row, lane);
      } else {
        if constexpr (PRE) {
#pragma unroll
          for (int s = 0; s < NKS; ++s) xf[0][s] = xpre[0][s];
        } else {
          const uint16_t* row[1] = {static_cast<const uint16_t*>(xin) + srow * kD};
          load_x<NKS>(xf, row, lane);
        }
        float ss = 0.f;
#pragma unroll
        for (int s = 0; s < NKS; ++s) ss = sumsq<F16>(xf[0][s], ss);
        ss += __shfl_xor(ss, 32, 64);
        nrm[0] = fmaxf(sqrtf(ss), 1e-8f);
      }
      if (lane < 32 && li < nv && myblk == 0) nrow[li] = nrm[0];
      // the MFMA result is y |x| / iscale (fp32 rows: 2^16 y)
      const float zs = F32 ? 65536.f : nrm[0] / iscale;
#pragma unroll
      for (int i = 0; i < 3; ++i) tho[i] = pof[i] * zs;
      thr[0] = prf[0] * zs;
    }

    // row dword of plane word r of block n: whole planes at word n, outlier
    // words after them (MSE keys: b0, b1, b2, parity; IP keys: b0, QJL, b1)
    auto dw = [](int r, int n) { return r < 2 ? 4 * r + n : 8 + n + (r == 3 ? NOB : 0); };
    const int64_t row = li < nv ? grp * t_stride + t0 + s0 + li : -1;
    uint32_t* dst = reinterpret_cast<uint32_t*>(kst) + row * RD;
    uint32_t kw[RD];  // this lane half's 16 bits of each row dword
#pragma unroll
    for (int i = 0; i < RD; ++i) kw[i] = 0u;

    static_for<NBK>([&](auto nc) {  // slots 32 n .. 32 n + 31
      constexpr int n = decltype(nc)::value;
      if (split && n != myblk) return;
      __builtin_amdgcn_sched_barrier(0);  // one slot block at a time (registers)
      constexpr bool OUT = n < NOB;
      constexpr int L = OUT ? 3 : 2;      // search levels
      constexpr int NW = OUT ? (IPM ? 3 : 4) : 2;  // row dwords of this block
      float yv[16];  // slot 32 n + 16 h + v of this lane's token
      if constexpr (FROM_Y) {
        const float4* y = reinterpret_cast<const float4*>(static_cast<const float*>(xin) +
                                                          srow * kD + 32 * n + 16 * hh);
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const float4 q = y[a];
          yv[4 * a] = q.x; yv[4 * a + 1] = q.y; yv[4 * a + 2] = q.z; yv[4 * a + 3] = q.w;
        }
      } else {
        qkv_f32x16 acc = {};
#pragma unroll
        for (int s = 0; s < NKS; ++s)
#pragma unroll
          for (int sp2 = 0; sp2 < 2; ++sp2) {
            const uint4 af = frag[((n * NKS + s) * 2 + sp2) * 64 + lane];
            acc = mma<F16>(af, xf[0][s], acc);
            if (F32 && sp2 == 0) acc = mma<F16>(af, xl[0][F32 ? s : 0], acc);
          }
#pragma unroll
        for (int v = 0; v < 16; ++v) yv[v] = acc[v];
      }
      // registers high to low: bit v of each accumulator is register v
      static_for<16>([&](auto vc) {
        constexpr int v = 15 - decltype(vc)::value;
        uint64_t m[L];
        if constexpr (FROM_Y)
          search_sym<L, IPM>(yv[v], OUT ? pov : prv, (cxw[n] >> v) & 1u, m);
        else
          search_sym_scaled<L>(yv[v], OUT ? tho : thr, m);
        if constexpr (IPM) {
          // b0 = MSE bit 0 (fine-count bit 1), QJL = fine-count bit 0,
          // outliers: b1 = MSE bit 1 (fine-count bit 2)
          kw[dw(0, n)] = shift_in(kw[dw(0, n)], m[1]);
          kw[dw(1, n)] = shift_in(kw[dw(1, n)], m[0]);
          if constexpr (OUT) kw[dw(2, n)] = shift_in(kw[dw(2, n)], m[2]);
        } else {
#pragma unroll
          for (int r = 0; r < L; ++r) kw[dw(r, n)] = shift_in(kw[dw(r, n)], m[r]);
        }
      });
      if constexpr (IPM)
        kw[dw(1, n)] ^= qflip[n];
      else if constexpr (OUT)
        kw[dw(3, n)] = kw[dw(0, n)] ^ kw[dw(1, n)] ^ kw[dw(2, n)];
      if (split) {
        // lane half h stores block n's words h LH ..
        constexpr int LH = (NW + 1) / 2;
#pragma unroll
        for (int i = 0; i < LH; ++i) {
          const int rb = i + LH < NW ? i + LH : i;
          const uint32_t w = merge_halves(kw[dw(i, n)], kw[dw(rb, n)]);
          if (row >= 0 && (hh == 0 || i + LH < NW)) dst[hh ? dw(rb, n) : dw(i, n)] = w;
        }
      }
    });

    if (!split) {
      // lane half h stores dwords h RDH .. of its token's row
      uint32_t ow[RDH];
#pragma unroll
      for (int i = 0; i < RDH; ++i) ow[i] = merge_halves(kw[i], kw[i + RDH < RD ? i + RDH : i]);
      if (row >= 0) {
        uint32_t* d = dst + hh * RDH;
        constexpr int VW = (RDH % 2 == 0 && RD % 2 == 0) ? 2 : 1;
#pragma unroll
        for (int i = 0; i < RDH; i += VW) {
          if (RD % 2 != 0 && hh == 1 && RDH + i >= RD) continue;
          if constexpr (VW == 2)
            *reinterpret_cast<uint2*>(d + i) = make_uint2(ow[i], ow[i + 1]);
          else
            d[i] = ow[i];
        }
      }
    }
    if constexpr (ONE) break;
  }
}

template <int NO, int XT, bool FROM_Y, bool IPM>
__global__ __launch_bounds__(kThreads, 2) void append_kmix_mfma(
    const void* __restrict__ xin, const float* __restrict__ nin, int64_t S, int64_t tpg,
    int64_t ntiles, const float* __restrict__ pi_perm, const float* __restrict__ signs_perm,
    Half po, Half pr, uint8_t* __restrict__ kst, float* __restrict__ knorm, int64_t t_stride,
    int64_t t0) {
  __shared__ uint4 frag[FROM_Y ? 1 : kFragN];  // Pi fragments (slot order, half-major per block)
  append_kmix_run<NO, XT, FROM_Y, IPM>(xin, nin, S, tpg, ntiles, pi_perm, signs_perm, po, pr, kst,
                                       knorm, t_stride, t0, frag, blockIdx.x, gridDim.x);
}

// ------------------------------------------------ quantizer-API compress

// MSEQuantizer.compress / InnerProductQuantizer.compress and fused_compress_*
// (quashkv/quantizer.py:113-131,211-242, quashkv/triton_kernels/compress.py:
// 210-303) on the MFMA: n rows of dimension D into one uint8 code (and, IP,
// one QJL bit) per coordinate, row-major, and the fp32 norms.  The rotation, search and tie rules are append_k_mfma's
// (tokens x coordinates); IP searches the fine list (L = MB + 1 levels), MSE
// the boundaries (L = bits levels).  A lane's code byte lands beside its
// 31 neighbours' (32 coordinates of one row per half-wave).
template <int L, bool IP, int XT, int D>
__global__ __launch_bounds__(kThreads, 4) void compress_mfma(
    const void* __restrict__ xin, int64_t n, int64_t ntiles, const float* __restrict__ pi,
    const float* __restrict__ signs, Half lst, uint8_t* __restrict__ codes,
    uint8_t* __restrict__ qjl, float* __restrict__ norms) {
  constexpr bool F16 = XT != 0, F32 = XT == 2;
  constexpr int NP = (1 << (L - 1)) - 1;  // positive half of the searched list
  constexpr int NBK = D / 32, NKS = D / 16;
  __shared__ uint4 frag[frag_n<D>()];
  __shared__ float4 inv_s[kWaves][kTok / 4];
  stage_pi<F16, D>(frag, pi, F16 ? kPScaleF16 : 1.f);
  __syncthreads();

  const int lane = threadIdx.x & 63, li = lane & 31, wv = threadIdx.x >> 6;
  uint32_t lv[NP > 0 ? NP : 1];
#pragma unroll
  for (int i = 0; i < NP; ++i) lv[i] = in_vgpr(lst.t[i]);
  uint32_t cx[NBK];  // IP: 1 where S >= 0 (the centroid level counts c <= y there)
  uint32_t neg[NBK];  // IP: 1 where S < 0
#pragma unroll
  for (int b = 0; b < NBK; ++b) {
    const bool ng = IP && signs[32 * b + li] < 0.f;
    cx[b] = ng ? 0u : 1u;
    neg[b] = ng ? 1u : 0u;
  }
  const float iscale = F16 ? 1.f / kPScaleF16 : 1.f;
  const int64_t wstep = int64_t(gridDim.x) * kWaves;

  for (int64_t tile = int64_t(blockIdx.x) * kWaves + wv; tile < ntiles; tile += wstep) {
    const int64_t s0 = tile * kTok;
    const int nv = static_cast<int>(min<int64_t>(kTok, n - s0));
    uint4 xf[kHalves][NKS];
    uint4 xl[kHalves][F32 ? NKS : 1];  // fp32 rows: the low fp16 parts
    float nrm[kHalves];
    if constexpr (F32) {
      const float* row[kHalves];
#pragma unroll
      for (int tt = 0; tt < kHalves; ++tt)
        row[tt] = static_cast<const float*>(xin) + (s0 + min(32 * tt + li, nv - 1)) * D;
      load_x_f32<NKS>(xf, xl, nrm, row, lane);
    } else {
      const uint16_t* row[kHalves];
#pragma unroll
      for (int tt = 0; tt < kHalves; ++tt)
        row[tt] = static_cast<const uint16_t*>(xin) + (s0 + min(32 * tt + li, nv - 1)) * D;
      load_x<NKS>(xf, row, lane);
#pragma unroll
      for (int tt = 0; tt < kHalves; ++tt) {
        float ss = 0.f;
#pragma unroll
        for (int s = 0; s < NKS; ++s) ss = sumsq<F16>(xf[tt][s], ss);
        ss += __shfl_xor(ss, 32, 64);
        nrm[tt] = fmaxf(sqrtf(ss), 1e-8f);
      }
    }
    float* invw = reinterpret_cast<float*>(&inv_s[wv][0]);
#pragma unroll
    for (int tt = 0; tt < kHalves; ++tt) {
      if (lane < 32) {
        if (32 * tt + li < nv) norms[s0 + 32 * tt + li] = nrm[tt];
        if (!F32) invw[32 * tt + li] = iscale / nrm[tt];
      }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes landed
    __builtin_amdgcn_wave_barrier();

    static_for<NBK>([&](auto nc) {  // coordinates 32 b .. 32 b + 31
      constexpr int b = decltype(nc)::value;
      __builtin_amdgcn_sched_barrier(0);
      qkv_f32x16 acc[kHalves] = {};
#pragma unroll
      for (int s = 0; s < NKS; ++s)
#pragma unroll
        for (int sp2 = 0; sp2 < 2; ++sp2) {
          const uint4 bf = frag[((b * NKS + s) * 2 + sp2) * 64 + lane];
#pragma unroll
          for (int tt = 0; tt < kHalves; ++tt) {
            acc[tt] = mma<F16>(xf[tt][s], bf, acc[tt]);
            if (F32 && sp2 == 0) acc[tt] = mma<F16>(xl[tt][F32 ? s : 0], bf, acc[tt]);
          }
        }
#pragma unroll
      for (int tt = 0; tt < kHalves; ++tt) {
        float4 iv4[4];
        if constexpr (!F32) {
#pragma unroll
          for (int a = 0; a < 4; ++a) iv4[a] = inv_s[wv][8 * tt + 2 * a + (lane >> 5)];
        }
        // this lane's first token 32 tt + 4 (l >> 5) at coordinate 32 b + (l & 31); the
        // others sit at fixed offsets from it
        const int64_t o0 = (s0 + 32 * tt + 4 * (lane >> 5)) * D + 32 * b + li;
        uint8_t* cb = codes + o0;
        uint8_t* qb = IP ? qjl + o0 : nullptr;
        const int tk0 = 32 * tt + 4 * (lane >> 5);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          float iv = 1.f / 65536.f;  // fp32 rows: scaled before the rotation
          if constexpr (!F32) {
            const float4 q4 = iv4[v >> 2];
            iv = (v & 3) == 0 ? q4.x : (v & 3) == 1 ? q4.y : (v & 3) == 2 ? q4.z : q4.w;
          }
          // token tk0 + 8 (v >> 2) + (v & 3)
          const int dt = 8 * (v >> 2) + (v & 3);
          const uint32_t f = search_sym_count<L, IP>(acc[tt][v] * iv, lv, cx[b]);
          if (tk0 + dt < nv) {
            if constexpr (IP) {
              cb[dt * D] = static_cast<uint8_t>(f >> 1);
              qb[dt * D] = static_cast<uint8_t>((f & 1u) ^ neg[b]);
            } else {
              cb[dt * D] = static_cast<uint8_t>(f);
            }
          }
        }
      }
    });
  }
}

// ---------------------------------------------------------------- values

// One wave per kTok store tokens [A0, A0 + kTok) of one group, A0 32-aligned,
// so the wave owns one whole V tile; tokens outside [t0, t0 + S) keep the bits
// already in the store.  FROM_Y: `xin` holds fp32 rotated unit rows and `nin`
// their norms, and the search is search_sym's exact one on y.
//
// Orientation: C = tokens x coordinates (A = x with the tile's token rows in
// half-major order, B = Pi), so lane l holds coordinate 32 mb + (l & 31) and,
// in register v, token 16 (l >> 5) + v of the tile.  Each compare mask is
// shifted into the lanes' own 16-token plane accumulators (shift_in), the two
// lane halves are merged into the tile's 32-token words (merge_halves), and
// each lane stores its coordinate's word of two planes.  The tokens' 1 / |x|
// reach the lanes through inv_s.
template <int VB, int XT, int D, bool PAGED, bool FROM_Y, bool ONE = false>
__device__ __forceinline__ void append_v_run(
    const void* __restrict__ xin, const float* __restrict__ nin, int64_t S, int64_t tpg,
    int64_t ntiles, const float* __restrict__ pi, Half bnd, uint32_t* __restrict__ vst,
    float* __restrict__ vnorm, int64_t t_stride, int64_t t0, QkvPages pg,
    uint4* __restrict__ frag, float4 (*inv_s)[kTok / 4], int bid, int nb, int nsplit = 1) {
  static_assert(kHalves == 1, "one 32-token MFMA row block (one V tile) per wave tile");
  constexpr bool F16 = XT != 0, F32 = XT == 2;  // fp16 MFMA / fp32 rows split for it
  constexpr int NP = (1 << (VB - 1)) - 1;  // positive half of the boundaries
  constexpr int NBK = D / 32;        // coordinate blocks
  constexpr int NKS = D / 16;        // k-steps
  constexpr int KH = (VB + 1) / 2;   // planes per lane half in a merge
  const int lane = threadIdx.x & 63, li = lane & 31, hh = lane >> 5;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // tile math on the SALU
  const int64_t a_base = t0 & ~int64_t(31);
  // ONE (as in append_k_run): the wave's rows loaded before the Pi staging
  // ONE, nsplit: the workgroups' tiles and coordinate blocks as in append_k_run
  const bool split = ONE && nsplit > 1;
  int myblk = 0;
  const int64_t gw = split ? one_first(bid, nb, NBK, wv, myblk)  // the wave's first tile
                           : int64_t(bid) * kWaves + wv;
  const int wt = half_major(li);  // tile token of this lane's A-operand row
  constexpr bool PRE = ONE && !FROM_Y && !F32;
  uint4 xpre[1][PRE ? NKS : 1];
  if constexpr (PRE) {
    const int64_t tile = gw;
    if (tile < ntiles) {
      const int64_t grp = tile_group(tile, tpg);
      const int64_t d0 = a_base + (tile - grp * tpg) * kTok - t0;
      const uint16_t* row[1] = {static_cast<const uint16_t*>(xin) +
                                (grp * S + min<int64_t>(max<int64_t>(d0 + wt, 0), S - 1)) * D};
      load_x<NKS>(xpre, row, lane);
    }
  }
  if constexpr (!FROM_Y) {
    stage_pi<F16, D>(frag, pi, F16 ? kPScaleF16 : 1.f, split ? myblk : -1);
    __syncthreads();
  }

  // the positive half of the boundaries: integer keys (FROM_Y), floats (on y;
  // fp32 rows compare the MFMA result 2^16 y against them times 2^16)
  uint32_t bv[NP > 0 ? NP : 1];
  float bp[NP > 0 ? NP : 1];
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    bv[i] = in_vgpr(bnd.t[i]);
    bp[i] = __uint_as_float(in_vgpr(bnd.t[i] >> 1)) * (F32 ? 65536.f : 1.f);
  }
  const float iscale = F16 ? 1.f / kPScaleF16 : 1.f;
  const int64_t wstep = int64_t(nb) * kWaves;

  for (int64_t tile = gw; tile < ntiles; tile += wstep) {
    const int64_t grp = tile_group(tile, tpg);
    const int64_t A0 = a_base + (tile - grp * tpg) * kTok;  // store token of tile token 0
    const int64_t d0 = A0 - t0;                              // its input index (may be < 0)
    QkvSpan sp{};
    if constexpr (PAGED) sp = qkv_span(pg, grp, t_stride, A0);
    uint4 xf[1][NKS];  // tokens outside [t0, t0 + S) read a valid row; bits not stored
    uint4 xl[1][F32 ? NKS : 1];  // fp32 rows: the low fp16 parts
    if constexpr (FROM_Y) {
      const int64_t si = d0 + li;
      if (lane < 32 && si >= 0 && si < S) {
        const int64_t t = A0 + li;
        const int64_t r = PAGED ? sp.row(t) : grp * t_stride + t;
        if (r >= 0) vnorm[r] = nin[grp * S + si];
      }
    } else {
      const int64_t si = d0 + wt;
      const int64_t src = grp * S + min<int64_t>(max<int64_t>(si, 0), S - 1);
      float nrm[1];
      if constexpr (F32) {
        const float* row[1] = {static_cast<const float*>(xin) + src * D};
        load_x_f32<NKS>(xf, xl, nrm, row, lane);
      } else {
        if constexpr (PRE) {
#pragma unroll
          for (int s = 0; s < NKS; ++s) xf[0][s] = xpre[0][s];
        } else {
          const uint16_t* row[1] = {static_cast<const uint16_t*>(xin) + src * D};
          load_x<NKS>(xf, row, lane);
        }
        float ss = 0.f;
#pragma unroll
        for (int s = 0; s < NKS; ++s) ss = sumsq<F16>(xf[0][s], ss);
        ss += __shfl_xor(ss, 32, 64);
        nrm[0] = fmaxf(sqrtf(ss), 1e-8f);
      }
      if (lane < 32 && si >= 0 && si < S) {
        const int64_t t = A0 + wt;
        const int64_t r = PAGED ? sp.row(t) : grp * t_stride + t;
        if (r >= 0 && myblk == 0) vnorm[r] = nrm[0];
      }
      if constexpr (!F32) {
        // 1 / |x| of tile token wt, read back by the lanes holding it
        if (lane < 32) reinterpret_cast<float*>(&inv_s[wv][0])[wt] = iscale / nrm[0];
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes landed
        __builtin_amdgcn_wave_barrier();
      }
    }
    // the appended tokens [lo, hi) of the tile; a page outside the pool takes
    // nothing
    const int64_t lo = max<int64_t>(t0 - A0, 0), hi = min<int64_t>(t0 + S - A0, 32);
    const uint32_t vm = hi - lo >= 32 ? 0xffffffffu
                        : hi > lo    ? ((1u << static_cast<int>(hi - lo)) - 1u) << lo
                                     : 0u;
    const int64_t vrow = PAGED ? sp.row(A0) : 0;
    const bool wr = vm != 0u && vrow >= 0;
    const int64_t vt = PAGED ? (vrow >> 5) : grp * (t_stride >> 5) + (A0 >> 5);
    uint32_t* vtile = vst + vt * (VB * D);

    static_for<NBK>([&](auto mc) {  // coordinates 32 mb .. 32 mb + 31
      constexpr int mb = decltype(mc)::value;
      if (split && mb != myblk) return;
      __builtin_amdgcn_sched_barrier(0);  // one coordinate block at a time (registers)
      float yv[16];  // token 16 h + v of the tile at coordinate 32 mb + (l & 31)
      if constexpr (FROM_Y) {
        const auto* y = static_cast<const float*>(xin);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int64_t si = min<int64_t>(max<int64_t>(d0 + 16 * hh + v, 0), S - 1);
          yv[v] = y[(grp * S + si) * D + 32 * mb + li];
        }
      } else {
        qkv_f32x16 acc = {};
#pragma unroll
        for (int s = 0; s < NKS; ++s)
#pragma unroll
          for (int sp2 = 0; sp2 < 2; ++sp2) {
            const uint4 bf = frag[((mb * NKS + s) * 2 + sp2) * 64 + lane];
            acc = mma<F16>(xf[0][s], bf, acc);
            if (F32 && sp2 == 0) acc = mma<F16>(xl[0][F32 ? s : 0], bf, acc);
          }
        if constexpr (F32) {
#pragma unroll
          for (int v = 0; v < 16; ++v) yv[v] = acc[v];
        } else {
          float4 iv4[4];
#pragma unroll
          for (int a = 0; a < 4; ++a) iv4[a] = inv_s[wv][4 * hh + a];
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const float4 q4 = iv4[v >> 2];
            const float iv = (v & 3) == 0 ? q4.x : (v & 3) == 1 ? q4.y : (v & 3) == 2 ? q4.z : q4.w;
            yv[v] = acc[v] * iv;
          }
        }
      }
      uint32_t va[VB];  // plane k: this lane half's 16 tokens (bit v = register v)
#pragma unroll
      for (int k = 0; k < VB; ++k) va[k] = 0u;
      static_for<16>([&](auto vc) {
        constexpr int v = 15 - decltype(vc)::value;
        uint64_t m[VB];
        if constexpr (FROM_Y)
          search_sym<VB, false>(yv[v], bv, 0u, m);
        else
          search_sym_scaled<VB>(yv[v], bp, m);
#pragma unroll
        for (int k = 0; k < VB; ++k) va[k] = shift_in(va[k], m[k]);
      });
      // lanes 0..31 store plane i, lanes 32..63 plane i + KH
#pragma unroll
      for (int i = 0; i < KH; ++i) {
        const int kb = i + KH < VB ? i + KH : i;
        const uint32_t w = merge_halves(va[i], va[kb]);
        if (wr && (hh == 0 || i + KH < VB)) {
          uint32_t* p = vtile + (hh ? kb : i) * D + 32 * mb + li;
          *p = vm == 0xffffffffu ? w : (*p & ~vm) | (w & vm);
        }
      }
    });
    if constexpr (ONE) break;
  }
}

template <int VB, int XT, int D, bool PAGED, bool FROM_Y>
__global__ __launch_bounds__(kThreads, PAGED ? 2 : 4) void append_v_mfma(
    const void* __restrict__ xin, const float* __restrict__ nin, int64_t S, int64_t tpg,
    int64_t ntiles, const float* __restrict__ pi, Half bnd, uint32_t* __restrict__ vst,
    float* __restrict__ vnorm, int64_t t_stride, int64_t t0, QkvPages pg) {
  __shared__ uint4 frag[FROM_Y ? 1 : frag_n<D>()];  // Pi operand fragments
  __shared__ float4 inv_s[kWaves][kTok / 4];         // 1 / norm of each wave's tokens
  append_v_run<VB, XT, D, PAGED, FROM_Y>(xin, nin, S, tpg, ntiles, pi, bnd, vst, vnorm, t_stride,
                                         t0, pg, frag, inv_s, blockIdx.x, gridDim.x);
}

// append_v_mfma over the contiguous stores of blockIdx.y's layer
template <int VB, int XT, int D>
__global__ __launch_bounds__(kThreads, 4) void append_v_layers(AppendLayers al, int64_t S,
                                                               int64_t tpg, int64_t ntiles,
                                                               Half bnd, int64_t t_stride,
                                                               int64_t t0) {
  __shared__ uint4 frag[frag_n<D>()];
  __shared__ float4 inv_s[kWaves][kTok / 4];
  const int l = blockIdx.y;
  append_v_run<VB, XT, D, false, false>(al.x[l], nullptr, S, tpg, ntiles, al.pi[l], bnd,
                                        static_cast<uint32_t*>(al.st[l]), al.nrm[l], t_stride,
                                        t0, QkvPages{}, frag, inv_s, blockIdx.x, gridDim.x);
}

}  // namespace
