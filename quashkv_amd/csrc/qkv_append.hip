// Fused compress straight into the cache store, for bf16 / fp16 K and V rows
// with d = 128: normalise -> rotate (MFMA) -> Lloyd-Max boundary search ->
// QJL sign -> bit planes, one pass over the inputs.
//
// Reference: QuashKVEngine.append (quashkv/engine.py:145-172) compresses keys
// with InnerProductQuantizer.compress (quashkv/quantizer.py:211-242) and values
// with MSEQuantizer.compress (quashkv/quantizer.py:113-131); the GPU operator
// surface is fused_compress_ip / fused_compress_mse
// (quashkv/triton_kernels/compress.py:210-303).  The codes land in the K-row and
// V-tile store formats that the decode kernel reads.
//
// Rotation.  z = x Pi^T runs on the 16x16x32 bf16 (fp16) MFMA with x as it is
// stored (a bf16 / fp16 value is exact in the operand type) and Pi split into
// a high and a low 16-bit part, Pi ~= Pi_hi + Pi_lo, accumulated in fp32: two
// MFMA passes carry ~16 (bf16) / ~22 (fp16) significant bits of Pi, against
// 24 for the reference's fp32 GEMM.  Codes computed from x may therefore
// differ from the reference's where y lies within ~1e-5 relative of a
// boundary (about 1e-6 of the coordinates); codes from an identical y go
// through qkv_compress(QKV_FLAG_PRE_ROTATED), which is exact.
//
// Boundary search without per-element codes.  For the value y of one
// coordinate, code = #{i : t_i < y} (torch.bucketize, right=False).  Bit k of
// that count is the XOR of the comparisons [y > t_i] over i = 2^k - 1,
// 2^k - 1 + 2^k, ..., so a wave compares its 64 values with every boundary
// (one v_cmp each, giving a 64-bit lane mask) and forms the bit planes with
// scalar XORs of the masks.  Keys interleave centroids and boundaries,
// c_0 < t_0 < c_1 < ... < c_{2^m-1}: the QJL bit [(y - c[code]) S_j >= 0] is
// the parity of #{f : f < y S_j} over that fine list (y S_j lies in
// (c_code', t_code'] exactly when the count is odd), using the codebook's
// symmetry (c_i = -c_{2^m-1-i}, t_i = -t_{2^m-2-i}) to fold the sign S_j into
// y: with y' = y S_j, code(y) = code'(y') for S_j = +1 and its complement for
// S_j = -1.  Pi is staged with its rows scaled by S, so the MFMA yields y S
// directly.  Exact ties (y equal to a boundary or centroid) are a measure-zero
// event on this path and resolve as [y' > f].
//
// Orientation.  Keys: C = tokens x coordinates, so a mask's 16-lane groups are
// 16 coordinates of one token -- two bytes of one K-row plane.  Values:
// C = coordinates x tokens, so a mask's 16-lane groups are 16 tokens of one
// coordinate -- half a V-tile word.  The MFMA operand layouts of the 16x16x32
// instructions are symmetric, so the same x and Pi register fragments serve
// both orders.  Plane words are assembled in SGPRs and placed into staging
// VGPRs with v_writelane, then stored with coalesced vector stores.

#include <cmath>
#include <type_traits>
#include <utility>

#include "qkv_common.h"

namespace {

typedef __bf16 qkv_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 qkv_f16x8 __attribute__((ext_vector_type(8)));
typedef float qkv_f32x4 __attribute__((ext_vector_type(4)));

constexpr int kD = 128;                 // head dim of this path
constexpr int kTok = 64;                // tokens per wave tile
constexpr int kWaves = 4;               // waves per workgroup
constexpr int kFragN = 8 * 4 * 2 * 64;  // Pi fragments [block][k-step][split][lane] (64 KiB)
constexpr float kPScaleF16 = 256.f;     // keeps the fp16 low part of Pi out of subnormals

struct Thresh {
  float v[15];  // ascending comparison list
};

template <bool F16>
__device__ __forceinline__ qkv_f32x4 mma(uint4 a, uint4 b, qkv_f32x4 c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(qkv_f16x8, a),
                                                  __builtin_bit_cast(qkv_f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(qkv_bf16x8, a),
                                                   __builtin_bit_cast(qkv_bf16x8, b), c, 0, 0, 0);
}

// Value `val` (wave-uniform) into lane L of `old`.
template <int L>
__device__ __forceinline__ uint32_t put_lane(uint32_t old, uint32_t val) {
  static_assert(L >= 0 && L < 64, "lane");
  uint32_t r;
  asm("v_writelane_b32 %0, %1, %2" : "=v"(r) : "s"(val), "i"(L), "0"(old));
  return r;
}

__device__ __forceinline__ uint64_t lanes_where(bool p) { return __builtin_amdgcn_ballot_w64(p); }

// 16-bit chunk G (lanes 16 G .. 16 G + 15) of mask a, with that of mask b in
// the high half: one scalar pack (s_pack_{ll,hh}_b32_b16) on wave-uniform masks.
template <int G>
__device__ __forceinline__ uint32_t chunk_pair(uint64_t a, uint64_t b) {
  const uint32_t x = static_cast<uint32_t>(a >> (32 * (G >> 1)));
  const uint32_t y = static_cast<uint32_t>(b >> (32 * (G >> 1)));
  uint32_t r;
  if constexpr ((G & 1) == 0)
    asm("s_pack_ll_b32_b16 %0, %1, %2" : "=s"(r) : "s"(x), "s"(y));
  else
    asm("s_pack_hh_b32_b16 %0, %1, %2" : "=s"(r) : "s"(x), "s"(y));
  return r;
}

// f(std::integral_constant<int, 0>), ..., f(<N - 1>): compile-time unrolled
// loops whose index feeds template arguments (v_writelane lane numbers).
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

template <bool F16>
__device__ __forceinline__ float half_lo(uint32_t w) {
  if constexpr (F16)
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w & 0xffffu)));
  else
    return __uint_as_float(w << 16);
}

template <bool F16>
__device__ __forceinline__ float half_hi(uint32_t w) {
  if constexpr (F16)
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
  else
    return __uint_as_float(w & 0xffff0000u);
}

template <bool F16>
__device__ __forceinline__ float sumsq(uint4 q, float s) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a = half_lo<F16>(w[i]), b = half_hi<F16>(w[i]);
    s = fmaf(a, a, s);
    s = fmaf(b, b, s);
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

template <bool F16>
__device__ __forceinline__ float from16(uint16_t h) {
  if constexpr (F16)
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
  else
    return qkv_bf16_to_f32(h);
}

// Stage the rotation operand in LDS.  Entry ((b * 4 + s) * 2 + split) * 64 + l
// holds, for lane l, Pi'[16 b + (l & 15)][32 s + 8 (l >> 4) + e], e = 0..7, as
// eight 16-bit values: the high part (split 0) or the low part (split 1) of
// Pi' = diag(rowsign) Pi * pscale (rowsign = S for keys, none for values).
template <bool F16>
__device__ void stage_pi(uint4* __restrict__ frag, const float* __restrict__ pi,
                         const float* __restrict__ rowsign, float pscale) {
  for (int e = threadIdx.x; e < kFragN; e += blockDim.x) {
    const int ln = e & 63, split = (e >> 6) & 1, s = (e >> 7) & 3, b = e >> 9;
    const int j = 16 * b + (ln & 15), k0 = 32 * s + 8 * (ln >> 4);
    const float4 p0 = *reinterpret_cast<const float4*>(pi + j * kD + k0);
    const float4 p1 = *reinterpret_cast<const float4*>(pi + j * kD + k0 + 4);
    const float sc = (rowsign ? rowsign[j] : 1.f) * pscale;  // +-2^k: exact
    const float p[8] = {p0.x * sc, p0.y * sc, p0.z * sc, p0.w * sc,
                        p1.x * sc, p1.y * sc, p1.z * sc, p1.w * sc};
    uint32_t h[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint16_t hi = to16<F16>(p[i]);
      h[i] = split == 0 ? hi : to16<F16>(p[i] - from16<F16>(hi));
    }
    frag[e] = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                         h[6] | (h[7] << 16));
  }
}

// Bit k of the thermometer count of masks m[0..n): XOR of m[i], i = 2^k - 1 (step 2^k).
template <int K, int N>
__device__ __forceinline__ uint64_t count_bit(const uint64_t* m) {
  uint64_t a = 0;
#pragma unroll
  for (int i = (1 << K) - 1; i < N; i += (1 << K)) a ^= m[i];
  return a;
}

// ------------------------------------------------------------------ keys

// One wave per tile of 64 consecutive tokens of one (b, h) group.  Input rows
// grp * S + s; store rows grp * t_stride + t0 + s ((MB + 1) * 16 bytes:
// MB MSE planes, then the QJL plane).
template <int MB, bool F16>
__global__ __launch_bounds__(256, 2) void append_k_mfma(
    const uint16_t* __restrict__ x, int64_t S, int64_t tpg, int64_t ntiles,
    const float* __restrict__ pi, const float* __restrict__ signs, Thresh fine,
    uint8_t* __restrict__ kst, float* __restrict__ knorm, int64_t t_stride, int64_t t0) {
  constexpr int NF = (2 << MB) - 1;  // c_0, t_0, c_1, ..., c_{2^MB - 1}
  constexpr int NT = (1 << MB) - 1;  // boundaries
  constexpr int NP = MB + 1;         // planes per row
  constexpr int RD = 4 * NP;         // dwords per row = staging dwords per lane
  __shared__ uint4 frag[kFragN];
  stage_pi<F16>(frag, pi, signs, F16 ? kPScaleF16 : 1.f);
  __syncthreads();

  const int lane = threadIdx.x & 63, g = lane >> 4, li = lane & 15;
  uint32_t sneg = 0;  // bit b: S < 0 at this lane's coordinate of block b
#pragma unroll
  for (int b = 0; b < 8; ++b) sneg |= (signs[16 * b + li] < 0.f ? 1u : 0u) << b;
  const float iscale = F16 ? 1.f / kPScaleF16 : 1.f;

  for (int64_t tile = int64_t(blockIdx.x) * kWaves + (threadIdx.x >> 6); tile < ntiles;
       tile += int64_t(gridDim.x) * kWaves) {
    const int64_t grp = tile / tpg;
    const int64_t s0 = (tile - grp * tpg) * kTok;
    const int nv = static_cast<int>(min<int64_t>(kTok, S - s0));
    const uint16_t* xt = x + (grp * S + s0) * kD;

    // A operand: lane (li, g) holds x[16 mt + li][32 s + 8 g .. + 7]
    uint4 xf[4][4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int s = 0; s < 4; ++s)
        xf[mt][s] = (16 * mt + li < nv)
                        ? *reinterpret_cast<const uint4*>(xt + (16 * mt + li) * kD + 32 * s + 8 * g)
                        : make_uint4(0u, 0u, 0u, 0u);

    // norms; inv[mt][v] = 1 / n of token 16 mt + 4 g + v (the C-row of VGPR v)
    float inv[4][4];
    float* nrow = knorm + grp * t_stride + t0 + s0;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      float ss = 0.f;
#pragma unroll
      for (int s = 0; s < 4; ++s) ss = sumsq<F16>(xf[mt][s], ss);
      ss += __shfl_xor(ss, 16, 64);
      ss += __shfl_xor(ss, 32, 64);
      const float nrm = fmaxf(sqrtf(ss), 1e-8f);
      if (g == 0 && 16 * mt + li < nv) nrow[16 * mt + li] = nrm;
      const float iv = iscale / nrm;
#pragma unroll
      for (int v = 0; v < 4; ++v) inv[mt][v] = __shfl(iv, 4 * g + v, 64);
    }

    uint32_t stg[RD];
#pragma unroll
    for (int i = 0; i < RD; ++i) stg[i] = 0u;

    static_for<4>([&](auto wc) {  // coordinates 32 w .. 32 w + 31 (blocks 2w, 2w+1)
      constexpr int w = decltype(wc)::value;
      qkv_f32x4 acc[2][4];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) acc[h][mt] = qkv_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int sp = 0; sp < 2; ++sp) {
            const uint4 bf = frag[(((2 * w + h) * 4 + s) * 2 + sp) * 64 + lane];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) acc[h][mt] = mma<F16>(xf[mt][s], bf, acc[h][mt]);
          }
      const uint64_t sn[2] = {lanes_where((sneg >> (2 * w)) & 1u),
                              lanes_where((sneg >> (2 * w + 1)) & 1u)};
      static_for<4>([&](auto mtc) {
        constexpr int mt = decltype(mtc)::value;
        static_for<4>([&](auto vc) {
          constexpr int v = decltype(vc)::value;
          uint64_t pl[2][NP];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const float ys = acc[h][mt][v] * inv[mt][v];  // y_j S_j
            uint64_t f[NF];
#pragma unroll
            for (int i = 0; i < NF; ++i) f[i] = lanes_where(ys > fine.v[i]);
            uint64_t m[NT];
#pragma unroll
            for (int i = 0; i < NT; ++i) m[i] = f[2 * i + 1];
            uint64_t q = 0;
#pragma unroll
            for (int i = 0; i < NF; ++i) q ^= f[i];
            static_for<MB>([&](auto kc) {
              pl[h][decltype(kc)::value] = count_bit<decltype(kc)::value, NT>(m) ^ sn[h];
            });
            pl[h][MB] = q;
          }
          // token 16 mt + 4 g2 + v: bits [16 g2, 16 g2 + 16) of each mask; the
          // two 16-coordinate blocks of the pair fill one dword of plane r
          static_for<4>([&](auto g2c) {
            constexpr int g2 = decltype(g2c)::value;
            static_for<NP>([&](auto rc) {
              constexpr int r = decltype(rc)::value;
              constexpr int D = (16 * mt + 4 * g2 + v) * RD + 4 * r + w;
              const uint32_t dw = chunk_pair<g2>(pl[0][r], pl[1][r]);
              stg[D >> 6] = put_lane<(D & 63)>(stg[D >> 6], dw);
            });
          });
        });
      });
    });

    uint32_t* dst = reinterpret_cast<uint32_t*>(kst + (grp * t_stride + t0 + s0) * (RD * 4));
#pragma unroll
    for (int i = 0; i < RD; ++i) {
      const int D = i * 64 + lane;
      if (D < nv * RD) dst[D] = stg[i];
    }
  }
}

// ---------------------------------------------------------------- values

// One wave per 64 store tokens [A0, A0 + 64) of one group, A0 = 32-aligned, so
// the wave owns two whole V tiles; tokens outside [t0, t0 + S) keep the bits
// already in the store.
template <int VB, bool F16>
__global__ __launch_bounds__(256, 2) void append_v_mfma(
    const uint16_t* __restrict__ x, int64_t S, int64_t tpg, int64_t ntiles,
    const float* __restrict__ pi, Thresh bnd, uint32_t* __restrict__ vst,
    float* __restrict__ vnorm, int64_t t_stride, int64_t t0) {
  constexpr int NB = (1 << VB) - 1;  // boundaries
  constexpr int NS = 4 * VB;         // staging dwords per lane: 2 tiles x VB planes x 128 / 64
  __shared__ uint4 frag[kFragN];
  stage_pi<F16>(frag, pi, nullptr, F16 ? kPScaleF16 : 1.f);
  __syncthreads();

  const int lane = threadIdx.x & 63, g = lane >> 4, li = lane & 15;
  const float iscale = F16 ? 1.f / kPScaleF16 : 1.f;
  const int64_t a_base = t0 & ~int64_t(31);
  const int64_t tiles_per_group = t_stride / 32;

  for (int64_t tile = int64_t(blockIdx.x) * kWaves + (threadIdx.x >> 6); tile < ntiles;
       tile += int64_t(gridDim.x) * kWaves) {
    const int64_t grp = tile / tpg;
    const int64_t A0 = a_base + (tile - grp * tpg) * kTok;  // store token of lane-token 0
    const int64_t d0 = A0 - t0;                              // its input index (may be < 0)
    const uint16_t* xg = x + grp * S * kD;

    // B operand: lane (li, g) holds x[token 16 n + li][32 s + 8 g .. + 7]
    uint4 xf[4][4];
    bool ok[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const int64_t si = d0 + 16 * n + li;
      ok[n] = si >= 0 && si < S;
#pragma unroll
      for (int s = 0; s < 4; ++s)
        xf[n][s] = ok[n] ? *reinterpret_cast<const uint4*>(xg + si * kD + 32 * s + 8 * g)
                         : make_uint4(0u, 0u, 0u, 0u);
    }
    float inv[4];  // token 16 n + li: the C-column of this lane
    float* nrow = vnorm + grp * t_stride + A0;
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      float ss = 0.f;
#pragma unroll
      for (int s = 0; s < 4; ++s) ss = sumsq<F16>(xf[n][s], ss);
      ss += __shfl_xor(ss, 16, 64);
      ss += __shfl_xor(ss, 32, 64);
      const float nrm = fmaxf(sqrtf(ss), 1e-8f);
      if (g == 0 && ok[n]) nrow[16 * n + li] = nrm;
      inv[n] = iscale / nrm;
    }

    uint32_t stg[NS];
#pragma unroll
    for (int i = 0; i < NS; ++i) stg[i] = 0u;

    static_for<8>([&](auto mbc) {  // coordinates 16 mb .. 16 mb + 15
      constexpr int mb = decltype(mbc)::value;
      qkv_f32x4 acc[4];
#pragma unroll
      for (int n = 0; n < 4; ++n) acc[n] = qkv_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int sp = 0; sp < 2; ++sp) {
          const uint4 af = frag[((mb * 4 + s) * 2 + sp) * 64 + lane];
#pragma unroll
          for (int n = 0; n < 4; ++n) acc[n] = mma<F16>(af, xf[n][s], acc[n]);
        }
      static_for<4>([&](auto vc) {
        constexpr int v = decltype(vc)::value;
        uint64_t pl[4][VB];
#pragma unroll
        for (int n = 0; n < 4; ++n) {
          const float ys = acc[n][v] * inv[n];
          uint64_t m[NB];
#pragma unroll
          for (int i = 0; i < NB; ++i) m[i] = lanes_where(ys > bnd.v[i]);
          static_for<VB>([&](auto kc) {
            pl[n][decltype(kc)::value] = count_bit<decltype(kc)::value, NB>(m);
          });
        }
        // coordinate 16 mb + 4 g2 + v of tile tau: tokens 32 tau + 0..15 | 16..31
        static_for<2>([&](auto tc) {
          constexpr int tau = decltype(tc)::value;
          static_for<4>([&](auto g2c) {
            constexpr int g2 = decltype(g2c)::value;
            static_for<VB>([&](auto kc) {
              constexpr int k = decltype(kc)::value;
              constexpr int D = (tau * VB + k) * 128 + 16 * mb + 4 * g2 + v;
              const uint32_t dw = chunk_pair<g2>(pl[2 * tau][k], pl[2 * tau + 1][k]);
              stg[D >> 6] = put_lane<(D & 63)>(stg[D >> 6], dw);
            });
          });
        });
      });
    });

    // store: staging dword i covers tile i / (2 VB), plane (i / 2) % VB,
    // coordinates 64 (i % 2) + lane
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int tau = i / (2 * VB), k = (i / 2) % VB, j = 64 * (i % 2) + lane;
      const int64_t tok0 = A0 + 32 * tau;
      const int64_t lo = max<int64_t>(t0 - tok0, 0), hi = min<int64_t>(t0 + S - tok0, 32);
      if (hi <= lo) continue;
      const uint32_t vm = (hi - lo == 32) ? 0xffffffffu
                                          : (((1u << (hi - lo)) - 1u) << lo);
      uint32_t* p = vst + ((grp * tiles_per_group + tok0 / 32) * VB + k) * kD + j;
      uint32_t val = stg[i];
      if (vm != 0xffffffffu) val = (*p & ~vm) | (val & vm);
      *p = val;
    }
  }
}

// -------------------------------------------------------------- host side

bool symmetric(const float* v, int n) {
  for (int i = 0; i < n; ++i)
    if (v[i] != -v[n - 1 - i]) return false;
  return true;
}

int append_blocks(int64_t ntiles) {
  const int64_t cap = int64_t(qkv_num_cus()) * 2;  // two 64-KiB-LDS workgroups per CU
  return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>((ntiles + kWaves - 1) / kWaves, cap)));
}

}  // namespace

extern "C" int qkv_store_append(int32_t in_dtype, const void* keys, const void* values,
                                int64_t groups, int64_t S, int32_t d, int32_t mbits,
                                int32_t vbits, const float* pi, const float* signs,
                                const float* kcent_host, const float* kbound_host,
                                const float* vbound_host, uint8_t* kstore, float* knorm,
                                uint32_t* vstore, float* vnorm, int64_t t_stride, int64_t t0,
                                void* stream) {
  QKV_REQUIRE(groups >= 0 && S >= 0 && t0 >= 0, "negative size");
  QKV_REQUIRE(t_stride % 32 == 0 && t0 + S <= t_stride,
              "store capacity %lld (multiple of 32) must hold tokens [%lld, %lld)",
              (long long)t_stride, (long long)t0, (long long)(t0 + S));
  if (in_dtype != QKV_BF16 && in_dtype != QKV_F16) {
    qkv_set_error("store append runs on bf16 / fp16 inputs (got dtype %d)", in_dtype);
    return QKV_E_UNSUPPORTED;
  }
  if (d != kD) {
    qkv_set_error("store append runs on head_dim 128 (got %d)", d);
    return QKV_E_UNSUPPORTED;
  }
  if (keys) {
    if (mbits < 1 || mbits > 3) {
      qkv_set_error("store append: key MSE bits %d not in 1..3", mbits);
      return QKV_E_UNSUPPORTED;
    }
    QKV_REQUIRE(pi && signs && kcent_host && kbound_host && kstore && knorm, "null pointer");
    QKV_REQUIRE(qkv_aligned(keys, 16) && qkv_aligned(kstore, 4), "keys 16-B / store 4-B aligned");
  }
  if (values) {
    QKV_REQUIRE(qkv_bits_ok(vbits), "value bits %d not in 1..4", vbits);
    QKV_REQUIRE(pi && vbound_host && vstore && vnorm, "null pointer");
    QKV_REQUIRE(qkv_aligned(values, 16) && qkv_aligned(vstore, 4),
                "values 16-B / store 4-B aligned");
  }
  QKV_REQUIRE(!pi || qkv_aligned(pi, 16), "pi must be 16-byte aligned");
  Thresh fine{}, bnd{};
  if (keys) {
    const int nc = 1 << mbits;
    for (int i = 0; i < nc; ++i) {
      fine.v[2 * i] = kcent_host[i];
      if (i + 1 < nc) fine.v[2 * i + 1] = kbound_host[i];
    }
    bool asc = true;
    for (int i = 0; i + 1 < 2 * nc - 1; ++i) asc = asc && fine.v[i] < fine.v[i + 1];
    if (!asc || !symmetric(fine.v, 2 * nc - 1)) {
      qkv_set_error("store append needs a symmetric key codebook with c_i < t_i < c_{i+1}");
      return QKV_E_UNSUPPORTED;
    }
  }
  if (values)
    for (int i = 0; i < (1 << vbits) - 1; ++i) bnd.v[i] = vbound_host[i];
  if (groups == 0 || S == 0) return QKV_OK;
  auto s = static_cast<hipStream_t>(stream);
  const bool f16 = in_dtype == QKV_F16;
  if (keys) {
    const int64_t tpg = (S + kTok - 1) / kTok, ntiles = groups * tpg;
    const dim3 grid(append_blocks(ntiles));
    const auto* xk = static_cast<const uint16_t*>(keys);
#define QKV_K(MB, F)                                                                        \
  hipLaunchKernelGGL((append_k_mfma<MB, F>), grid, dim3(256), 0, s, xk, S, tpg, ntiles, pi, \
                     signs, fine, kstore, knorm, t_stride, t0)
    switch (mbits * 2 + (f16 ? 1 : 0)) {
      case 2: QKV_K(1, false); break;
      case 3: QKV_K(1, true); break;
      case 4: QKV_K(2, false); break;
      case 5: QKV_K(2, true); break;
      case 6: QKV_K(3, false); break;
      case 7: QKV_K(3, true); break;
    }
#undef QKV_K
    QKV_LAUNCHED();
  }
  if (values) {
    const int64_t a_base = t0 & ~int64_t(31);
    const int64_t tpg = (t0 + S - a_base + kTok - 1) / kTok, ntiles = groups * tpg;
    const dim3 grid(append_blocks(ntiles));
    const auto* xv = static_cast<const uint16_t*>(values);
#define QKV_V(VB, F)                                                                        \
  hipLaunchKernelGGL((append_v_mfma<VB, F>), grid, dim3(256), 0, s, xv, S, tpg, ntiles, pi, \
                     bnd, vstore, vnorm, t_stride, t0)
    switch (vbits * 2 + (f16 ? 1 : 0)) {
      case 2: QKV_V(1, false); break;
      case 3: QKV_V(1, true); break;
      case 4: QKV_V(2, false); break;
      case 5: QKV_V(2, true); break;
      case 6: QKV_V(3, false); break;
      case 7: QKV_V(3, true); break;
      case 8: QKV_V(4, false); break;
      case 9: QKV_V(4, true); break;
    }
#undef QKV_V
    QKV_LAUNCHED();
  }
  return QKV_OK;
}
