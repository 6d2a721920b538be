// Device-side definitions of the decode-attention kernels (qkv_attention.hip):
// parameter blocks, the odd Walsh subsets of a symmetric codebook, DPP wave
// reductions and the fp8 x fp4 score-operand helpers.
#pragma once

#include <math.h>

#include "qkv_common.h"

typedef int qkv_v4i __attribute__((ext_vector_type(4)));
typedef int qkv_v8i __attribute__((ext_vector_type(8)));
typedef float qkv_v4f __attribute__((ext_vector_type(4)));

namespace qkv_attn {

struct Tables {
  float kc[16];      // key MSE centroids
  float vc[16];      // value centroids
  float kg[4];       // key Walsh coefficient of (2 b_r - 1), r < mbits
  float kconst;      // g_empty - sum_r kg[r]
  float vg[8];       // value Walsh coefficients, odd subsets (odd_subset order)
  float vconst;      // g_empty - sum vg (the plane form's constant)
  int mfma_ok;       // both codebooks admit the plane decomposition, key MSE bits <= 2
  int fused_ok;      // the same with key MSE bits <= 3 (decode_fused, d = 128)
  // mixed-precision keys over slots (outlier channels first), rows of whole
  // dwords:
  //   kmix 1, MSE keys 3-bit outlier / 2-bit regular (no QJL):
  //     [b0 of every slot][b1 of every slot][b2 of the n_out outlier slots]
  //     [their parity b0^b1^b2]
  //   kmix 2, IP keys with a 2-bit outlier / 1-bit regular MSE stage:
  //     [b0 of every slot][QJL of every slot][b1 of the outlier slots]
  int kmix;
  int n_out;
  float kgo[4];      // outlier Walsh coefficients: b0, b1 (, b2, b0b1b2)
  float kgr[2];      // regular Walsh coefficients: b0 (, b1)
  float kco, kcr;    // -(sum of the coefficients) per kind
};

// Per-layer pointers of a layer-batched decode call (one model step over
// n <= kMaxLayers layers that share shapes and codebooks), passed by value as
// kernel arguments.  The workspace then holds the layers as one batch of
// B * n sequences (layer l, sequence b <-> batch index l B + b).  The
// single-layer entry points use entry 0.
constexpr int kMaxLayers = 32;
struct QLayers {  // query, rotation (row-major d x d), QJL signs
  const void* q[kMaxLayers];
  const float* pi[kMaxLayers];
  const float* signs[kMaxLayers];
};
struct KVLayers {  // the store
  const uint8_t* kst[kMaxLayers];
  const float* knorm[kMaxLayers];
  const uint32_t* vst[kMaxLayers];
  const float* vnorm[kMaxLayers];
  const int32_t* ptab;  // paged store: page of sequence b's token t at
  int32_t pmax;         // ptab[b * pmax + (t >> plg)] (nullptr: contiguous
  int32_t plg;          // streams of t_stride rows); pages of 1 << plg tokens
  int32_t npages;       // pages in the pool: a tile on a page outside [0, npages)
                        // is read from page 0 and masked (contributes nothing)
  // Per-sequence key ranges (nullptr: all T): sequence b attends to the keys
  // [klo[b], khi[b]) of its T cached tokens, the rest masked like padding.
  const int32_t* klo;
  const int32_t* khi;
  int64_t cbase;        // causal: query i sits at cbase - Q + i (0: at khi[b] - Q + i)
};

// The key range and causal position of sequence b (every layer shares them),
// for a workgroup-uniform b: the values are read into scalar registers.
struct SeqRange {
  int64_t lo, hi;  // attended keys [lo, hi)
  int64_t cpos;    // causal: query i at cpos - Q + i sees keys t <= cpos - Q + i
};
__device__ __forceinline__ SeqRange seq_range(const KVLayers& kv, int64_t b, int64_t T) {
  SeqRange r;
  r.lo = kv.klo ? max<int64_t>(0, __builtin_amdgcn_readfirstlane(kv.klo[b])) : 0;
  r.hi = kv.khi ? min<int64_t>(T, __builtin_amdgcn_readfirstlane(kv.khi[b])) : T;
  r.cpos = kv.cbase > 0 ? kv.cbase : r.hi;
  return r;
}
struct OutLayers {  // un-rotation and output
  const float* pi[kMaxLayers];
  void* out[kMaxLayers];
};

// Odd-size subsets of the code bits (bit masks), in a fixed order shared by
// the host (coefficients) and the device (plane words).
__host__ __device__ constexpr uint32_t odd_subset(int bits, int s) {
  return bits == 1 ? 1u
       : bits == 2 ? (s == 0 ? 1u : 2u)
       : bits == 3 ? (s < 3 ? (1u << s) : 7u)
       : (s < 4 ? (1u << s) : (s == 4 ? 7u : s == 5 ? 11u : s == 6 ? 13u : 14u));
}
__host__ __device__ constexpr int n_odd_subsets(int bits) {
  return bits == 1 ? 1 : bits == 2 ? 2 : bits == 3 ? 4 : 8;
}

constexpr int kSplitMax = 2048;  // tokens per split on the MFMA path (LDS scores)
static_assert(kSplitMax / 64 <= 64, "a split's tiles fit one page entry per lane");
constexpr int kRowsM = 4;        // query rows per workgroup on the MFMA path
constexpr int kNUMax = 6;        // score MFMAs per 16 tokens (d = 128, 2 MSE bits)

__device__ __forceinline__ qkv_v4i mfma_i8(qkv_v4i a, qkv_v4i b, qkv_v4i c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ int64_t shfl_xor_i64(int64_t v, int mask) {
  const int lo = __shfl_xor(static_cast<int>(static_cast<uint64_t>(v) & 0xffffffffu), mask, 64);
  const int hi = __shfl_xor(static_cast<int>(static_cast<uint64_t>(v) >> 32), mask, 64);
  return static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) |
                              static_cast<uint32_t>(lo));
}

// lane l's value of a per-lane int64 (wave-uniform result)
__device__ __forceinline__ int64_t readlane_i64(int64_t v, int l) {
  const uint32_t lo = __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint64_t>(v)), l);
  const uint32_t hi = __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint64_t>(v) >> 32), l);
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}
__device__ __forceinline__ int64_t wave_sum_i64(int64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += shfl_xor_i64(v, o);
  return v;
}

// Wait states between an MFMA chain and the first VALU read of its result.
// The compiler's padding for this hazard was found short when a branch sits
// between the last MFMA and the read (3 wait states on the taken path, where
// an 8-pass XDL result needs more), which returned stale accumulators.  The
// scheduling barriers keep the reads after an explicit 20-wait-state pad,
// enough for the longest (16-pass) MFMA.
__device__ __forceinline__ void mfma_settle() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Sum over the wave through DPP lane moves (no LDS round trips): prefix sums
// within each 16-lane row (row_shr 1, 2, 4, 8), then the row totals folded
// into lane 63 (row_bcast 15 into rows 1 and 3, row_bcast 31 into rows 2
// and 3), read back to every lane.
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xf,
                                                        true));
}
// max of v and the DPP-moved v in one v_max_f32_dpp (lanes without a source,
// or outside the row mask, keep v: the destination is v itself).  fmaxf over
// a moved copy costs four instructions here (copy, DPP move, the NaN-quieting
// max of the moved value, max), since the compiler neither folds the move into
// the max nor drops the quieting; the values reduced here are never NaN.
// The s_nop gives the two wait states a DPP read of a VGPR written by the
// previous VALU instruction needs.
#define QKV_DPP_MAX(NAME, CTRL)                                                        \
  __device__ __forceinline__ float NAME(float v) {                                     \
    asm volatile("s_nop 1\n\tv_max_f32_dpp %0, %0, %0 " CTRL : "+v"(v));                \
    return v;                                                                          \
  }
QKV_DPP_MAX(dmax_shr1, "row_shr:1 row_mask:0xf bank_mask:0xf")
QKV_DPP_MAX(dmax_shr2, "row_shr:2 row_mask:0xf bank_mask:0xf")
QKV_DPP_MAX(dmax_shr4, "row_shr:4 row_mask:0xf bank_mask:0xf")
QKV_DPP_MAX(dmax_shr8, "row_shr:8 row_mask:0xf bank_mask:0xf")
QKV_DPP_MAX(dmax_bc15, "row_bcast:15 row_mask:0xa bank_mask:0xf")
QKV_DPP_MAX(dmax_bc31, "row_bcast:31 row_mask:0xc bank_mask:0xf")
QKV_DPP_MAX(dmax_swap1, "quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf")
QKV_DPP_MAX(dmax_swap2, "quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf")
QKV_DPP_MAX(dmax_hmirror, "row_half_mirror row_mask:0xf bank_mask:0xf")
#undef QKV_DPP_MAX
// Max over each 16-lane row, left in the row's last lane (prefix maxima).
__device__ __forceinline__ float row_max_last(float v) {
  return dmax_shr8(dmax_shr4(dmax_shr2(dmax_shr1(v))));
}
// Max over the wave, read back to every lane.
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = dmax_bc31(dmax_bc15(row_max_last(v)));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v = dpp_add<0x111>(v);
  v = dpp_add<0x112>(v);
  v = dpp_add<0x114>(v);
  v = dpp_add<0x118>(v);
  v = dpp_add<0x142, 0xa>(v);
  v = dpp_add<0x143, 0xc>(v);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Max over each aligned group of 8 lanes, in every lane of the group
// (quad_perm swaps of neighbours and pairs, then the half-row mirror).
__device__ __forceinline__ float max8_dpp(float v) {
  return dmax_hmirror(dmax_swap2(dmax_swap1(v)));
}

// ---- fp4 key operands of the fused d = 128 decode
//
// The score MFMA there is v_mfma_scale_f32_16x16x128_f8f6f4 with A = the
// query weights as fp8 (e4m3) digits and B = the K-row bits as fp4 (e2m1)
// values, four bit-to-operand operations per 32 bits against eight for int8
// bytes.  B: lane group g of a 16-token MFMA u takes K-row dword
// w = g DPL + u and spreads its 32 bits over 32 fp4 elements by bit class
// c = bit & 3: element 8 c + (bit >> 2) holds bit * {0.5, 1, 2}[c] for c < 3
// (masks 0x11111111 << c) and 0.5 (1 - 2 bit) for c = 3
// ((x & 0x88888888) | 0x11111111).  A row 4 r + d holds digit d of query row
// r's weights W scaled by the class ({2, 1, 0.5, -1}; class 3 leaves W / 2 in
// the row constant), as fp8 values q_d with
//   W' 2^-sigma ~= q_0 + q_1 / 16 + q_2 / 256 + q_3 / 4096,
// q_d the round-to-nearest fp8 of the remaining residual times 16^d, and the
// MFMA's per-row E8M0 scale 2^(sigma - 4 d); |W'| 2^-sigma <= 224 keeps every
// digit inside the fp8 range.  A's K order: lane group ga, byte ea <->
// k = 16 ga + (ea & 15) + 64 (ea >> 4); B's: lane group gb, element eb <->
// k = 32 gb + eb.
//
// The value side stays on the exact int8 MFMA: the f8f6f4 MFMA sums its
// products with an error near 2^-10 of the largest one when the fp8 operands
// span many binades, which the key weights (bounded by the rotation) absorb
// within the score tolerance but the softmax-weighted value digits p |v| of a
// peaked distribution do not.

// A constant held in a VGPR: (x & c1) | c2 with c1, c2 in VGPRs is one
// v_bitop3, where two literal operands would take two instructions.
__device__ __forceinline__ uint32_t vgpr_u32(uint32_t x) {
  uint32_t r;
  asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "s"(x));
  return r;
}

// Four fp8 (e4m3) digits of x, |x| <= 224: digit d in byte d.
__device__ __forceinline__ uint32_t fp8_digits(float x) {
  uint32_t out = 0;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const int p = __builtin_amdgcn_cvt_pk_fp8_f32(x, 0.f, 0, false);
    out |= static_cast<uint32_t>(p & 0xff) << (8 * d);
    x = (x - __builtin_amdgcn_cvt_f32_fp8(p, 0)) * 16.f;
  }
  return out;
}

// First row dword that lane group g of a row of RDW dwords loads: groups own
// dwords [g DPL, (g + 1) DPL) clipped to the row, and a group whose range
// passes the row's end loads the row's last DPL dwords instead (its operand
// bytes outside the dwords it owns are zero).
template <int DPL, int RDW>
__host__ __device__ constexpr int krow_base(int g) {
  return g * DPL < RDW - DPL ? g * DPL : RDW - DPL;
}

// Byte of the A-operand image (DPL MFMAs x 64 lanes x 32 bytes) holding row
// bit p (dword p >> 5, bit p & 31) for A row m.
// PMAJ (plane-major rows): lane group g takes dword g of each 128-bit plane
// of a virtual row, MFMA u plane u -- IP keys of 3 MSE bits (virtual planes
// b0, b1, b2, b0^b1^b2, QJL; the parity dword computed from the loaded ones)
// and 96-dim rows (planes of 3 dwords; lane group 3 has no data).
template <int DPL, int RDW, bool PMAJ>
__device__ __forceinline__ int kf4_byte(int p, int m) {
  const int w = p >> 5, bit = p & 31;
  const int gb = PMAJ ? (w & 3) : w / DPL;
  const int u = PMAJ ? (w >> 2) : w - krow_base<DPL, RDW>(gb);
  const int k = 32 * gb + 8 * (bit & 3) + (bit >> 2);
  const int ga = (k & 63) >> 4, ea = (k & 15) + 16 * (k >> 6);
  return (u * 64 + m + 16 * ga) * 32 + ea;
}

// Class factor of row bit p.
__device__ __forceinline__ float kf4_factor(int p) {
  const int c = p & 3;
  return c == 0 ? 2.f : c == 1 ? 1.f : c == 2 ? 0.5f : -1.f;
}

// The row's exponent sigma from the bound wmax >= max |W|: 2 wmax 2^-sigma <= 224.
__device__ __forceinline__ int kf4_sigma(float wmax) {
  int e = 0;
  if (wmax > 0.f) frexpf(wmax * (2.f / 224.f), &e);
  return e;
}

// The digit bytes of weight W at row bit p of query row r into the image sb;
// returns W's share of the row constant.
template <int DPL, int RDW, bool PMAJ>
__device__ __forceinline__ float kf4_put(uint8_t* sb, int p, float W, int sigma, int r) {
  const uint32_t dg = fp8_digits(ldexpf(W * kf4_factor(p), -sigma));
#pragma unroll
  for (int d = 0; d < 4; ++d)
    sb[kf4_byte<DPL, RDW, PMAJ>(p, 4 * r + d)] = static_cast<uint8_t>(dg >> (8 * d));
  return (p & 3) == 3 ? 0.5f * W : 0.f;
}

// Score weights of slot j of one query row (v = q~_j, w = alpha |v| S_j) at
// their K-row bits through put(bit, W); returns the slot's share of the row's
// MSE constant: v for IP keys (whose constant is kconst sum v), the slot's
// codebook constant times v for mixed keys.
template <int MB, typename P>
__device__ __forceinline__ float key_weights(const Tables& tb, int j, float v, float w, P&& put) {
  constexpr int D = 128;
  if (tb.kmix) {
    const bool outl = j < tb.n_out;
    put(j, 2.f * (outl ? tb.kgo[0] : tb.kgr[0]) * v);
    if (tb.kmix == 1) {
      put(D + j, 2.f * (outl ? tb.kgo[1] : tb.kgr[1]) * v);
      if (outl) {
        put(2 * D + j, 2.f * tb.kgo[2] * v);
        put(2 * D + tb.n_out + j, 2.f * tb.kgo[3] * v);
      }
    } else {
      put(D + j, 2.f * w);
      if (outl) put(2 * D + j, 2.f * tb.kgo[1] * v);
    }
    return (outl ? tb.kco : tb.kcr) * v;
  }
#pragma unroll
  for (int pl = 0; pl < MB; ++pl) put(pl * D + j, 2.f * tb.kg[pl] * v);
  put(MB * D + j, 2.f * w);
  return v;
}

// Float4 i of a 128 x 128 row-major matrix holding the DS x DS matrix at src
// in its top-left corner, zero elsewhere.
template <int DS>
__device__ __forceinline__ float4 pi_f4(const float4* __restrict__ src, int i) {
  if constexpr (DS == 128) {
    return src[i];
  } else {
    const int row = i >> 5, c4 = i & 31;
    return row < DS && c4 < DS / 4 ? src[row * (DS / 4) + c4] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

// Workgroup barrier ordering LDS accesses only: outstanding global loads (the
// prefetched chunks) stay in flight across it.
__device__ __forceinline__ void lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <typename T>
__device__ __forceinline__ T ldnt(const T* p) {
  return __builtin_nontemporal_load(p);
}

constexpr float kMFloor = -1e30f;  // running maxima start here (finite: no inf - inf)

}  // namespace qkv_attn
