// Shared host/device helpers for the quashkv_amd HIP kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/quashkv_amd.h"

// ---------------------------------------------------------------- host side

void qkv_set_error(const char* fmt, ...);

#define QKV_REQUIRE(cond, ...)                 \
  do {                                         \
    if (!(cond)) {                             \
      qkv_set_error(__VA_ARGS__);              \
      return QKV_E_INVALID;                    \
    }                                          \
  } while (0)

#define QKV_HIP(call)                                                     \
  do {                                                                    \
    hipError_t e_ = (call);                                               \
    if (e_ != hipSuccess) {                                               \
      qkv_set_error("HIP error %s at %s:%d", hipGetErrorString(e_),       \
                    __FILE__, __LINE__);                                  \
      return QKV_E_HIP;                                                   \
    }                                                                     \
  } while (0)

// Launch check: a failed launch is reported as a HIP error.
#define QKV_LAUNCHED() QKV_HIP(hipGetLastError())

static inline bool qkv_bits_ok(int bits) { return bits >= 1 && bits <= 4; }
static inline bool qkv_dtype_ok(int dt) { return dt == QKV_F32 || dt == QKV_F16 || dt == QKV_BF16; }
static inline bool qkv_d_ok(int d) { return d == 64 || d == 96 || d == 128; }
static inline bool qkv_aligned(const void* p, int a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

__host__ __device__ inline int64_t qkv_row_bytes(int d, int bits) {
  switch (bits) {
    case 8: return d;
    case 1: return (d + 7) / 8;
    case 2: return (d + 3) / 4;
    case 3: return 3 * ((d + 7) / 8);
    case 4: return (d + 1) / 2;
    default: return -1;
  }
}

static inline int qkv_num_cus() {
  static int n = 0;
  if (n == 0) {
    int dev = 0;
    hipDeviceProp_t p;
    if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&p, dev) == hipSuccess)
      n = p.multiProcessorCount;
    if (n <= 0) n = 256;
  }
  return n;
}

// -------------------------------------------------------------- device side

__device__ __forceinline__ float qkv_bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

__device__ __forceinline__ uint16_t qkv_f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40);  // NaN
  u += 0x7fffu + ((u >> 16) & 1u);  // round to nearest even
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float qkv_load(const void* p, int64_t i, int dt) {
  if (dt == QKV_F32) return static_cast<const float*>(p)[i];
  if (dt == QKV_F16) return static_cast<float>(static_cast<const _Float16*>(p)[i]);
  return qkv_bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
}

__device__ __forceinline__ void qkv_store(void* p, int64_t i, float v, int dt) {
  if (dt == QKV_F32) static_cast<float*>(p)[i] = v;
  else if (dt == QKV_F16) static_cast<_Float16*>(p)[i] = static_cast<_Float16>(v);
  else static_cast<uint16_t*>(p)[i] = qkv_f32_to_bf16(v);
}

// Code j of a row in the pack_bits layout (bits in {1,2,3,4}) or raw uint8 (8).
__device__ __forceinline__ uint32_t qkv_get_code(const uint8_t* __restrict__ row, int j, int bits) {
  switch (bits) {
    case 1: return (row[j >> 3] >> (j & 7)) & 1u;
    case 2: return (row[j >> 2] >> ((j & 3) * 2)) & 3u;
    case 4: return (row[j >> 1] >> ((j & 1) * 4)) & 15u;
    case 3: {
      const uint8_t* p = row + 3 * (j >> 3);
      uint32_t w = p[0] | (uint32_t(p[1]) << 8) | (uint32_t(p[2]) << 16);
      return (w >> (3 * (j & 7))) & 7u;
    }
    default: return row[j];
  }
}

// Byte b of the packed row of `codes` (d uint8 values), mirroring pack_bits'
// arithmetic exactly (quashkv/packing.py:43-89): 1/2-bit bytes are the sum of
// uint8-shifted values mod 256, 4-bit is lo | (hi << 4) in uint8, 3-bit splits
// the OR of (v_i << 3i) as a 32-bit word.
__device__ __forceinline__ uint8_t qkv_pack_byte(const uint8_t* __restrict__ codes, int b, int d, int bits) {
  if (bits == 3) {
    const int g = b / 3, k = b - 3 * (b / 3);
    uint32_t w = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int j = 8 * g + i;
      const uint32_t v = j < d ? codes[j] : 0u;
      w |= v << (3 * i);
    }
    return static_cast<uint8_t>((w >> (8 * k)) & 0xffu);
  }
  if (bits == 4) {
    const int j = 2 * b;
    const uint32_t lo = codes[j];
    const uint32_t hi = (j + 1 < d) ? codes[j + 1] : 0u;
    return static_cast<uint8_t>(lo | ((hi << 4) & 0xffu));
  }
  const int per = 8 / bits;
  uint32_t s = 0;
  for (int i = 0; i < per; ++i) {
    const int j = per * b + i;
    const uint32_t v = j < d ? codes[j] : 0u;
    s += (v << (bits * i)) & 0xffu;
  }
  return static_cast<uint8_t>(s & 0xffu);
}

// Row index of vector r in grouped-row addressing.
__device__ __forceinline__ int64_t qkv_grouped_row(int64_t r, int64_t seq, int64_t gstride) {
  const int64_t g = r / seq;
  return g * gstride + (r - g * seq);
}

template <typename T>
__device__ __forceinline__ T qkv_wave_sum(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

template <typename T>
__device__ __forceinline__ T qkv_wave_max(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// ------------------------------------------------ decompress (shared host side)

// Arguments of one decompress call (validated by the C ABI entry points).
struct QkvDecompressArgs {
  int mode, fmt;
  const uint8_t* codes;
  const uint8_t* qjl;
  const float* norms;
  int64_t n;
  int d, bits;
  const float* pi;
  const float* cents;
  const float* signs;
  float qjl_scale;
  int64_t in_seq, in_gstride;
  void* out;
  int out_dtype;
  const uint8_t* sel;  // mixed precision: per-coordinate codebook selector
  const float* alt_cents;
  int alt_bits;
};

// The MFMA decompress kernels take d = 64 / 128 with aligned operands;
// qkv_decompress_mfma launches them.
bool qkv_decompress_mfma_ok(const QkvDecompressArgs& a);
int qkv_decompress_mfma(const QkvDecompressArgs& a, hipStream_t s);

// ------------------------------------------------------ paged cache stores

// A paged store: pages of 64 tokens, each holding those tokens of all H kv
// heads of one sequence; tab[b * pmax + t / 64] is the page of sequence b's
// token t.  tab == nullptr: the contiguous store (stream grp = b * H + h at
// rows grp * t_stride ..).  Page pg's stream h then occupies the 64 rows
// (pg * H + h) * 64 .. of the same row / tile arrays.
struct QkvPages {
  const int32_t* tab;
  int32_t pmax;    // pages per sequence in the table
  int32_t H;       // kv heads
  int32_t lg;      // log2 of the tokens per page
  int32_t npages;  // pages in the pool: entries outside [0, npages) are never written
};

// Pages hold 64 << k tokens, k = 0 .. 5 (whole 64-token tiles, at most one
// split's worth).
constexpr int kPageLgMin = 6, kPageLgMax = 11;

// log2 of a page token count, or -1 when it is not 64 << k, k = 0 .. 5.
inline int qkv_page_lg(int32_t page_tokens) {
  for (int lg = kPageLgMin; lg <= kPageLgMax; ++lg)
    if (page_tokens == (1 << lg)) return lg;
  return -1;
}

// Store rows of the 64-token span [t, t + 64) of stream grp.  On a paged
// store the span meets at most two pages, looked up once; row(t) >> 5 is the
// token's 32-token V tile (store capacity a multiple of 32).
struct QkvSpan {
  int64_t base0, base1;  // store row of the first token of page p0 and of p0 + 1
                         // (-1: the table names a page outside the pool)
  int64_t p0;
  int lg;                // log2 of the page (64-token blocks on a contiguous store)
  // store row of token t, or -1 when its page is outside the pool (callers
  // then write nothing)
  __device__ __forceinline__ int64_t row(int64_t t) const {
    const int64_t b = (t >> lg) == p0 ? base0 : base1;
    return b < 0 ? -1 : b + (t & ((int64_t(1) << lg) - 1));
  }
};

// Span rows of stream grp from token t (t and every token the caller asks
// for lie below the table's pages_per_seq pages).
__device__ __forceinline__ QkvSpan qkv_span(const QkvPages& pg, int64_t grp, int64_t t_stride,
                                            int64_t t) {
  QkvSpan s;
  if (pg.tab == nullptr) {
    s.lg = 6;
    s.p0 = t >> 6;
    s.base0 = grp * t_stride + (s.p0 << 6);
    s.base1 = s.base0 + 64;
    return s;
  }
  s.lg = pg.lg;
  s.p0 = t >> pg.lg;
  const int g = static_cast<int>(grp), b = g / pg.H, h = g - b * pg.H;
  const int32_t* tb = pg.tab + int64_t(b) * pg.pmax;
  const int p = static_cast<int>(s.p0);
  const int64_t pa = tb[p];
  const int64_t pb = p + 1 < pg.pmax ? tb[p + 1] : pa;
  s.base0 = pa >= 0 && pa < pg.npages ? (pa * pg.H + h) << pg.lg : -1;
  s.base1 = pb >= 0 && pb < pg.npages ? (pb * pg.H + h) << pg.lg : -1;
  return s;
}

