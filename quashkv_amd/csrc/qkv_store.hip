// Cache store formats and their converters.
//
// The engine keeps its compressed cache in two bit-plane formats that the
// MFMA decode kernel streams directly (the reference keeps a Python list of
// per-append pack_bits tensors, quashkv/engine.py:145-172; the formats here
// hold the same bits, re-arranged):
//
//   K rows ("kplanes"): one row per token of (mbits + 1) * d / 8 bytes:
//       [MSE bit-plane 0][MSE bit-plane 1]...[QJL plane]
//     plane r holds bit r of every coordinate's code, coordinate j at bit
//     (j % 8) of byte j / 8 (LSB first, the 1-bit pack_bits layout,
//     quashkv/packing.py:43-52).  Rows use grouped-row addressing.
//
//   V tiles ("vtiles"): tokens in tiles of 32; per (sequence, kv head):
//       word[tile][plane k][coordinate j] (uint32), bit (t % 32) = bit k of
//       the code of token t at coordinate j.
//     vbits * d * 4 bytes per 32 tokens == the pack_bits size.
//
//   Mixed K rows ("kmixed", d = 128): 48 bytes per token over coordinates
//   permuted outliers first (slot j holds rotated channel perm[j]):
//       [plane b0 (16 B)][plane b1 (16 B)][plane 2 (16 B)]
//     plane 2 holds b2 of slots 0 .. n_out-1 at bits 0.., and their parity
//     b0^b1^b2 at bits 64..; outlier slots carry 3-bit codes, the others
//     2-bit ones.
//
// Converters to and from one-uint8-per-code tensors serve the reference's
// block views (CompressedKVBlock, quashkv/engine.py:30-51) and the tests.
#include "qkv_common.h"

namespace {

// one thread per (row, plane dword)
__global__ void kplanes_pack_kernel(const uint8_t* __restrict__ codes,
                                    const uint8_t* __restrict__ qjl, int64_t n, int d, int mbits,
                                    uint8_t* __restrict__ dst, int64_t row_bytes, int64_t seq,
                                    int64_t gstride) {
  const int wpp = d / 32;                     // dwords per plane
  const int nplanes = mbits + (qjl ? 1 : 0);
  const int64_t total = n * nplanes * wpp;
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t r = i / (nplanes * wpp);
    const int rem = static_cast<int>(i - r * nplanes * wpp);
    const int plane = rem / wpp, w = rem - plane * wpp;
    uint32_t word = 0;
    if (plane < mbits) {
      const uint8_t* c = codes + r * d + 32 * w;
      for (int b = 0; b < 32; ++b) word |= ((uint32_t(c[b]) >> plane) & 1u) << b;
    } else {
      const uint8_t* c = qjl + r * d + 32 * w;
      for (int b = 0; b < 32; ++b) word |= (uint32_t(c[b]) & 1u) << b;
    }
    const int64_t row = qkv_grouped_row(r, seq, gstride);
    uint32_t* out = reinterpret_cast<uint32_t*>(dst + row * row_bytes);
    out[plane * wpp + w] = word;
  }
}

// one thread per (row, coordinate)
__global__ void kplanes_unpack_kernel(const uint8_t* __restrict__ src, int64_t row_bytes,
                                      int64_t n, int d, int mbits, int64_t seq, int64_t gstride,
                                      uint8_t* __restrict__ codes, uint8_t* __restrict__ qjl) {
  const int64_t total = n * d;
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t r = i / d;
    const int j = static_cast<int>(i - r * d);
    const uint8_t* row = src + qkv_grouped_row(r, seq, gstride) * row_bytes;
    uint32_t c = 0;
    for (int p = 0; p < mbits; ++p) c |= ((row[p * (d / 8) + (j >> 3)] >> (j & 7)) & 1u) << p;
    if (codes) codes[i] = static_cast<uint8_t>(c);
    if (qjl) qjl[i] = (row[mbits * (d / 8) + (j >> 3)] >> (j & 7)) & 1u;
  }
}

// one thread per (group, tile, plane, coordinate) word touched by tokens
// [t0, t0 + S) of each group; bits of other tokens are preserved.
__global__ void vtiles_pack_kernel(const uint8_t* __restrict__ codes, int64_t G, int64_t S,
                                   int d, int vbits, uint32_t* __restrict__ dst,
                                   int64_t tiles_per_group, int64_t t0) {
  const int64_t tb = t0 / 32, te = (t0 + S + 31) / 32;  // tiles touched
  const int64_t nt = te - tb;
  const int64_t per_tile = int64_t(vbits) * d;
  const int64_t total = G * nt * per_tile;
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t g = i / (nt * per_tile);
    int64_t rem = i - g * nt * per_tile;
    const int64_t tt = rem / per_tile;
    rem -= tt * per_tile;
    const int k = static_cast<int>(rem / d), j = static_cast<int>(rem - int64_t(k) * d);
    const int64_t tile = tb + tt;
    const int64_t lo = max<int64_t>(tile * 32, t0), hi = min<int64_t>(tile * 32 + 32, t0 + S);
    uint32_t mask = 0, bits = 0;
    for (int64_t t = lo; t < hi; ++t) {
      const uint32_t c = codes[(g * S + (t - t0)) * d + j];
      mask |= 1u << (t & 31);
      bits |= ((c >> k) & 1u) << (t & 31);
    }
    uint32_t* w = dst + (g * tiles_per_group + tile) * per_tile + int64_t(k) * d + j;
    *w = (*w & ~mask) | bits;
  }
}

// one thread per (group, token, coordinate) of tokens [t0, t0 + S)
__global__ void vtiles_unpack_kernel(const uint32_t* __restrict__ src, int64_t G, int64_t S,
                                     int d, int vbits, int64_t tiles_per_group, int64_t t0,
                                     uint8_t* __restrict__ codes) {
  const int64_t total = G * S * d;
  const int64_t per_tile = int64_t(vbits) * d;
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t g = i / (S * d);
    int64_t rem = i - g * S * d;
    const int64_t s = rem / d;
    const int j = static_cast<int>(rem - s * d);
    const int64_t t = t0 + s;
    const uint32_t* w = src + (g * tiles_per_group + t / 32) * per_tile + j;
    uint32_t c = 0;
    for (int k = 0; k < vbits; ++k) c |= ((w[int64_t(k) * d] >> (t & 31)) & 1u) << k;
    codes[i] = static_cast<uint8_t>(c);
  }
}

int grid_for(int64_t total) {
  int64_t blocks = (total + 255) / 256;
  const int64_t cap = int64_t(qkv_num_cus()) * 16;
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  return static_cast<int>(blocks);
}

int check_d(int d) {
  if (d <= 0 || d % 32 != 0 || d > 256) {
    qkv_set_error("head_dim %d unsupported by the cache formats (multiple of 32, <= 256)", d);
    return QKV_E_UNSUPPORTED;
  }
  return QKV_OK;
}


struct Perm128 {
  uint8_t p[128];  // slot -> channel
};

// Mixed-precision K rows over slots (slot j = channel perm[j], the NO = n_out
// outlier channels first), RD = kmixed_row_dwords(ipm, n_out) dwords:
//   MSE keys (ipm = 0): [b0 x 4][b1 x 4][b2 of outliers][parity of outliers]
//   IP keys  (ipm = 1): [b0 x 4][QJL x 4][b1 of outliers]
__host__ __device__ inline int kmixed_row_dwords(int ipm, int n_out) {
  return ipm ? 8 + n_out / 32 : 8 + n_out / 16;
}

// one thread per (row, row dword); qjl (IP keys) holds one bit per uint8
__global__ void kmixed_pack_kernel(const uint8_t* __restrict__ codes,
                                   const uint8_t* __restrict__ qjl, int64_t n, Perm128 perm,
                                   int n_out, int ipm, uint8_t* __restrict__ dst, int64_t seq,
                                   int64_t gstride) {
  const int rd = kmixed_row_dwords(ipm, n_out), nob = n_out / 32;
  const int64_t total = n * rd;
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t r = i / rd;
    const int w = static_cast<int>(i - r * rd);
    const uint8_t* c = codes + r * 128;
    uint32_t word = 0;
    for (int b = 0; b < 32; ++b) {
      uint32_t bit;
      if (w < 4) {
        bit = c[perm.p[32 * w + b]] & 1u;
      } else if (w < 8) {
        const int ch = perm.p[32 * (w - 4) + b];
        bit = ipm ? qjl[r * 128 + ch] & 1u : (c[ch] >> 1) & 1u;
      } else {
        const int k = (w - 8) / nob;  // 0: b2 (MSE) / b1 (IP); 1: parity (MSE)
        const uint32_t code = c[perm.p[32 * (w - 8 - k * nob) + b]];
        bit = ipm ? (code >> 1) & 1u
                  : (k == 0 ? (code >> 2) & 1u : (code ^ (code >> 1) ^ (code >> 2)) & 1u);
      }
      word |= bit << b;
    }
    const int64_t row = qkv_grouped_row(r, seq, gstride);
    reinterpret_cast<uint32_t*>(dst + row * (4 * rd))[w] = word;
  }
}

// one thread per (row, slot)
__global__ void kmixed_unpack_kernel(const uint8_t* __restrict__ src, int64_t n, Perm128 perm,
                                     int n_out, int ipm, int64_t seq, int64_t gstride,
                                     uint8_t* __restrict__ codes, uint8_t* __restrict__ qjl) {
  const int rd = kmixed_row_dwords(ipm, n_out);
  const int64_t total = n * 128;
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t r = i >> 7;
    const int j = static_cast<int>(i & 127);
    const uint8_t* row = src + qkv_grouped_row(r, seq, gstride) * (4 * rd);
    auto bit = [&](int byte0) { return (uint32_t(row[byte0 + (j >> 3)]) >> (j & 7)) & 1u; };
    uint32_t code = bit(0);
    const int ch = perm.p[j];
    if (ipm) {
      qjl[r * 128 + ch] = static_cast<uint8_t>(bit(16));
      if (j < n_out) code |= bit(32) << 1;
    } else {
      code |= bit(16) << 1;
      if (j < n_out) code |= bit(32) << 2;
    }
    codes[r * 128 + ch] = static_cast<uint8_t>(code);
  }
}

bool make_perm(const int32_t* perm_host, int n_out, Perm128* out) {
  if (n_out != 32 && n_out != 64) return false;
  bool seen[128] = {};
  for (int j = 0; j < 128; ++j) {
    const int32_t c = perm_host[j];
    if (c < 0 || c >= 128 || seen[c]) return false;
    seen[c] = true;
    out->p[j] = static_cast<uint8_t>(c);
  }
  return true;
}
}  // namespace

extern "C" int64_t qkv_kplanes_row_bytes(int32_t d, int32_t mbits, int32_t with_qjl) {
  if (d <= 0 || d % 32 != 0 || mbits < 0 || mbits > 4) return -1;
  return int64_t(mbits + (with_qjl ? 1 : 0)) * d / 8;
}

extern "C" int64_t qkv_vtiles_bytes(int32_t d, int32_t vbits, int64_t tokens) {
  if (d <= 0 || d % 32 != 0 || vbits < 1 || vbits > 4 || tokens < 0) return -1;
  return (tokens + 31) / 32 * 4 * int64_t(vbits) * d;
}

extern "C" int qkv_kplanes_pack(const uint8_t* codes, const uint8_t* qjl, int64_t n, int32_t d,
                                int32_t mbits, uint8_t* dst, int64_t row_bytes, int64_t seq,
                                int64_t group_stride, void* stream) {
  int st = check_d(d);
  if (st != QKV_OK) return st;
  QKV_REQUIRE(mbits >= 1 && mbits <= 4, "mse bits must be in {1, 2, 3, 4}, got %d", mbits);
  QKV_REQUIRE(n >= 0, "negative row count");
  if (n == 0) return QKV_OK;
  QKV_REQUIRE(codes && dst, "null pointer");
  QKV_REQUIRE(row_bytes >= qkv_kplanes_row_bytes(d, mbits, qjl != nullptr) && row_bytes % 4 == 0,
              "bad K row stride %lld", (long long)row_bytes);
  QKV_REQUIRE(qkv_aligned(dst, 4), "K rows must be 4-byte aligned");
  QKV_REQUIRE(seq > 0 && group_stride >= seq, "bad grouped-row layout");
  const int64_t total = n * (mbits + (qjl ? 1 : 0)) * (d / 32);
  hipLaunchKernelGGL(kplanes_pack_kernel, dim3(grid_for(total)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), codes, qjl, n, d, mbits, dst, row_bytes,
                     seq, group_stride);
  QKV_LAUNCHED();
  return QKV_OK;
}

extern "C" int qkv_kplanes_unpack(const uint8_t* src, int64_t row_bytes, int64_t n, int32_t d,
                                  int32_t mbits, int64_t seq, int64_t group_stride,
                                  uint8_t* codes, uint8_t* qjl, void* stream) {
  int st = check_d(d);
  if (st != QKV_OK) return st;
  QKV_REQUIRE(mbits >= 1 && mbits <= 4, "mse bits must be in {1, 2, 3, 4}, got %d", mbits);
  QKV_REQUIRE(n >= 0, "negative row count");
  if (n == 0) return QKV_OK;
  QKV_REQUIRE(src && (codes || qjl), "null pointer");
  QKV_REQUIRE(row_bytes >= qkv_kplanes_row_bytes(d, mbits, qjl != nullptr),
              "bad K row stride %lld", (long long)row_bytes);
  QKV_REQUIRE(seq > 0 && group_stride >= seq, "bad grouped-row layout");
  hipLaunchKernelGGL(kplanes_unpack_kernel, dim3(grid_for(n * d)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), src, row_bytes, n, d, mbits, seq,
                     group_stride, codes, qjl);
  QKV_LAUNCHED();
  return QKV_OK;
}

extern "C" int qkv_vtiles_pack(const uint8_t* codes, int64_t groups, int64_t S, int32_t d,
                               int32_t vbits, uint32_t* dst, int64_t tiles_per_group,
                               int64_t t0, void* stream) {
  int st = check_d(d);
  if (st != QKV_OK) return st;
  QKV_REQUIRE(qkv_bits_ok(vbits), "bits must be in {1, 2, 3, 4}, got %d", vbits);
  QKV_REQUIRE(groups >= 0 && S >= 0 && t0 >= 0, "invalid shape");
  if (groups == 0 || S == 0) return QKV_OK;
  QKV_REQUIRE(codes && dst, "null pointer");
  QKV_REQUIRE((t0 + S + 31) / 32 <= tiles_per_group, "tokens [%lld, %lld) exceed %lld tiles",
              (long long)t0, (long long)(t0 + S), (long long)tiles_per_group);
  const int64_t nt = (t0 + S + 31) / 32 - t0 / 32;
  const int64_t total = groups * nt * vbits * d;
  hipLaunchKernelGGL(vtiles_pack_kernel, dim3(grid_for(total)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), codes, groups, S, d, vbits, dst,
                     tiles_per_group, t0);
  QKV_LAUNCHED();
  return QKV_OK;
}

extern "C" int qkv_vtiles_unpack(const uint32_t* src, int64_t groups, int64_t S, int32_t d,
                                 int32_t vbits, int64_t tiles_per_group, int64_t t0,
                                 uint8_t* codes, void* stream) {
  int st = check_d(d);
  if (st != QKV_OK) return st;
  QKV_REQUIRE(qkv_bits_ok(vbits), "bits must be in {1, 2, 3, 4}, got %d", vbits);
  QKV_REQUIRE(groups >= 0 && S >= 0 && t0 >= 0, "invalid shape");
  if (groups == 0 || S == 0) return QKV_OK;
  QKV_REQUIRE(codes && src, "null pointer");
  QKV_REQUIRE((t0 + S + 31) / 32 <= tiles_per_group, "tokens [%lld, %lld) exceed %lld tiles",
              (long long)t0, (long long)(t0 + S), (long long)tiles_per_group);
  hipLaunchKernelGGL(vtiles_unpack_kernel, dim3(grid_for(groups * S * d)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), src, groups, S, d, vbits,
                     tiles_per_group, t0, codes);
  QKV_LAUNCHED();
  return QKV_OK;
}


namespace {

int kmixed_pack_impl(const uint8_t* codes, const uint8_t* qjl, int ipm, int64_t n,
                     const int32_t* perm_host, int32_t n_out, uint8_t* dst, int64_t seq,
                     int64_t group_stride, void* stream) {
  QKV_REQUIRE(n >= 0, "negative row count");
  QKV_REQUIRE(perm_host, "null pointer");
  Perm128 perm;
  QKV_REQUIRE(make_perm(perm_host, n_out, &perm),
              "perm must be a permutation of 0..127 and n_out 32 or 64");
  if (n == 0) return QKV_OK;
  QKV_REQUIRE(codes && dst && (!ipm || qjl), "null pointer");
  QKV_REQUIRE(qkv_aligned(dst, 4), "K rows must be 4-byte aligned");
  QKV_REQUIRE(seq > 0 && group_stride >= seq, "bad grouped-row layout");
  hipLaunchKernelGGL(kmixed_pack_kernel, dim3(grid_for(n * kmixed_row_dwords(ipm, n_out))),
                     dim3(256), 0, static_cast<hipStream_t>(stream), codes, qjl, n, perm, n_out,
                     ipm, dst, seq, group_stride);
  QKV_LAUNCHED();
  return QKV_OK;
}

int kmixed_unpack_impl(const uint8_t* src, int ipm, int64_t n, const int32_t* perm_host,
                       int32_t n_out, int64_t seq, int64_t group_stride, uint8_t* codes,
                       uint8_t* qjl, void* stream) {
  QKV_REQUIRE(n >= 0, "negative row count");
  QKV_REQUIRE(perm_host, "null pointer");
  Perm128 perm;
  QKV_REQUIRE(make_perm(perm_host, n_out, &perm),
              "perm must be a permutation of 0..127 and n_out 32 or 64");
  if (n == 0) return QKV_OK;
  QKV_REQUIRE(src && codes && (!ipm || qjl), "null pointer");
  QKV_REQUIRE(seq > 0 && group_stride >= seq, "bad grouped-row layout");
  hipLaunchKernelGGL(kmixed_unpack_kernel, dim3(grid_for(n * 128)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), src, n, perm, n_out, ipm, seq,
                     group_stride, codes, qjl);
  QKV_LAUNCHED();
  return QKV_OK;
}

}  // namespace

extern "C" int qkv_kmixed_pack(const uint8_t* codes, int64_t n, const int32_t* perm_host,
                               int32_t n_out, uint8_t* dst, int64_t seq, int64_t group_stride,
                               void* stream) {
  return kmixed_pack_impl(codes, nullptr, 0, n, perm_host, n_out, dst, seq, group_stride,
                          stream);
}

extern "C" int qkv_kmixed_unpack(const uint8_t* src, int64_t n, const int32_t* perm_host,
                                 int32_t n_out, int64_t seq, int64_t group_stride,
                                 uint8_t* codes, void* stream) {
  return kmixed_unpack_impl(src, 0, n, perm_host, n_out, seq, group_stride, codes, nullptr,
                            stream);
}

extern "C" int qkv_kipmixed_pack(const uint8_t* codes, const uint8_t* qjl, int64_t n,
                                 const int32_t* perm_host, int32_t n_out, uint8_t* dst,
                                 int64_t seq, int64_t group_stride, void* stream) {
  return kmixed_pack_impl(codes, qjl, 1, n, perm_host, n_out, dst, seq, group_stride, stream);
}

extern "C" int qkv_kipmixed_unpack(const uint8_t* src, int64_t n, const int32_t* perm_host,
                                   int32_t n_out, int64_t seq, int64_t group_stride,
                                   uint8_t* codes, uint8_t* qjl, void* stream) {
  return kmixed_unpack_impl(src, 1, n, perm_host, n_out, seq, group_stride, codes, qjl,
                            stream);
}
