// Measurement helper: the read-only HBM ceiling of the device.
//
// The decode kernels are read-dominated (packed K/V in, a few KB of partials
// out), so their roofline fraction is judged against what a plain streaming
// read reaches on the same box: every lane reads 16-byte words of a buffer
// larger than the 256 MB MALL, UNROLL of them in flight per iteration, and
// folds them into one word per workgroup (the only store).  No reference
// counterpart; bench.py reports the best of a few launch shapes.
#include "qkv_common.h"

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int UNROLL, bool NT>
__global__ __launch_bounds__(256) void read_probe(const u32x4* __restrict__ src, int64_t n16,
                                                  uint32_t* __restrict__ sink) {
  const int64_t stride = int64_t(gridDim.x) * 256;
  int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  uint32_t acc = 0;
  for (; i + (UNROLL - 1) * stride < n16; i += UNROLL * stride) {
    u32x4 v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u)
      v[u] = NT ? __builtin_nontemporal_load(src + i + u * stride) : src[i + u * stride];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < n16; i += stride) {
    const u32x4 v = src[i];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  // fold the block into one word (keeps the loads live)
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) acc ^= static_cast<uint32_t>(__shfl_xor(static_cast<int>(acc), o, 64));
  __shared__ uint32_t w[4];
  if ((threadIdx.x & 63) == 0) w[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) sink[blockIdx.x] = w[0] ^ w[1] ^ w[2] ^ w[3];
}

}  // namespace

extern "C" int qkv_hbm_read_probe(const void* buf, int64_t bytes, uint32_t* sink, int32_t grid,
                                  int32_t unroll, int32_t nontemporal, void* stream) {
  QKV_REQUIRE(buf && sink, "null pointer");
  QKV_REQUIRE(qkv_aligned(buf, 16) && bytes > 0 && bytes % 16 == 0,
              "buffer must be 16-byte aligned and a positive multiple of 16 bytes");
  QKV_REQUIRE(grid > 0 && grid <= 1 << 20, "grid %d out of range", grid);
  QKV_REQUIRE(unroll == 4 || unroll == 8 || unroll == 16, "unroll must be 4, 8 or 16");
  auto s = static_cast<hipStream_t>(stream);
  const auto* src = static_cast<const u32x4*>(buf);
  const int64_t n16 = bytes / 16;
#define QKV_RP(U, NTV) hipLaunchKernelGGL((read_probe<U, NTV>), dim3(grid), dim3(256), 0, s, src, n16, sink)
  if (nontemporal) {
    if (unroll == 4) QKV_RP(4, true); else if (unroll == 8) QKV_RP(8, true); else QKV_RP(16, true);
  } else {
    if (unroll == 4) QKV_RP(4, false); else if (unroll == 8) QKV_RP(8, false); else QKV_RP(16, false);
  }
#undef QKV_RP
  QKV_LAUNCHED();
  return QKV_OK;
}
