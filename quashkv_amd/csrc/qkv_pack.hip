// pack_bits / unpack_bits on the GPU (reference: quashkv/packing.py:22-165),
// plus the library-wide error state.
#include <stdarg.h>
#include <stdio.h>

#include "qkv_common.h"

static thread_local char g_err[512] = "";

void qkv_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

extern "C" const char* qkv_last_error(void) { return g_err; }
extern "C" int qkv_abi_version(void) { return QKV_ABI_VERSION; }

extern "C" int64_t qkv_packed_row_bytes(int32_t d, int32_t bits) {
  if (d <= 0) return -1;
  return qkv_row_bytes(d, bits);
}

// One thread per output byte.  Each wave covers 64 consecutive bytes of the
// packed stream, so stores are fully coalesced; the (up to 8) code loads per
// byte hit the same few cache lines per row.
__global__ void qkv_pack_kernel(const uint8_t* __restrict__ codes, uint8_t* __restrict__ packed,
                                int64_t rows, int d, int bits, int64_t pb) {
  const int64_t total = rows * pb;
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t r = i / pb;
    const int b = static_cast<int>(i - r * pb);
    packed[i] = qkv_pack_byte(codes + r * d, b, d, bits);
  }
}

// One thread per output code.
__global__ void qkv_unpack_kernel(const uint8_t* __restrict__ packed, int64_t pstride,
                                  uint8_t* __restrict__ codes, int64_t rows, int d, int bits) {
  const int64_t total = rows * d;
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t r = i / d;
    const int j = static_cast<int>(i - r * d);
    codes[i] = static_cast<uint8_t>(qkv_get_code(packed + r * pstride, j, bits));
  }
}

static int grid_for(int64_t total) {
  int64_t blocks = (total + 255) / 256;
  const int64_t cap = int64_t(qkv_num_cus()) * 16;
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  return static_cast<int>(blocks);
}

extern "C" int qkv_pack_bits(const uint8_t* codes, uint8_t* packed, int64_t rows, int32_t d,
                             int32_t bits, void* stream) {
  QKV_REQUIRE(qkv_bits_ok(bits), "Unsupported bits: %d", bits);
  QKV_REQUIRE(d > 0 && rows >= 0, "invalid shape rows=%lld d=%d", (long long)rows, d);
  if (rows == 0) return QKV_OK;
  QKV_REQUIRE(codes && packed, "null pointer");
  const int64_t pb = qkv_row_bytes(d, bits);
  hipLaunchKernelGGL(qkv_pack_kernel, dim3(grid_for(rows * pb)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), codes, packed, rows, d, bits, pb);
  QKV_LAUNCHED();
  return QKV_OK;
}

extern "C" int qkv_unpack_bits(const uint8_t* packed, int64_t packed_row_bytes, uint8_t* codes,
                               int64_t rows, int32_t d, int32_t bits, void* stream) {
  QKV_REQUIRE(qkv_bits_ok(bits), "Unsupported bits: %d", bits);
  QKV_REQUIRE(d > 0 && rows >= 0, "invalid shape rows=%lld d=%d", (long long)rows, d);
  QKV_REQUIRE(packed_row_bytes >= qkv_row_bytes(d, bits),
              "packed rows of %lld bytes cannot hold %d %d-bit codes",
              (long long)packed_row_bytes, d, bits);
  if (rows == 0) return QKV_OK;
  QKV_REQUIRE(codes && packed, "null pointer");
  hipLaunchKernelGGL(qkv_unpack_kernel, dim3(grid_for(rows * d)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), packed, packed_row_bytes, codes, rows, d,
                     bits);
  QKV_LAUNCHED();
  return QKV_OK;
}

// ----------------------------------------------------------------------------
// Codebook primitives on arbitrary-shape tensors.
//   qkv_quantize mode 0: code = #{i : t_i < y}        (quashkv/codebook.py:239-259)
//                mode 1: first argmin_i |y - c_i|     (quashkv/codebook.py:209-224)
//   qkv_dequantize:      c[code], NaN for codes >= count (the reference raises)
//   qkv_ip_dot:          n (<q~, c[code]> + alpha sum |q~| (2b-1) S)
//                        (quashkv/quantizer.py:244-279), one wave per vector.
// ----------------------------------------------------------------------------

__global__ void qkv_quantize_kernel(const float* __restrict__ y, int64_t n,
                                    const float* __restrict__ table, int count, int mode,
                                    uint8_t* __restrict__ out) {
  __shared__ float tb[16];
  if (threadIdx.x < 16) tb[threadIdx.x] = threadIdx.x < count ? table[threadIdx.x] : 0.f;
  __syncthreads();
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n;
       i += int64_t(gridDim.x) * blockDim.x) {
    const float v = y[i];
    int code = 0;
    if (mode == 0) {
      for (int k = 0; k < count; ++k) code += (v > tb[k]) ? 1 : 0;
    } else {
      float best = fabsf(v - tb[0]);
      for (int k = 1; k < count; ++k) {
        const float dk = fabsf(v - tb[k]);
        if (dk < best) {
          best = dk;
          code = k;
        }
      }
    }
    out[i] = static_cast<uint8_t>(code);
  }
}

__global__ void qkv_dequantize_kernel(const uint8_t* __restrict__ codes, int64_t n,
                                      const float* __restrict__ cents, int count,
                                      float* __restrict__ out) {
  __shared__ float cb[256];
  for (int k = threadIdx.x; k < 256; k += blockDim.x) cb[k] = k < count ? cents[k] : __builtin_nanf("");
  __syncthreads();
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n;
       i += int64_t(gridDim.x) * blockDim.x)
    out[i] = cb[codes[i]];
}

__global__ void qkv_ip_dot_kernel(const uint8_t* __restrict__ codes, const uint8_t* __restrict__ qjl,
                                  const float* __restrict__ norms, const float* __restrict__ q_rot,
                                  int64_t n, int d, const float* __restrict__ cents, int count,
                                  const float* __restrict__ signs, float alpha,
                                  float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = (blockIdx.x * int64_t(blockDim.x) + threadIdx.x) >> 6;
  const int64_t nwaves = (int64_t(gridDim.x) * blockDim.x) >> 6;
  for (int64_t r = wave; r < n; r += nwaves) {
    float mse = 0.f, corr = 0.f;
    for (int j = lane; j < d; j += 64) {
      const float q = q_rot[r * d + j];
      const int c = codes[r * d + j];
      const float cv = c < count ? cents[c] : __builtin_nanf("");
      mse = fmaf(q, cv, mse);
      const float sv = qjl[r * d + j] ? 1.f : -1.f;
      corr = fmaf(fabsf(q) * sv, signs[j], corr);
    }
    mse = qkv_wave_sum(mse);
    corr = qkv_wave_sum(corr);
    if (lane == 0) out[r] = norms[r] * (mse + alpha * corr);
  }
}

extern "C" int qkv_quantize(const float* y, int64_t n, const float* table, int32_t count,
                            int32_t mode, uint8_t* out, void* stream) {
  QKV_REQUIRE(mode == 0 || mode == 1, "unknown quantize mode %d", mode);
  QKV_REQUIRE(count >= 1 && count <= 16, "table size %d out of range", count);
  QKV_REQUIRE(n >= 0, "negative size");
  if (n == 0) return QKV_OK;
  QKV_REQUIRE(y && table && out, "null pointer");
  hipLaunchKernelGGL(qkv_quantize_kernel, dim3(grid_for(n)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), y, n, table, count, mode, out);
  QKV_LAUNCHED();
  return QKV_OK;
}

extern "C" int qkv_dequantize(const uint8_t* codes, int64_t n, const float* cents, int32_t count,
                              float* out, void* stream) {
  QKV_REQUIRE(count >= 1 && count <= 256, "table size %d out of range", count);
  QKV_REQUIRE(n >= 0, "negative size");
  if (n == 0) return QKV_OK;
  QKV_REQUIRE(codes && cents && out, "null pointer");
  hipLaunchKernelGGL(qkv_dequantize_kernel, dim3(grid_for(n)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), codes, n, cents, count, out);
  QKV_LAUNCHED();
  return QKV_OK;
}

extern "C" int qkv_ip_dot(const uint8_t* codes, const uint8_t* qjl, const float* norms,
                          const float* q_rot, int64_t n, int32_t d, const float* cents,
                          int32_t count, const float* signs, float alpha, float* out,
                          void* stream) {
  QKV_REQUIRE(d > 0 && n >= 0, "invalid shape");
  QKV_REQUIRE(count >= 1 && count <= 256, "table size %d out of range", count);
  if (n == 0) return QKV_OK;
  QKV_REQUIRE(codes && qjl && norms && q_rot && cents && signs && out, "null pointer");
  int64_t blocks = (n * 64 + 255) / 256;
  const int64_t cap = int64_t(qkv_num_cus()) * 16;
  if (blocks > cap) blocks = cap;
  hipLaunchKernelGGL(qkv_ip_dot_kernel, dim3(static_cast<int>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), codes, qjl, norms, q_rot, n, d, cents,
                     count, signs, alpha, out);
  QKV_LAUNCHED();
  return QKV_OK;
}
