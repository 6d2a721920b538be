// Fused compress and decompress (generic VALU path).
//
// compress:   n = max(||x||, 1e-8); u = x / n; y = u Pi^T; code = #{t_i < y}
//             [IP: bit = ((y - c[code]) * S >= 0)]; packed stores.
//             Reference: quashkv/triton_kernels/compress.py:34-97 (PyTorch path),
//             quashkv/quantizer.py:113-131, 211-242.
// decompress: x^ = ((c[code] [+ alpha S (2b-1)]) Pi) * n.
//             Reference: quashkv/triton_kernels/decompress.py:32-96,
//             quashkv/quantizer.py:133-147.
//
// One workgroup of 128 threads owns ROWS vectors at a time; thread j owns
// output coordinate j.  Pi (or Pi^T) is staged once per workgroup in LDS
// (64 KB at d = 128) and the grid is persistent over row tiles.
#include "qkv_common.h"

namespace {

constexpr int kThreads = 128;
constexpr int kRows = 8;

template <int D>
__global__ __launch_bounds__(kThreads) void compress_generic(
    int mode, int in_dtype, int flags, const void* __restrict__ x, int64_t n,
    const float* __restrict__ pi, const float* __restrict__ bounds,
    const float* __restrict__ cents, int bits, const float* __restrict__ signs,
    uint8_t* __restrict__ codes, uint8_t* __restrict__ qjl, float* __restrict__ norms,
    int64_t out_seq, int64_t out_gstride, const uint8_t* __restrict__ sel,
    const float* __restrict__ alt_bounds, const float* __restrict__ alt_cents, int alt_bits) {
  __shared__ float piT[D * D];          // piT[k * D + j] = Pi[j][k]
  __shared__ float us[D * kRows];       // us[k * kRows + r] = u_r[k]
  __shared__ uint8_t cs[kRows * D];     // codes of the tile
  __shared__ uint8_t qs[kRows * D];     // QJL bits of the tile
  __shared__ float nrm[kRows];
  __shared__ float part[2][kRows];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const bool pre_rot = (flags & QKV_FLAG_PRE_ROTATED) != 0;
  const bool packed = (flags & QKV_FLAG_PACKED) != 0;
  // mixed precision: coordinates with sel[j] != 0 use the alternate codebook
  const bool alt = sel != nullptr && tid < D && sel[tid] != 0;
  const int nb = (1 << (alt ? alt_bits : bits)) - 1;
  const float* tb = alt ? alt_bounds : bounds;
  const float* cb = alt ? alt_cents : cents;

  if (!pre_rot) {
    for (int i = tid; i < D * D; i += kThreads) {
      const int j = i / D, k = i - j * D;
      piT[k * D + j] = pi[i];
    }
  }
  float t[15], c[16];
#pragma unroll
  for (int i = 0; i < 15; ++i) t[i] = i < nb ? tb[i] : 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) c[i] = i <= nb ? cb[i] : 0.f;
  const float sj = (mode == QKV_MODE_IP && tid < D) ? signs[tid] : 1.f;
  const int64_t pb = packed ? qkv_row_bytes(D, bits) : D;
  const int64_t pq = packed ? qkv_row_bytes(D, 1) : D;
  __syncthreads();

  for (int64_t r0 = int64_t(blockIdx.x) * kRows; r0 < n; r0 += int64_t(gridDim.x) * kRows) {
    const int nr = static_cast<int>(min<int64_t>(kRows, n - r0));
    float y[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r)
      y[r] = (tid < D && r < nr) ? qkv_load(x, (r0 + r) * D + tid, in_dtype) : 0.f;

    if (!pre_rot) {
      // norms (wave tree + 2-wave combine)
#pragma unroll
      for (int r = 0; r < kRows; ++r) {
        const float s = qkv_wave_sum(y[r] * y[r]);
        if (lane == 0) part[wave][r] = s;
      }
      __syncthreads();
      if (tid < kRows) nrm[tid] = fmaxf(sqrtf(part[0][tid] + part[1][tid]), 1e-8f);
      __syncthreads();
      if (tid < D) {
#pragma unroll
        for (int r = 0; r < kRows; ++r) us[tid * kRows + r] = y[r] / nrm[r];
      }
      __syncthreads();
#pragma unroll
      for (int r = 0; r < kRows; ++r) y[r] = 0.f;
      if (tid < D) {
        for (int k = 0; k < D; ++k) {
          const float p = piT[k * D + tid];
#pragma unroll
          for (int r = 0; r < kRows; ++r) y[r] = fmaf(us[k * kRows + r], p, y[r]);
        }
      }
    }

    if (tid < D) {
#pragma unroll
      for (int r = 0; r < kRows; ++r) {
        int code = 0;
#pragma unroll
        for (int i = 0; i < 15; ++i) code += (i < nb && y[r] > t[i]) ? 1 : 0;
        cs[r * D + tid] = static_cast<uint8_t>(code);
        if (mode == QKV_MODE_IP) {
          float cv = c[0];
#pragma unroll
          for (int i = 1; i < 16; ++i) cv = (code == i) ? c[i] : cv;
          const float res = y[r] - cv;
          qs[r * D + tid] = (res * sj >= 0.f) ? 1 : 0;
        }
      }
    }
    __syncthreads();

    // stores (packed bytes or raw codes), grouped-row addressed
    for (int i = tid; i < nr * pb; i += kThreads) {
      const int r = i / static_cast<int>(pb);
      const int b = i - r * static_cast<int>(pb);
      const int64_t row = qkv_grouped_row(r0 + r, out_seq, out_gstride);
      codes[row * pb + b] = packed ? qkv_pack_byte(cs + r * D, b, D, bits) : cs[r * D + b];
    }
    if (mode == QKV_MODE_IP) {
      for (int i = tid; i < nr * pq; i += kThreads) {
        const int r = i / static_cast<int>(pq);
        const int b = i - r * static_cast<int>(pq);
        const int64_t row = qkv_grouped_row(r0 + r, out_seq, out_gstride);
        qjl[row * pq + b] = packed ? qkv_pack_byte(qs + r * D, b, D, 1) : qs[r * D + b];
      }
    }
    if (!pre_rot && tid < nr) norms[qkv_grouped_row(r0 + tid, out_seq, out_gstride)] = nrm[tid];
    __syncthreads();
  }
}

template <int D>
__global__ __launch_bounds__(kThreads) void decompress_generic(
    int mode, int fmt, const uint8_t* __restrict__ codes, const uint8_t* __restrict__ qjl,
    const float* __restrict__ norms, int64_t n, int bits, const float* __restrict__ pi,
    const float* __restrict__ cents, const float* __restrict__ signs, float qjl_scale,
    int64_t in_seq, int64_t in_gstride, void* __restrict__ out, int out_dtype,
    const uint8_t* __restrict__ sel, const float* __restrict__ alt_cents, int alt_bits) {
  __shared__ float pis[D * D];      // Pi row-major
  __shared__ float cs[D * kRows];   // cs[k * kRows + r] = rotated-domain value
  __shared__ float ns[kRows];
  __shared__ float cl[2][16];       // centroid tables (codes are masked to 4 bits)
  const int tid = threadIdx.x;
  for (int i = tid; i < D * D; i += kThreads) pis[i] = pi[i];
  if (tid < 16) cl[0][tid] = tid < (1 << bits) ? cents[tid] : 0.f;
  if (tid < 16 && sel) cl[1][tid] = tid < (1 << alt_bits) ? alt_cents[tid] : 0.f;
  // mixed precision: coordinates with sel[j] != 0 use the alternate codebook
  const int tsel = (sel != nullptr && tid < D && sel[tid] != 0) ? 1 : 0;
  const int cb = fmt == QKV_FMT_PACKED ? bits : 8;
  const int qb = fmt == QKV_FMT_PACKED ? 1 : 8;
  const int64_t pb = fmt == QKV_FMT_PACKED ? qkv_row_bytes(D, bits)
                   : fmt == QKV_FMT_KPLANES ? int64_t(bits + 1) * D / 8 : D;
  const int64_t pq = fmt == QKV_FMT_PACKED ? qkv_row_bytes(D, 1) : D;
  const float qs = (mode == QKV_MODE_IP && tid < D) ? qjl_scale * signs[tid] : 0.f;
  __syncthreads();

  for (int64_t r0 = int64_t(blockIdx.x) * kRows; r0 < n; r0 += int64_t(gridDim.x) * kRows) {
    const int nr = static_cast<int>(min<int64_t>(kRows, n - r0));
    if (tid < D) {
#pragma unroll
      for (int r = 0; r < kRows; ++r) {
        float v = 0.f;
        if (r < nr) {
          uint32_t code, bit = 0;
          if (fmt == QKV_FMT_VTILES) {
            const int64_t g = (r0 + r) / in_seq, t = (r0 + r) - g * in_seq;
            const uint32_t* w = reinterpret_cast<const uint32_t*>(codes) +
                                ((g * in_gstride + (t >> 5)) * bits) * D + tid;
            code = 0;
            for (int k = 0; k < bits; ++k) code |= ((w[k * D] >> (t & 31)) & 1u) << k;
          } else {
            const int64_t row = qkv_grouped_row(r0 + r, in_seq, in_gstride);
            if (fmt == QKV_FMT_KPLANES) {
              const uint8_t* kr = codes + row * pb;
              code = 0;
              for (int p = 0; p < bits; ++p)
                code |= ((kr[p * (D / 8) + (tid >> 3)] >> (tid & 7)) & 1u) << p;
              bit = (kr[bits * (D / 8) + (tid >> 3)] >> (tid & 7)) & 1u;
            } else {
              code = qkv_get_code(codes + row * pb, tid, cb);
              if (mode == QKV_MODE_IP) bit = qkv_get_code(qjl + row * pq, tid, qb);
            }
          }
          v = cl[tsel][code & 15u];
          if (mode == QKV_MODE_IP) v += qs * (bit ? 1.f : -1.f);
        }
        cs[tid * kRows + r] = v;
      }
    }
    if (tid < nr) {
      int64_t nrow;
      if (fmt == QKV_FMT_VTILES) {
        const int64_t g = (r0 + tid) / in_seq;
        nrow = g * in_gstride * 32 + ((r0 + tid) - g * in_seq);
      } else {
        nrow = qkv_grouped_row(r0 + tid, in_seq, in_gstride);
      }
      ns[tid] = norms[nrow];
    }
    __syncthreads();
    if (tid < D) {
      float acc[kRows];
#pragma unroll
      for (int r = 0; r < kRows; ++r) acc[r] = 0.f;
      for (int k = 0; k < D; ++k) {
        const float p = pis[k * D + tid];
#pragma unroll
        for (int r = 0; r < kRows; ++r) acc[r] = fmaf(cs[k * kRows + r], p, acc[r]);
      }
#pragma unroll
      for (int r = 0; r < kRows; ++r)
        if (r < nr) qkv_store(out, (r0 + r) * D + tid, acc[r] * ns[r], out_dtype);
    }
    __syncthreads();
  }
}

int grid_rows(int64_t n) {
  int64_t g = (n + kRows - 1) / kRows;
  const int64_t cap = int64_t(qkv_num_cus()) * 2;
  if (g > cap) g = cap;
  return static_cast<int>(g < 1 ? 1 : g);
}

}  // namespace

static int compress_impl(int32_t mode, int32_t in_dtype, int32_t flags, const void* x,
                         int64_t n, int32_t d, const float* pi, const float* boundaries,
                         const float* centroids, int32_t bits, const float* signs,
                         uint8_t* codes, uint8_t* qjl, float* norms, int64_t out_seq,
                         int64_t out_group_stride, const uint8_t* sel, const float* alt_bounds,
                         const float* alt_cents, int32_t alt_bits, void* stream) {
  QKV_REQUIRE(mode == QKV_MODE_MSE || mode == QKV_MODE_IP, "unknown mode %d", mode);
  QKV_REQUIRE(qkv_dtype_ok(in_dtype), "unsupported input dtype %d", in_dtype);
  QKV_REQUIRE(qkv_bits_ok(bits), "bits must be in {1, 2, 3, 4}, got %d", bits);
  if (!qkv_d_ok(d)) {
    qkv_set_error("head_dim %d unsupported (64, 96 or 128)", d);
    return QKV_E_UNSUPPORTED;
  }
  QKV_REQUIRE(n >= 0, "negative row count");
  if (n == 0) return QKV_OK;
  const bool pre_rot = (flags & QKV_FLAG_PRE_ROTATED) != 0;
  QKV_REQUIRE(x && boundaries && centroids && codes, "null pointer");
  QKV_REQUIRE(pre_rot || (pi && norms), "null pointer (pi / norms)");
  QKV_REQUIRE(mode != QKV_MODE_IP || (signs && qjl), "null pointer (signs / qjl)");
  QKV_REQUIRE(out_seq > 0 && out_group_stride >= out_seq, "bad grouped-row layout");
  auto s = static_cast<hipStream_t>(stream);
  switch (d) {
#define QKV_CASE(DD)                                                                          \
  case DD:                                                                                    \
    hipLaunchKernelGGL(compress_generic<DD>, dim3(grid_rows(n)), dim3(kThreads), 0, s, mode, \
                       in_dtype, flags, x, n, pi, boundaries, centroids, bits, signs, codes,  \
                       qjl, norms, out_seq, out_group_stride, sel, alt_bounds, alt_cents,     \
                       alt_bits);                                                             \
    break;
    QKV_CASE(64)
    QKV_CASE(96)
    QKV_CASE(128)
#undef QKV_CASE
  }
  QKV_LAUNCHED();
  return QKV_OK;
}

static int decompress_impl(int32_t mode, int32_t fmt, const uint8_t* codes,
                           const uint8_t* qjl, const float* norms, int64_t n, int32_t d,
                           int32_t bits, const float* pi, const float* centroids,
                           const float* signs, float qjl_scale, int64_t in_seq,
                           int64_t in_group_stride, void* out, int32_t out_dtype,
                           const uint8_t* sel, const float* alt_cents, int32_t alt_bits,
                           void* stream) {
  QKV_REQUIRE(mode == QKV_MODE_MSE || mode == QKV_MODE_IP, "unknown mode %d", mode);
  QKV_REQUIRE(qkv_dtype_ok(out_dtype), "unsupported output dtype %d", out_dtype);
  QKV_REQUIRE(qkv_bits_ok(bits), "bits must be in {1, 2, 3, 4}, got %d", bits);
  if (!qkv_d_ok(d)) {
    qkv_set_error("head_dim %d unsupported (64, 96 or 128)", d);
    return QKV_E_UNSUPPORTED;
  }
  QKV_REQUIRE(n >= 0, "negative row count");
  if (n == 0) return QKV_OK;
  QKV_REQUIRE(fmt >= QKV_FMT_UNPACKED && fmt <= QKV_FMT_VTILES, "unknown code format %d", fmt);
  QKV_REQUIRE(codes && norms && pi && centroids && out, "null pointer");
  QKV_REQUIRE(mode != QKV_MODE_IP || signs, "null pointer (signs)");
  QKV_REQUIRE(mode != QKV_MODE_IP || qjl || fmt == QKV_FMT_KPLANES, "null pointer (qjl)");
  QKV_REQUIRE(mode != QKV_MODE_IP || fmt != QKV_FMT_VTILES, "V tiles carry no QJL plane");
  if (fmt == QKV_FMT_VTILES)
    QKV_REQUIRE(in_seq > 0 && in_group_stride * 32 >= in_seq, "bad V tile layout");
  else
    QKV_REQUIRE(in_seq > 0 && in_group_stride >= in_seq, "bad grouped-row layout");
  auto s = static_cast<hipStream_t>(stream);
  const QkvDecompressArgs args{mode,      fmt,     codes,   qjl,       norms,    n,
                               d,         bits,    pi,      centroids, signs,    qjl_scale,
                               in_seq,    in_group_stride,  out,       out_dtype, sel,
                               alt_cents, alt_bits};
  if (qkv_decompress_mfma_ok(args)) {
    qkv_decompress_mfma(args, s);
    QKV_LAUNCHED();
    return QKV_OK;
  }
  switch (d) {
#define QKV_CASE(DD)                                                                         \
  case DD:                                                                                   \
    hipLaunchKernelGGL(decompress_generic<DD>, dim3(grid_rows(n)), dim3(kThreads), 0, s,    \
                       mode, fmt, codes, qjl, norms, n, bits, pi, centroids, signs,          \
                       qjl_scale, in_seq, in_group_stride, out, out_dtype, sel, alt_cents,   \
                       alt_bits);                                                            \
    break;
    QKV_CASE(64)
    QKV_CASE(96)
    QKV_CASE(128)
#undef QKV_CASE
  }
  QKV_LAUNCHED();
  return QKV_OK;
}

extern "C" int qkv_compress(int32_t mode, int32_t in_dtype, int32_t flags, const void* x,
                            int64_t n, int32_t d, const float* pi, const float* boundaries,
                            const float* centroids, int32_t bits, const float* signs,
                            uint8_t* codes, uint8_t* qjl, float* norms, int64_t out_seq,
                            int64_t out_group_stride, void* stream) {
  return compress_impl(mode, in_dtype, flags, x, n, d, pi, boundaries, centroids, bits, signs,
                       codes, qjl, norms, out_seq, out_group_stride, nullptr, nullptr, nullptr,
                       0, stream);
}

extern "C" int qkv_decompress(int32_t mode, int32_t fmt, const uint8_t* codes,
                              const uint8_t* qjl, const float* norms, int64_t n, int32_t d,
                              int32_t bits, const float* pi, const float* centroids,
                              const float* signs, float qjl_scale, int64_t in_seq,
                              int64_t in_group_stride, void* out, int32_t out_dtype,
                              void* stream) {
  return decompress_impl(mode, fmt, codes, qjl, norms, n, d, bits, pi, centroids, signs,
                         qjl_scale, in_seq, in_group_stride, out, out_dtype, nullptr, nullptr,
                         0, stream);
}

extern "C" int qkv_compress_mixed(int32_t mode, int32_t in_dtype, int32_t flags, const void* x,
                                  int64_t n, int32_t d, const float* pi,
                                  const uint8_t* outlier_mask, const float* out_bounds,
                                  const float* out_cents, int32_t out_bits,
                                  const float* reg_bounds, const float* reg_cents,
                                  int32_t reg_bits, const float* signs, uint8_t* codes,
                                  uint8_t* qjl, float* norms, int64_t out_seq,
                                  int64_t out_group_stride, void* stream) {
  QKV_REQUIRE((flags & QKV_FLAG_PACKED) == 0, "mixed-precision codes are stored unpacked");
  QKV_REQUIRE(outlier_mask && out_bounds && out_cents, "null pointer (outlier tables)");
  QKV_REQUIRE(qkv_bits_ok(out_bits), "outlier bits must be in {1, 2, 3, 4}, got %d", out_bits);
  return compress_impl(mode, in_dtype, flags, x, n, d, pi, reg_bounds, reg_cents, reg_bits,
                       signs, codes, qjl, norms, out_seq, out_group_stride, outlier_mask,
                       out_bounds, out_cents, out_bits, stream);
}

extern "C" int qkv_decompress_mixed(int32_t mode, const uint8_t* codes, const uint8_t* qjl,
                                    const float* norms, int64_t n, int32_t d,
                                    const uint8_t* outlier_mask, const float* out_cents,
                                    int32_t out_bits, const float* reg_cents, int32_t reg_bits,
                                    const float* pi, const float* signs, float qjl_scale,
                                    int64_t in_seq, int64_t in_group_stride, void* out,
                                    int32_t out_dtype, void* stream) {
  QKV_REQUIRE(outlier_mask && out_cents, "null pointer (outlier tables)");
  QKV_REQUIRE(qkv_bits_ok(out_bits), "outlier bits must be in {1, 2, 3, 4}, got %d", out_bits);
  return decompress_impl(mode, QKV_FMT_UNPACKED, codes, qjl, norms, n, d, reg_bits, pi,
                         reg_cents, signs, qjl_scale, in_seq, in_group_stride, out, out_dtype,
                         outlier_mask, out_cents, out_bits, stream);
}
