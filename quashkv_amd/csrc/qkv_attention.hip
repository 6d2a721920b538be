// Split-K decode attention over the compressed cache (generic VALU path).
//
// score(q, t) = n_k,t * (sum_j q~_j c_k[code_tj] + alpha sum_j |q~_j| S_j (2b_tj - 1)) * scale
// out         = (sum_t softmax(score)_t n_v,t c_v[vcode_t]) Pi
// with q~ = q Pi^T.  Reference: quashkv/engine.py:204-299 (naive) and
// quashkv/triton_kernels/attention.py:55-149 (online softmax).  Unlike the
// reference, values are accumulated in the ROTATED domain and un-rotated once
// per query row in the combine kernel (linearity of x -> x Pi).
//
// Kernels:
//   qrot_kernel    q~ and w = alpha |q~| S for every query row (once per call)
//   split_kernel   one workgroup per (split, kv-head x row-chunk, batch):
//                  online softmax over its token range, partial (m, l, O~)
//   combine_kernel merges the splits' partials (log-sum-exp), divides by
//                  max(l, 1e-8) and applies Pi once.
// GQA: query head h reads kv head h / G; the G*Q query rows of one kv head
// ("rows") share every K/V byte the workgroup streams.
#include <math.h>

#include "qkv_common.h"

namespace {

constexpr int kTile = 256;     // tokens per tile == threads per workgroup
constexpr int kMaxRows = 32;   // query rows per workgroup (row chunk)
constexpr int kRowBlk = 8;     // rows scored per pass over a key row

struct AttnWs {
  float* qw;      // [B][Hkv][R][2][D]   q~ then w
  float* part_o;  // [S][B][Hkv][R][D]   un-normalised rotated-domain outputs
  float* part_ml; // [S][B][Hkv][R][2]   running max, running sum
};

__host__ __device__ inline int64_t ws_qw_floats(int B, int Hkv, int R, int D) {
  return int64_t(B) * Hkv * R * 2 * D;
}
__host__ __device__ inline int64_t ws_po_floats(int S, int B, int Hkv, int R, int D) {
  return int64_t(S) * B * Hkv * R * D;
}
__host__ __device__ inline int64_t ws_ml_floats(int S, int B, int Hkv, int R) {
  return int64_t(S) * B * Hkv * R * 2;
}

// q~_j = sum_k q_k Pi[j][k];  w_j = alpha |q~_j| S_j.  One block per query row.
template <int D>
__global__ __launch_bounds__(128) void qrot_kernel(const void* __restrict__ q, int q_dtype,
                                                   const float* __restrict__ pi,
                                                   const float* __restrict__ signs, float alpha,
                                                   int Hq, int Hkv, int Q,
                                                   float* __restrict__ qw) {
  __shared__ float qs[D];
  const int row = blockIdx.x;  // (b, h, qi) flattened
  const int tid = threadIdx.x;
  if (tid < D) qs[tid] = qkv_load(q, int64_t(row) * D + tid, q_dtype);
  __syncthreads();
  if (tid >= D) return;
  const int qi = row % Q;
  const int h = (row / Q) % Hq;
  const int b = row / (Q * Hq);
  const int G = Hq / Hkv;
  const int hkv = h / G, g = h - hkv * G;
  const int R = G * Q;
  const int r = g * Q + qi;
  float acc = 0.f;
  const float* prow = pi + int64_t(tid) * D;
  for (int k = 0; k < D; ++k) acc = fmaf(qs[k], prow[k], acc);
  float* dst = qw + ((int64_t(b) * Hkv + hkv) * R + r) * 2 * D;
  dst[tid] = acc;
  dst[D + tid] = alpha * fabsf(acc) * signs[tid];
}

template <int D>
__global__ __launch_bounds__(kTile) void split_kernel(
    const float* __restrict__ qw, const uint8_t* __restrict__ kcodes,
    const uint8_t* __restrict__ kqjl, const float* __restrict__ knorm,
    const uint8_t* __restrict__ vcodes, const float* __restrict__ vnorm, int64_t t_stride,
    int64_t T, int Hkv, int R, int Q, int row_chunks, int kbits, int vbits, int packed,
    const float* __restrict__ kcent, const float* __restrict__ vcent, float scale, int causal,
    int64_t split_len, int n_splits, float* __restrict__ part_o, float* __restrict__ part_ml) {
  __shared__ float qs[kMaxRows][D];
  __shared__ float ws[kMaxRows][D];
  __shared__ float ps[kMaxRows][kTile];   // scores, then probabilities; reused at the end
  __shared__ float vn[kTile];
  __shared__ float red[kMaxRows][4];
  __shared__ float ms[kMaxRows], ls[kMaxRows], al[kMaxRows];
  __shared__ float kc[16], vc[16];

  const int split = blockIdx.x;
  const int hkv = blockIdx.y / row_chunks;
  const int chunk = blockIdx.y - hkv * row_chunks;
  const int b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r_begin = chunk * kMaxRows;
  const int nr = min(kMaxRows, R - r_begin);

  const int kb = packed ? kbits : 8, qb = packed ? 1 : 8, vb = packed ? vbits : 8;
  const int64_t pk = qkv_row_bytes(D, kb), pq = qkv_row_bytes(D, qb), pv = qkv_row_bytes(D, vb);
  const int64_t bh = int64_t(b) * Hkv + hkv;
  const uint8_t* kbase = kcodes + bh * t_stride * pk;
  const uint8_t* qbase = kqjl + bh * t_stride * pq;
  const uint8_t* vbase = vcodes + bh * t_stride * pv;
  const float* knb = knorm + bh * t_stride;
  const float* vnb = vnorm + bh * t_stride;

  const float* qsrc = qw + (bh * R + r_begin) * 2 * D;
  for (int i = tid; i < nr * D; i += kTile) {
    const int r = i / D, j = i - r * D;
    qs[r][j] = qsrc[r * 2 * D + j];
    ws[r][j] = qsrc[r * 2 * D + D + j];
  }
  if (tid < 16) {
    kc[tid] = tid < (1 << kbits) ? kcent[tid] : 0.f;
    vc[tid] = tid < (1 << vbits) ? vcent[tid] : 0.f;
  }
  if (tid < kMaxRows) {
    ms[tid] = -INFINITY;
    ls[tid] = 0.f;
  }

  const int64_t t_begin = int64_t(split) * split_len;
  const int64_t t_end = min<int64_t>(T, t_begin + split_len);

  // PV thread layout: coordinate j, token half hf of the tile
  const int pj = tid & 127, hf = tid >> 7;
  float acc[kMaxRows];
#pragma unroll
  for (int r = 0; r < kMaxRows; ++r) acc[r] = 0.f;
  __syncthreads();

  for (int64_t t0 = t_begin; t0 < t_end; t0 += kTile) {
    const int64_t t = t0 + tid;
    const bool valid = t < t_end;
    // ---- scores: one token per thread, rows in blocks of kRowBlk
    const uint8_t* krow = kbase + (valid ? t : t_begin) * pk;
    const uint8_t* qrow = qbase + (valid ? t : t_begin) * pq;
    const float kn = valid ? knb[t] * scale : 0.f;
    for (int rb = 0; rb < nr; rb += kRowBlk) {
      float s[kRowBlk];
#pragma unroll
      for (int i = 0; i < kRowBlk; ++i) s[i] = 0.f;
      for (int j = 0; j < D; ++j) {
        const float c = kc[qkv_get_code(krow, j, kb) & 15u];
        const float z = qkv_get_code(qrow, j, qb) ? 1.f : -1.f;
#pragma unroll
        for (int i = 0; i < kRowBlk; ++i) {
          const int r = min(rb + i, kMaxRows - 1);
          s[i] = fmaf(qs[r][j], c, s[i]);
          s[i] = fmaf(ws[r][j], z, s[i]);
        }
      }
#pragma unroll
      for (int i = 0; i < kRowBlk; ++i) {
        const int r = rb + i;
        if (r < nr) {
          float v = kn * s[i];
          if (!valid) v = -INFINITY;
          if (causal) {
            const int qi = (r_begin + r) % Q;
            if (t > T - Q + qi) v = -INFINITY;
          }
          ps[r][tid] = v;
        }
      }
    }
    vn[tid] = valid ? vnb[t] : 0.f;
    __syncthreads();

    // ---- tile max per row
    for (int r = 0; r < nr; ++r) {
      const float m = qkv_wave_max(ps[r][tid]);
      if (lane == 0) red[r][wave] = m;
    }
    __syncthreads();
    if (tid < nr) {
      const float tm = fmaxf(fmaxf(red[tid][0], red[tid][1]), fmaxf(red[tid][2], red[tid][3]));
      const float mo = ms[tid];
      const float mn = fmaxf(mo, tm);
      al[tid] = (mn == -INFINITY) ? 1.f : expf(mo - mn);
      ms[tid] = mn;
    }
    __syncthreads();
    // ---- probabilities and row sums
    for (int r = 0; r < nr; ++r) {
      const float mn = ms[r];
      const float p = (mn == -INFINITY) ? 0.f : expf(ps[r][tid] - mn);
      ps[r][tid] = p;
      const float sum = qkv_wave_sum(p);
      if (lane == 0) red[r][wave] = sum;
    }
    __syncthreads();
    if (tid < nr) ls[tid] = ls[tid] * al[tid] + (red[tid][0] + red[tid][1]) + (red[tid][2] + red[tid][3]);

    // ---- P V in the rotated domain
#pragma unroll
    for (int r = 0; r < kMaxRows; ++r) acc[r] *= (r < nr) ? al[r] : 1.f;
    if (pj < D) {
      const int tt0 = hf * (kTile / 2);
      for (int tt = tt0; tt < tt0 + kTile / 2; ++tt) {
        const int64_t tk = t0 + tt;
        if (tk >= t_end) break;
        const float v = vc[qkv_get_code(vbase + tk * pv, pj, vb) & 15u] * vn[tt];
#pragma unroll
        for (int r = 0; r < kMaxRows; ++r)
          if (r < nr) acc[r] = fmaf(ps[r][tt], v, acc[r]);
      }
    }
    __syncthreads();
  }

  // ---- reduce the two token halves and write the partials
  float* red_o = &ps[0][0];  // kMaxRows x 128 floats
  if (hf == 1 && pj < D) {
#pragma unroll
    for (int r = 0; r < kMaxRows; ++r)
      if (r < nr) red_o[r * 128 + pj] = acc[r];
  }
  __syncthreads();
  const int64_t base = ((int64_t(split) * gridDim.z + b) * Hkv + hkv) * R + r_begin;
  if (hf == 0 && pj < D) {
#pragma unroll
    for (int r = 0; r < kMaxRows; ++r)
      if (r < nr) part_o[(base + r) * D + pj] = acc[r] + red_o[r * 128 + pj];
  }
  if (tid < nr) {
    part_ml[(base + tid) * 2 + 0] = ms[tid];
    part_ml[(base + tid) * 2 + 1] = ls[tid];
  }
}

// One block per (b, hkv, r) query row: merge splits, normalise, un-rotate.
template <int D>
__global__ __launch_bounds__(128) void combine_kernel(const float* __restrict__ part_o,
                                                      const float* __restrict__ part_ml,
                                                      const float* __restrict__ pi, int n_splits,
                                                      int B, int Hkv, int R, int Q, int Hq,
                                                      void* __restrict__ out, int out_dtype) {
  __shared__ float o[D];
  __shared__ float wgt[1024];
  __shared__ float lsum;
  const int row = blockIdx.x;  // ((b * Hkv) + hkv) * R + r
  const int tid = threadIdx.x;
  const int64_t stride = int64_t(B) * Hkv * R;
  if (tid == 0) {
    float M = -INFINITY;
    for (int s = 0; s < n_splits; ++s) M = fmaxf(M, part_ml[(s * stride + row) * 2]);
    float L = 0.f;
    for (int s = 0; s < n_splits; ++s) {
      const float m = part_ml[(s * stride + row) * 2];
      const float w = (m == -INFINITY) ? 0.f : expf(m - M);
      wgt[s] = w;
      L = fmaf(w, part_ml[(s * stride + row) * 2 + 1], L);
    }
    lsum = fmaxf(L, 1e-8f);
  }
  __syncthreads();
  if (tid < D) {
    float a = 0.f;
    for (int s = 0; s < n_splits; ++s) a = fmaf(wgt[s], part_o[(s * stride + row) * D + tid], a);
    o[tid] = a / lsum;
  }
  __syncthreads();
  if (tid >= D) return;
  float acc = 0.f;
  for (int k = 0; k < D; ++k) acc = fmaf(o[k], pi[k * D + tid], acc);
  const int r = row % R;
  const int hkv = (row / R) % Hkv;
  const int b = row / (R * Hkv);
  const int G = Hq / Hkv;
  const int g = r / Q, qi = r - (r / Q) * Q;
  const int h = hkv * G + g;
  qkv_store(out, ((int64_t(b) * Hq + h) * Q + qi) * D + tid, acc, out_dtype);
}

}  // namespace

extern "C" int32_t qkv_attention_splits(int32_t B, int32_t Hq, int32_t Hkv, int32_t Q,
                                        int32_t d, int64_t T) {
  (void)d;
  if (B <= 0 || Hkv <= 0 || Hq <= 0 || Q <= 0 || T <= 0) return 1;
  const int R = (Hq / Hkv) * Q;
  const int chunks = (R + kMaxRows - 1) / kMaxRows;
  const int64_t groups = int64_t(B) * Hkv * chunks;
  const int64_t target = int64_t(qkv_num_cus()) * 4;
  int64_t s = (target + groups - 1) / groups;
  const int64_t max_s = (T + kTile - 1) / kTile;
  if (s > max_s) s = max_s;
  if (s > 1024) s = 1024;
  if (s < 1) s = 1;
  return static_cast<int32_t>(s);
}

extern "C" int64_t qkv_attention_workspace_bytes(int32_t B, int32_t Hq, int32_t Hkv, int32_t Q,
                                                 int32_t d, int32_t n_splits) {
  if (B <= 0 || Hkv <= 0 || Hq <= 0 || Q <= 0 || d <= 0 || n_splits <= 0) return -1;
  const int R = (Hq / Hkv) * Q;
  return 4 * (ws_qw_floats(B, Hkv, R, d) + ws_po_floats(n_splits, B, Hkv, R, d) +
              ws_ml_floats(n_splits, B, Hkv, R));
}

static int validate_common(int32_t B, int32_t Hq, int32_t Hkv, int32_t Q, int32_t d,
                           int32_t n_splits, const void* workspace, int64_t ws_bytes) {
  if (!qkv_d_ok(d)) {
    qkv_set_error("head_dim %d unsupported (64, 96 or 128)", d);
    return QKV_E_UNSUPPORTED;
  }
  QKV_REQUIRE(B > 0 && Hq > 0 && Hkv > 0 && Q > 0, "invalid shape");
  QKV_REQUIRE(Hq % Hkv == 0, "query heads (%d) must be a multiple of kv heads (%d)", Hq, Hkv);
  QKV_REQUIRE(B <= 65535, "batch too large");
  QKV_REQUIRE(n_splits >= 1 && n_splits <= 1024, "n_splits %d out of range", n_splits);
  const int R = (Hq / Hkv) * Q;
  const int chunks = (R + kMaxRows - 1) / kMaxRows;
  QKV_REQUIRE(int64_t(Hkv) * chunks <= 65535, "too many kv heads x row chunks");
  QKV_REQUIRE(workspace != nullptr, "null workspace");
  QKV_REQUIRE(qkv_aligned(workspace, 16), "workspace must be 16-byte aligned");
  const int64_t need = qkv_attention_workspace_bytes(B, Hq, Hkv, Q, d, n_splits);
  QKV_REQUIRE(ws_bytes >= need, "workspace too small: %lld < %lld", (long long)ws_bytes,
              (long long)need);
  return QKV_OK;
}

extern "C" int qkv_attention_prepare(const void* q, int32_t q_dtype, int32_t B, int32_t Hq,
                                     int32_t Hkv, int32_t Q, int32_t d, const float* pi,
                                     const float* signs, float qjl_scale, void* workspace,
                                     int64_t ws_bytes, int32_t n_splits, void* stream) {
  QKV_REQUIRE(qkv_dtype_ok(q_dtype), "unsupported query dtype %d", q_dtype);
  int st = validate_common(B, Hq, Hkv, Q, d, n_splits, workspace, ws_bytes);
  if (st != QKV_OK) return st;
  QKV_REQUIRE(q && pi && signs, "null pointer");
  float* qw = static_cast<float*>(workspace);
  auto s = static_cast<hipStream_t>(stream);
  switch (d) {
#define QKV_CASE(DD)                                                                        \
  case DD:                                                                                  \
    hipLaunchKernelGGL(qrot_kernel<DD>, dim3(B * Hq * Q), dim3(128), 0, s, q, q_dtype, pi, \
                       signs, qjl_scale, Hq, Hkv, Q, qw);                                   \
    break;
    QKV_CASE(64)
    QKV_CASE(96)
    QKV_CASE(128)
#undef QKV_CASE
  }
  QKV_LAUNCHED();
  return QKV_OK;
}

extern "C" int qkv_attention_partial(const uint8_t* kcodes, const uint8_t* kqjl,
                                     const float* knorm, const uint8_t* vcodes,
                                     const float* vnorm, int64_t t_stride, int64_t T, int32_t B,
                                     int32_t Hq, int32_t Hkv, int32_t Q, int32_t d,
                                     int32_t kbits, int32_t vbits, int32_t packed,
                                     const float* kcent, const float* vcent, float scale,
                                     int32_t causal, void* workspace, int64_t ws_bytes,
                                     int32_t n_splits, void* stream) {
  QKV_REQUIRE(qkv_bits_ok(kbits) && qkv_bits_ok(vbits), "bits must be in {1, 2, 3, 4}");
  QKV_REQUIRE(T > 0, "No compressed KV blocks in cache. Call append() first.");
  QKV_REQUIRE(t_stride >= T, "t_stride %lld < T %lld", (long long)t_stride, (long long)T);
  int st = validate_common(B, Hq, Hkv, Q, d, n_splits, workspace, ws_bytes);
  if (st != QKV_OK) return st;
  QKV_REQUIRE(kcodes && kqjl && knorm && vcodes && vnorm && kcent && vcent, "null pointer");
  const int R = (Hq / Hkv) * Q;
  const int chunks = (R + kMaxRows - 1) / kMaxRows;
  const int64_t split_len = ((T + n_splits - 1) / n_splits + kTile - 1) / kTile * kTile;
  float* qw = static_cast<float*>(workspace);
  float* po = qw + ws_qw_floats(B, Hkv, R, d);
  float* pml = po + ws_po_floats(n_splits, B, Hkv, R, d);
  auto s = static_cast<hipStream_t>(stream);
  switch (d) {
#define QKV_CASE(DD)                                                                           \
  case DD:                                                                                     \
    hipLaunchKernelGGL(split_kernel<DD>, dim3(n_splits, Hkv * chunks, B), dim3(kTile), 0, s,  \
                       qw, kcodes, kqjl, knorm, vcodes, vnorm, t_stride, T, Hkv, R, Q, chunks, \
                       kbits, vbits, packed, kcent, vcent, scale, causal, split_len, n_splits, \
                       po, pml);                                                               \
    break;
    QKV_CASE(64)
    QKV_CASE(96)
    QKV_CASE(128)
#undef QKV_CASE
  }
  QKV_LAUNCHED();
  return QKV_OK;
}

extern "C" int qkv_attention_combine(int32_t B, int32_t Hq, int32_t Hkv, int32_t Q, int32_t d,
                                     const float* pi, void* out, int32_t out_dtype,
                                     void* workspace, int64_t ws_bytes, int32_t n_splits,
                                     void* stream) {
  QKV_REQUIRE(qkv_dtype_ok(out_dtype), "unsupported output dtype %d", out_dtype);
  int st = validate_common(B, Hq, Hkv, Q, d, n_splits, workspace, ws_bytes);
  if (st != QKV_OK) return st;
  QKV_REQUIRE(pi && out, "null pointer");
  const int R = (Hq / Hkv) * Q;
  float* qw = static_cast<float*>(workspace);
  float* po = qw + ws_qw_floats(B, Hkv, R, d);
  float* pml = po + ws_po_floats(n_splits, B, Hkv, R, d);
  auto s = static_cast<hipStream_t>(stream);
  switch (d) {
#define QKV_CASE(DD)                                                                         \
  case DD:                                                                                   \
    hipLaunchKernelGGL(combine_kernel<DD>, dim3(B * Hkv * R), dim3(128), 0, s, po, pml, pi, \
                       n_splits, B, Hkv, R, Q, Hq, out, out_dtype);                          \
    break;
    QKV_CASE(64)
    QKV_CASE(96)
    QKV_CASE(128)
#undef QKV_CASE
  }
  QKV_LAUNCHED();
  return QKV_OK;
}

extern "C" int qkv_decode_attention(const void* q, int32_t q_dtype, const uint8_t* kcodes,
                                    const uint8_t* kqjl, const float* knorm,
                                    const uint8_t* vcodes, const float* vnorm, int64_t t_stride,
                                    int64_t T, int32_t B, int32_t Hq, int32_t Hkv, int32_t Q,
                                    int32_t d, int32_t kbits, int32_t vbits, int32_t packed,
                                    const float* pi, const float* kcent, const float* vcent,
                                    const float* signs, float qjl_scale, float scale,
                                    int32_t causal, void* out, int32_t out_dtype,
                                    void* workspace, int64_t ws_bytes, int32_t n_splits,
                                    void* stream) {
  // validate everything before the first launch
  QKV_REQUIRE(qkv_dtype_ok(q_dtype) && qkv_dtype_ok(out_dtype), "unsupported dtype");
  QKV_REQUIRE(qkv_bits_ok(kbits) && qkv_bits_ok(vbits), "bits must be in {1, 2, 3, 4}");
  QKV_REQUIRE(T > 0, "No compressed KV blocks in cache. Call append() first.");
  QKV_REQUIRE(t_stride >= T, "t_stride %lld < T %lld", (long long)t_stride, (long long)T);
  int st = validate_common(B, Hq, Hkv, Q, d, n_splits, workspace, ws_bytes);
  if (st != QKV_OK) return st;
  QKV_REQUIRE(q && kcodes && kqjl && knorm && vcodes && vnorm && pi && kcent && vcent && signs &&
                  out,
              "null pointer");
  st = qkv_attention_prepare(q, q_dtype, B, Hq, Hkv, Q, d, pi, signs, qjl_scale, workspace,
                             ws_bytes, n_splits, stream);
  if (st != QKV_OK) return st;
  st = qkv_attention_partial(kcodes, kqjl, knorm, vcodes, vnorm, t_stride, T, B, Hq, Hkv, Q, d,
                             kbits, vbits, packed, kcent, vcent, scale, causal, workspace,
                             ws_bytes, n_splits, stream);
  if (st != QKV_OK) return st;
  return qkv_attention_combine(B, Hq, Hkv, Q, d, pi, out, out_dtype, workspace, ws_bytes,
                               n_splits, stream);
}
