// One launch for the key and the value half of a store append: the workgroups
// of the key kernel body (append_k_run, or append_kmix_run for mixed-precision
// keys) and of append_v_run (qkv_append_dev.h) in one grid, so that a small
// append -- one decode token per layer, a short chunk -- runs both halves side
// by side on different CUs and pays one launch instead of two.  Instantiated
// for value bits = key MSE bits + 1 (key_bits == value_bits in the reference's
// QuashKVEngine(key_bits, value_bits), quashkv/engine.py:77-101, whose default
// is 3 / 3) and, with mixed-precision keys, value bits 2..4; other
// combinations launch the two kernels.

#include "qkv_append_dev.h"

namespace {

// grid = (key workgroups + value workgroups, layers): x < kblocks runs the key
// append of layer blockIdx.y over kblocks workgroups, the rest its value
// append; each wave takes one tile or, nsplit = d / 32, one 32-coordinate
// block of one tile (the launchers check that the grid covers that), and its
// rows load while Pi is staged.
template <int MB, int VB, int XT, int D>
__global__ __launch_bounds__(kThreads, 4) void append_kv_layers(
    AppendLayers ak, AppendLayers av, int kblocks, int64_t S, int64_t ktpg, int64_t kntiles,
    int64_t vtpg, int64_t vntiles, Half fine, Half bnd, int64_t t_stride, int64_t t0,
    int nsplit) {
  __shared__ uint4 frag[frag_n<D>()];         // the running half's Pi fragments
  __shared__ float4 inv_s[kWaves][kTok / 4];  // value half: 1 / norm of each wave's tokens
  const int l = blockIdx.y, b = blockIdx.x;
  if (b < kblocks)
    append_k_run<MB, XT, D, false, false, true>(ak.x[l], nullptr, S, ktpg, kntiles, ak.pi[l],
                                          ak.signs[l], fine, static_cast<uint8_t*>(ak.st[l]),
                                          ak.nrm[l], t_stride, t0, QkvPages{}, frag, b,
                                          kblocks, nsplit);
  else
    append_v_run<VB, XT, D, false, false, true>(av.x[l], nullptr, S, vtpg, vntiles, av.pi[l], bnd,
                                          static_cast<uint32_t*>(av.st[l]), av.nrm[l], t_stride,
                                          t0, QkvPages{}, frag, inv_s, b - kblocks,
                                          static_cast<int>(gridDim.x) - kblocks, nsplit);
}

// The same over a paged store (two workgroups per CU, as the paged kernels).
template <int MB, int VB, int XT, int D>
__global__ __launch_bounds__(kThreads, 2) void append_kv_paged(
    const void* __restrict__ keys, const void* __restrict__ values, int kblocks, int64_t S,
    int64_t ktpg, int64_t kntiles, int64_t vtpg, int64_t vntiles, const float* __restrict__ kpi,
    const float* __restrict__ signs, const float* __restrict__ vpi, Half fine, Half bnd,
    uint8_t* __restrict__ kpool, float* __restrict__ knorm, uint32_t* __restrict__ vpool,
    float* __restrict__ vnorm, int64_t t_stride, int64_t t0, QkvPages pg, int nsplit) {
  __shared__ uint4 frag[frag_n<D>()];
  __shared__ float4 inv_s[kWaves][kTok / 4];
  const int b = blockIdx.x;
  if (b < kblocks)
    append_k_run<MB, XT, D, true, false, true>(keys, nullptr, S, ktpg, kntiles, kpi, signs, fine,
                                               kpool, knorm, t_stride, t0, pg, frag, b,
                                               kblocks, nsplit);
  else
    append_v_run<VB, XT, D, true, false, true>(values, nullptr, S, vtpg, vntiles, vpi, bnd, vpool,
                                               vnorm, t_stride, t0, pg, frag, inv_s, b - kblocks,
                                               static_cast<int>(gridDim.x) - kblocks, nsplit);
}

// Mixed-precision keys and their values: x < kblocks runs append_kmix_run over
// kblocks workgroups, the rest append_v_run.
template <int NO, bool IPM, int VB, int XT>
__global__ __launch_bounds__(kThreads, 2) void append_kmixv(
    const void* __restrict__ keys, const void* __restrict__ values, int kblocks, int64_t S,
    int64_t ktpg, int64_t kntiles, int64_t vtpg, int64_t vntiles,
    const float* __restrict__ pi_perm, const float* __restrict__ signs_perm, Half po, Half pr,
    uint8_t* __restrict__ kst, float* __restrict__ knorm, const float* __restrict__ vpi, Half bnd,
    uint32_t* __restrict__ vst, float* __restrict__ vnorm, int64_t t_stride, int64_t t0,
    int nsplit) {
  __shared__ uint4 frag[kFragN];
  __shared__ float4 inv_s[kWaves][kTok / 4];
  const int b = blockIdx.x;
  if (b < kblocks)
    append_kmix_run<NO, XT, false, IPM, true>(keys, nullptr, S, ktpg, kntiles, pi_perm, signs_perm, po,
                                        pr, kst, knorm, t_stride, t0, frag, b, kblocks, nsplit);
  else
    append_v_run<VB, XT, kD, false, false, true>(values, nullptr, S, vtpg, vntiles, vpi, bnd, vst,
                                           vnorm, t_stride, t0, QkvPages{}, frag, inv_s,
                                           b - kblocks, static_cast<int>(gridDim.x) - kblocks,
                                           nsplit);
}

}  // namespace

namespace qkv_app {

bool launch_append_kmixv(int n_out, bool ipm, int vbits, int xt, const void* keys,
                         const void* values, int kblocks, int vblocks, int64_t S, int64_t ktpg,
                         int64_t kntiles, int64_t vtpg, int64_t vntiles, const float* pi_perm,
                         const float* signs_perm, Half po, Half pr, uint8_t* kst, float* knorm,
                         const float* vpi, Half bnd, uint32_t* vst, float* vnorm,
                         int64_t t_stride, int64_t t0, int nsplit, hipStream_t s) {
  if ((n_out != 32 && n_out != 64) || vbits < 2 || vbits > 4 || xt < 0 || xt > 2) return false;
  // the kernel bodies run one tile (nsplit = 4: one slot block of one tile) per wave
  if ((nsplit != 1 && nsplit != 4) || kblocks < one_blocks(kntiles, nsplit) ||
      vblocks < one_blocks(vntiles, nsplit))
    return false;
  const dim3 grid(kblocks + vblocks);
#define QKV_KMV(NOV, IP, VB, F)                                                                 \
  hipLaunchKernelGGL((append_kmixv<NOV, IP, VB, F>), grid, dim3(kThreads), 0, s, keys, values,  \
                     kblocks, S, ktpg, kntiles, vtpg, vntiles, pi_perm, signs_perm, po, pr, kst, \
                     knorm, vpi, bnd, vst, vnorm, t_stride, t0, nsplit)
#define QKV_KMV_F(NOV, IP, VB)        \
  switch (xt) {                      \
    case 0: QKV_KMV(NOV, IP, VB, 0); break; \
    case 1: QKV_KMV(NOV, IP, VB, 1); break; \
    default: QKV_KMV(NOV, IP, VB, 2); break; \
  }
#define QKV_KMV_V(NOV, IP)               \
  switch (vbits) {                      \
    case 2: QKV_KMV_F(NOV, IP, 2); break; \
    case 3: QKV_KMV_F(NOV, IP, 3); break; \
    default: QKV_KMV_F(NOV, IP, 4); break; \
  }
  if (n_out == 32) {
    if (ipm) {
      QKV_KMV_V(32, true)
    } else {
      QKV_KMV_V(32, false)
    }
  } else {
    if (ipm) {
      QKV_KMV_V(64, true)
    } else {
      QKV_KMV_V(64, false)
    }
  }
#undef QKV_KMV_V
#undef QKV_KMV_F
#undef QKV_KMV
  return true;
}

bool launch_append_kv_paged(int mbits, int vbits, int xt, int d, const void* keys,
                            const void* values, int kblocks, int vblocks, int64_t S,
                            int64_t ktpg, int64_t kntiles, int64_t vtpg, int64_t vntiles,
                            const float* kpi, const float* signs, const float* vpi, Half fine,
                            Half bnd, uint8_t* kpool, float* knorm, uint32_t* vpool,
                            float* vnorm, int64_t t_stride, int64_t t0, const QkvPages& pg,
                            int nsplit, hipStream_t s) {
  if (vbits != mbits + 1 || (d != 128 && d != 64) || xt < 0 || xt > 2) return false;
  if ((nsplit != 1 && nsplit != d / 32) || kblocks < one_blocks(kntiles, nsplit) ||
      vblocks < one_blocks(vntiles, nsplit))
    return false;
  const dim3 grid(kblocks + vblocks);
#define QKV_KVP(MB, F, DD)                                                                     \
  hipLaunchKernelGGL((append_kv_paged<MB, MB + 1, F, DD>), grid, dim3(kThreads), 0, s, keys,    \
                     values, kblocks, S, ktpg, kntiles, vtpg, vntiles, kpi, signs, vpi, fine,   \
                     bnd, kpool, knorm, vpool, vnorm, t_stride, t0, pg, nsplit)
#define QKV_KVPD(DD)                   \
  switch (mbits * 3 + xt) {            \
    case 3: QKV_KVP(1, 0, DD); break;  \
    case 4: QKV_KVP(1, 1, DD); break;  \
    case 5: QKV_KVP(1, 2, DD); break;  \
    case 6: QKV_KVP(2, 0, DD); break;  \
    case 7: QKV_KVP(2, 1, DD); break;  \
    case 8: QKV_KVP(2, 2, DD); break;  \
    case 9: QKV_KVP(3, 0, DD); break;  \
    case 10: QKV_KVP(3, 1, DD); break; \
    case 11: QKV_KVP(3, 2, DD); break; \
    default: return false;             \
  }
  if (d == 128) {
    QKV_KVPD(128)
  } else {
    QKV_KVPD(64)
  }
#undef QKV_KVPD
#undef QKV_KVP
  return true;
}

bool launch_append_kv(int mbits, int vbits, int xt, int d, const AppendLayers& ak,
                      const AppendLayers& av, int n_layers, int kblocks, int vblocks, int64_t S,
                      int64_t ktpg, int64_t kntiles, int64_t vtpg, int64_t vntiles, Half fine,
                      Half bnd, int64_t t_stride, int64_t t0, int nsplit, hipStream_t s) {
  if (vbits != mbits + 1 || (d != 128 && d != 64) || xt < 0 || xt > 2) return false;
  // the kernel bodies run one tile (nsplit = d / 32: one coordinate block of one
  // tile) per wave
  if ((nsplit != 1 && nsplit != d / 32) || kblocks < one_blocks(kntiles, nsplit) ||
      vblocks < one_blocks(vntiles, nsplit))
    return false;
  const dim3 grid(kblocks + vblocks, n_layers);
#define QKV_KV(MB, F, DD)                                                                      \
  hipLaunchKernelGGL((append_kv_layers<MB, MB + 1, F, DD>), grid, dim3(kThreads), 0, s, ak, av, \
                     kblocks, S, ktpg, kntiles, vtpg, vntiles, fine, bnd, t_stride, t0, nsplit)
#define QKV_KVD(DD)                  \
  switch (mbits * 3 + xt) {          \
    case 3: QKV_KV(1, 0, DD); break;  \
    case 4: QKV_KV(1, 1, DD); break;  \
    case 5: QKV_KV(1, 2, DD); break;  \
    case 6: QKV_KV(2, 0, DD); break;  \
    case 7: QKV_KV(2, 1, DD); break;  \
    case 8: QKV_KV(2, 2, DD); break;  \
    case 9: QKV_KV(3, 0, DD); break;  \
    case 10: QKV_KV(3, 1, DD); break; \
    case 11: QKV_KV(3, 2, DD); break; \
    default: return false;           \
  }
  if (d == 128) {
    QKV_KVD(128)
  } else {
    QKV_KVD(64)
  }
#undef QKV_KVD
#undef QKV_KV
  return true;
}

}  // namespace qkv_app
