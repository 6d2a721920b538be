// One launch for the key and the value half of a store append: the workgroups
// of append_k_run and of append_v_run (qkv_append_dev.h) in one grid, so that
// a small append -- one decode token per layer, a short chunk -- runs both
// halves side by side on different CUs and pays one launch instead of two.
// Instantiated for value bits = key MSE bits + 1 (key_bits == value_bits in
// the reference's QuashKVEngine(key_bits, value_bits), quashkv/engine.py:62-90,
// whose default is 3 / 3); other combinations launch the two kernels.

#include "qkv_append_dev.h"

namespace {

// grid = (key workgroups + value workgroups, layers): x < kblocks runs the key
// append of layer blockIdx.y over kblocks workgroups, the rest its value append.
template <int MB, int VB, int XT, int D>
__global__ __launch_bounds__(kThreads, 4) void append_kv_layers(
    AppendLayers ak, AppendLayers av, int kblocks, int64_t S, int64_t ktpg, int64_t kntiles,
    int64_t vtpg, int64_t vntiles, Half fine, Half bnd, int64_t t_stride, int64_t t0) {
  __shared__ uint4 frag[frag_n<D>()];         // the running half's Pi fragments
  __shared__ float4 inv_s[kWaves][kTok / 4];  // key half: 1 / norm of each wave's tokens
  const int l = blockIdx.y, b = blockIdx.x;
  if (b < kblocks)
    append_k_run<MB, XT, D, false, false>(ak.x[l], nullptr, S, ktpg, kntiles, ak.pi[l],
                                          ak.signs[l], fine, static_cast<uint8_t*>(ak.st[l]),
                                          ak.nrm[l], t_stride, t0, QkvPages{}, frag, inv_s, b,
                                          kblocks);
  else
    append_v_run<VB, XT, D, false, false>(av.x[l], nullptr, S, vtpg, vntiles, av.pi[l], bnd,
                                          static_cast<uint32_t*>(av.st[l]), av.nrm[l], t_stride,
                                          t0, QkvPages{}, frag, b - kblocks,
                                          static_cast<int>(gridDim.x) - kblocks);
}

}  // namespace

namespace qkv_app {

bool launch_append_kv(int mbits, int vbits, int xt, int d, const AppendLayers& ak,
                      const AppendLayers& av, int n_layers, int kblocks, int vblocks, int64_t S,
                      int64_t ktpg, int64_t kntiles, int64_t vtpg, int64_t vntiles, Half fine,
                      Half bnd, int64_t t_stride, int64_t t0, hipStream_t s) {
  if (vbits != mbits + 1 || (d != 128 && d != 64) || xt < 0 || xt > 2) return false;
  const dim3 grid(kblocks + vblocks, n_layers);
#define QKV_KV(MB, F, DD)                                                                      \
  hipLaunchKernelGGL((append_kv_layers<MB, MB + 1, F, DD>), grid, dim3(kThreads), 0, s, ak, av, \
                     kblocks, S, ktpg, kntiles, vtpg, vntiles, fine, bnd, t_stride, t0)
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
