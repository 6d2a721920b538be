// C ABI of the fused store append (compress straight into the K-row / V-tile
// store): argument checks, search lists and launches of the kernels in
// qkv_append_dev.h.

#include "qkv_append_dev.h"

namespace {

bool symmetric(const float* v, int n) {
  for (int i = 0; i < n; ++i)
    if (v[i] != -v[n - 1 - i]) return false;
  return true;
}

// Integer keys 2 bits(p) of the positive half of an ascending list v[0 .. n-1]
// symmetric about 0 (n odd); false unless those entries are positive and finite.
bool positive_half(const float* v, int n, Half* h) {
  for (int i = 0; i < n / 2; ++i) {
    const float p = v[n / 2 + 1 + i];
    if (!(p > 0.f) || !std::isfinite(p)) return false;
    uint32_t b;
    std::memcpy(&b, &p, 4);
    h->t[i] = 2u * b;
  }
  return true;
}

// The search lists of the store append: the key fine list (centroids and
// boundaries interleaved) and the value boundaries, as positive halves of
// integer keys; QKV_E_UNSUPPORTED unless they are ascending and symmetric.
int append_lists(bool keys, bool values, int mbits, int vbits, const float* kcent_host,
                 const float* kbound_host, const float* vbound_host, Half* fine, Half* bnd) {
  if (keys) {
    const int nc = 1 << mbits;
    float fl[15];
    for (int i = 0; i < nc; ++i) {
      fl[2 * i] = kcent_host[i];
      if (i + 1 < nc) fl[2 * i + 1] = kbound_host[i];
    }
    bool asc = true;
    for (int i = 0; i + 1 < 2 * nc - 1; ++i) asc = asc && fl[i] < fl[i + 1];
    if (!asc || !symmetric(fl, 2 * nc - 1) || !positive_half(fl, 2 * nc - 1, fine)) {
      qkv_set_error("store append needs a symmetric key codebook with c_i < t_i < c_{i+1}");
      return QKV_E_UNSUPPORTED;
    }
  }
  if (values) {
    const int nb = (1 << vbits) - 1;
    bool asc = true;
    for (int i = 0; i + 1 < nb; ++i) asc = asc && vbound_host[i] < vbound_host[i + 1];
    if (!asc || !symmetric(vbound_host, nb) || !positive_half(vbound_host, nb, bnd)) {
      qkv_set_error("store append needs ascending value boundaries symmetric about 0");
      return QKV_E_UNSUPPORTED;
    }
  }
  return QKV_OK;
}

int append_blocks(int64_t ntiles) {
  const int64_t cap = int64_t(qkv_num_cus()) * 2;  // two 64-KiB-LDS workgroups per CU
  return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>((ntiles + kWaves - 1) / kWaves, cap)));
}

// qkv_store_append and its variants.  rotated: keys / values are fp32 rotated
// unit rows y with their norms in knorm_in / vnorm_in (in_dtype unused).
int store_append_impl(int32_t in_dtype, const void* keys, const void* values, bool rotated,
                      const float* knorm_in, const float* vnorm_in, int64_t groups, int64_t S,
                      int32_t d, int32_t mbits, int32_t vbits, const float* kpi,
                      const float* signs, const float* kcent_host, const float* kbound_host,
                      const float* vbound_host, uint8_t* kstore, float* knorm, uint32_t* vstore,
                      float* vnorm, int64_t t_stride, int64_t t0, QkvPages pg, void* stream,
                      const float* vpi) {
  QKV_REQUIRE(groups >= 0 && S >= 0 && t0 >= 0, "negative size");
  QKV_REQUIRE(S / kTok + 2 <= ((int64_t(1) << 31) - 1) / std::max<int64_t>(groups, 1),
              "append of %lld groups x %lld tokens: more than 2^31 tiles", (long long)groups,
              (long long)S);
  if (pg.tab == nullptr) {
    QKV_REQUIRE(t_stride % 32 == 0 && t0 + S <= t_stride,
                "store capacity %lld (multiple of 32) must hold tokens [%lld, %lld)",
                (long long)t_stride, (long long)t0, (long long)(t0 + S));
  } else {
    QKV_REQUIRE(!rotated, "the rotated append writes the contiguous store only");
    QKV_REQUIRE(pg.H > 0 && groups % pg.H == 0, "groups must be batch x kv heads");
    QKV_REQUIRE(t0 + S <= (int64_t(pg.pmax) << pg.lg),
                "page table of %d pages of %d tokens per sequence must hold tokens "
                "[%lld, %lld)", pg.pmax, 1 << pg.lg, (long long)t0, (long long)(t0 + S));
  }
  QKV_REQUIRE(qkv_dtype_ok(in_dtype), "unsupported input dtype %d", in_dtype);
  if (d != 128 && d != 96 && d != 64) {
    qkv_set_error("store append runs on head_dim 128, 96 or 64 (got %d)", d);
    return QKV_E_UNSUPPORTED;
  }
  const int in_align = rotated ? 4 : 16;
  if (keys) {
    if (mbits < 1 || mbits > 3) {
      qkv_set_error("store append: key MSE bits %d not in 1..3", mbits);
      return QKV_E_UNSUPPORTED;
    }
    QKV_REQUIRE((rotated || kpi) && signs && kcent_host && kbound_host && kstore && knorm &&
                    (!rotated || knorm_in),
                "null pointer");
    QKV_REQUIRE(qkv_aligned(keys, in_align) && qkv_aligned(kstore, 4),
                "keys %d-B / store 4-B aligned", in_align);
  }
  if (values) {
    QKV_REQUIRE(qkv_bits_ok(vbits), "value bits %d not in 1..4", vbits);
    QKV_REQUIRE((rotated || vpi) && vbound_host && vstore && vnorm && (!rotated || vnorm_in),
                "null pointer");
    QKV_REQUIRE(qkv_aligned(values, in_align) && qkv_aligned(vstore, 4),
                "values %d-B / store 4-B aligned", in_align);
  }
  QKV_REQUIRE((!kpi || qkv_aligned(kpi, 16)) && (!vpi || qkv_aligned(vpi, 16)),
              "pi must be 16-byte aligned");
  Half fine{}, bnd{};
  if (const int st = append_lists(keys != nullptr, values != nullptr, mbits, vbits, kcent_host,
                                  kbound_host, vbound_host, &fine, &bnd))
    return st;
  if (groups == 0 || S == 0) return QKV_OK;
  auto s = static_cast<hipStream_t>(stream);
  const int xt = in_dtype == QKV_F32 ? 2 : in_dtype == QKV_F16 ? 1 : 0;  // the kernels' XT
  if (keys && values && !rotated) {
    // both halves in one launch when their workgroups are resident at once
    const int64_t ktpg = (S + kTok - 1) / kTok, kn = groups * ktpg;
    const int64_t vtpg = (t0 + S - (t0 & ~int64_t(31)) + kTok - 1) / kTok, vn = groups * vtpg;
    // a wave per 32-coordinate block of a tile while that fits one workgroup per
    // CU, else a wave per tile while two per CU hold every workgroup
    int ns = d / 32;
    int kb = static_cast<int>(std::min<int64_t>(one_blocks(kn, ns), 1 << 20));
    int vb = static_cast<int>(std::min<int64_t>(one_blocks(vn, ns), 1 << 20));
    if (kb + vb > qkv_num_cus()) {
      ns = 1;
      kb = append_blocks(kn);
      vb = append_blocks(vn);
    }
    if (kb + vb <= 2 * qkv_num_cus() && pg.tab != nullptr) {
      if (qkv_app::launch_append_kv_paged(mbits, vbits, xt, d, keys, values, kb, vb, S, ktpg, kn,
                                          vtpg, vn, kpi, signs, vpi, fine, bnd, kstore, knorm,
                                          vstore, vnorm, t_stride, t0, pg, ns, s)) {
        QKV_LAUNCHED();
        return QKV_OK;
      }
    } else if (kb + vb <= 2 * qkv_num_cus()) {
      AppendLayers ak{}, av{};
      ak.x[0] = keys;
      ak.pi[0] = kpi;
      ak.signs[0] = signs;
      ak.st[0] = kstore;
      ak.nrm[0] = knorm;
      av.x[0] = values;
      av.pi[0] = vpi;
      av.st[0] = vstore;
      av.nrm[0] = vnorm;
      if (qkv_app::launch_append_kv(mbits, vbits, xt, d, ak, av, 1, kb, vb, S, ktpg, kn, vtpg, vn,
                                    fine, bnd, t_stride, t0, ns, s)) {
        QKV_LAUNCHED();
        return QKV_OK;
      }
    }
  }
  if (keys) {
    const int64_t tpg = (S + kTok - 1) / kTok, ntiles = groups * tpg;
    const dim3 grid(append_blocks(ntiles));
#define QKV_K(MB, F, DD)                                                                       \
  if (rotated)                                                                                 \
    hipLaunchKernelGGL((append_k_mfma<MB, 0, DD, false, true>), grid, dim3(kThreads), 0, s,     \
                       keys, knorm_in, S, tpg, ntiles, kpi, signs, fine, kstore, knorm,          \
                       t_stride, t0, pg);                                                      \
  else if (pg.tab)                                                                             \
    hipLaunchKernelGGL((append_k_mfma<MB, F, DD, true, false>), grid, dim3(kThreads), 0, s,     \
                       keys, nullptr, S, tpg, ntiles, kpi, signs, fine, kstore, knorm,           \
                       t_stride, t0, pg);                                                      \
  else                                                                                         \
    hipLaunchKernelGGL((append_k_mfma<MB, F, DD, false, false>), grid, dim3(kThreads), 0, s,    \
                       keys, nullptr, S, tpg, ntiles, kpi, signs, fine, kstore, knorm,           \
                       t_stride, t0, pg)
#define QKV_KD(DD)                                  \
  switch (mbits * 3 + xt) {                         \
    case 3: QKV_K(1, 0, DD); break;                 \
    case 4: QKV_K(1, 1, DD); break;                 \
    case 5: QKV_K(1, 2, DD); break;                 \
    case 6: QKV_K(2, 0, DD); break;                 \
    case 7: QKV_K(2, 1, DD); break;                 \
    case 8: QKV_K(2, 2, DD); break;                 \
    case 9: QKV_K(3, 0, DD); break;                 \
    case 10: QKV_K(3, 1, DD); break;                \
    case 11: QKV_K(3, 2, DD); break;                \
  }
    if (d == 128) {
      QKV_KD(128)
    } else if (d == 96) {
      QKV_KD(96)
    } else {
      QKV_KD(64)
    }
#undef QKV_KD
#undef QKV_K
    QKV_LAUNCHED();
  }
  if (values) {
    const int64_t a_base = t0 & ~int64_t(31);
    const int64_t tpg = (t0 + S - a_base + kTok - 1) / kTok, ntiles = groups * tpg;
    const dim3 grid(append_blocks(ntiles));
#define QKV_V(VB, F, DD)                                                                       \
  if (rotated)                                                                                 \
    hipLaunchKernelGGL((append_v_mfma<VB, 0, DD, false, true>), grid, dim3(kThreads), 0, s,     \
                       values, vnorm_in, S, tpg, ntiles, vpi, bnd, vstore, vnorm, t_stride, t0,  \
                       pg);                                                                    \
  else if (pg.tab)                                                                             \
    hipLaunchKernelGGL((append_v_mfma<VB, F, DD, true, false>), grid, dim3(kThreads), 0, s,     \
                       values, nullptr, S, tpg, ntiles, vpi, bnd, vstore, vnorm, t_stride, t0,   \
                       pg);                                                                    \
  else                                                                                         \
    hipLaunchKernelGGL((append_v_mfma<VB, F, DD, false, false>), grid, dim3(kThreads), 0, s,    \
                       values, nullptr, S, tpg, ntiles, vpi, bnd, vstore, vnorm, t_stride, t0,   \
                       pg)
#define QKV_VD(DD)                                  \
  switch (vbits * 3 + xt) {                         \
    case 3: QKV_V(1, 0, DD); break;                 \
    case 4: QKV_V(1, 1, DD); break;                 \
    case 5: QKV_V(1, 2, DD); break;                 \
    case 6: QKV_V(2, 0, DD); break;                 \
    case 7: QKV_V(2, 1, DD); break;                 \
    case 8: QKV_V(2, 2, DD); break;                 \
    case 9: QKV_V(3, 0, DD); break;                 \
    case 10: QKV_V(3, 1, DD); break;                \
    case 11: QKV_V(3, 2, DD); break;                \
    case 12: QKV_V(4, 0, DD); break;                \
    case 13: QKV_V(4, 1, DD); break;                \
    case 14: QKV_V(4, 2, DD); break;                \
  }
    if (d == 128) {
      QKV_VD(128)
    } else if (d == 96) {
      QKV_VD(96)
    } else {
      QKV_VD(64)
    }
#undef QKV_VD
#undef QKV_V
    QKV_LAUNCHED();
  }
  return QKV_OK;
}

// qkv_store_append_layers: one K and one V launch over n_layers contiguous
// stores that share shapes, codebooks, capacity and length (grid.y = layer).
int store_append_layers_impl(int32_t n_layers, int32_t in_dtype, const void* const* keys,
                             const void* const* values, int64_t groups, int64_t S, int32_t d,
                             int32_t mbits, int32_t vbits, const float* const* kpi,
                             const float* const* signs, const float* const* vpi,
                             const float* kcent_host, const float* kbound_host,
                             const float* vbound_host, uint8_t* const* kstore,
                             float* const* knorm, uint32_t* const* vstore,
                             float* const* vnorm, int64_t t_stride, int64_t t0, void* stream) {
  QKV_REQUIRE(n_layers >= 1 && n_layers <= kMaxAppendLayers, "n_layers %d not in 1..%d",
              n_layers, kMaxAppendLayers);
  QKV_REQUIRE(keys && values && kpi && signs && vpi && kstore && knorm && vstore && vnorm &&
                  kcent_host && kbound_host && vbound_host,
              "null pointer");
  QKV_REQUIRE(groups >= 0 && S >= 0 && t0 >= 0, "negative size");
  QKV_REQUIRE(S / kTok + 2 <= ((int64_t(1) << 31) - 1) / std::max<int64_t>(groups, 1),
              "append of %lld groups x %lld tokens: more than 2^31 tiles", (long long)groups,
              (long long)S);
  QKV_REQUIRE(t_stride % 32 == 0 && t0 + S <= t_stride,
              "store capacity %lld (multiple of 32) must hold tokens [%lld, %lld)",
              (long long)t_stride, (long long)t0, (long long)(t0 + S));
  QKV_REQUIRE(qkv_dtype_ok(in_dtype), "unsupported input dtype %d", in_dtype);
  if (d != 128 && d != 96 && d != 64) {
    qkv_set_error("store append runs on head_dim 128, 96 or 64 (got %d)", d);
    return QKV_E_UNSUPPORTED;
  }
  if (mbits < 1 || mbits > 3) {
    qkv_set_error("store append: key MSE bits %d not in 1..3", mbits);
    return QKV_E_UNSUPPORTED;
  }
  QKV_REQUIRE(qkv_bits_ok(vbits), "value bits %d not in 1..4", vbits);
  AppendLayers ak{}, av{};
  for (int l = 0; l < n_layers; ++l) {
    QKV_REQUIRE(keys[l] && values[l] && kpi[l] && signs[l] && vpi[l] && kstore[l] && knorm[l] &&
                    vstore[l] && vnorm[l],
                "null pointer (layer %d)", l);
    QKV_REQUIRE(qkv_aligned(keys[l], 16) && qkv_aligned(values[l], 16) &&
                    qkv_aligned(kpi[l], 16) && qkv_aligned(vpi[l], 16) &&
                    qkv_aligned(kstore[l], 4) && qkv_aligned(vstore[l], 4),
                "layer %d: rows and pi 16-B, stores 4-B aligned", l);
    ak.x[l] = keys[l];
    ak.pi[l] = kpi[l];
    ak.signs[l] = signs[l];
    ak.st[l] = kstore[l];
    ak.nrm[l] = knorm[l];
    av.x[l] = values[l];
    av.pi[l] = vpi[l];
    av.st[l] = vstore[l];
    av.nrm[l] = vnorm[l];
  }
  Half fine{}, bnd{};
  if (const int st = append_lists(true, true, mbits, vbits, kcent_host, kbound_host, vbound_host,
                                  &fine, &bnd))
    return st;
  if (groups == 0 || S == 0) return QKV_OK;
  auto s = static_cast<hipStream_t>(stream);
  const int xt = in_dtype == QKV_F32 ? 2 : in_dtype == QKV_F16 ? 1 : 0;
  // workgroups per layer: the tiles' waves, at most two workgroups per CU over all layers
  auto blocks = [&](int64_t ntiles) {
    const int64_t cap = std::max<int64_t>(1, int64_t(qkv_num_cus()) * 2 / n_layers);
    return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>((ntiles + kWaves - 1) / kWaves, cap)));
  };
  {
    // both halves in one launch when all their workgroups are resident at once
    const int64_t ktpg = (S + kTok - 1) / kTok, kn = groups * ktpg;
    const int64_t vtpg = (t0 + S - (t0 & ~int64_t(31)) + kTok - 1) / kTok, vn = groups * vtpg;
    // a wave per 32-coordinate block of a tile while that fits one workgroup per
    // CU, else a wave per tile while two per CU hold every workgroup
    int ns = d / 32;
    int kb = static_cast<int>(std::min<int64_t>(one_blocks(kn, ns), 1 << 20));
    int vb = static_cast<int>(std::min<int64_t>(one_blocks(vn, ns), 1 << 20));
    if (int64_t(kb + vb) * n_layers > qkv_num_cus()) {
      ns = 1;
      kb = blocks(kn);
      vb = blocks(vn);
    }
    if (int64_t(kb + vb) * n_layers <= 2 * qkv_num_cus() &&
        qkv_app::launch_append_kv(mbits, vbits, xt, d, ak, av, n_layers, kb, vb, S, ktpg, kn,
                                  vtpg, vn, fine, bnd, t_stride, t0, ns, s)) {
      QKV_LAUNCHED();
      return QKV_OK;
    }
  }
  {
    const int64_t tpg = (S + kTok - 1) / kTok, ntiles = groups * tpg;
    const dim3 grid(blocks(ntiles), n_layers);
#define QKV_K(MB, F, DD)                                                                     \
  hipLaunchKernelGGL((append_k_layers<MB, F, DD>), grid, dim3(kThreads), 0, s, ak, S, tpg,    \
                     ntiles, fine, t_stride, t0)
#define QKV_KD(DD)                  \
  switch (mbits * 3 + xt) {         \
    case 3: QKV_K(1, 0, DD); break; \
    case 4: QKV_K(1, 1, DD); break; \
    case 5: QKV_K(1, 2, DD); break; \
    case 6: QKV_K(2, 0, DD); break; \
    case 7: QKV_K(2, 1, DD); break; \
    case 8: QKV_K(2, 2, DD); break; \
    case 9: QKV_K(3, 0, DD); break; \
    case 10: QKV_K(3, 1, DD); break; \
    case 11: QKV_K(3, 2, DD); break; \
  }
    if (d == 128) {
      QKV_KD(128)
    } else if (d == 96) {
      QKV_KD(96)
    } else {
      QKV_KD(64)
    }
#undef QKV_KD
#undef QKV_K
    QKV_LAUNCHED();
  }
  {
    const int64_t a_base = t0 & ~int64_t(31);
    const int64_t tpg = (t0 + S - a_base + kTok - 1) / kTok, ntiles = groups * tpg;
    const dim3 grid(blocks(ntiles), n_layers);
#define QKV_V(VB, F, DD)                                                                     \
  hipLaunchKernelGGL((append_v_layers<VB, F, DD>), grid, dim3(kThreads), 0, s, av, S, tpg,    \
                     ntiles, bnd, t_stride, t0)
#define QKV_VD(DD)                   \
  switch (vbits * 3 + xt) {          \
    case 3: QKV_V(1, 0, DD); break;  \
    case 4: QKV_V(1, 1, DD); break;  \
    case 5: QKV_V(1, 2, DD); break;  \
    case 6: QKV_V(2, 0, DD); break;  \
    case 7: QKV_V(2, 1, DD); break;  \
    case 8: QKV_V(2, 2, DD); break;  \
    case 9: QKV_V(3, 0, DD); break;  \
    case 10: QKV_V(3, 1, DD); break; \
    case 11: QKV_V(3, 2, DD); break; \
    case 12: QKV_V(4, 0, DD); break; \
    case 13: QKV_V(4, 1, DD); break; \
    case 14: QKV_V(4, 2, DD); break; \
  }
    if (d == 128) {
      QKV_VD(128)
    } else if (d == 96) {
      QKV_VD(96)
    } else {
      QKV_VD(64)
    }
#undef QKV_VD
#undef QKV_V
    QKV_LAUNCHED();
  }
  return QKV_OK;
}

// The kmixed key append (x or, rotated, y in slot order with its norms).
// Fine list c_0 < t_0 < c_1 < ... < c_{2^bits - 1} of a codebook into fl.
int fine_list(const float* cent, const float* bound, int bits, float* fl) {
  const int nc = 1 << bits;
  for (int i = 0; i < nc; ++i) {
    fl[2 * i] = cent[i];
    if (i + 1 < nc) fl[2 * i + 1] = bound[i];
  }
  return 2 * nc - 1;
}

// Mixed-precision key append.  ipm = false: MSE keys, 3-bit outlier / 2-bit
// regular boundaries (out_bound 7, reg_bound 3 entries).  ipm = true: IP keys
// with a 2-bit outlier / 1-bit regular MSE stage, searched over the fine
// lists built from the centroids (4, 2) and boundaries (3, 1); signs_perm is S
// in slot order.
int kmixed_append_impl(int32_t in_dtype, const void* keys, bool rotated, const float* norm_in,
                       int64_t groups, int64_t S, int32_t d, const float* pi_perm,
                       int32_t n_out, bool ipm, const float* signs_perm,
                       const float* out_cent_host, const float* reg_cent_host,
                       const float* out_bound_host, const float* reg_bound_host,
                       uint8_t* kstore, float* knorm, int64_t t_stride, int64_t t0,
                       void* stream, Half* po_out = nullptr, Half* pr_out = nullptr) {
  QKV_REQUIRE(groups >= 0 && S >= 0 && t0 >= 0, "negative size");
  QKV_REQUIRE(S / kTok + 2 <= ((int64_t(1) << 31) - 1) / std::max<int64_t>(groups, 1),
              "append of %lld groups x %lld tokens: more than 2^31 tiles", (long long)groups,
              (long long)S);
  QKV_REQUIRE(t0 + S <= t_stride, "store capacity %lld must hold tokens [%lld, %lld)",
              (long long)t_stride, (long long)t0, (long long)(t0 + S));
  QKV_REQUIRE(qkv_dtype_ok(in_dtype), "unsupported input dtype %d", in_dtype);
  if (d != kD || (n_out != 32 && n_out != 64)) {
    qkv_set_error("mixed-precision keys run on head_dim 128 with 32 or 64 outlier channels");
    return QKV_E_UNSUPPORTED;
  }
  QKV_REQUIRE(keys && (rotated || pi_perm) && out_bound_host && reg_bound_host && kstore &&
                  knorm && (!rotated || norm_in) &&
                  (!ipm || (signs_perm && out_cent_host && reg_cent_host)),
              "null pointer");
  QKV_REQUIRE(qkv_aligned(keys, rotated ? 4 : 16) && qkv_aligned(kstore, 4) &&
                  (rotated || qkv_aligned(pi_perm, 16)),
              "keys / pi aligned (16-B input rows, 4-B rotated rows) and store 4-B aligned");
  float lo[7], lr[3];
  if (ipm) {
    fine_list(out_cent_host, out_bound_host, 2, lo);
    fine_list(reg_cent_host, reg_bound_host, 1, lr);
  } else {
    for (int i = 0; i < 7; ++i) lo[i] = out_bound_host[i];
    for (int i = 0; i < 3; ++i) lr[i] = reg_bound_host[i];
  }
  Half po{}, pr{};
  bool asc = true;
  for (int i = 0; i + 1 < 7; ++i) asc = asc && lo[i] < lo[i + 1];
  for (int i = 0; i + 1 < 3; ++i) asc = asc && lr[i] < lr[i + 1];
  if (!asc || !symmetric(lo, 7) || !symmetric(lr, 3) || !positive_half(lo, 7, &po) ||
      !positive_half(lr, 3, &pr)) {
    qkv_set_error("mixed-precision keys need ascending %s symmetric about 0",
                  ipm ? "fine lists c_i < t_i < c_{i+1}" : "boundaries");
    return QKV_E_UNSUPPORTED;
  }
  if (po_out) {  // checks and lists only (the caller launches)
    *po_out = po;
    *pr_out = pr;
    return QKV_OK;
  }
  if (groups == 0 || S == 0) return QKV_OK;
  auto s = static_cast<hipStream_t>(stream);
  const int64_t tpg = (S + kTok - 1) / kTok, ntiles = groups * tpg;
  const dim3 grid(append_blocks(ntiles));
  const int xt = in_dtype == QKV_F32 ? 2 : in_dtype == QKV_F16 ? 1 : 0;  // the kernel's XT
#define QKV_KM(NOV, F, FY, IP)                                                                 \
  hipLaunchKernelGGL((append_kmix_mfma<NOV, F, FY, IP>), grid, dim3(kThreads), 0, s, keys,     \
                     norm_in, S, tpg, ntiles, pi_perm, signs_perm, po, pr, kstore, knorm,      \
                     t_stride, t0)
#define QKV_KM_IN(NOV, IP)                \
  do {                                    \
    if (rotated)                          \
      QKV_KM(NOV, 0, true, IP);           \
    else if (xt == 2)                     \
      QKV_KM(NOV, 2, false, IP);          \
    else if (xt == 1)                     \
      QKV_KM(NOV, 1, false, IP);          \
    else                                  \
      QKV_KM(NOV, 0, false, IP);          \
  } while (0)
  if (n_out == 32) {
    if (ipm) QKV_KM_IN(32, true);
    else QKV_KM_IN(32, false);
  } else {
    if (ipm) QKV_KM_IN(64, true);
    else QKV_KM_IN(64, false);
  }
#undef QKV_KM_IN
#undef QKV_KM
  QKV_LAUNCHED();
  return QKV_OK;
}

// qkv_store_append_kmixed_kv: the kmixed / kipmixed key append and the value
// append of the same tokens; one launch when both halves' workgroups are
// resident at once, else the two kernels.  Every argument is checked before
// anything is launched.
int kmixed_kv_impl(int32_t in_dtype, const void* keys, const void* values, int64_t groups,
                   int64_t S, int32_t d, const float* pi_perm, const float* signs_perm,
                   int32_t n_out, bool ipm, const float* out_cent_host,
                   const float* out_bound_host, const float* reg_cent_host,
                   const float* reg_bound_host, uint8_t* kstore, float* knorm, int32_t vbits,
                   const float* vpi, const float* vbound_host, uint32_t* vstore, float* vnorm,
                   int64_t t_stride, int64_t t0, void* stream) {
  Half po{}, pr{};
  if (const int st = kmixed_append_impl(in_dtype, keys, false, nullptr, groups, S, d, pi_perm,
                                        n_out, ipm, signs_perm, out_cent_host, reg_cent_host,
                                        out_bound_host, reg_bound_host, kstore, knorm, t_stride,
                                        t0, stream, &po, &pr))
    return st;
  QKV_REQUIRE(qkv_bits_ok(vbits), "value bits %d not in 1..4", vbits);
  QKV_REQUIRE(values && vpi && vbound_host && vstore && vnorm, "null pointer");
  QKV_REQUIRE(qkv_aligned(values, 16) && qkv_aligned(vpi, 16) && qkv_aligned(vstore, 4),
              "values / pi 16-B, store 4-B aligned");
  QKV_REQUIRE(t_stride % 32 == 0, "store capacity %lld must be a multiple of 32",
              (long long)t_stride);
  Half fine{}, bnd{};
  if (const int st = append_lists(false, true, 2, vbits, nullptr, nullptr, vbound_host, &fine,
                                  &bnd))
    return st;
  if (groups == 0 || S == 0) return QKV_OK;
  const int64_t ktpg = (S + kTok - 1) / kTok, kn = groups * ktpg;
  const int64_t vtpg = (t0 + S - (t0 & ~int64_t(31)) + kTok - 1) / kTok, vn = groups * vtpg;
  // a wave per 32-slot block of a tile while two workgroups per CU hold every
  // workgroup (cfg4's 2048-token chunks: 512 workgroups, 12 us per chunk
  // against 14.5 us for a wave per tile), else a wave per tile
  int ns = 4;
  int kb = static_cast<int>(std::min<int64_t>(one_blocks(kn, ns), 1 << 20));
  int vb = static_cast<int>(std::min<int64_t>(one_blocks(vn, ns), 1 << 20));
  if (kb + vb > 2 * qkv_num_cus()) {
    ns = 1;
    kb = append_blocks(kn);
    vb = append_blocks(vn);
  }
  const int xt = in_dtype == QKV_F32 ? 2 : in_dtype == QKV_F16 ? 1 : 0;
  if (kb + vb <= 2 * qkv_num_cus() &&
      qkv_app::launch_append_kmixv(n_out, ipm, vbits, xt, keys, values, kb, vb, S, ktpg, kn, vtpg,
                                   vn, pi_perm, signs_perm, po, pr, kstore, knorm, vpi, bnd,
                                   vstore, vnorm, t_stride, t0, ns,
                                   static_cast<hipStream_t>(stream))) {
    QKV_LAUNCHED();
    return QKV_OK;
  }
  if (const int st = kmixed_append_impl(in_dtype, keys, false, nullptr, groups, S, d, pi_perm,
                                        n_out, ipm, signs_perm, out_cent_host, reg_cent_host,
                                        out_bound_host, reg_bound_host, kstore, knorm, t_stride,
                                        t0, stream))
    return st;
  return store_append_impl(in_dtype, nullptr, values, false, nullptr, nullptr, groups, S, d, 2,
                           vbits, nullptr, nullptr, nullptr, nullptr, vbound_host, nullptr, nullptr,
                           vstore, vnorm, t_stride, t0, QkvPages{}, stream, vpi);
}

}  // namespace

extern "C" int qkv_store_append(int32_t in_dtype, const void* keys, const void* values,
                                int64_t groups, int64_t S, int32_t d, int32_t mbits,
                                int32_t vbits, const float* pi, const float* signs,
                                const float* kcent_host, const float* kbound_host,
                                const float* vbound_host, uint8_t* kstore, float* knorm,
                                uint32_t* vstore, float* vnorm, int64_t t_stride, int64_t t0,
                                void* stream) {
  return store_append_impl(in_dtype, keys, values, false, nullptr, nullptr, groups, S, d, mbits,
                           vbits, pi, signs, kcent_host, kbound_host, vbound_host, kstore, knorm,
                           vstore, vnorm, t_stride, t0, QkvPages{nullptr, 0, 1, 6, 0}, stream, pi);
}

extern "C" int qkv_store_append_layers(int32_t n_layers, int32_t in_dtype,
                                       const void* const* keys, const void* const* values,
                                       int64_t groups, int64_t S, int32_t d, int32_t mbits,
                                       int32_t vbits, const float* const* kpi,
                                       const float* const* signs, const float* const* vpi,
                                       const float* kcent_host, const float* kbound_host,
                                       const float* vbound_host, uint8_t* const* kstore,
                                       float* const* knorm, uint32_t* const* vstore,
                                       float* const* vnorm, int64_t t_stride, int64_t t0,
                                       void* stream) {
  return store_append_layers_impl(n_layers, in_dtype, keys, values, groups, S, d, mbits, vbits,
                                  kpi, signs, vpi, kcent_host, kbound_host, vbound_host, kstore,
                                  knorm, vstore, vnorm, t_stride, t0, stream);
}

extern "C" int qkv_store_append_rotated(const float* yk, const float* knorm_in, const float* yv,
                                        const float* vnorm_in, int64_t groups, int64_t S,
                                        int32_t d, int32_t mbits, int32_t vbits,
                                        const float* signs, const float* kcent_host,
                                        const float* kbound_host, const float* vbound_host,
                                        uint8_t* kstore, float* knorm, uint32_t* vstore,
                                        float* vnorm, int64_t t_stride, int64_t t0,
                                        void* stream) {
  return store_append_impl(QKV_F32, yk, yv, true, knorm_in, vnorm_in, groups, S, d, mbits,
                           vbits, nullptr, signs, kcent_host, kbound_host, vbound_host, kstore,
                           knorm, vstore, vnorm, t_stride, t0, QkvPages{nullptr, 0, 1, 6, 0},
                           stream, nullptr);
}

extern "C" int qkv_paged_store_append(int32_t in_dtype, const void* keys, const void* values,
                                      int32_t B, int32_t H, int64_t S, int32_t d, int32_t mbits,
                                      int32_t vbits, const float* pi, const float* signs,
                                      const float* kcent_host, const float* kbound_host,
                                      const float* vbound_host, uint8_t* kpool, float* knorm,
                                      uint32_t* vpool, float* vnorm, const int32_t* page_table,
                                      int32_t pages_per_seq, int32_t page_tokens,
                                      int32_t num_pages, int64_t t0, void* stream) {
  QKV_REQUIRE(B >= 0 && H > 0 && int64_t(B) * H < (int64_t(1) << 31), "invalid shape");
  QKV_REQUIRE(page_table && pages_per_seq > 0, "null page table");
  QKV_REQUIRE(num_pages > 0, "num_pages %d must be positive", num_pages);
  const int lg = qkv_page_lg(page_tokens);
  QKV_REQUIRE(lg > 0, "page_tokens %d must be 64, 128, ..., 2048", page_tokens);
  QKV_REQUIRE(qkv_aligned(page_table, 4), "page table 4-B aligned");
  return store_append_impl(in_dtype, keys, values, false, nullptr, nullptr, int64_t(B) * H, S, d,
                           mbits, vbits, pi, signs, kcent_host, kbound_host, vbound_host, kpool,
                           knorm, vpool, vnorm, page_tokens, t0,
                           QkvPages{page_table, pages_per_seq, H, lg, num_pages}, stream, pi);
}

extern "C" int qkv_paged_store_append_kv(
    int32_t in_dtype, const void* keys, const void* values, int32_t B, int32_t H, int64_t S,
    int32_t d, int32_t mbits, int32_t vbits, const float* kpi, const float* signs,
    const float* vpi, const float* kcent_host, const float* kbound_host,
    const float* vbound_host, uint8_t* kpool, float* knorm, uint32_t* vpool, float* vnorm,
    const int32_t* page_table, int32_t pages_per_seq, int32_t page_tokens, int32_t num_pages,
    int64_t t0, void* stream) {
  QKV_REQUIRE(keys && values, "null pointer");
  QKV_REQUIRE(B >= 0 && H > 0 && int64_t(B) * H < (int64_t(1) << 31), "invalid shape");
  QKV_REQUIRE(page_table && pages_per_seq > 0, "null page table");
  QKV_REQUIRE(num_pages > 0, "num_pages %d must be positive", num_pages);
  const int lg = qkv_page_lg(page_tokens);
  QKV_REQUIRE(lg > 0, "page_tokens %d must be 64, 128, ..., 2048", page_tokens);
  QKV_REQUIRE(qkv_aligned(page_table, 4), "page table 4-B aligned");
  return store_append_impl(in_dtype, keys, values, false, nullptr, nullptr, int64_t(B) * H, S, d,
                           mbits, vbits, kpi, signs, kcent_host, kbound_host, vbound_host, kpool,
                           knorm, vpool, vnorm, page_tokens, t0,
                           QkvPages{page_table, pages_per_seq, H, lg, num_pages}, stream, vpi);
}

extern "C" int qkv_store_append_kmixed(int32_t in_dtype, const void* keys, int64_t groups,
                                       int64_t S, int32_t d, const float* pi_perm,
                                       int32_t n_out, const float* out_bound_host,
                                       const float* reg_bound_host, uint8_t* kstore,
                                       float* knorm, int64_t t_stride, int64_t t0,
                                       void* stream) {
  return kmixed_append_impl(in_dtype, keys, false, nullptr, groups, S, d, pi_perm, n_out, false,
                            nullptr, nullptr, nullptr, out_bound_host, reg_bound_host, kstore,
                            knorm, t_stride, t0, stream);
}

extern "C" int qkv_store_append_kmixed_rotated(const float* y_slots, const float* norm_in,
                                               int64_t groups, int64_t S, int32_t d,
                                               int32_t n_out, const float* out_bound_host,
                                               const float* reg_bound_host, uint8_t* kstore,
                                               float* knorm, int64_t t_stride, int64_t t0,
                                               void* stream) {
  return kmixed_append_impl(QKV_F32, y_slots, true, norm_in, groups, S, d, nullptr, n_out, false,
                            nullptr, nullptr, nullptr, out_bound_host, reg_bound_host, kstore,
                            knorm, t_stride, t0, stream);
}

extern "C" int qkv_store_append_kipmixed(int32_t in_dtype, const void* keys, int64_t groups,
                                         int64_t S, int32_t d, const float* pi_perm,
                                         const float* signs_perm, int32_t n_out,
                                         const float* out_cent_host, const float* out_bound_host,
                                         const float* reg_cent_host, const float* reg_bound_host,
                                         uint8_t* kstore, float* knorm, int64_t t_stride,
                                         int64_t t0, void* stream) {
  return kmixed_append_impl(in_dtype, keys, false, nullptr, groups, S, d, pi_perm, n_out, true,
                            signs_perm, out_cent_host, reg_cent_host, out_bound_host,
                            reg_bound_host, kstore, knorm, t_stride, t0, stream);
}

extern "C" int qkv_store_append_kmixed_kv(
    int32_t in_dtype, const void* keys, const void* values, int64_t groups, int64_t S, int32_t d,
    const float* pi_perm, const float* signs_perm, int32_t n_out, int32_t ip,
    const float* out_cent_host, const float* out_bound_host, const float* reg_cent_host,
    const float* reg_bound_host, uint8_t* kstore, float* knorm, int32_t vbits, const float* vpi,
    const float* vbound_host, uint32_t* vstore, float* vnorm, int64_t t_stride, int64_t t0,
    void* stream) {
  return kmixed_kv_impl(in_dtype, keys, values, groups, S, d, pi_perm, signs_perm, n_out, ip != 0,
                        out_cent_host, out_bound_host, reg_cent_host, reg_bound_host, kstore,
                        knorm, vbits, vpi, vbound_host, vstore, vnorm, t_stride, t0, stream);
}

extern "C" int qkv_store_append_kipmixed_rotated(const float* y_slots, const float* norm_in,
                                                 int64_t groups, int64_t S, int32_t d,
                                                 const float* signs_perm, int32_t n_out,
                                                 const float* out_cent_host,
                                                 const float* out_bound_host,
                                                 const float* reg_cent_host,
                                                 const float* reg_bound_host, uint8_t* kstore,
                                                 float* knorm, int64_t t_stride, int64_t t0,
                                                 void* stream) {
  return kmixed_append_impl(QKV_F32, y_slots, true, norm_in, groups, S, d, nullptr, n_out, true,
                            signs_perm, out_cent_host, reg_cent_host, out_bound_host,
                            reg_bound_host, kstore, knorm, t_stride, t0, stream);
}

extern "C" int qkv_compress_mfma(int32_t mode, int32_t in_dtype, const void* x, int64_t n,
                                 int32_t d, const float* pi, const float* cent_host,
                                 const float* bound_host, int32_t bits, const float* signs,
                                 uint8_t* codes, uint8_t* qjl, float* norms, int64_t out_seq,
                                 int64_t out_group_stride, void* stream) {
  QKV_REQUIRE(mode == QKV_MODE_MSE || mode == QKV_MODE_IP, "mode must be MSE or IP");
  QKV_REQUIRE(qkv_dtype_ok(in_dtype), "unsupported input dtype %d", in_dtype);
  QKV_REQUIRE(n >= 0, "negative row count");
  const bool ip = mode == QKV_MODE_IP;
  if ((d != 128 && d != 96 && d != 64) || bits < 1 || bits > (ip ? 3 : 4)) {
    qkv_set_error("MFMA compress runs on head_dim 128, 96 or 64 with %s bits in 1..%d",
                  ip ? "key MSE" : "value", ip ? 3 : 4);
    return QKV_E_UNSUPPORTED;
  }
  QKV_REQUIRE(pi && bound_host && (!ip || (cent_host && signs)), "null pointer");
  // the searched list: IP the fine list c_0 < t_0 < ... < c_{2^bits-1}, MSE the boundaries
  float lst[15];
  int nl;
  if (ip) {
    nl = fine_list(cent_host, bound_host, bits, lst);
  } else {
    nl = (1 << bits) - 1;
    for (int i = 0; i < nl; ++i) lst[i] = bound_host[i];
  }
  bool asc = true;
  for (int i = 0; i + 1 < nl; ++i) asc = asc && lst[i] < lst[i + 1];
  Half h{};
  if (!asc || !symmetric(lst, nl) || !positive_half(lst, nl, &h)) {
    qkv_set_error("MFMA compress needs a codebook symmetric about 0%s",
                  ip ? " with c_i < t_i < c_{i+1}" : "");
    return QKV_E_UNSUPPORTED;
  }
  if (n == 0) return QKV_OK;
  const int64_t seq = out_seq > 0 ? out_seq : n;
  const int64_t gst = out_group_stride > 0 ? out_group_stride : seq;
  QKV_REQUIRE(x && codes && norms && (!ip || qjl), "null pointer");
  QKV_REQUIRE(qkv_aligned(x, 16) && qkv_aligned(pi, 16), "x rows and pi must be 16-byte aligned");
  QKV_REQUIRE(gst >= seq, "bad grouped-row layout");
  if (gst != seq && seq < n) {
    qkv_set_error("MFMA compress writes dense rows (grouped layouts: qkv_compress)");
    return QKV_E_UNSUPPORTED;
  }
  auto s = static_cast<hipStream_t>(stream);
  const int64_t ntiles = (n + kTok - 1) / kTok;
  const dim3 grid(append_blocks(ntiles));
  const int xt = in_dtype == QKV_F32 ? 2 : in_dtype == QKV_F16 ? 1 : 0;
#define QKV_C(LV, IPV, XTV, DD)                                                                 \
  hipLaunchKernelGGL((compress_mfma<LV, IPV, XTV, DD>), grid, dim3(kThreads), 0, s, x, n,      \
                     ntiles, pi, signs, h, codes, qjl, norms)
#define QKV_CX(LV, IPV, DD)        \
  do {                             \
    if (xt == 2)                   \
      QKV_C(LV, IPV, 2, DD);       \
    else if (xt == 1)              \
      QKV_C(LV, IPV, 1, DD);       \
    else                           \
      QKV_C(LV, IPV, 0, DD);       \
  } while (0)
#define QKV_CD(DD)                                         \
  do {                                                     \
    if (ip) {                                              \
      if (bits == 1) QKV_CX(2, true, DD);                  \
      else if (bits == 2) QKV_CX(3, true, DD);             \
      else QKV_CX(4, true, DD);                            \
    } else {                                               \
      if (bits == 1) QKV_CX(1, false, DD);                 \
      else if (bits == 2) QKV_CX(2, false, DD);            \
      else if (bits == 3) QKV_CX(3, false, DD);            \
      else QKV_CX(4, false, DD);                           \
    }                                                      \
  } while (0)
  if (d == 128)
    QKV_CD(128);
  else if (d == 96)
    QKV_CD(96);
  else
    QKV_CD(64);
#undef QKV_CD
#undef QKV_CX
#undef QKV_C
  QKV_LAUNCHED();
  return QKV_OK;
}
