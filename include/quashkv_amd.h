/*
 * quashkv_amd -- C ABI of the MI355X (gfx950) TurboQuant hot path.
 *
 * Every entry point:
 *   - takes plain device pointers, sizes and a hipStream_t passed as void*;
 *   - validates its arguments on the host BEFORE any launch;
 *   - launches asynchronously on `stream` and never synchronises;
 *   - never allocates or frees device memory (callers pass outputs and the
 *     attention workspace, sized by qkv_attention_workspace_bytes);
 *   - returns QKV_OK (0) or a QKV_E_* status; qkv_last_error() then holds a
 *     thread-local message.
 *
 * Layout conventions (shared with the reference's PyTorch tensors):
 *   - Pi is the d x d rotation, row-major fp32; y = u Pi^T rotates, x = y Pi
 *     un-rotates (quashkv/quantizer.py:105-111).
 *   - Code rows use the reference's pack_bits layout (quashkv/packing.py:8-14):
 *     LSB-first, 1/2/4-bit groups per byte, 3-bit groups of 8 codes in a
 *     little-endian 24-bit word; bits = 8 means one uint8 per code (unpacked).
 *   - "Grouped rows": vector r of a call lives at row
 *       (r / seq) * group_stride + (r % seq)
 *     of the code/norm buffers, so a (B, H, S, d) input can be written into,
 *     or read from, a (B, H, T_capacity, row_bytes) cache at any offset.
 *
 * The reference interface each function replaces is cited as path:line
 * relative to the reference package root.
 */
#ifndef QUASHKV_AMD_H
#define QUASHKV_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QKV_ABI_VERSION 1

/* status codes */
#define QKV_OK 0
#define QKV_E_INVALID 1     /* bad argument (maps to ValueError) */
#define QKV_E_UNSUPPORTED 2 /* valid but unsupported shape/bits (maps to ValueError) */
#define QKV_E_HIP 3         /* HIP runtime error (maps to RuntimeError) */

/* element types */
#define QKV_F32 0
#define QKV_F16 1
#define QKV_BF16 2

/* compress / decompress modes */
#define QKV_MODE_MSE 0 /* MSEQuantizer */
#define QKV_MODE_IP 1  /* InnerProductQuantizer: (b-1)-bit MSE + 1-bit QJL */

/* code formats of qkv_decompress (store formats: see "Cache store formats") */
#define QKV_FMT_UNPACKED 0 /* one uint8 per code */
#define QKV_FMT_PACKED 1   /* pack_bits rows */
#define QKV_FMT_KPLANES 2  /* K store rows: `bits` MSE planes + QJL plane */
#define QKV_FMT_VTILES 3   /* V store tiles */

/* compress flags */
#define QKV_FLAG_PACKED 1      /* write packed rows (else one uint8 per code) */
#define QKV_FLAG_PRE_ROTATED 2 /* x is already y = u Pi^T: skip norm + rotation
                                  (parity entry: codes from identical y) */

int qkv_abi_version(void);
const char* qkv_last_error(void);

/* Bytes per packed row as pack_bits lays it out: 3*ceil(d/8) for 3-bit,
 * ceil(d*bits/8) otherwise, d for bits = 8 (quashkv/packing.py:43-89).
 * Returns -1 for unsupported bits. */
int64_t qkv_packed_row_bytes(int32_t d, int32_t bits);

/* pack_bits(indices, bits) -- quashkv/packing.py:22-94.
 * codes: rows x d uint8, packed: rows x qkv_packed_row_bytes(d, bits). */
int qkv_pack_bits(const uint8_t* codes, uint8_t* packed, int64_t rows,
                  int32_t d, int32_t bits, void* stream);

/* unpack_bits(packed, bits, d) -- quashkv/packing.py:97-159.
 * packed rows are packed_row_bytes apart; codes: rows x d uint8. */
int qkv_unpack_bits(const uint8_t* packed, int64_t packed_row_bytes,
                    uint8_t* codes, int64_t rows, int32_t d, int32_t bits,
                    void* stream);

/* LloydMaxCodebook.quantize_boundary (mode 0; quashkv/codebook.py:239-259,
 * == torch.bucketize, quashkv/triton_kernels/compress.py:57) and
 * LloydMaxCodebook.quantize (mode 1, first nearest centroid;
 * quashkv/codebook.py:209-224) on n contiguous fp32 values.
 * table: boundaries (mode 0) or centroids (mode 1), count <= 16 entries. */
int qkv_quantize(const float* y, int64_t n, const float* table, int32_t count,
                 int32_t mode, uint8_t* out, void* stream);

/* LloydMaxCodebook.dequantize -- quashkv/codebook.py:226-237: out = c[code];
 * codes >= count give NaN (the reference raises an index error). */
int qkv_dequantize(const uint8_t* codes, int64_t n, const float* cents,
                   int32_t count, float* out, void* stream);

/* InnerProductQuantizer.decompress_for_dot -- quashkv/quantizer.py:244-279:
 * out[r] = n_r (<q_rot_r, c[code_r]> + alpha sum_j |q_rot_rj| (2b_rj-1) S_j)
 * over unpacked uint8 codes/bits, n rows of d. */
int qkv_ip_dot(const uint8_t* codes, const uint8_t* qjl, const float* norms,
               const float* q_rot, int64_t n, int32_t d, const float* cents,
               int32_t count, const float* signs, float alpha, float* out,
               void* stream);

/* Fused compress: normalise -> rotate -> boundary search [-> QJL sign] -> store.
 * Replaces fused_compress_mse / fused_compress_ip
 * (quashkv/triton_kernels/compress.py:210-303) and MSEQuantizer.compress /
 * InnerProductQuantizer.compress (quashkv/quantizer.py:113-131, 211-242).
 *   mode       QKV_MODE_MSE or QKV_MODE_IP
 *   x          n x d, in_dtype (F32/F16/BF16), contiguous
 *   pi         d x d fp32 rotation
 *   boundaries 2^bits - 1 fp32, ascending; centroids 2^bits fp32
 *   bits       MSE code bits (1..4); for IP this is total_bits - 1
 *   signs      d fp32 (+-1), IP only (may be NULL for MSE)
 *   codes      grouped rows of qkv_packed_row_bytes(d, bits) (or d if unpacked)
 *   qjl        grouped rows of the 1-bit QJL signs (IP only)
 *   norms      grouped fp32 norms max(||x||, 1e-8) (ignored if PRE_ROTATED)
 *   out_seq, out_group_stride  grouped-row addressing of codes/qjl/norms
 * This is the VALU kernel for any d, tables and flags; d = 128 / 96 / 64 with
 * symmetric codebooks run faster on qkv_compress_mfma below. */
int qkv_compress(int32_t mode, int32_t in_dtype, int32_t flags,
                 const void* x, int64_t n, int32_t d,
                 const float* pi, const float* boundaries,
                 const float* centroids, int32_t bits, const float* signs,
                 uint8_t* codes, uint8_t* qjl, float* norms,
                 int64_t out_seq, int64_t out_group_stride, void* stream);

/* qkv_compress's unpacked output (one uint8 code, and for IP one QJL bit, per
 * coordinate; norms max(||x||, 1e-8)) on the MFMA for dense rows (out_seq =
 * n or out_group_stride = out_seq; grouped layouts: QKV_E_UNSUPPORTED), for the
 * same reference operators (quashkv/quantizer.py:113-131, 211-242,
 * quashkv/triton_kernels/compress.py:210-303): the rotation, search and tie
 * rules of qkv_store_append.  d = 128, 96 or 64; cent_host / bound_host are HOST
 * copies of the codebook (2^bits centroids, 2^bits - 1 boundaries), which
 * must be symmetric about 0 (else QKV_E_UNSUPPORTED, as for other d or bits
 * beyond 1..3 (IP) / 1..4 (MSE)); x and pi 16-byte aligned. */
int qkv_compress_mfma(int32_t mode, int32_t in_dtype, const void* x, int64_t n, int32_t d,
                      const float* pi, const float* cent_host, const float* bound_host,
                      int32_t bits, const float* signs, uint8_t* codes, uint8_t* qjl,
                      float* norms, int64_t out_seq, int64_t out_group_stride, void* stream);

/* Fused decompress: unpack -> centroid gather [+ alpha S (2b-1)] -> Pi -> *norm.
 * Replaces fused_decompress_mse / fused_decompress_ip
 * (quashkv/triton_kernels/decompress.py:194-285), MSEQuantizer.decompress
 * (quashkv/quantizer.py:133-147) and QuashKVCache's key/value reconstruction
 * (quashkv/integrations/hf_cache.py:96-121, mode MSE with the key codebook).
 *   fmt        QKV_FMT_UNPACKED / PACKED: code rows (qjl rows alike) at grouped
 *              rows (in_seq, in_group_stride);
 *              QKV_FMT_KPLANES: K store rows (qjl unused: the row holds it);
 *              QKV_FMT_VTILES: V store tiles, in_seq tokens per group (from
 *              token 0), in_group_stride tiles per group, norms at
 *              group * 32 * in_group_stride + token (MSE mode only)
 *   out        n x d, out_dtype, contiguous
 * d = 64 / 96 / 128 run on the matrix cores (fp16 high/low split of Pi and
 * of the values, fp32 accumulation: within ~3e-6 relative of an fp32
 * evaluation); they need 16-byte aligned out and V-tile pointers, unpacked
 * code pointers 16-byte (8-byte at d = 96) and packed / K-row pointers
 * 4-byte (2-byte at d = 64) aligned.  Other pointers use a VALU kernel with
 * fp32 arithmetic. */
int qkv_decompress(int32_t mode, int32_t fmt,
                   const uint8_t* codes, const uint8_t* qjl, const float* norms,
                   int64_t n, int32_t d, int32_t bits,
                   const float* pi, const float* centroids, const float* signs,
                   float qjl_scale, int64_t in_seq, int64_t in_group_stride,
                   void* out, int32_t out_dtype, void* stream);

/* Mixed precision (quashkv/mixed_precision.py:25-322): qkv_compress /
 * qkv_decompress with a per-coordinate choice of codebook.  Coordinate j uses
 * the outlier codebook where outlier_mask[j] != 0 (d bytes), else the regular
 * one.  Replaces MixedPrecisionMSEQuantizer.compress/decompress (:132-187;
 * mode MSE) and MixedPrecisionIPQuantizer.compress (:271-322; mode IP: the
 * QJL residual uses each coordinate's own codebook).  Codes are one uint8 per
 * coordinate (the reference stores them unpacked); grouped-row addressing as
 * above. */
int qkv_compress_mixed(int32_t mode, int32_t in_dtype, int32_t flags, const void* x,
                       int64_t n, int32_t d, const float* pi, const uint8_t* outlier_mask,
                       const float* out_bounds, const float* out_cents, int32_t out_bits,
                       const float* reg_bounds, const float* reg_cents, int32_t reg_bits,
                       const float* signs, uint8_t* codes, uint8_t* qjl, float* norms,
                       int64_t out_seq, int64_t out_group_stride, void* stream);
int qkv_decompress_mixed(int32_t mode, const uint8_t* codes, const uint8_t* qjl,
                         const float* norms, int64_t n, int32_t d,
                         const uint8_t* outlier_mask, const float* out_cents,
                         int32_t out_bits, const float* reg_cents, int32_t reg_bits,
                         const float* pi, const float* signs, float qjl_scale,
                         int64_t in_seq, int64_t in_group_stride, void* out,
                         int32_t out_dtype, void* stream);

/* ------------------------------------------------------------------------
 * Cache store formats (the engine's compressed KV cache; see qkv_store.hip).
 *
 *   K rows  ("kplanes"): one row per token, (mbits + 1) * d / 8 bytes:
 *           [MSE bit-plane 0] ... [MSE bit-plane mbits-1] [QJL plane];
 *           plane r holds bit r of each coordinate's code, coordinate j at
 *           bit j % 8 of byte j / 8.  Grouped-row addressing as above.
 *   V tiles ("vtiles"): per (sequence, kv head), tokens in tiles of 32;
 *           uint32 word[tile][plane k][coordinate j], bit (t % 32) = bit k of
 *           the code of token t at coordinate j.
 * Both hold exactly the bits of the reference's pack_bits tensors
 * (quashkv/engine.py:156-160), re-arranged so that the decode kernel can feed
 * bit planes to the matrix cores.  d must be a multiple of 32.
 * ---------------------------------------------------------------------- */

/* Bytes of one K row: (mbits + with_qjl) * d / 8; -1 if unsupported. */
int64_t qkv_kplanes_row_bytes(int32_t d, int32_t mbits, int32_t with_qjl);

/* Bytes of `tokens` tokens of V tiles (rounded up to whole tiles). */
int64_t qkv_vtiles_bytes(int32_t d, int32_t vbits, int64_t tokens);

/* n rows of one-uint8-per-code MSE codes (and QJL bits, may be NULL) into K
 * rows of stride row_bytes at grouped rows (seq, group_stride). */
int qkv_kplanes_pack(const uint8_t* codes, const uint8_t* qjl, int64_t n, int32_t d,
                     int32_t mbits, uint8_t* dst, int64_t row_bytes, int64_t seq,
                     int64_t group_stride, void* stream);

/* Inverse of qkv_kplanes_pack (codes and/or qjl may be NULL). */
int qkv_kplanes_unpack(const uint8_t* src, int64_t row_bytes, int64_t n, int32_t d,
                       int32_t mbits, int64_t seq, int64_t group_stride,
                       uint8_t* codes, uint8_t* qjl, void* stream);

/* codes: groups x S x d uint8 written as tokens [t0, t0 + S) of each group's
 * V tiles (tiles_per_group tiles per group); other tokens' bits are kept. */
int qkv_vtiles_pack(const uint8_t* codes, int64_t groups, int64_t S, int32_t d,
                    int32_t vbits, uint32_t* dst, int64_t tiles_per_group, int64_t t0,
                    void* stream);

/* Fused compress of new K and V rows straight into the store: normalise ->
 * rotate (MFMA, Pi split into two 16-bit parts) -> Lloyd-Max boundary search
 * -> QJL sign -> K-row / V-tile bit planes and norms.
 * Replaces the compress half of QuashKVEngine.append (quashkv/engine.py:
 * 145-172: InnerProductQuantizer.compress for keys, quashkv/quantizer.py:
 * 211-242, MSEQuantizer.compress for values, quashkv/quantizer.py:113-131).
 *   in_dtype   QKV_BF16, QKV_F16 or QKV_F32 (fp32 rows are divided by their
 *              norm first and split into fp16 hi + lo for the fp16 MFMA)
 *   keys, values  groups x S x d rows (d = 128, 96 or 64), 16-byte aligned;
 *              either may be NULL to append only the other
 *   mbits      key MSE bits (1..3; key total bits - 1), vbits value bits (1..4)
 *   kcent_host, kbound_host  HOST arrays of the key MSE codebook (2^mbits
 *              centroids, 2^mbits - 1 boundaries; must be symmetric);
 *   vbound_host  HOST array of the 2^vbits - 1 value boundaries
 *   kstore/knorm/vstore/vnorm  the store of groups x t_stride tokens; tokens
 *              [t0, t0 + S) of every group are written, all others kept
 * Codes equal the reference's except where the rotated value lies within
 * ~1e-5 relative of a boundary (the rotation carries ~16 significant bits of
 * Pi for bf16 inputs, ~22 for fp16 and fp32). */
int qkv_store_append(int32_t in_dtype, const void* keys, const void* values,
                     int64_t groups, int64_t S, int32_t d, int32_t mbits,
                     int32_t vbits, const float* pi, const float* signs,
                     const float* kcent_host, const float* kbound_host,
                     const float* vbound_host, uint8_t* kstore, float* knorm,
                     uint32_t* vstore, float* vnorm, int64_t t_stride, int64_t t0,
                     void* stream);

/* qkv_store_append over n_layers (1..32) contiguous stores that share shapes,
 * bit widths, codebooks, capacity t_stride and length t0 -- one decode step's
 * new token(s) for every layer of a model, in one K and one V launch instead
 * of one pair per layer (QuashKVEngine.append per layer, quashkv/engine.py:
 * 145-172).  keys, values, kpi, signs, vpi (the key quantizer's Pi and S, the
 * value quantizer's Pi), kstore, knorm, vstore and vnorm are HOST arrays of
 * n_layers device pointers, each as in qkv_store_append (keys and values both
 * required); the codebook tables are shared. */
int qkv_store_append_layers(int32_t n_layers, int32_t in_dtype, const void* const* keys,
                            const void* const* values, int64_t groups, int64_t S, int32_t d,
                            int32_t mbits, int32_t vbits, const float* const* kpi,
                            const float* const* signs, const float* const* vpi,
                            const float* kcent_host, const float* kbound_host,
                            const float* vbound_host, uint8_t* const* kstore,
                            float* const* knorm, uint32_t* const* vstore, float* const* vnorm,
                            int64_t t_stride, int64_t t0, void* stream);

/* qkv_store_append from rotated unit vectors: the search, QJL and store code
 * of qkv_store_append (the same device code, with the normalisation and the
 * rotation skipped) on given fp32 rows y = (x / |x|) Pi^T, groups x S x d,
 * with the norms to store (groups x S).  Replaces the code stage of
 * InnerProductQuantizer.compress (quashkv/quantizer.py:225-242) for keys and
 * of MSEQuantizer.compress (quashkv/quantizer.py:124-131) for values: codes
 * equal quantize_boundary(y) = #{i : t_i < y} and the QJL bits
 * [(y - c[code]) S >= 0] bit for bit, exact ties included.  yk or yv may be
 * NULL to append only the other; rows 4-byte aligned.  Contiguous store only. */
int qkv_store_append_rotated(const float* yk, const float* knorm_in, const float* yv,
                             const float* vnorm_in, int64_t groups, int64_t S, int32_t d,
                             int32_t mbits, int32_t vbits, const float* signs,
                             const float* kcent_host, const float* kbound_host,
                             const float* vbound_host, uint8_t* kstore, float* knorm,
                             uint32_t* vstore, float* vnorm, int64_t t_stride, int64_t t0,
                             void* stream);

/* Inverse of qkv_vtiles_pack: tokens [t0, t0 + S) -> groups x S x d uint8. */
int qkv_vtiles_unpack(const uint32_t* src, int64_t groups, int64_t S, int32_t d,
                      int32_t vbits, int64_t tiles_per_group, int64_t t0, uint8_t* codes,
                      void* stream);

/* ------------------------------------------------------------------------
 * Decode attention over the store.
 * Replaces QuashKVEngine.attention (quashkv/engine.py:204-299) and
 * fused_quantized_attention (quashkv/triton_kernels/attention.py:307-394),
 * with GQA: query head h reads kv head h / (Hq / Hkv).
 *   q          B x Hq x Q x d, q_dtype, contiguous
 *   kstore     B x Hkv x t_stride K rows (kbits = MSE bits of the keys)
 *   knorm      B x Hkv x t_stride fp32
 *   vstore     B x Hkv x (t_stride / 32) V tiles (vbits)
 *   vnorm      B x Hkv x t_stride fp32
 *   t_stride   token capacity (multiple of 32; 64 for the MFMA path)
 *   T          valid tokens (<= t_stride); causal masks kv_pos > T - Q + i
 *   kcent_host, vcent_host  HOST arrays of the 2^kbits / 2^vbits centroids
 *   out        B x Hq x Q x d, out_dtype
 *   workspace  >= qkv_attention_workspace_bytes(..., n_splits), 256-B aligned
 * Symmetric codebooks (all Lloyd-Max codebooks are) with d = 128 and
 * kbits <= 2 run on the integer-MFMA kernel; other shapes on a VALU kernel.
 * ---------------------------------------------------------------------- */

/* Split-K count the library would use for a decode-attention call. */
int32_t qkv_attention_splits(int32_t B, int32_t Hq, int32_t Hkv, int32_t Q,
                             int32_t d, int64_t T);

/* Workspace bytes qkv_decode_attention needs for `n_splits` splits. */
int64_t qkv_attention_workspace_bytes(int32_t B, int32_t Hq, int32_t Hkv,
                                      int32_t Q, int32_t d, int32_t n_splits);

/* 1 if a call with these parameters runs an MFMA kernel (symmetric codebooks,
 * key MSE bits <= 3, t_stride a multiple of 64), 0 for the VALU kernel, -1
 * for invalid arguments. */
int32_t qkv_attention_path(int32_t d, int32_t kbits, int32_t vbits,
                           const float* kcent_host, const float* vcent_host,
                           int64_t t_stride, int64_t T, int32_t n_splits);

int qkv_decode_attention(const void* q, int32_t q_dtype, const uint8_t* kstore,
                         const float* knorm, const uint32_t* vstore,
                         const float* vnorm, int64_t t_stride, int64_t T,
                         int32_t B, int32_t Hq, int32_t Hkv, int32_t Q,
                         int32_t d, int32_t kbits, int32_t vbits,
                         const float* pi, const float* kcent_host,
                         const float* vcent_host, const float* signs,
                         float qjl_scale, float scale, int32_t causal,
                         void* out, int32_t out_dtype, void* workspace,
                         int64_t ws_bytes, int32_t n_splits, void* stream);

/* qkv_decode_attention with per-sequence key ranges and a causal query
 * position.  Replaces the causal placement of fused_quantized_attention
 * (queries at total_kv_tokens - Q + i, quashkv/triton_kernels/attention.py:
 * 118-121) and the padding mask that HF attention applies to the reference's
 * reconstructed keys (quashkv/integrations/hf_cache.py:123-152, a left-padded
 * batch masks each sequence's leading pad positions).
 *   kv_start, kv_end  B int32 (device memory) or NULL: sequence b attends to
 *                     the keys [kv_start[b], kv_end[b]) of its T cached tokens
 *                     (NULL: 0 and T; values are clamped to [0, T]); keys
 *                     outside contribute nothing, and a sequence with none
 *                     gives zeros
 *   q_end             causal only: query i of every sequence sits at position
 *                     q_end - Q + i and sees the keys t <= q_end - Q + i;
 *                     q_end = 0 places it at kv_end[b] - Q + i (T - Q + i)
 * Other arguments as qkv_decode_attention; same workspace. */
int qkv_decode_attention_ranges(const void* q, int32_t q_dtype, const uint8_t* kstore,
                                const float* knorm, const uint32_t* vstore,
                                const float* vnorm, int64_t t_stride, int64_t T,
                                const int32_t* kv_start, const int32_t* kv_end,
                                int64_t q_end, int32_t B, int32_t Hq, int32_t Hkv,
                                int32_t Q, int32_t d, int32_t kbits, int32_t vbits,
                                const float* pi, const float* kcent_host,
                                const float* vcent_host, const float* signs,
                                float qjl_scale, float scale, int32_t causal,
                                void* out, int32_t out_dtype, void* workspace,
                                int64_t ws_bytes, int32_t n_splits, void* stream);

/* No counterpart in the reference: qkv_decode_attention for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments and results as
 * qkv_decode_attention without `workspace` / `ws_bytes`: the workspace is a
 * static device array of QKV_NOALLOC_SCRATCH_BYTES held by the library on
 * each GPU it runs on until the process ends.  A call whose workspace
 * (qkv_attention_workspace_bytes) exceeds that size returns QKV_E_INVALID.
 * The library allocates nothing on this path.  Calls that overlap on one GPU
 * (different streams or threads) share the array and race; the last call's
 * contents stay in it. */
#define QKV_NOALLOC_SCRATCH_BYTES (16 << 20)
int qkv_decode_attention_noalloc(const void* q, int32_t q_dtype, const uint8_t* kstore,
                                 const float* knorm, const uint32_t* vstore,
                                 const float* vnorm, int64_t t_stride, int64_t T,
                                 int32_t B, int32_t Hq, int32_t Hkv, int32_t Q,
                                 int32_t d, int32_t kbits, int32_t vbits,
                                 const float* pi, const float* kcent_host,
                                 const float* vcent_host, const float* signs,
                                 float qjl_scale, float scale, int32_t causal,
                                 void* out, int32_t out_dtype, int32_t n_splits,
                                 void* stream);

/* The phases qkv_decode_attention runs, exposed so a caller can overlap or
 * time them separately (same arguments and workspace, one stream):
 *   prepare  q~ = q Pi^T, w = alpha |q~| S and the MFMA query operands
 *            (quashkv/engine.py:237-238, quashkv/triton_kernels/attention.py:94,111)
 *   partial  split-K online-softmax partials (m, l, O~) over the cache
 *            (quashkv/engine.py:245-289, quashkv/triton_kernels/attention.py:97-145)
 *   combine  log-sum-exp merge of the splits, / max(l, 1e-8), x Pi once, store
 *            (quashkv/engine.py:292-297, quashkv/triton_kernels/attention.py:147-149)
 *   run      partial + combine
 * pi (d x d fp32, row-major) must be 16-byte aligned. */
int qkv_attention_prepare(const void* q, int32_t q_dtype, int32_t B, int32_t Hq,
                          int32_t Hkv, int32_t Q, int32_t d, int32_t kbits,
                          int32_t vbits, const float* pi, const float* kcent_host,
                          const float* vcent_host, const float* signs, float qjl_scale,
                          void* workspace, int64_t ws_bytes, int32_t n_splits,
                          void* stream);
int qkv_attention_partial(const uint8_t* kstore, const float* knorm,
                          const uint32_t* vstore, const float* vnorm,
                          int64_t t_stride, int64_t T, int32_t B, int32_t Hq,
                          int32_t Hkv, int32_t Q, int32_t d, int32_t kbits,
                          int32_t vbits, const float* kcent_host,
                          const float* vcent_host, float scale, int32_t causal,
                          void* workspace, int64_t ws_bytes, int32_t n_splits,
                          void* stream);
int qkv_attention_combine(int32_t B, int32_t Hq, int32_t Hkv, int32_t Q, int32_t d,
                          const float* pi, void* out, int32_t out_dtype,
                          void* workspace, int64_t ws_bytes, int32_t n_splits,
                          void* stream);
int qkv_attention_run(const uint8_t* kstore, const float* knorm,
                      const uint32_t* vstore, const float* vnorm, int64_t t_stride,
                      int64_t T, int32_t B, int32_t Hq, int32_t Hkv, int32_t Q,
                      int32_t d, int32_t kbits, int32_t vbits, const float* pi,
                      const float* kcent_host, const float* vcent_host, float scale,
                      int32_t causal, void* out, int32_t out_dtype, void* workspace,
                      int64_t ws_bytes, int32_t n_splits, void* stream);

/* One decode step over n_layers (1..32) layers sharing shapes, bit widths and
 * codebooks -- a model's layers, each with its own store, Pi, S, query and
 * output -- in one launch (decode_fused / decode_small; plus the merge of the
 * splits when there are several) instead of n_layers calls (quashkv/engine.py:
 * 204-299 per layer).  q, kstore, knorm, vstore, vnorm, pi, signs and out are
 * HOST arrays of n_layers device pointers, each as in qkv_decode_attention;
 * the other arguments are shared.  The workspace and split count are those of
 * a batch of B * n_layers sequences (qkv_attention_splits /
 * qkv_attention_workspace_bytes with B * n_layers).  MFMA path only
 * (QKV_E_UNSUPPORTED otherwise). */
int qkv_decode_attention_layers(int32_t n_layers, const void* const* q, int32_t q_dtype,
                                const uint8_t* const* kstore, const float* const* knorm,
                                const uint32_t* const* vstore, const float* const* vnorm,
                                int64_t t_stride, int64_t T, int32_t B, int32_t Hq,
                                int32_t Hkv, int32_t Q, int32_t d, int32_t kbits,
                                int32_t vbits, const float* const* pi,
                                const float* kcent_host, const float* vcent_host,
                                const float* const* signs, float qjl_scale, float scale,
                                int32_t causal, void* const* out, int32_t out_dtype,
                                void* workspace, int64_t ws_bytes, int32_t n_splits,
                                void* stream);

/* ------------------------------------------------------------------------
 * Mixed-precision keys in the store (quashkv/mixed_precision.py).  The
 * reference has no packed format or attention for these keys; it keeps one
 * uint8 per code and reconstructs keys with decompress (:160-187; the IP
 * quantizer's :283-297 adds one uint8 QJL bit per coordinate).  Here keys
 * live in rows of whole dwords (d = 128) over coordinates permuted outliers
 * first -- slot j holds rotated channel perm[j]:
 *   kmixed   MixedPrecisionMSEQuantizer (:25-197), 3-bit outlier / 2-bit
 *            regular channels: [plane b0][plane b1][b2 of the n_out outlier
 *            slots][their parity b0^b1^b2], 32 + n_out / 4 bytes (40 or 48);
 *   kipmixed MixedPrecisionIPQuantizer (:200-322) with outlier_bits 3 /
 *            regular_bits 2, i.e. a 2-bit outlier / 1-bit regular MSE stage
 *            plus a QJL bit on every coordinate: [plane b0][QJL plane][b1 of
 *            the outlier slots], 32 + n_out / 8 bytes (36 or 40).
 *   perm_host  HOST int32[128], a permutation with the n_out outlier
 *              channels (ascending) first, then the regular ones (ascending)
 *   pi_perm    device d x d fp32: row j = Pi row perm[j]
 *   signs_perm device fp32[128]: S[perm[j]] (kipmixed)
 *   n_out      32 or 64 (else QKV_E_UNSUPPORTED)
 * ---------------------------------------------------------------------- */

/* One-uint8-per-code mixed codes (n x 128, channel order) into kmixed rows at
 * grouped rows (seq, group_stride), and back. */
int qkv_kmixed_pack(const uint8_t* codes, int64_t n, const int32_t* perm_host,
                    int32_t n_out, uint8_t* dst, int64_t seq, int64_t group_stride,
                    void* stream);
int qkv_kmixed_unpack(const uint8_t* src, int64_t n, const int32_t* perm_host,
                      int32_t n_out, int64_t seq, int64_t group_stride, uint8_t* codes,
                      void* stream);
/* The same for kipmixed rows: MSE codes and QJL bits (one uint8 each, n x 128,
 * channel order), as MixedPrecisionIPQuantizer.compress returns them
 * (quashkv/mixed_precision.py:271-297). */
int qkv_kipmixed_pack(const uint8_t* codes, const uint8_t* qjl, int64_t n,
                      const int32_t* perm_host, int32_t n_out, uint8_t* dst, int64_t seq,
                      int64_t group_stride, void* stream);
int qkv_kipmixed_unpack(const uint8_t* src, int64_t n, const int32_t* perm_host,
                        int32_t n_out, int64_t seq, int64_t group_stride, uint8_t* codes,
                        uint8_t* qjl, void* stream);

/* Fused compress of bf16, fp16 or fp32 keys (groups x S x 128) straight into
 * kmixed rows and norms at tokens [t0, t0 + S) of each group: the key half of
 * qkv_store_append with MixedPrecisionMSEQuantizer.compress
 * (quashkv/mixed_precision.py:132-158) in place of InnerProductQuantizer.
 * out_bound_host (7) / reg_bound_host (3): HOST boundaries of the 3-bit and
 * 2-bit codebooks (symmetric). */
int qkv_store_append_kmixed(int32_t in_dtype, const void* keys, int64_t groups, int64_t S,
                            int32_t d, const float* pi_perm, int32_t n_out,
                            const float* out_bound_host, const float* reg_bound_host,
                            uint8_t* kstore, float* knorm, int64_t t_stride, int64_t t0,
                            void* stream);

/* qkv_store_append_kmixed from rotated unit vectors in slot order (row j of
 * y_slots' last axis = rotated channel perm[j]) with their norms: the kmixed
 * search and row store of qkv_store_append_kmixed on given y, codes equal to
 * MixedPrecisionMSEQuantizer's per-channel quantize_boundary
 * (quashkv/mixed_precision.py:140-158) bit for bit. */
int qkv_store_append_kmixed_rotated(const float* y_slots, const float* norm_in, int64_t groups,
                                    int64_t S, int32_t d, int32_t n_out,
                                    const float* out_bound_host, const float* reg_bound_host,
                                    uint8_t* kstore, float* knorm, int64_t t_stride, int64_t t0,
                                    void* stream);

/* Fused compress of bf16, fp16 or fp32 keys into kipmixed rows and norms:
 * MixedPrecisionIPQuantizer.compress (quashkv/mixed_precision.py:271-297) --
 * per-channel boundary codes, QJL bit [(y - c[code]) S >= 0] -- straight into
 * the store.  out_cent_host (4) / out_bound_host (3): HOST 2-bit outlier
 * codebook; reg_cent_host (2) / reg_bound_host (1): 1-bit regular codebook
 * (both symmetric). */
int qkv_store_append_kipmixed(int32_t in_dtype, const void* keys, int64_t groups, int64_t S,
                              int32_t d, const float* pi_perm, const float* signs_perm,
                              int32_t n_out, const float* out_cent_host,
                              const float* out_bound_host, const float* reg_cent_host,
                              const float* reg_bound_host, uint8_t* kstore, float* knorm,
                              int64_t t_stride, int64_t t0, void* stream);
/* qkv_store_append_kipmixed from rotated unit vectors in slot order with
 * their norms; codes and QJL bits equal the reference's
 * (quashkv/mixed_precision.py:283-297) bit for bit, ties included. */
int qkv_store_append_kipmixed_rotated(const float* y_slots, const float* norm_in,
                                      int64_t groups, int64_t S, int32_t d,
                                      const float* signs_perm, int32_t n_out,
                                      const float* out_cent_host, const float* out_bound_host,
                                      const float* reg_cent_host, const float* reg_bound_host,
                                      uint8_t* kstore, float* knorm, int64_t t_stride,
                                      int64_t t0, void* stream);

/* QuashKVEngine.append (quashkv/engine.py:145-172: compress_keys, then
 * compress_values) with a mixed-precision key quantizer: the key half of
 * qkv_store_append_kmixed (ip = 0; signs_perm, out_cent_host and
 * reg_cent_host may be NULL) or qkv_store_append_kipmixed (ip = 1) and the
 * value half of qkv_store_append (vbits, vpi, vbound_host, vstore, vnorm) in
 * one call, results identical to those two calls.  Small appends (a chunk of
 * a few thousand tokens per kv head) run both halves in one launch; every
 * argument is checked before anything is launched. */
int qkv_store_append_kmixed_kv(int32_t in_dtype, const void* keys, const void* values,
                               int64_t groups, int64_t S, int32_t d, const float* pi_perm,
                               const float* signs_perm, int32_t n_out, int32_t ip,
                               const float* out_cent_host, const float* out_bound_host,
                               const float* reg_cent_host, const float* reg_bound_host,
                               uint8_t* kstore, float* knorm, int32_t vbits, const float* vpi,
                               const float* vbound_host, uint32_t* vstore, float* vnorm,
                               int64_t t_stride, int64_t t0, void* stream);

/* Decode attention over kmixed K rows and V tiles: scores
 * n_k <q Pi^T, c_channel[code]> (the reference's decompress-then-attend,
 * quashkv/mixed_precision.py:160-187 with quashkv/engine.py:245-297), values
 * un-rotated by pi_v.  out_cent_host (8) / reg_cent_host (4): HOST centroids. */
int qkv_decode_attention_kmixed(const void* q, int32_t q_dtype, const uint8_t* kstore,
                                const float* knorm, const uint32_t* vstore,
                                const float* vnorm, int64_t t_stride, int64_t T, int32_t B,
                                int32_t Hq, int32_t Hkv, int32_t Q, int32_t d, int32_t vbits,
                                const float* pi_perm, int32_t n_out,
                                const float* out_cent_host, const float* reg_cent_host,
                                const float* pi_v, const float* vcent_host, float scale,
                                int32_t causal, void* out, int32_t out_dtype,
                                void* workspace, int64_t ws_bytes, int32_t n_splits,
                                void* stream);
/* Decode attention over kipmixed K rows: scores as decompress_for_dot
 * (quashkv/quantizer.py:244-279) with each channel's MSE codebook,
 * n_k (<q~, c_channel[code]> + qjl_scale sum_j |q~_j| (2 b_j - 1) S_j),
 * q~ = q Pi^T; the rest as qkv_decode_attention_kmixed.  out_cent_host (4) /
 * reg_cent_host (2): HOST centroids of the 2-bit and 1-bit MSE codebooks. */
int qkv_decode_attention_kipmixed(const void* q, int32_t q_dtype, const uint8_t* kstore,
                                  const float* knorm, const uint32_t* vstore,
                                  const float* vnorm, int64_t t_stride, int64_t T, int32_t B,
                                  int32_t Hq, int32_t Hkv, int32_t Q, int32_t d, int32_t vbits,
                                  const float* pi_perm, const float* signs_perm,
                                  float qjl_scale, int32_t n_out, const float* out_cent_host,
                                  const float* reg_cent_host, const float* pi_v,
                                  const float* vcent_host, float scale, int32_t causal,
                                  void* out, int32_t out_dtype, void* workspace,
                                  int64_t ws_bytes, int32_t n_splits, void* stream);

/* ------------------------------------------------------------------------
 * Maximum inner-product search over K rows (the index form of the key store).
 * Replaces QuashIndex.search (quashkv/nn_search/index.py:121-163): for M
 * queries against N database rows,
 *   score = n_x (<q Pi^T, c[code]> + qjl_scale sum_j |q~_j| S_j (2 b_j - 1))
 * (no 1/sqrt(d)), then the k largest per query, descending; equal scores
 * list the lower index first.  The (M, N) score matrix is never formed.
 *   queries    M x d, q_dtype
 *   d          64, 96 or 128; mbits key MSE bits 1..3 (index bits - 1)
 *   kcent_host HOST array of the 2^mbits MSE centroids (symmetric)
 *   kstore     N K rows of (mbits + 1) * d / 8 bytes (qkv_kplanes_pack layout)
 *   norms      N fp32
 *   k          <= 256 after clamping to N
 *   out_scores M x k fp32, out_indices M x k int64
 *   workspace  >= qkv_mips_workspace_bytes(M, d, mbits, k, N), 256-B aligned
 * ---------------------------------------------------------------------- */
int64_t qkv_mips_workspace_bytes(int32_t M, int32_t d, int32_t mbits, int32_t k,
                                 int64_t N);
int qkv_mips_search(const void* queries, int32_t q_dtype, int32_t M, int32_t d,
                    int32_t mbits, const float* pi, const float* signs,
                    const float* kcent_host, float qjl_scale, const uint8_t* kstore,
                    const float* norms, int64_t N, int32_t k, float* out_scores,
                    int64_t* out_indices, void* workspace, int64_t ws_bytes,
                    void* stream);

/* ------------------------------------------------------------------------
 * Paged cache store (the "preallocated, paged packed-cache format" the
 * reference's vLLM page manager leaves unimplemented: QuashKVPageManager,
 * quashkv/integrations/vllm_backend.py:82-195, whose block_size is unused).
 * A page holds P = page_tokens tokens (64, 128, ..., 2048) of all H kv heads
 * of one sequence, in the K-row and V-tile formats above: for page p, head h,
 *   kpool   rows (p H + h) P .. + P - 1, (mbits + 1) d / 8 bytes each
 *   knorm / vnorm   the same rows, fp32
 *   vpool   32-token tiles (p H + h) P / 32 .. + P / 32 - 1, vbits x d uint32
 * page_table[b * pages_per_seq + t / P] is the page of sequence b's token t
 * (int32, device).  Every sequence of a call holds the same token count.
 * num_pages is the pool's page count: an entry outside [0, num_pages) is
 * never written through (appends drop those tokens) and its tiles are read
 * from page 0 and masked out of attention, so a bad table cannot make the
 * kernels touch memory outside the pool.
 * ---------------------------------------------------------------------- */

/* qkv_store_append into a paged store: B sequences' new tokens
 * [t0, t0 + S) (keys / values (B, H, S, d), bf16, fp16 or fp32, d = 64, 96
 * or 128);
 * the pages covering them must be in the table.  Same arguments otherwise. */
int qkv_paged_store_append(int32_t in_dtype, const void* keys, const void* values,
                           int32_t B, int32_t H, int64_t S, int32_t d, int32_t mbits,
                           int32_t vbits, const float* pi, const float* signs,
                           const float* kcent_host, const float* kbound_host,
                           const float* vbound_host, uint8_t* kpool, float* knorm,
                           uint32_t* vpool, float* vnorm, const int32_t* page_table,
                           int32_t pages_per_seq, int32_t page_tokens, int32_t num_pages,
                           int64_t t0, void* stream);

/* QuashKVEngine.append (quashkv/engine.py:145-172) into a paged store: keys
 * and values of the same tokens in one call, each with its own rotation (kpi:
 * the key quantizer's Pi, vpi: the value quantizer's), results identical to
 * qkv_paged_store_append called for the keys and then for the values.  Small
 * appends (a decode step's token per sequence) run both halves in one
 * launch; every argument is checked before anything is launched. */
int qkv_paged_store_append_kv(int32_t in_dtype, const void* keys, const void* values, int32_t B,
                              int32_t H, int64_t S, int32_t d, int32_t mbits, int32_t vbits,
                              const float* kpi, const float* signs, const float* vpi,
                              const float* kcent_host, const float* kbound_host,
                              const float* vbound_host, uint8_t* kpool, float* knorm,
                              uint32_t* vpool, float* vnorm, const int32_t* page_table,
                              int32_t pages_per_seq, int32_t page_tokens, int32_t num_pages,
                              int64_t t0, void* stream);

/* qkv_decode_attention over a paged store of T tokens per sequence (the MFMA
 * path: symmetric codebooks, key MSE bits <= 3, d = 64, 96 or 128; returns
 * QKV_E_UNSUPPORTED otherwise).  Same arguments as qkv_decode_attention with
 * (kpool, knorm, vpool, vnorm, page_table, pages_per_seq, page_tokens) for the
 * store. */
int qkv_paged_decode_attention(const void* q, int32_t q_dtype, const uint8_t* kpool,
                               const float* knorm, const uint32_t* vpool, const float* vnorm,
                               const int32_t* page_table, int32_t pages_per_seq,
                               int32_t page_tokens, int32_t num_pages, int64_t T,
                               int32_t B, int32_t Hq, int32_t Hkv, int32_t Q, int32_t d,
                               int32_t kbits, int32_t vbits, const float* pi,
                               const float* kcent_host, const float* vcent_host,
                               const float* signs, float qjl_scale, float scale,
                               int32_t causal, void* out, int32_t out_dtype, void* workspace,
                               int64_t ws_bytes, int32_t n_splits, void* stream);

/* qkv_decode_attention_layers over paged stores: per-layer pools (host arrays
 * of n_layers device pointers) and one page table shared by all layers (a
 * serving engine's block table); workspace sized for B x n_layers sequences. */
int qkv_paged_decode_attention_layers(
    int32_t n_layers, const void* const* q, int32_t q_dtype, const uint8_t* const* kpool,
    const float* const* knorm, const uint32_t* const* vpool, const float* const* vnorm,
    const int32_t* page_table, int32_t pages_per_seq, int32_t page_tokens, int32_t num_pages,
    int64_t T,
    int32_t B, int32_t Hq, int32_t Hkv, int32_t Q, int32_t d, int32_t kbits, int32_t vbits,
    const float* const* pi, const float* kcent_host, const float* vcent_host,
    const float* const* signs, float qjl_scale, float scale, int32_t causal, void* const* out,
    int32_t out_dtype, void* workspace, int64_t ws_bytes, int32_t n_splits, void* stream);

/* ------------------------------------------------------------------------
 * Measurement helper (no reference counterpart): streams `bytes` (a multiple
 * of 16, 16-byte aligned) of `buf` with 16-byte loads, `unroll` (4, 8, 16)
 * per lane in flight, nontemporal loads if `nontemporal`, over `grid`
 * workgroups of 256, and writes one folded word per workgroup to sink[grid].
 * The read-only HBM ceiling the decode kernels' roofline is compared with.
 * ---------------------------------------------------------------------- */
int qkv_hbm_read_probe(const void* buf, int64_t bytes, uint32_t* sink, int32_t grid,
                       int32_t unroll, int32_t nontemporal, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QUASHKV_AMD_H */
