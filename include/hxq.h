/*
 * hxq.h -- C ABI of libhxq.so, the MI355X (gfx950) HXQ compressed-linear
 * hot path.
 *
 * Conventions (all entry points):
 *   - every pointer is a device pointer, caller-owned, contiguous, row-major;
 *   - work is enqueued on `stream` (hipStream_t; NULL = default stream) and the
 *     call returns without synchronising;
 *   - return value is an hxq_status; on error hxq_last_error() (thread-local)
 *     says what was wrong.  Nothing is launched when an argument is rejected;
 *   - no entry point allocates device memory; none keeps state between calls;
 *   - results are deterministic (no floating-point atomics).
 *
 * Tensor format (CDNAv3 + per-group affine extension):
 *   indices       uint8 [out_features, in_features]     (CDNAv3 indices.bin)
 *   codebook      fp32  [256]                            (CDNAv3 codebook.npy)
 *   group_scale   fp32  [out_features, in_features/group_size] or NULL
 *   group_offset  fp32  [out_features, in_features/group_size] or NULL
 *   sidecar as CSR over output rows, built from the flat sidecar positions
 *   (CDNAv3 sidecar.npz: positions int64, values fp16->fp32):
 *     sc_row_ptr  int32 [out_features + 1]
 *     sc_col      int32 [nnz]
 *     sc_val      fp32  [nnz]   replacement value      (dequant)
 *     sc_delta    fp32  [nnz]   value - W_affine[pos]  (contractions)
 *   Reconstructed weight:
 *     W[o,k] = fl(fl(codebook[idx[o,k]] * s[o,k/G]) + off[o,k/G])  (affine)
 *     W[o,k] = codebook[idx[o,k]]                                   (no affine)
 *     W[o,k] = sc_val  where (o,k) is a sidecar position (replacement).
 *   GEMMs with bf16/fp16 activations multiply W rounded to the activation
 *   type, the affine taken there as one rounding, fl(codebook * s + off),
 *   as the reference's GPU kernel computes it
 *   (triton_affine_group_matmul.py:99); everything that produces or
 *   contracts fp32 W uses the two-rounding form above.
 */
#ifndef HXQ_H
#define HXQ_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum hxq_status {
    HXQ_OK = 0,
    HXQ_ERR_INVALID_ARG = 1,
    HXQ_ERR_UNSUPPORTED = 2,
    HXQ_ERR_HIP = 3
} hxq_status;

typedef enum hxq_dtype {
    HXQ_F32 = 0,
    HXQ_BF16 = 1,
    HXQ_F16 = 2
} hxq_dtype;

/* Index formats (the packed index data per weight):
 *   HXQ_FMT_SCALAR   uint8 index into a <= 256-entry fp32 codebook, optional
 *                    per-group affine: W = fl(fl(cb[q] * s) + o) (1 B/weight).
 *   HXQ_FMT_VQ2_U16  2-D VQ: one uint16 index per weight pair into a
 *                    [n_codes <= 4096, 2] fp32 codebook, W[o, 2j + d] =
 *                    cb[q[o, j]][d] (1 B/weight; reference
 *                    triton_vq2d_matmul.py:1-24).
 *   HXQ_FMT_VQ2_P12  the same with the pair indices packed 12-bit, two per
 *                    3 bytes (a = byte0 | (byte1 & 15) << 8, b = byte1 >> 4 |
 *                    byte2 << 4; reference index_packing.py:1-13), rows of
 *                    in/2 indices (in % 4 == 0) (0.75 B/weight).
 *   HXQ_FMT_AF6      6-bit levels packed four per 3 bytes (q0 = b0 & 63,
 *                    q1 = b0 >> 6 | (b1 & 15) << 2, q2 = b1 >> 4 | (b2 & 3) << 4,
 *                    q3 = b2 >> 2), no codebook: W = fl(fl(q * s) + o) with
 *                    the per-group fp32 scale/offset (reference
 *                    triton_affine_group_matmul.py:181-259, 366-383)
 *                    (0.75 B/weight).
 *   HXQ_FMT_SCALAR_U16  uint16 index into a <= 4096-entry fp32 codebook (a
 *                    scalar codebook above 256 entries: reference
 *                    helix_linear.py:166-176 int16 indices, writer index_dtype
 *                    "uint16", hxq_writer_v3.py:187-198), optional per-group
 *                    affine as HXQ_FMT_SCALAR (2 B/weight).
 * Both packed forms are little-endian bit streams (field i at bit 12i / 6i of
 * the row's bytes).  The uint8 affine-group format of the same reference file
 * is HXQ_FMT_SCALAR with the identity codebook cb[j] = j. */
typedef enum hxq_format {
    HXQ_FMT_SCALAR = 0,
    HXQ_FMT_VQ2_U16 = 1,
    HXQ_FMT_VQ2_P12 = 2,
    HXQ_FMT_AF6 = 3,
    HXQ_FMT_SCALAR_U16 = 4
} hxq_format;

/* Message for the last failed call on this thread ("" if none). */
const char *hxq_last_error(void);

/*
 * ABI version of this library (bumped on any signature or struct-layout
 * change).  A caller compares hxq_abi_version() with the HXQ_ABI_VERSION it
 * was built against and refuses to run on a mismatch.
 *   1: first release.
 *   2: hxq_expert_bank gained sc_grp_ptr / sc_grp_key / sc_grp_val (the
 *      per-step sidecar lists of the register-dequant grouped GEMM).
 *   3: wide scalar encoder entry points (hxq_assign_nearest_wide,
 *      hxq_kmeans_run_wide, hxq_affine_fit_wide); hxq_kmeans_workspace_bytes
 *      sizes for codebooks of up to 4096 entries.
 */
#define HXQ_ABI_VERSION 3
int hxq_abi_version(void);

/*
 * Clocks the current device reports: peak engine clock and memory clock in
 * kHz, memory bus width in bits (for printing next to the published peaks).
 * No counterpart in the reference (its benchmarks hard-code device figures).
 */
int hxq_device_clocks(int32_t *clock_khz, int32_t *mem_clock_khz, int32_t *bus_width_bits);

/*
 * Reconstruct rows [row_begin, row_end) of W into w_out
 * (fp32 [row_end-row_begin, in_features]); bit-exact with the reference
 * reader.
 * Replaces: CDNAv3Reader.reconstruct / reconstruct_block
 *   (helix_substrate/hxq_reader_v3.py:102-140, 142-187) and
 *   HelixLinear.decode_weight / _dequant_tile (helix_linear.py:735-781, 881-888).
 * Requires in_features % 16 == 0; group_size % 16 == 0 when affine is used.
 */
int hxq_dequant_f32(const uint8_t *indices, const float *codebook,
                    const float *group_scale, const float *group_offset,
                    int32_t group_size, const int32_t *sc_row_ptr,
                    const int32_t *sc_col, const float *sc_val,
                    int64_t out_features, int64_t in_features,
                    int64_t row_begin, int64_t row_end, float *w_out,
                    hipStream_t stream);

/*
 * Decode GEMV: y[n, :] = x[n, :] @ W^T (+ bias) for n < n_rows (1 <= n_rows <= 4).
 * x is fp32/bf16/fp16 [n_rows, in_features]; arithmetic and accumulation in
 * fp32; y is written in y_dtype [n_rows, out_features].
 * Replaces: fused_vq_matmul with N == 1 -> _vq_decode_dotprod_kernel +
 *   _sidecar_fused_kernel + bias (helix_substrate/triton_vq_matmul.py:521-633,
 *   670-692, 724-725), called from HelixLinear._forward_fused
 *   (helix_linear.py:468-502).
 * Requires in_features % 16 == 0, group_size % 16 == 0 (affine).
 */
int hxq_gemv(const void *x, int32_t x_dtype, const uint8_t *indices,
             const float *codebook, const float *group_scale,
             const float *group_offset, int32_t group_size,
             const int32_t *sc_row_ptr, const int32_t *sc_col,
             const float *sc_delta, const float *bias, void *y,
             int32_t y_dtype, int64_t n_rows, int64_t out_features,
             int64_t in_features, hipStream_t stream);

/*
 * Several HXQ matrices that read the same activation (q/k/v, gate/up) in one
 * launch.  Each descriptor is one HelixLinear; all share in_features and
 * group_size.  At most HXQ_MAX_MULTI matrices.
 * Replaces: consecutive HelixLinear.forward calls on one input
 *   (helix_linear.py:318-361), one fused_vq_matmul each.
 */
#define HXQ_MAX_MULTI 8
typedef struct hxq_matrix {
    const uint8_t *indices;
    const float *codebook;
    const float *group_scale;
    const float *group_offset;
    const int32_t *sc_row_ptr;
    const int32_t *sc_col;
    const float *sc_delta;
    const float *bias;
    void *y;
    int64_t out_features;
} hxq_matrix;

/*
 * hxq_gemv_fmt: hxq_gemv for any index format (HXQ_FMT_*); y = x W^T (+ bias),
 * 1-4 activation rows, fp32 accumulation, sidecar CSR in weight coordinates
 * (sc_delta = value - reconstruction).  Pair formats take `codebook`
 * [n_codes, 2] and no affine; HXQ_FMT_AF6 takes the affine and no codebook;
 * HXQ_FMT_SCALAR_U16 takes `codebook` [n_codes <= 4096] and an optional
 * affine.  Indices must lie below n_codes (reads past it give 0).
 * Replaces: the decode branches of fused_vq2d_matmul
 * (triton_vq2d_matmul.py:171-280, with the 12-bit gather of
 * triton_gather_12bit.py:43-157) and fused_affine_group_matmul_packed6
 * (triton_affine_group_matmul.py:181-259, 262-363).
 * hxq_dequant_fmt: the reconstruction W (fp32 rows [row_begin, row_end)),
 * sidecar values replacing (as hxq_dequant_f32); replaces naive_vq2d_matmul's
 * W / dequant_vq2d_tile (triton_vq2d_matmul.py:283-336) and
 * unpack_12bit_rows (index_packing.py:75-95).
 */
int hxq_gemv_fmt(const void *x, int32_t x_dtype, int32_t format, const uint8_t *indices,
                 const float *codebook, int32_t n_codes, const float *group_scale,
                 const float *group_offset, int32_t group_size, const int32_t *sc_row_ptr,
                 const int32_t *sc_col, const float *sc_delta, const float *bias, void *y,
                 int32_t y_dtype, int64_t n_rows, int64_t out_features, int64_t in_features,
                 hipStream_t stream);
int hxq_dequant_fmt(int32_t format, const uint8_t *indices, const float *codebook,
                    int32_t n_codes, const float *group_scale, const float *group_offset,
                    int32_t group_size, const int32_t *sc_row_ptr, const int32_t *sc_col,
                    const float *sc_val, int64_t out_features, int64_t in_features,
                    int64_t row_begin, int64_t row_end, float *w_out, hipStream_t stream);

int hxq_gemv_multi(const void *x, int32_t x_dtype, const hxq_matrix *mats,
                   int32_t n_mats, int32_t group_size, int32_t y_dtype,
                   int64_t in_features, hipStream_t stream);

/*
 * hxq_gemv_multi with the activation built on load (one fp32 row, K =
 * in_features), so a decoder step needs no separate norm / SiLU launch:
 *   _rmsnorm: r = x + delta (delta NULL: r = x); h = bf16(norm_w * r *
 *     rsqrt(mean(r^2) + eps)); y_m = W_m h.  res_out (optional, must not alias
 *     x or delta) receives r, written once.
 *   _silu:    h = bf16(silu(gate) * up); y_m = W_m h.
 * No reference counterparts: they fuse transformers' Qwen2RMSNorm
 * (models/qwen2/modeling_qwen2.py:247-253) / Qwen2MLP act(gate) * up into the
 * HelixLinear.forward GEMV that follows them.
 */
int hxq_gemv_multi_rmsnorm(const float *x, const float *delta, const float *norm_w, float eps,
                           float *res_out, const hxq_matrix *mats, int32_t n_mats,
                           int32_t group_size, int32_t y_dtype, int64_t in_features,
                           hipStream_t stream);
int hxq_gemv_multi_silu(const float *gate, const float *up, const hxq_matrix *mats,
                        int32_t n_mats, int32_t group_size, int32_t y_dtype, int64_t in_features,
                        hipStream_t stream);

/*
 * Prefill GEMM: Y[m, :] = X[m, :] @ W^T (+ bias), X bf16 or fp16 [m_rows,
 * in_features], W dequantised tile by tile into LDS (sidecar values replace
 * their elements, then W is rounded to X's 16-bit type) and multiplied with
 * MFMA, fp32 accumulation; Y in y_dtype [m_rows, out_features].
 * The affine factors come in the GEMM's layout group_affine fp32
 * [in/G][out][2] = {scale, offset} (NULL = no affine), built from the
 * [out, in/G] scale/offset arrays by hxq_affine_pack.
 * Replaces: fused_vq_matmul with N > 1 -> _vq_gather_matmul_tiled_kernel +
 *   scatter_add sidecar + bias (helix_substrate/triton_vq_matmul.py:634-661,
 *   693-698, 724-725) and HelixLinear._forward_buffered (helix_linear.py:556-634).
 * Requires in_features % 64 == 0 and, with affine, group_size % 64 == 0.
 * sc_val are the replacement values (as for hxq_dequant_f32); columns
 * ascending within a row.
 */
int hxq_gemm(const void *x, int32_t x_dtype, const uint8_t *indices,
             const float *codebook, const float *group_affine, int32_t group_size,
             const int32_t *sc_row_ptr, const int32_t *sc_col,
             const float *sc_val, const float *bias, void *y, int32_t y_dtype,
             int64_t m_rows, int64_t out_features, int64_t in_features,
             hipStream_t stream);
/*
 * hxq_gemm_ws: hxq_gemm with a workspace.  When the output tiles
 * (128 x 256) cover under half of the compute units, K is split into up to 8
 * ranges run in parallel, each writing fp32 partials to the workspace, and a
 * second launch adds the ranges in order (then the bias) into y; results are
 * deterministic.  workspace_bytes >= hxq_gemm_workspace_bytes(m_rows,
 * out_features, in_features) (0 when no split is planned; a NULL workspace
 * runs unsplit, as hxq_gemm does).
 * Replaces: the same reference paths as hxq_gemm.
 */
int64_t hxq_gemm_workspace_bytes(int64_t m_rows, int64_t out_features, int64_t in_features);
int hxq_gemm_ws(const void *x, int32_t x_dtype, const uint8_t *indices,
                const float *codebook, const float *group_affine, int32_t group_size,
                const int32_t *sc_row_ptr, const int32_t *sc_col, const float *sc_val,
                const float *bias, void *y, int32_t y_dtype, int64_t m_rows,
                int64_t out_features, int64_t in_features, void *workspace,
                int64_t workspace_bytes, hipStream_t stream);

/*
 * hxq_prefill_gemm: the prefill GEMM Y = X W^T (+ bias) with W dequantised
 * straight into the MFMA operand registers (X [m_rows, in] in bf16 or fp16:
 * 16-bit MFMA on W rounded to X's type; or fp32: fp32 MFMA on the exact fp32
 * W; fp32 accumulation, y in y_dtype; in_features % 64 == 0), for every
 * index format (HXQ_FMT_*): uint8 with the 256-entry
 * codebook, uint16 with n_codes entries, pair codebooks [n_codes, 2] (uint16
 * or 12-bit packed indices, no affine) and 6-bit levels (affine, no
 * codebook).  The sidecar comes in the kernel's order: for each group of 64
 * output rows g (rows [64g, 64g + 64)), its entries sorted by column then row
 * (stable): sc_grp_key uint32 (col << 6) | (row - 64g), sc_grp_val fp32
 * replacement values, and sc_grp_ptr int32 [ceil(out/64) * (in/64) + 1]
 * whose element g * (in/64) + t is the first entry of group g with a column
 * in K step t ([64t, 64t + 64)) or later, the last element being the entry
 * count (NULL sc_grp_ptr = no sidecar).  group_affine is fp32
 * [ceil(in / group_size), out, 2] {scale, offset} (the layout hxq_affine_pack
 * writes) for any group_size that is a positive multiple of 16; a caller
 * whose true K is not a multiple of 64 pads X and the index rows with zero
 * columns up to in_features and the affine with groups of (0, 0), so the
 * padded columns contribute nothing.  Shapes with few output tiles split K: a
 * workspace of hxq_prefill_gemm_workspace_bytes(...) bytes holds fp32
 * partials, reduced in order (deterministic).
 * Replaces: fused_vq_matmul's N > 1 path (triton_vq_matmul.py:249-334,
 * 634-661, 693-698, 724-725) and HelixLinear._forward_buffered
 * (helix_linear.py:556-634).
 */
int64_t hxq_prefill_gemm_workspace_bytes(int64_t m_rows, int64_t out_features,
                                         int64_t in_features);
int hxq_prefill_gemm(const void *x, int32_t x_dtype, int32_t format, const uint8_t *indices,
                     const float *codebook, int32_t n_codes, const float *group_affine,
                     int32_t group_size,
                     const int32_t *sc_grp_ptr, const uint32_t *sc_grp_key,
                     const float *sc_grp_val, const float *bias, void *y, int32_t y_dtype,
                     int64_t m_rows, int64_t out_features, int64_t in_features,
                     void *workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * hxq_gemm_noalloc: hxq_gemm_ws without a workspace argument and without any
 * allocation: the split-K partials live in a static device array of
 * hxq_gemm_noalloc_max_bytes() bytes (64 MiB) that each GPU the library runs
 * on holds until the process ends.  Same arguments and results as
 * hxq_gemm_ws (same kernels, same K split).  Shapes whose partials need more
 * than the array (hxq_gemm_workspace_bytes above the maximum) are rejected
 * with HXQ_ERR_INVALID_ARG.  Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (several streams) race.  The stream must
 * belong to the current device.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).
 */
int64_t hxq_gemm_noalloc_max_bytes(void);
int hxq_gemm_noalloc(const void *x, int32_t x_dtype, const uint8_t *indices,
                     const float *codebook, const float *group_affine, int32_t group_size,
                     const int32_t *sc_row_ptr, const int32_t *sc_col, const float *sc_val,
                     const float *bias, void *y, int32_t y_dtype, int64_t m_rows,
                     int64_t out_features, int64_t in_features, hipStream_t stream);

/*
 * group_affine[g][o] = {group_scale[o][g], group_offset[o][g]} (fp32): the
 * GEMM layout of the per-group affine factors (n_groups = in/G).
 * No reference counterpart: the affine extension has no reference layout;
 * HelixLinear builds this once as a derived buffer.
 */
int hxq_affine_pack(const float *group_scale, const float *group_offset, int64_t out_features,
                    int64_t n_groups, float *group_affine, hipStream_t stream);

/*
 * Mixture-of-experts FFN over HXQ experts (OLMoE-style SwiGLU experts).
 * The reference has no MoE kernel: HelixLinear replaces per-expert nn.Linear
 * modules only (helix_substrate/hf_quantizer.py:231-249), so each expert runs
 * HelixLinear.forward (helix_linear.py:318-361) on its routed tokens.  These
 * entry points run all experts of a layer in one grouped launch instead.
 *
 * An expert bank stacks the per-expert HXQ arrays along a leading expert
 * axis: indices [E, out, in] u8, codebook [E, 256], group_affine
 * [E, in/G, out, 2] in the GEMM layout (hxq_affine_pack per expert; NULL = no
 * affine), sc_row_ptr [E, out+1] holding ABSOLUTE offsets into sc_col/sc_val
 * (replacement values), columns ascending within a row.
 */
typedef struct hxq_expert_bank {
    const uint8_t *indices;
    const float *codebook;
    const float *group_affine;
    const int32_t *sc_row_ptr;
    const int32_t *sc_col;
    const float *sc_val;
    /* The same sidecar in the prefill GEMM's order (see hxq_prefill_gemm), per
     * expert: sc_grp_ptr [E, ceil(out/64) * in/64 + 1] holding ABSOLUTE
     * offsets into sc_grp_key / sc_grp_val.  With it (or without any
     * sidecar) the grouped entry points below run the register-dequant MFMA
     * kernel of hxq_prefill_gemm; NULL with a CSR sidecar: the LDS-dequant
     * kernel of hxq_gemm. */
    const int32_t *sc_grp_ptr;
    const uint32_t *sc_grp_key;
    const float *sc_grp_val;
} hxq_expert_bank;

/*
 * Routing: p = softmax(logits[t, :]) (fp32 [n_tokens, n_experts], n_experts <=
 * 256, top_k <= 64); the top_k
 * experts by logit (ties -> lower id) with weights p (renormalised to sum 1
 * when `renormalize`); then the expert-sorted assignment list: expert e owns
 * sorted positions [expert_offsets[e], expert_offsets[e+1]) in token order,
 * sorted_rows[pos] = token, assign_pos[t*top_k + s] = pos of slot s of t.
 * Outputs: topk_ids i32 / topk_weights f32 [n_tokens, top_k], expert_counts
 * [E], expert_offsets [E+1], sorted_rows / assign_pos [n_tokens*top_k].
 * Replaces: the router of transformers' OlmoeSparseMoeBlock (softmax ->
 * topk, norm_topk_prob=False), which the reference leaves to the HF model.
 */
int hxq_moe_route(const float *logits, int64_t n_tokens, int32_t n_experts, int32_t top_k,
                  int32_t renormalize, int32_t *topk_ids, float *topk_weights,
                  int32_t *expert_counts, int32_t *expert_offsets, int32_t *sorted_rows,
                  int32_t *assign_pos, hipStream_t stream);

/*
 * Grouped GEMM: for each expert e and each sorted position pos in its
 * segment, Y[pos, :] = X[row(pos), :] @ W_e^T with row(pos) = sorted_rows[pos]
 * (or pos itself when sorted_rows is NULL, X then holding n_assign rows).
 * X bf16/fp16 [x_rows, in]; Y y_dtype [n_assign, out].  W_e dequantised
 * straight into MFMA operand registers as in hxq_prefill_gemm (uint8
 * indices; banks with sc_grp_*) or into LDS as in hxq_gemm (otherwise).
 * Replaces: HelixLinear.forward per expert (helix_linear.py:318-361) on that
 * expert's token rows.
 */
int hxq_moe_grouped_gemm(const void *x, int32_t x_dtype, int64_t x_rows,
                         const int32_t *sorted_rows, const int32_t *expert_offsets,
                         int64_t n_assign, int32_t n_experts, const hxq_expert_bank *bank,
                         int32_t group_size, void *y, int32_t y_dtype, int64_t out_features,
                         int64_t in_features, hipStream_t stream);

/*
 * Whole SwiGLU MoE FFN from a routing (hxq_moe_route):
 *   H = silu(X Wg_e^T) * (X Wu_e^T)   (x's dtype)
 *   O = H Wd_e^T                       (sorted order; x's dtype with register-dequant
 *                                       banks, as the reference's experts return it,
 *                                       else fp32)
 * With register-dequant banks (sc_grp_*, see hxq_expert_bank) gate and up
 * run as one grouped launch into [n_assign, 2 * intermediate] in x's dtype
 * (each projection's output rounded like the module's; the workspace holds
 * it), then the SiLU product; otherwise one LDS-dequant launch with the
 * SiLU-product epilogue on the fp32 sums.
 *   y[t] = sum_s topk_weights[t, s] * O[assign_pos[t*top_k + s]]  (slots in order, fp32 sum)
 * x bf16/fp16 [n_tokens, hidden], or fp32 (fp32 MFMA on the exact fp32 W,
 * fp32 H; register-dequant banks only); y y_dtype [n_tokens, hidden].  `workspace`
 * (device, 256-B aligned, >= hxq_moe_ffn_workspace_bytes) holds H, O and the
 * gate/up outputs.
 * Replaces: the expert loop of OlmoeSparseMoeBlock.forward with HelixLinear
 * experts (helix_linear.py:318-361 per expert projection).
 */
int64_t hxq_moe_ffn_workspace_bytes(int64_t n_tokens, int64_t hidden, int64_t intermediate,
                                    int32_t top_k);

int hxq_moe_ffn(const void *x, int32_t x_dtype, int64_t n_tokens, int64_t hidden,
                int64_t intermediate, int32_t n_experts, int32_t top_k,
                const float *topk_weights, const int32_t *expert_offsets,
                const int32_t *sorted_rows, const int32_t *assign_pos,
                const hxq_expert_bank *gate, const hxq_expert_bank *up,
                const hxq_expert_bank *down, int32_t group_size, void *workspace,
                int64_t workspace_bytes, void *y, int32_t y_dtype, hipStream_t stream);

/*
 * Mamba2 mixer around the scan.  in_proj's output row is laid out
 *   [d_mlp | d_mlp | gate (d_inner) | xBC (d_inner + 2*ngroups*state) | dt (heads)]
 * (proj_width = 2*d_mlp + 2*d_inner + 2*ngroups*state + heads), as split by
 * the reference mixer (helix_substrate/mamba_scan_chunked.py:256-261).
 *
 * hxq_mamba2_conv_split (prefill): causal depthwise conv1d of width `width`
 * over xBC with left zero padding, + conv_b, SiLU, split into x [b, L, d_inner]
 * (= [b, L, heads, d_inner/heads]), B and C [b, L, ngroups, state]
 * (out_dtype); dt[b, L, heads] = clamp(softplus(dt_raw + dt_bias), dt_min,
 * dt_max) in fp32.  conv_w fp32 [conv_dim, width]; conv_state (optional, fp32
 * [b, conv_dim, width]) receives the last `width` raw xBC inputs.
 * Replaces: mamba_scan_chunked.py:296-310 (conv + act + split) and :356-357
 *   (dt transform) of _chunked_scan_forward.
 */
int hxq_mamba2_conv_split(const void *proj, int32_t proj_dtype, const float *conv_w,
                          const float *conv_b, const float *dt_bias, float dt_min, float dt_max,
                          int64_t batch, int64_t seqlen, int64_t d_mlp, int64_t d_inner,
                          int64_t ngroups, int64_t state, int64_t heads, int64_t width,
                          void *x, void *B, void *C, int32_t out_dtype, float *dt,
                          float *conv_state, hipStream_t stream);

/*
 * hxq_mamba2_conv_step (decode, one token per batch row): conv_state rolls
 * left by one and takes the new raw xBC input, x/B/C = silu(sum(conv_state *
 * conv_w) + conv_b) and dt as above.  proj [b, proj_width].
 * Replaces: mamba_scan_chunked.py:269-282 (single-token conv update).
 */
int hxq_mamba2_conv_step(const void *proj, int32_t proj_dtype, const float *conv_w,
                         const float *conv_b, const float *dt_bias, float dt_min, float dt_max,
                         int64_t batch, int64_t d_mlp, int64_t d_inner, int64_t ngroups,
                         int64_t state, int64_t heads, int64_t width, float *conv_state,
                         void *x, void *B, void *C, int32_t out_dtype, float *dt,
                         hipStream_t stream);

/*
 * Gated RMSNorm: h = y * silu(gate); out = weight * h * rsqrt(mean(h^2) + eps)
 * per row, the mean taken over groups of group_size columns (0 = the whole
 * row).  y [rows, width]; gate rows are gate_row_stride elements apart (a
 * column slice of in_proj's output); weight fp32 [width].
 * Replaces: self.norm(y, gate) (mamba_scan_chunked.py:384; transformers
 *   MambaRMSNormGated.forward, models/mamba2/modeling_mamba2.py:111-120).
 */
int hxq_gated_rmsnorm(const void *y, int32_t y_dtype, const void *gate, int32_t gate_dtype,
                      int64_t gate_row_stride, const float *weight, float eps, int64_t rows,
                      int64_t width, int64_t group_size, void *out, int32_t out_dtype,
                      hipStream_t stream);

/*
 * Batch-1 decoder step pieces around the HXQ GEMVs (Qwen2-shaped greedy
 * decoding).  The position `pos` is a device int so one captured HIP graph
 * replays every step; hxq_argmax advances it.  No reference counterparts:
 * the reference runs these parts in transformers' Qwen2 model (models/qwen2/
 * modeling_qwen2.py: Qwen2RMSNorm :247-253, apply_rotary_pos_emb :113-135,
 * eager attention :150-170, Qwen2MLP) around HelixLinear projections.
 *
 * hxq_add_rmsnorm: x fp32 [rows, hidden] += delta (optional, delta_dtype);
 *   out = weight * x * rsqrt(mean(x^2) + eps) in out_dtype.
 * hxq_rope_kv_append: qkv fp32 [(n_heads + 2 n_kv) * D] of one token; rotates
 *   q and k at *pos (rotate_half, inv_freq = theta^(-2i/D)), writes q_out fp32
 *   [n_heads*D] and k/v rows *pos of the caches [max_seq, n_kv, D].
 * hxq_attn_decode: per query head softmax(q.k_t / sqrt(D), t <= *pos) . v_t,
 *   GQA (head h reads kv head h / (n_heads/n_kv)); out [n_heads*D]; D = 128.
 * hxq_silu_mul: out = silu(gate) * up (fp32 inputs).
 * hxq_dense_gemv_bf16: y fp32 [rows] = W bf16 [rows, in] . x (the
 *   uncompressed LM head).
 * hxq_argmax: *out_id = argmax(logits) (ties -> lowest index); ++*pos when
 *   pos is not NULL; workspace: device scratch of >= 2048 bytes (partials).
 * hxq_dense_gemv_bf16 needs in_features % 8 == 0 and a 16-byte aligned weight.
 */
int hxq_add_rmsnorm(float *x, const void *delta, int32_t delta_dtype, const float *weight,
                    float eps, int64_t rows, int64_t hidden, void *out, int32_t out_dtype,
                    hipStream_t stream);
int hxq_rope_kv_append(const float *qkv, const int32_t *pos, int32_t n_heads, int32_t n_kv_heads,
                       int32_t head_dim, float theta, float *q_out, void *k_cache, void *v_cache,
                       int32_t cache_dtype, int32_t max_seq, hipStream_t stream);
int hxq_attn_decode(const float *q, const void *k_cache, const void *v_cache,
                    int32_t cache_dtype, const int32_t *pos, int32_t n_heads,
                    int32_t n_kv_heads, int32_t head_dim, int32_t max_seq, void *out,
                    int32_t out_dtype, hipStream_t stream);
int hxq_silu_mul(const float *gate, const float *up, int64_t n, void *out, int32_t out_dtype,
                 hipStream_t stream);
/* hxq_attn_rope_decode: hxq_rope_kv_append + hxq_attn_decode in one launch
 * (qkv fp32 row in; k/v of position *pos stored into the caches). */
int hxq_attn_rope_decode(const float *qkv, const int32_t *pos, int32_t n_heads,
                         int32_t n_kv_heads, int32_t head_dim, float theta, void *k_cache,
                         void *v_cache, int32_t cache_dtype, int32_t max_seq, void *out,
                         int32_t out_dtype, hipStream_t stream);
int hxq_dense_gemv_bf16(const uint16_t *weight, const void *x, int32_t x_dtype, int64_t rows,
                        int64_t in_features, float *y, hipStream_t stream);
int hxq_argmax(const float *logits, int64_t n, int32_t *out_id, int32_t *pos,
               void *workspace, hipStream_t stream);

/*
 * CDNAv3 encoder (k-means codebook, assignment, percentile sidecar), with the
 * reference's numpy results reproduced bit for bit (fp32 argmin with first
 * index on ties; cluster means as numpy's fp32 pairwise sums over 8192-element
 * blocks; numpy's 'linear' percentiles).
 *
 * hxq_assign_nearest: indices[i] = argmin_j |x[i] - codebook[j]| (k <= 256).
 *   Replaces: CDNAv3Writer._chunked_assign / _gpu_assign
 *   (helix_substrate/hxq_writer_v3.py:449-487).
 * hxq_kmeans_init: sorts x (keys in the workspace, kept for hxq_kmeans_run)
 *   and counts its distinct values into *n_unique (device int32).
 * hxq_kmeans_run: k centroids initialised at the percentiles
 *   percentiles01[j] (fp64, the reference's np.linspace(0, 100, k) / 100) of
 *   the sorted sample, then up to max_iters Lloyd steps on the device, stopping
 *   when the largest centroid move is below rtol * (c[k-1] - c[0]); writes
 *   codebook fp32 [k], assignments u8 [n] (of the last assignment step) and
 *   *iters (device int32).  Same workspace as hxq_kmeans_init, called before
 *   on the same x.  max_iters >= 1 (with none the reference has no
 *   assignments).
 *   Replaces: _simple_kmeans (helix_substrate/hxq_encoder.py:107-177).
 * hxq_select_f32: values[r] = the ranks[r]-th smallest element (0-based,
 *   numpy sort order, NaN last) for m <= 4 ranks (device int64 ranks);
 *   *nan_count (optional, device) = number of NaNs.
 * hxq_outliers_f32: positions (ascending) and values of x < lohi[0] or
 *   x > lohi[1] (device fp32 thresholds); *count (device int64) = total, at
 *   most `capacity` written.
 *   With hxq_select_f32 these replace find_outliers_percentile
 *   (helix_substrate/generate_sidecars_v3.py:18-40).
 */
int hxq_assign_nearest(const float *x, int64_t n, const float *codebook, int32_t k,
                       uint8_t *indices, hipStream_t stream);
int64_t hxq_sort_workspace_bytes(int64_t n);
int64_t hxq_kmeans_workspace_bytes(int64_t n);
int hxq_kmeans_init(const float *x, int64_t n, void *workspace, int64_t workspace_bytes,
                    int32_t *n_unique, hipStream_t stream);
int hxq_kmeans_run(const float *x, int64_t n, const double *percentiles01, int32_t k,
                   int32_t max_iters, double rtol, void *workspace, int64_t workspace_bytes,
                   float *codebook, uint8_t *assignments, int32_t *iters, hipStream_t stream);
/*
 * Wide scalar codebooks (257..4096 entries, uint16 indices): the same
 * algorithms and arithmetic as hxq_assign_nearest / hxq_kmeans_run /
 * hxq_affine_fit with k <= 4096 (the same k-means workspace).
 *   Replace: the scalar path of CDNAv3Writer._write_quantized for
 *   n_clusters > 256 (helix_substrate/hxq_writer_v3.py:189-198, uint16
 *   indices), _simple_kmeans on its GPU branch (_gpu_kmeans,
 *   helix_substrate/hxq_encoder.py:180-207: integer assignments, so every
 *   cluster above 255 is updated; the CPU branch's uint8 cast at :160 would
 *   fold clusters mod 256).
 */
int hxq_assign_nearest_wide(const float *x, int64_t n, const float *codebook, int32_t k,
                            uint16_t *indices, hipStream_t stream);
int hxq_kmeans_run_wide(const float *x, int64_t n, const double *percentiles01, int32_t k,
                        int32_t max_iters, double rtol, void *workspace, int64_t workspace_bytes,
                        float *codebook, uint16_t *assignments, int32_t *iters, hipStream_t stream);
int64_t hxq_select_workspace_bytes(void);
int hxq_select_f32(const float *x, int64_t n, const int64_t *ranks, int32_t m, float *values,
                   int32_t *nan_count, void *workspace, int64_t workspace_bytes,
                   hipStream_t stream);
/*
 * Pair-codebook (vector_dim 2) encoder steps, with the reference's numpy CPU
 * arithmetic reproduced bit for bit.  x is fp32 [n, 2] (adjacent column
 * pairs of the weight), the codebook fp32 [k, 2], 1 <= k <= 4096.
 *
 * hxq_vq2_assign: indices[i] = argmin_j fl(fl(|x_i|^2 + |c_j|^2) - 2 x_i.c_j)
 *   with |v|^2 = fl(fl(v0 v0) + fl(v1 v1)), x.c = fma(x1, c1, fl(x0 c0)),
 *   first index on ties.  workspace >= 16 * k bytes.
 *   Replaces: the assignment of _vector_kmeans (helix_substrate/
 *   hxq_encoder.py:280-289, 305-313) and CDNAv3Writer._chunked_vector_assign
 *   (helix_substrate/hxq_writer_v3.py:373-420).
 * hxq_vq2_update: new_centroids[j] = fp32(sum of the pairs assigned to j /
 *   fp32 count) with fp64 sums (a fixed-order two-level sum), or centroids[j]
 *   if none is; *max_delta (device fp32) = max |new - old|.  indices < k.
 *   workspace >= hxq_vq2_workspace_bytes(n, k) (at most about 42 MB at
 *   k = 4096).  new_centroids must not alias centroids.
 *   Replaces: the bincount update of _vector_kmeans
 *   (helix_substrate/hxq_encoder.py:291-303).
 * hxq_vq2_min_dist: dmin[i] = max(0, min_j d(x[rows[i]], c_j)) (the same
 *   fp32 distance; rows NULL: row i, m <= n) -- the seeding distances of the
 *   k-means++ initialisation (helix_substrate/hxq_encoder.py:241-251,
 *   np.maximum(dists, 0) then min over the seeds).  An out-of-range row gives
 *   NaN.  workspace >= 16 * k bytes.
 * The seeding's draws (a sequential RandomState(42) stream) stay on the
 * host, as in the reference.
 */
int64_t hxq_vq2_workspace_bytes(int64_t n, int32_t k);
int hxq_vq2_assign(const float *x, int64_t n, const float *codebook, int32_t k,
                   uint16_t *indices, void *workspace, int64_t workspace_bytes,
                   hipStream_t stream);
int hxq_vq2_min_dist(const float *x, int64_t n, const int64_t *rows, int64_t m,
                     const float *codebook, int32_t k, float *dmin, void *workspace,
                     int64_t workspace_bytes, hipStream_t stream);
int hxq_vq2_update(const float *x, int64_t n, const uint16_t *indices, int32_t k,
                   const float *centroids, float *new_centroids, float *max_delta,
                   void *workspace, int64_t workspace_bytes, hipStream_t stream);
/*
 * hxq_affine_fit: per-group affine of the encoder (an extension with no
 * reference counterpart: the benchmark configs' group_scale / group_offset,
 * fp32 [rows, cols / group_size]).  For each row and group of group_size
 * columns, (s, o) minimise sum (s * codebook[idx] + o - w)^2 over the group's
 * elements whose flat position is not in exclude_positions (the sidecar,
 * which replaces them); fp64 sums in a fixed order (lane l of a 64-lane wave
 * adds elements l, l + 64, ... in turn, then a xor butterfly 32 ... 1),
 * closed form in fp64, rounded to fp32.  Groups with fewer than two elements
 * or a zero determinant keep s = 1 and o = mean(w - c) (0 if empty).
 * workspace: hxq_affine_fit_workspace_bytes(rows, cols) bytes (an exclusion
 * bitmap), needed only when n_exclude > 0; positions must be < rows * cols.
 */
int64_t hxq_affine_fit_workspace_bytes(int64_t rows, int64_t cols);
int hxq_affine_fit(const float *w, const uint8_t *indices, const float *codebook, int32_t k,
                   int64_t rows, int64_t cols, int32_t group_size,
                   const int64_t *exclude_positions, int64_t n_exclude, void *workspace,
                   int64_t workspace_bytes, float *scale, float *offset, hipStream_t stream);
/* hxq_affine_fit for uint16 indices and codebooks of up to 4096 entries. */
int hxq_affine_fit_wide(const float *w, const uint16_t *indices, const float *codebook, int32_t k,
                        int64_t rows, int64_t cols, int32_t group_size,
                        const int64_t *exclude_positions, int64_t n_exclude, void *workspace,
                        int64_t workspace_bytes, float *scale, float *offset, hipStream_t stream);
int64_t hxq_outliers_workspace_bytes(int64_t n);
int hxq_outliers_f32(const float *x, int64_t n, const float *lohi, int64_t capacity,
                     int64_t *positions, float *values, int64_t *count, void *workspace,
                     int64_t workspace_bytes, hipStream_t stream);

/*
 * Whole greedy decode step in ONE launch per token (persistent kernel, one
 * 16-wave block per compute unit; inside a layer the stages exchange
 * activations as epoch-tagged words that consumers poll, with each stage's
 * compressed weights fetched before it waits; a grid barrier only before the
 * LM head and the argmax).
 * Per layer: r = x + delta, q/k/v = W norm(r) (+bias); RoPE, KV append and
 * GQA attention; o = W_o attn; r' = r + o, act = silu(W_g norm(r')) *
 * (W_u norm(r')); delta = W_d act.  Then logits = E norm(x + delta) (tied
 * bf16 embedding E), *token = argmax (ties -> lowest id), ++*pos.  The step
 * embeds *token at position *pos; out_ids[i] (optional) receives the token
 * fed into step i.  Same math as the per-kernel sequence above.
 * No reference counterpart: it replaces the HF decoder-layer loop around
 * HelixLinear.forward (helix_linear.py:318-361) for benchmark config 1.
 *
 * hxq_decoder_layer holds one layer's seven HXQ matrices (the y fields are
 * ignored), fp32 norm weights and bf16 caches [max_seq, n_kv_heads, 128].
 * hxq_decoder: sizes, a HOST array of layers, device embedding / final norm,
 * device token and position words, device fp32 logits [vocab].
 * Limits: hidden 512..3584 (multiple of 512), head_dim 128, max_seq <= 1024,
 * n_heads <= number of compute units, intermediate <= 16384 (above hidden
 * 2048: <= 24576 within the 160 KB LDS budget, e.g. Qwen2.5-7B's 18944).
 * hxq_decoder_init copies the layer table into `workspace` (device, 256-byte
 * aligned, >= hxq_decoder_workspace_bytes) and clears the barrier state;
 * hxq_decoder_step runs n_steps tokens (n_steps launches, no host sync);
 * hxq_decoder_error copies the barrier error word (0 = fine; 1 = a wait
 * for other blocks timed out; 2 = token/position out of range) to *err_out and
 * synchronises the stream.  A workspace serves one stream at a time.
 */
typedef struct hxq_decoder_layer {
    hxq_matrix q, k, v, o, gate, up, down;
    const float *in_norm;
    const float *post_norm;
    uint16_t *k_cache;
    uint16_t *v_cache;
} hxq_decoder_layer;

typedef struct hxq_decoder {
    int32_t hidden, n_layers, n_heads, n_kv_heads, head_dim, intermediate, vocab, max_seq;
    int32_t group_size;
    float rms_eps;
    float rope_theta;
    const hxq_decoder_layer *layers;
    const uint16_t *embed;
    const float *final_norm;
    int32_t *token;
    int32_t *pos;
    float *logits;
} hxq_decoder;

int64_t hxq_decoder_workspace_bytes(const hxq_decoder *d);
int hxq_decoder_init(const hxq_decoder *d, void *workspace, int64_t workspace_bytes,
                     hipStream_t stream);
int hxq_decoder_step(const hxq_decoder *d, void *workspace, int32_t n_steps, int32_t *out_ids,
                     hipStream_t stream);
int hxq_decoder_error(const void *workspace, const hxq_decoder *d, int32_t *err_out,
                      hipStream_t stream);

/*
 * Selective scan (Mamba/Mamba2), fp32 state, chunk-parallel:
 *   a_t = exp(A[h] dt[b,t,h]);  h_t = a_t h_{t-1} + dt[b,t,h] x[b,t,h,p] B[b,t,g,n]
 *   y[b,t,h,p] = sum_n h_t C[b,t,g,n] + D[h] x[b,t,h,p],  g = h / (heads/ngroups)
 * Layouts: x [batch, seqlen, heads, head_dim]; dt [batch, seqlen, heads];
 * A, D fp32 [heads]; B, C [batch, seqlen, ngroups, state]; h0 / h_final fp32
 * [batch, heads, head_dim, state] (h0 NULL = zeros, h_final may be NULL);
 * y [batch, seqlen, heads, head_dim].  x/dt/B/C/y dtypes: HXQ_F32/BF16/F16.
 * `workspace` (device, >= hxq_ssm_scan_workspace_bytes(...)) holds the chunk
 * states; state must be 16, 32, 64, 128 or 256.
 * Replaces: chunked_scan / sequential_scan (helix_substrate/mamba_scan_chunked.py:
 *   42-86, 89-213) and triton_scan (triton_mamba_scan.py:373-416).
 */
int64_t hxq_ssm_scan_workspace_bytes(int64_t batch, int64_t seqlen, int64_t heads,
                                     int64_t head_dim, int64_t state, int64_t chunk);

int hxq_ssm_chunk_scan(const void *x, int32_t x_dtype, const void *dt, int32_t dt_dtype,
                       const float *A, const void *B, const void *C, int32_t bc_dtype,
                       const float *D, const float *h0, void *y, int32_t y_dtype,
                       float *h_final, int64_t batch, int64_t seqlen, int64_t heads,
                       int64_t head_dim, int64_t state, int64_t ngroups, int64_t chunk,
                       void *workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * One decode step; h (fp32 [batch, heads, head_dim, state]) is updated in place.
 * x [batch, heads, head_dim], dt [batch, heads], B/C [batch, ngroups, state],
 * y [batch, heads, head_dim].
 * Replaces: triton_mamba_decode_step (triton_mamba_scan.py:312-366) and the
 *   single-token branch of chunked_scan (mamba_scan_chunked.py:150-159).
 */
int hxq_ssm_decode_step(const void *x, int32_t x_dtype, const void *dt, int32_t dt_dtype,
                        const float *A, const void *B, const void *C, int32_t bc_dtype,
                        const float *D, float *h, void *y, int32_t y_dtype, int64_t batch,
                        int64_t heads, int64_t head_dim, int64_t state, int64_t ngroups,
                        hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* HXQ_H */
