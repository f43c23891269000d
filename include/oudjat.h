/*
 * oudjat.h -- C ABI of the gfx950 token-correction library (liboudjat_hip.so).
 *
 * The library implements the server-side DINOv3 token-correction pass of AppCorr ("Oudjat"):
 * top-k token selection, row gather/scatter, the in-place K/V row rewrite, sparse-query attention,
 * the selected-row GEMMs with their fused epilogues, the residual reconstruct/scatter/persist step
 * and NVFP4 quantize/dequantize.
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers. bf16 tensors are passed as uint16_t bit patterns.
 *   - Strides and row strides are in ELEMENTS of the tensor's own type unless the name ends in
 *     `_bytes`. Index tensors are int64 (torch.long), contiguous.
 *   - `stream` is a hipStream_t (NULL = the legacy default stream). Every call only enqueues work
 *     on that stream: no host synchronisation, no device-to-host reads, no allocation.
 *   - The return value is an oudjat status. OUDJAT_OK is 0; anything else means nothing was
 *     launched (argument/shape/layout errors) or the launch failed. oudjat_last_error() gives a
 *     message for the calling thread's most recent failure.
 *   - Scatter entry points assume the (batch, token) pairs of one call are unique.
 *
 * Reference interfaces named below are files of ckswjd99-lab/AppCorr, cited as path:line.
 */
#ifndef OUDJAT_H
#define OUDJAT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* oudjat_stream_t; /* hipStream_t */

enum oudjat_status {
  OUDJAT_OK = 0,
  OUDJAT_ERR_INVALID_ARGUMENT = 1, /* null pointer, negative size, bad enum */
  OUDJAT_ERR_UNSUPPORTED_SHAPE = 2, /* a dimension the kernels do not handle (e.g. K % 64 != 0) */
  OUDJAT_ERR_UNSUPPORTED_LAYOUT = 3, /* strides or alignment the kernels do not handle */
  OUDJAT_ERR_TOO_LARGE = 4,         /* exceeds a documented maximum (e.g. LDS capacity) */
  OUDJAT_ERR_LAUNCH = 5,            /* the kernel launch itself failed */
  OUDJAT_ERR_HIP = 6                /* another HIP runtime call failed */
};

/* GEMM epilogues for oudjat_linear_bf16. acc = A.W^T in fp32; every bf16() is one RNE rounding. */
enum oudjat_epilogue {
  OUDJAT_EPI_BIAS = 0,          /* C = bf16(acc + bias)                                  */
  OUDJAT_EPI_BIAS_GELU = 1,     /* C = bf16(gelu_erf(bf16(acc + bias)))                  */
  OUDJAT_EPI_BIAS_LS_RESID = 2, /* C = bf16(resid + bf16(acc + bias) * gamma)            */
  OUDJAT_EPI_BIAS_LS = 3,       /* C = bf16(bf16(acc + bias) * gamma)                    */
  OUDJAT_EPI_BIAS_SILU_MUL = 4, /* C = bf16(bf16(silu(bf16(acc + bias))) * resid)        */
  /* Flag OR-ed into any of the above but the GELU one (oudjat_linear_bf16): the accumulator is first
   * rounded to bf16 and then scaled, bf16(acc + bias) becoming bf16(bf16(acc) * acc_scale + bias) -- an
   * NVFP4 linear's bf16 _scaled_mm output followed by its scale and bias (fp4_fast_linear.py:221-283);
   * the bias must then be 16-byte aligned. */
  OUDJAT_EPI_RAW_BF16 = 16
};

/* Importance modes for oudjat_patch_importance. */
enum oudjat_importance {
  OUDJAT_IMPORTANCE_L2 = 0,     /* sqrt(sum d^2)   */
  OUDJAT_IMPORTANCE_ENERGY = 1, /* sum d^2         */
  OUDJAT_IMPORTANCE_RMS = 2     /* sqrt(mean d^2)  */
};

/* ABI version of this header (bumped on any signature change). */
int oudjat_abi_version(void);
const char* oudjat_status_string(int status);
const char* oudjat_last_error(void);

/* Runtime self-test: launches y = 2x on 8 floats and checks the result (the one entry point that
 * synchronises). Replaces verify_triton_runtime
 * (appcorr/models/dinov3/layers/triton_kernels/_strict.py:74-125). */
int oudjat_selftest(oudjat_stream_t stream);

/* Row 1 -- per-patch importance from a residual delta [rows, dim] fp32.
 * Replaces _compute_patch_residual_rms (offload/server/model/dinov3_classifier.py:91-122) and the
 * mobile residual energy (offload/policies/transmission/progressive.py:19-22). */
int oudjat_patch_importance(const float* delta, int64_t rows, int64_t dim, int64_t row_stride,
                            int mode, float* out, oudjat_stream_t stream);

/* Next-rank row f4 -- per-patch pixel-residual importance of HWC images, the residual formed on the
 * fly. Replaces _compute_patch_residual_rms (offload/server/model/dinov3_classifier.py:91-122:
 * mode RMS, curr / prev the decoded frames, image_idx the active images) and the mobile crop scores
 * _compute_patch_residual_rms / _energy (offload/policies/transmission/progressive.py:14-22: prev
 * NULL, curr the int16 Laplacian residual).
 * curr, prev [n_images, H, W, C] row-major, dtype 0 = uint8, 1 = int16, 2 = fp32; prev may be NULL;
 * image_idx [n_out] int64 selects the images scored (NULL: images 0 .. n_out-1; an index outside
 * [0, n_images) scores NaN). out [n_out, (H/ph) * (W/pw)] fp32, patches row-major.
 * d = fp32(curr) - fp32(prev); each d*d rounded to fp32; the sum over the patch's ph*pw*C values
 * in float64 in a fixed order (exact for uint8 / int16), then rounded: ENERGY = fp32(sum),
 * RMS = sqrt(fp32(sum / n)), L2 = sqrt(fp32(sum)), square roots correctly rounded.
 * Requires H % ph == 0, W % pw == 0, (W/pw) * ph <= 8192. */
int oudjat_patch_residual_score(const void* curr, const void* prev, int dtype, int64_t n_images,
                                const int64_t* image_idx, int64_t n_out, int64_t H, int64_t W, int64_t C,
                                int64_t ph, int64_t pw, int mode, float* out, oudjat_stream_t stream);

/* Next-rank row f4 -- image-residual token pruning, the kept set and its statistics:
 * _apply_image_residual_token_pruning (offload/server/model/dinov3_classifier.py:124-196, :143-154).
 * r[b, p] = rms[b, spatial[b, p]] (NaN for an index outside [0, G)); keep = r >= thres (fp32) or r
 * among the min(min_keep, P) largest of the row (torch.topk; ties to the lower candidate index, NaN
 * largest, as oudjat_topk_plan). keep [B, P] (1 byte), kept_count [B] int32,
 * kept_mass[b] = sum_p r * keep, full_mass[b] = sum_p r (float64 sums in a fixed order, rounded to fp32;
 * an unkept inf / NaN makes kept_mass NaN as r * keep.float() does). P <= 16384. */
int oudjat_residual_prune_keep(const float* rms, int64_t B, int64_t rms_stride_b, int64_t G,
                               const int64_t* spatial, int64_t spatial_stride_b, int64_t P, float thres,
                               int64_t min_keep, uint8_t* keep, int32_t* kept_count, float* kept_mass,
                               float* full_mass, oudjat_stream_t stream);

/* Next-rank row f4 -- the pruned candidate list (dinov3_classifier.py:163-196) at `width` (the largest
 * kept count, read back by the caller as the reference does): pruned_dindice [B, num_pre + width] =
 * dindice[b, :num_pre], then spatial[b, p] + num_pre of the kept candidates in candidate order, then
 * num_pre (a zero spatial index) for the rest; kept_local_idx [B, width] = the kept candidate
 * positions, 0 past the count. */
int oudjat_residual_prune_compact(const uint8_t* keep, int64_t B, int64_t P, const int64_t* spatial,
                                  int64_t spatial_stride_b, const int64_t* dindice, int64_t dindice_stride_b,
                                  int64_t num_pre, int64_t width, int64_t* pruned_dindice,
                                  int64_t* kept_local_idx, oudjat_stream_t stream);

/* Rows 2+3 -- top-k selection and the sync-free packed query plan, one workgroup per image.
 * Replaces torch.topk in _select_patch_keep_mask (appcorr/models/dinov3/layers/block.py:358-395)
 * and _build_packed_query_state_fixed_k / _all_keep (block.py:397-490).
 * scores [B, P] fp32 (row stride score_stride_b); k in [0, P]; dindice [B, num_pre + P] int64.
 * Keeps the k largest scores per row; among equal scores the lower candidate index wins
 * (-0.0 == +0.0; NaN ranks above +inf). Kept candidates are emitted in ascending candidate order.
 * Outputs (T = num_pre + k, M = B * T):
 *   update_indice [B, T], active_batch_idx [M], active_pos_idx [M], active_token_idx [M],
 *   active_patch_mask [M] (1 byte: token >= num_pre), active_rope_idx [M] (max(token-num_pre, 0)),
 *   keep_mask [B, P] (1 byte, may be NULL),
 *   row_slot [B, num_tokens] int32 (packed row b*T+s of token t of image b, or -1; may be NULL).
 * Limits: P <= 16384, (P + num_tokens) * 4 bytes <= 144 KiB. */
/* Rows 2+3 -- the plan's running statistics, _compute_partial_token_plan_stats
 * (appcorr/models/dinov3/layers/block.py:762-788): out[5] fp32 = {sum(scores * keep),
 * sum(scores), sum(keep), B * P, B} for scores [B, P] fp32 (row stride score_stride_b) and the
 * keep_mask [B, P] of oudjat_topk_plan. One workgroup, fixed summation order (deterministic);
 * an unkept -inf score makes the first sum NaN, as (scores * keep.float()).sum() does. */
int oudjat_plan_stats(const float* scores, int64_t B, int64_t P, int64_t score_stride_b,
                      const uint8_t* keep_mask, float* out, oudjat_stream_t stream);

int oudjat_topk_plan(const float* scores, int64_t B, int64_t P, int64_t score_stride_b, int64_t k,
                     const int64_t* dindice, int64_t dindice_stride_b, int64_t num_pre,
                     int64_t num_tokens, int64_t* update_indice, int64_t* active_batch_idx,
                     int64_t* active_pos_idx, int64_t* active_token_idx,
                     uint8_t* active_patch_mask, int64_t* active_rope_idx, uint8_t* keep_mask,
                     int32_t* row_slot, oudjat_stream_t stream);

/* Threshold selection (next-rank row f3) -- the kept mask and per-image kept count of
 * _select_patch_keep_mask's threshold branch (appcorr/models/dinov3/layers/block.py:374-376):
 * keep_mask[b, p] = scores[b, p] >= thres, compared in fp32 as torch compares an fp32 tensor with a
 * Python float (the float rounded to fp32 first; NaN never kept); kept_count[b] int32. keep_mask may
 * be NULL. This is what the padded builder (block.py:562-621) reads back to size its plan. */
int oudjat_threshold_keep(const float* scores, int64_t B, int64_t P, int64_t score_stride_b, float thres,
                          uint8_t* keep_mask, int32_t* kept_count, oudjat_stream_t stream);

/* Threshold selection and its packed query plan at a fixed width of `width` patch slots (T =
 * num_pre + width rows per image, M = B * T). Replaces _build_packed_query_state_thres_static
 * (block.py:492-560, fill_mode 0, width = min(token_keep_cap, P)) and _build_packed_query_state
 * (block.py:562-621, fill_mode 1, width = the largest kept count from oudjat_threshold_keep).
 * Kept candidates (scores >= thres, as above) fill slots num_pre.. in candidate order; kept ranks at
 * or past `width` are dropped. Slots past an image's kept count:
 *   fill_mode 0: the image's last kept candidate (candidate 0 if it keeps none), query_valid 1 --
 *     block.py:536-541;
 *   fill_mode 1: update_indice 0 and query_valid 0 (block.py:571-599); the packed rows (active_*)
 *     repeat the image's last valid row -- its last kept candidate, else its last pretoken -- which
 *     computes and writes exactly what that row does, so the rows at query_valid equal the
 *     reference's compacted PackedQueryState. An image with no valid row at all (num_pre == 0 and
 *     nothing kept) must not reach this mode; the caller checks kept_count first.
 * Outputs: update_indice [B, T], active_batch_idx/pos_idx/token_idx [M], active_patch_mask [M],
 * active_rope_idx [M] as oudjat_topk_plan; query_valid [B, T] (1 byte); keep_mask [B, P] (may be
 * NULL); kept_count [B] int32; row_slot [B, num_tokens] int32 = the first packed row holding the token,
 * or -1 (may be NULL). Limits: width <= P <= 16384, num_tokens * 4 bytes <= 144 KiB. */
int oudjat_threshold_plan(const float* scores, int64_t B, int64_t P, int64_t score_stride_b, float thres,
                          int64_t width, int fill_mode, const int64_t* dindice, int64_t dindice_stride_b,
                          int64_t num_pre, int64_t num_tokens, int64_t* update_indice,
                          int64_t* active_batch_idx, int64_t* active_pos_idx, int64_t* active_token_idx,
                          uint8_t* active_patch_mask, int64_t* active_rope_idx, uint8_t* query_valid,
                          uint8_t* keep_mask, int32_t* kept_count, int32_t* row_slot,
                          oudjat_stream_t stream);

/* Rows 4 and 11 -- dst[i, :] = src[batch_idx[i], token_idx[i], :] for row_bytes contiguous bytes.
 * Replaces gather_rows_triton (appcorr/models/dinov3/layers/triton_kernels/token_update.py:455-473).
 * Strides are in bytes. */
int oudjat_gather_rows(const void* src, int64_t src_stride_b_bytes, int64_t src_stride_n_bytes,
                       int64_t row_bytes, const int64_t* batch_idx, const int64_t* token_idx,
                       int64_t n, void* dst, int64_t dst_row_stride_bytes, oudjat_stream_t stream);

/* Rows 8 and 9 -- dst[batch_idx[i], token_idx[i], :] = src[i, :] (the in-place K/V rewrite and the
 * query scatter). Replaces scatter_rows_triton (token_update.py:417-452); src_row_stride_bytes
 * covers row views such as qkv_new[:, 1:] whose row stride is 3C while the row is 2C. */
int oudjat_scatter_rows(void* dst, int64_t dst_stride_b_bytes, int64_t dst_stride_n_bytes,
                        int64_t row_bytes, const int64_t* batch_idx, const int64_t* token_idx,
                        int64_t n, const void* src, int64_t src_row_stride_bytes,
                        oudjat_stream_t stream);

/* Row 15 -- x_out[batch_idx[i], token_idx[i], :] = bf16(x_attn[i] + x_delta[i]) (bf16, C columns).
 * Replaces active_token_update_triton (token_update.py:297-347). */
int oudjat_active_token_update(uint16_t* x_out, int64_t stride_b, int64_t stride_n,
                               const int64_t* batch_idx, const int64_t* token_idx, int64_t n,
                               const uint16_t* x_attn, int64_t attn_row_stride,
                               const uint16_t* x_delta, int64_t delta_row_stride, int64_t C,
                               oudjat_stream_t stream);

/* Rows 14+15+16 fused -- for every row r of [rows, C] (rows = B*N, contiguous):
 *   slot = row_slot[r];
 *   slot < 0 : x_out[r] = bf16(x[r] + blocks_out_sum[r])
 *   slot >= 0: x_out[r] = bf16(x_attn[slot] + mlp[slot]);
 *              blocks_out_sum[r] = bf16(bf16(x_attn[slot] - x_act[slot]) + mlp[slot])
 * x_out may alias x (inplace_residual_add). Replaces block.py:1140-1179 (x + blocks_out_sum,
 * active_token_update_triton, and the blocks_out_sum index_put_). */
int oudjat_reconstruct_scatter_persist(const uint16_t* x, uint16_t* blocks_out_sum,
                                       const int32_t* row_slot, const uint16_t* x_act,
                                       const uint16_t* x_attn, const uint16_t* mlp, int64_t rows,
                                       int64_t C, uint16_t* x_out, oudjat_stream_t stream);

/* Rows 14-16, selected half, for selected rows kept packed across blocks (the executor's multi-block
 * correction, dinov3_classifier.py:591-663 over block.py:1140-1179): for packed row i
 *   x_new[i] = bf16(x_attn[i] + mlp[i]);  bos[b_i, t_i] = bf16(bf16(x_attn[i] - x_act[i]) + mlp[i])
 * with b_i = batch_idx[i], t_i = token_idx[i]; bos addressed with element strides (b, n). */
int oudjat_packed_residual_persist(const uint16_t* x_act, const uint16_t* x_attn, const uint16_t* mlp,
                                   int64_t rows, int64_t C, const int64_t* batch_idx,
                                   const int64_t* token_idx, uint16_t* bos, int64_t bos_stride_b,
                                   int64_t bos_stride_n, uint16_t* x_new, oudjat_stream_t stream);

/* oudjat_packed_residual_persist fused with the next block's first LayerNorm (block.py:1114 of
 * block l + 1 after block.py:1140-1179 of block l): additionally ln_out[i] = LayerNorm(x_new[i]) with
 * weight ln_w, bias ln_b, eps, computed on the bf16 x_new exactly as oudjat_layernorm_rows does.
 * x_act, x_attn, mlp, x_new, ln_out: [rows, C] contiguous. */
int oudjat_packed_residual_persist_ln(const uint16_t* x_act, const uint16_t* x_attn, const uint16_t* mlp,
                                      int64_t rows, int64_t C, const int64_t* batch_idx,
                                      const int64_t* token_idx, uint16_t* bos, int64_t bos_stride_b,
                                      int64_t bos_stride_n, uint16_t* x_new, const uint16_t* ln_w,
                                      const uint16_t* ln_b, float eps, uint16_t* ln_out,
                                      oudjat_stream_t stream);

/* Row 14 over a run of n_blocks correction blocks (block.py:1143-1149 applied block after block):
 * x, out [rows, C] (rows = B*N, contiguous; out may alias x); row r with row_slot[r] >= 0 takes
 * x_packed[row_slot[r]]; every other row takes x + bos_0 + ... + bos_{n-1} rounded to bf16 after
 * each addition, bos_rows = device array of n_blocks pointers to [rows, C] blocks_out_sum tensors. */
int oudjat_fold_residual_rows(const uint16_t* x, int64_t rows, int64_t C, const int32_t* row_slot,
                              const uint16_t* x_packed, const uint16_t* const* bos_rows,
                              int64_t n_blocks, uint16_t* out, oudjat_stream_t stream);

/* Row 12 -- out = bf16(x + attn * gamma[c]) over [rows, C] contiguous.
 * Replaces fused_layerscale_add (token_update.py:10-60). */
int oudjat_fused_layerscale_add(const uint16_t* x, const uint16_t* attn, const uint16_t* gamma,
                                int64_t rows, int64_t C, uint16_t* out, oudjat_stream_t stream);

/* The approximate block's two residual sums in one launch (block.py:336-347, the cache producer):
 * bos = bf16(inc + mlp) (inc = ls1(attn), the cached {tag}_blocks_out_sum) and out = bf16(x_attn + mlp)
 * (the block output), all [rows, C] bf16 contiguous -- the same bits as two oudjat_fused_layerscale_add
 * calls with a gamma of ones. 16-byte aligned rows, C % 8 == 0, C <= 8192. */
int oudjat_residual_pair(const uint16_t* inc, const uint16_t* x_attn, const uint16_t* mlp, int64_t rows, int64_t C,
                         uint16_t* bos, uint16_t* out, oudjat_stream_t stream);

/* Row 7 -- rotate-half RoPE on q and k rows [n, H, Dh] in place, fp32 math, rows with
 * patch_mask == 0 untouched; table row rope_idx[i] of sin/cos [*, Dh] fp32.
 * Replaces apply_rope_active_inplace_triton (appcorr/models/dinov3/layers/triton_kernels/rope.py:186-240). */
int oudjat_rope_active_inplace(uint16_t* q, int64_t q_stride_t, int64_t q_stride_h, uint16_t* k,
                               int64_t k_stride_t, int64_t k_stride_h, const float* sin_table,
                               const float* cos_table, int64_t table_stride,
                               const uint8_t* patch_mask, const int64_t* rope_idx, int64_t n,
                               int64_t H, int64_t Dh, oudjat_stream_t stream);

/* Rows 6-9 fused -- post-QKV step of SelfAttention.correct_partial_token
 * (appcorr/models/dinov3/layers/attention.py:415-454): qkv [M, 3, H, Dh] bf16 contiguous;
 * RoPE on q and k of patch rows; k, v rows written into kv[b, t, 0|1, H, Dh] (row stride
 * kv_stride_n, batch stride kv_stride_b, elements); q written packed into q_out [M, H, Dh]. */
int oudjat_qkv_rope_kv_scatter(const uint16_t* qkv, int64_t M, int64_t H, int64_t Dh,
                               const float* sin_table, const float* cos_table,
                               int64_t table_stride, const uint8_t* patch_mask,
                               const int64_t* rope_idx, const int64_t* batch_idx,
                               const int64_t* token_idx, uint16_t* kv, int64_t kv_stride_b,
                               int64_t kv_stride_n, uint16_t* q_out, oudjat_stream_t stream);

/* Row 5 -- LayerNorm over the last dim (fp32 statistics, biased variance, affine), bf16 in/out.
 * Replaces nn.LayerNorm(eps=1e-5) at block.py:1114,1141. C % 8 == 0, C <= 8192. */
int oudjat_layernorm_rows(const uint16_t* x, int64_t rows, int64_t C, int64_t x_row_stride,
                          const uint16_t* weight, const uint16_t* bias, float eps, uint16_t* out,
                          int64_t out_row_stride, oudjat_stream_t stream);

/* Row 5 -- oudjat_layernorm_rows (same output bits) that also reads one 32-bit word of every whole
 * 128-byte line of the read-only device region [prefetch, prefetch + prefetch_bytes) in the same
 * launch, so that the region is resident in the last-level cache when the kernels after it run:
 * block.py:1141's norm2 warming the weights of the MLP's second linear (ffn_layers.py:48), whose
 * first-touch misses would otherwise wait on HBM. Nothing is written to the region. The reference's
 * LayerNorm has no such argument (a cache hint with no effect on results). prefetch_bytes >= 0;
 * prefetch 4-byte aligned and non-NULL when prefetch_bytes > 0; 0 bytes is oudjat_layernorm_rows. */
int oudjat_layernorm_rows_prefetch(const uint16_t* x, int64_t rows, int64_t C, int64_t x_row_stride,
                                   const uint16_t* weight, const uint16_t* bias, float eps, uint16_t* out,
                                   int64_t out_row_stride, const void* prefetch, int64_t prefetch_bytes,
                                   oudjat_stream_t stream);

/* Rows 6, 11, 12, 13 -- C[M, N] = epilogue(A[M, K] . W[N, K]^T) on bf16 MFMA with fp32 accumulate.
 * Replaces the qkv / proj / fc1 / fc2 nn.Linear calls (attention.py:415,532; ffn_layers.py:43-49)
 * and the LayerScale / residual ops folded into their epilogues (block.py:1129-1141); the SwiGLU
 * gate silu(w1 x) * (w2 x) (ffn_layers.py:106-115) is the SILU_MUL epilogue with resid = w2 x.
 * bias, gamma, resid may be NULL where the epilogue does not use them (bias NULL = 0).
 * acc_scale multiplies the fp32 accumulator before the first rounding: every epilogue starts from
 * bf16(acc * acc_scale + bias) (one rounding; 1.0 gives bf16(acc + bias) exactly). It carries the
 * per-tensor scales of an FP8 GEMM (torch._scaled_mm's scale_a * scale_b, fp8_fast_linear.py:187-194)
 * whose e4m3 operands were passed as their exact bf16 values.
 * workspace (fp32, workspace_elems elements, may be NULL): scratch for split K. When the output tiles
 * of a shape would leave most of the GPU idle (a small M), the call may split K over S slices that run
 * side by side, writing fp32 partial tiles to the workspace, and sum them in slice order in a second
 * launch that applies the epilogue; it does so only if S * M * N <= workspace_elems
 * (oudjat_linear_workspace_elems gives that size; 0: the shape never splits). A split result differs
 * from the unsplit one only in the fp32 summation order; both are deterministic.
 * K % 64 == 0, N % 64 == 0, all leading dimensions % 8 == 0 and 16-byte aligned pointers. */
int oudjat_linear_bf16(const uint16_t* A, int64_t M, int64_t K, int64_t lda, const uint16_t* W,
                       int64_t N, int64_t ldw, const uint16_t* bias, int epilogue,
                       const uint16_t* gamma, const uint16_t* resid, int64_t ldr, uint16_t* C,
                       int64_t ldc, float acc_scale, float* workspace, int64_t workspace_elems,
                       oudjat_stream_t stream);

/* Rows 6, 11, 12, 13 -- oudjat_linear_bf16 (same output bits) that also reads one 32-bit word of
 * every whole 128-byte line of the read-only device region [warm, warm + warm_bytes) into the caches
 * from the CUs the launch leaves idle: when the product is not split and has fewer output tiles than
 * the GPU has CUs, the launch carries extra workgroups that do only that, on the otherwise idle CUs
 * (the weight of a later launch: the correction block's proj warming its fc1 weight, fc1 its fc2
 * weight, fc2 the next block's qkv weight). Elsewhere it is oudjat_linear_bf16. The reference's
 * linears have no such argument (a cache hint with no effect on results). warm_bytes >= 0; warm 4-byte
 * aligned and non-NULL when warm_bytes > 0. */
int oudjat_linear_bf16_warm(const uint16_t* A, int64_t M, int64_t K, int64_t lda, const uint16_t* W,
                            int64_t N, int64_t ldw, const uint16_t* bias, int epilogue,
                            const uint16_t* gamma, const uint16_t* resid, int64_t ldr, uint16_t* C,
                            int64_t ldc, float acc_scale, float* workspace, int64_t workspace_elems,
                            const void* warm, int64_t warm_bytes, oudjat_stream_t stream);

/* The number of warming workgroups an oudjat_linear_bf16_warm call of this shape and epilogue (with
 * 16-byte aligned operands and the workspace oudjat_linear_workspace_elems names) adds: 0 when its
 * tiles fill the GPU or it splits K, so that a caller can warm the region some other way. No
 * counterpart in the reference. */
int64_t oudjat_linear_warm_slots(int64_t M, int64_t N, int64_t K, int epilogue);

/* The workspace (fp32 elements) oudjat_linear_bf16 can use for an M x N x K product with this
 * epilogue; 0 when it would not split K. No counterpart in the reference (cuBLAS sizes its own). */
int64_t oudjat_linear_workspace_elems(int64_t M, int64_t N, int64_t K, int epilogue);

/* Rows 13 + 14-16 across a kernel boundary -- the fc2 (or SwiGLU w3) product of a correction block,
 * split K, with its reduce left to the residual step (ffn_layers.py:24-115 into block.py:1140-1186):
 * the partial GEMM of oudjat_linear_bf16 alone. Writes the S fp32 slices [S, M, N] of A . W^T to
 * workspace and S to *slices (host memory); fails with OUDJAT_ERR_UNSUPPORTED_SHAPE when the product
 * would not split K (oudjat_linear_workspace_elems(M, N, K, OUDJAT_EPI_BIAS_LS) == 0) or the workspace
 * is shorter than that. Same operand rules as oudjat_linear_bf16; 16-byte aligned workspace. */
int oudjat_linear_splitk_partial(const uint16_t* A, int64_t M, int64_t K, int64_t lda, const uint16_t* W,
                                 int64_t N, int64_t ldw, float* workspace, int64_t workspace_elems,
                                 int64_t* slices, oudjat_stream_t stream);

/* The reduce of oudjat_linear_splitk_partial's slices with the LayerScale epilogue, fused with
 * oudjat_packed_residual_persist_ln (block.py:1140-1186, then :1114 of the next block):
 * mlp = bf16(bf16(sum_s partials[s] * acc_scale + fc_bias) * ls_gamma) (slices summed in order, as
 * oudjat_linear_bf16's split-K reduce), then x_new, the blocks_out_sum rows and LayerNorm(x_new)
 * exactly as oudjat_packed_residual_persist_ln computes them from that mlp. ln_w, ln_b and ln_out are
 * all NULL for the last block of a run (no LayerNorm). partials [slices, rows, C] fp32; fc_bias may be
 * NULL; 16-byte aligned rows, C % 8 == 0, C <= 8192. */
int oudjat_splitk_ls_packed_residual(const float* partials, int64_t slices, const uint16_t* fc_bias,
                                     const uint16_t* ls_gamma, float acc_scale, const uint16_t* x_act,
                                     const uint16_t* x_attn, int64_t rows, int64_t C,
                                     const int64_t* batch_idx, const int64_t* token_idx, uint16_t* bos,
                                     int64_t bos_stride_b, int64_t bos_stride_n, uint16_t* x_new,
                                     const uint16_t* ln_w, const uint16_t* ln_b, float eps, uint16_t* ln_out,
                                     oudjat_stream_t stream);

/* Rows 6-9 fused into the QKV GEMM -- SelfAttention.correct_partial_token up to the attention call
 * (appcorr/models/dinov3/layers/attention.py:415-454): qkv = A . W^T + bias for A [M, K] and
 * W [3*H*Dh, K] (never materialised), then RoPE on q and k of patch rows (rotate-half, fp32, tables
 * [*, Dh] fp32 with row stride table_stride), q written packed into q_out [M, H, Dh] and k, v into
 * kv[b, t, 0|1, H, Dh] at b = batch_idx[m], t = token_idx[m] (strides in elements).
 * Same arithmetic as oudjat_linear_bf16 (OUDJAT_EPI_BIAS, same acc_scale) followed by
 * oudjat_qkv_rope_kv_scatter.
 * K % 64 == 0, Dh in {16, 32, 64, 128}, H*Dh % 128 == 0; 16-byte aligned operands and rows. */
int oudjat_linear_qkv_rope_kv(const uint16_t* A, int64_t M, int64_t K, int64_t lda, const uint16_t* W,
                              int64_t ldw, const uint16_t* bias, int64_t H, int64_t Dh,
                              const float* sin_table, const float* cos_table, int64_t table_stride,
                              const uint8_t* patch_mask, const int64_t* rope_idx,
                              const int64_t* batch_idx, const int64_t* token_idx, uint16_t* kv,
                              int64_t kv_stride_b, int64_t kv_stride_n, uint16_t* q_out,
                              float acc_scale, oudjat_stream_t stream);

/* Rows 6-9 -- oudjat_linear_qkv_rope_kv (same outputs) with the warm region of
 * oudjat_linear_bf16_warm read from its idle CUs (the correction block's qkv warming its proj weight,
 * ffn_layers.py:43-49). No such argument in the reference (a cache hint with no effect on results). */
int oudjat_linear_qkv_rope_kv_warm(const uint16_t* A, int64_t M, int64_t K, int64_t lda, const uint16_t* W,
                                   int64_t ldw, const uint16_t* bias, int64_t H, int64_t Dh,
                                   const float* sin_table, const float* cos_table, int64_t table_stride,
                                   const uint8_t* patch_mask, const int64_t* rope_idx,
                                   const int64_t* batch_idx, const int64_t* token_idx, uint16_t* kv,
                                   int64_t kv_stride_b, int64_t kv_stride_n, uint16_t* q_out,
                                   float acc_scale, const void* warm, int64_t warm_bytes,
                                   oudjat_stream_t stream);

/* oudjat_linear_qkv_rope_kv for an NVFP4 qkv linear (fp4_fast_linear.py:221-283, then
 * attention.py:415-454): qkv = bf16(bf16(A . W^T) * out_scale + bias) (bias NULL: bf16(bf16(A . W^T) *
 * out_scale)), A the NVFP4 operand x_hat and W the weight's x_hat, then the same RoPE and K/V / q writes;
 * equal to oudjat_linear_bf16 (OUDJAT_EPI_BIAS | OUDJAT_EPI_RAW_BF16) followed by
 * oudjat_qkv_rope_kv_scatter_scaled. Same requirements as oudjat_linear_qkv_rope_kv. */
int oudjat_linear_qkv_rope_kv_nvfp4(const uint16_t* A, int64_t M, int64_t K, int64_t lda, const uint16_t* W,
                                    int64_t ldw, const uint16_t* bias, int64_t H, int64_t Dh,
                                    const float* sin_table, const float* cos_table, int64_t table_stride,
                                    const uint8_t* patch_mask, const int64_t* rope_idx, const int64_t* batch_idx,
                                    const int64_t* token_idx, uint16_t* kv, int64_t kv_stride_b,
                                    int64_t kv_stride_n, uint16_t* q_out, float out_scale,
                                    oudjat_stream_t stream);

/* The SwiGLU pair of NVFP4 linears up to w3's operand in one GEMM (fp4_fast_linear.py:221-283 for w2,
 * then the fused SwiGLU epilogue, token_update.py:620-669, then w3's activation quantizer): with
 * x2 = bf16(A . W^T) (A the shared NVFP4 operand x_hat, W w2's weight x_hat [N, K]) and x1 = w1's bf16
 * output [M, N] (row stride ld1), a = x1 s1 + b1 and b = x2 s2 + b2 in fp32, h = bf16((a sigmoid(a)) b),
 * and xhat [M, N] (row stride ldc) receives the NVFP4 operand of h with tensor scale *tensor_scale --
 * bit-identical to oudjat_linear_bf16 (w2, OUDJAT_EPI_BIAS) followed by oudjat_swiglu_scaled_nvfp4 when
 * both run the same tiles. b1, b2: both or neither. K % 64 == 0, N % 256 == 0; 16-byte aligned
 * operands and rows. */
int oudjat_linear_swiglu_nvfp4(const uint16_t* A, int64_t M, int64_t K, int64_t lda, const uint16_t* W, int64_t N,
                               int64_t ldw, const uint16_t* x1, int64_t ld1, float s1, const uint16_t* b1,
                               float s2, const uint16_t* b2, const float* tensor_scale, uint16_t* xhat, int64_t ldc,
                               oudjat_stream_t stream);

/* Row 10 -- sparse-query attention: for each image b, head h and query t < T,
 *   out[b*T + t, h*Dh:(h+1)*Dh] = softmax(q . K^T * scale) . V over ALL N cached keys, no mask.
 * q [B*T, H, Dh] packed (row stride q_row_stride); K = kv[b, n, 0, h, :], V = kv[b, n, 1, h, :]
 * addressed as b*kv_stride_b + n*kv_stride_n + {0|1}*kv_stride_kv + h*kv_stride_h.
 * Replaces F.scaled_dot_product_attention over the cache (attention.py:456-532). Dh in {64, 128};
 * 16-byte aligned q and kv rows. */
int oudjat_sparse_query_attention(const uint16_t* q, int64_t q_row_stride, int64_t B, int64_t T,
                                  int64_t H, int64_t Dh, const uint16_t* kv, int64_t kv_stride_b,
                                  int64_t kv_stride_n, int64_t kv_stride_kv, int64_t kv_stride_h,
                                  int64_t N, float scale, uint16_t* out, int64_t out_row_stride,
                                  oudjat_stream_t stream);

/* Row 10 with a workspace (the same SDPA call site, attention.py:456-532): the same result as
 * oudjat_sparse_query_attention, except that when few (image, head) pairs would leave most CUs idle
 * (Dh = 64, B*H at most half the CU count) the keys are split into contiguous ranges over several
 * workgroups per pair, whose fp32 partial outputs, running maxima and sums go to `workspace` and
 * are merged by a second launch (deterministic, in range order; within the unsplit kernel's error
 * bound, since each range rounds its probabilities to bf16 relative to its own running max, results
 * may differ from the unsplit ones by a bf16 ulp or two). It splits only if workspace is 16-byte aligned and
 * holds oudjat_sparse_query_attention_workspace_elems(B, T, H, Dh, N) fp32 elements; otherwise, or
 * when that size is 0, it runs exactly as oudjat_sparse_query_attention. */
int oudjat_sparse_query_attention_ws(const uint16_t* q, int64_t q_row_stride, int64_t B, int64_t T,
                                     int64_t H, int64_t Dh, const uint16_t* kv, int64_t kv_stride_b,
                                     int64_t kv_stride_n, int64_t kv_stride_kv, int64_t kv_stride_h,
                                     int64_t N, float scale, uint16_t* out, int64_t out_row_stride,
                                     float* workspace, int64_t workspace_elems, oudjat_stream_t stream);

/* Row 10 in the approximate pass with the row log-sum-exp (the cuDNN SDPA call that returns its LSE,
 * appcorr/models/dinov3/layers/triton_kernels/attention_pscore.py:136-168): the output of
 * oudjat_sparse_query_attention (bit for bit at Dh = 128; at Dh = 64 the register-staged kernel,
 * bit-identical on every row of a full 32-query wave) and lse[(b*H + h)*T + t] = ln sum_n exp(q . k_n *
 * scale), fp32, from an fp32 sum of the unrounded probabilities. lse: B*H*T fp32, 4-byte aligned. */
int oudjat_sparse_query_attention_lse(const uint16_t* q, int64_t q_row_stride, int64_t B, int64_t T,
                                      int64_t H, int64_t Dh, const uint16_t* kv, int64_t kv_stride_b,
                                      int64_t kv_stride_n, int64_t kv_stride_kv, int64_t kv_stride_h,
                                      int64_t N, float scale, uint16_t* out, int64_t out_row_stride,
                                      float* lse, oudjat_stream_t stream);

/* Row 10 + the FP8 route's attn.proj input (attention.py:497-532 with attn.proj a frozen FastFP8Linear,
 * fp8_fast_linear.py:183-196; fp4_fast_linear.py:309-311 routes proj to FP8 in the NVFP4 mode):
 * oudjat_sparse_query_attention whose output is written as the e4m3fn codes that FastFP8Linear's
 * activation quantizer gives on it (oudjat_fp8_quantize mode 0 with act_inv_scale, the bf16 inverse
 * activation scale as fp32, applied to the bf16 attention output), one byte per element: the operand of
 * oudjat_linear_fp8, in one launch. Dh == 128 only (OUDJAT_ERR_UNSUPPORTED_SHAPE otherwise);
 * out_row_stride in bytes, 4-byte aligned rows; other arguments as oudjat_sparse_query_attention. */
int oudjat_sparse_query_attention_fp8(const uint16_t* q, int64_t q_row_stride, int64_t B, int64_t T,
                                      int64_t H, int64_t Dh, const uint16_t* kv, int64_t kv_stride_b,
                                      int64_t kv_stride_n, int64_t kv_stride_kv, int64_t kv_stride_h,
                                      int64_t N, float scale, const float* act_inv_scale, uint8_t* out,
                                      int64_t out_row_stride, oudjat_stream_t stream);

/* fp32 elements of workspace oudjat_sparse_query_attention_ws uses for this shape (0: it never
 * splits the keys of this shape). */
int64_t oudjat_sparse_query_attention_workspace_elems(int64_t B, int64_t T, int64_t H, int64_t Dh,
                                                      int64_t N);

/* Approximate-pass server score with one query per (image, head) -- cls_attn_prob and, with the
 * pseudo query of oudjat_pseudo_query, patch_pseudo_attn_prob (the cache producer,
 * appcorr/models/dinov3/layers/attention.py:254-273):
 *   s[b,h,n] = bf16(bf16(q[b,h] . K[b,n,h]) * scale); p = bf16(softmax_n(s)) (fp32 max, exp, sum and
 *   division); out[b, n] = bf16(fl(sum_h p[b,h,n]) * fl(1/H))
 * -- the rounding points of torch's bf16 matmul, scalar multiply, softmax and mean. Each fp32
 * accumulation and exponential is evaluated exactly (float64, one rounding), so the result is
 * deterministic. q[b, h, :] at q + b*q_stride_b + h*q_stride_h; K[b, n, h, :] at
 * k + b*k_stride_b + n*k_stride_n + h*k_stride_h (the K half of the {tag}_kv cache, K after RoPE).
 * workspace: B*H*N fp32 (the per-head probabilities; its contents are not used after the call).
 * out: [B, N] at row stride out_stride_b, fp32 (out_bf16 = 0, cls_attn_prob's .to(float32)) or bf16
 * bits (out_bf16 = 1, the pseudo score's bf16 tensor). Dh in {64, 128}; N <= 8192; 16-byte aligned
 * q and K rows. */
int oudjat_query_attention_prob(const uint16_t* q, int64_t q_stride_b, int64_t q_stride_h, int64_t B,
                                int64_t H, int64_t Dh, const uint16_t* k, int64_t k_stride_b,
                                int64_t k_stride_n, int64_t k_stride_h, int64_t N, float scale,
                                float* workspace, void* out, int64_t out_stride_b, int out_bf16,
                                oudjat_stream_t stream);

/* No counterpart in the reference: oudjat_query_attention_prob for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * arguments and results without `workspace`: the per-head probabilities go to a library-owned device
 * array of OUDJAT_QUERY_PROB_NOALLOC_MAX fp32 (4 MiB), which each GPU the library runs on holds until
 * the process ends. B*H*N above that returns OUDJAT_ERR_TOO_LARGE. Nothing is allocated. All calls on
 * one GPU share the array: calls that overlap in time on one GPU (unordered streams) race. */
#define OUDJAT_QUERY_PROB_NOALLOC_MAX (1 << 20)
int oudjat_query_attention_prob_noalloc(const uint16_t* q, int64_t q_stride_b, int64_t q_stride_h, int64_t B,
                                        int64_t H, int64_t Dh, const uint16_t* k, int64_t k_stride_b,
                                        int64_t k_stride_n, int64_t k_stride_h, int64_t N, float scale,
                                        void* out, int64_t out_stride_b, int out_bf16, oudjat_stream_t stream);

/* The pseudo query of patch_pseudo_attn_prob (attention.py:254-259) for every (image b, head h)
 * from the P patch queries q[b, t, h, :] at q + b*q_stride_b + t*q_stride_t + h*q_stride_h (after
 * RoPE), with torch's bf16 rounding points (mean, vector norm, clamp_min(bf16 eps), division,
 * product; accumulations exact):
 *   q_mean = bf16(mean_t q_t); qmn = max(bf16(|q_mean|), 2^-7); target = bf16(mean_t bf16(|q_t|))
 *   out[b, h, :] = bf16(q_mean * bf16(target / qmn))          out: [B, H, Dh] bf16 contiguous.
 * Dh in {64, 128}; 16-byte aligned rows. */
int oudjat_pseudo_query(const uint16_t* q, int64_t q_stride_b, int64_t q_stride_t, int64_t q_stride_h,
                        int64_t B, int64_t P, int64_t H, int64_t Dh, uint16_t* out, oudjat_stream_t stream);

/* Approximate-pass dense server score: the mean attention probability of every key over heads and all
 * N queries, without materialising the [B, H, N, N] probabilities (next-rank row f1).
 *   mode 0 (patch_attn_prob, attention.py:251-253): s = bf16(bf16(q . k) * scale),
 *     p = bf16(exp(s - max) / sum) (torch softmax of the bf16 scores), hm = bf16(fl(sum_h p) * fl(1/H)),
 *     out[b, n] = bf16(fl(sum_t hm[t, n]) * fl(1/N));
 *   mode 1 (patch_attn_prob_layermean on 32 heads of 128, N <= 4096: the fused kernel of
 *     triton_kernels/attention_pscore.py:20-98, 172-241): s = (q . k) * scale in fp32,
 *     p = exp2(s log2e - lse log2e) from the row log-sum-exp, out = bf16(fl(sum_{t,h} p) * fl(1/(H N))).
 * q [B * N, H, Dh] packed rows (row stride q_row_stride elements, after RoPE); K [b, n, h, :] at
 * kv + b*kv_stride_b + n*kv_stride_n + h*kv_stride_h (the K half of {tag}_kv). q . k is an fp32 MFMA
 * accumulation and exp is the fp32 device exponential: agreement with an exact evaluation is to fp32
 * rounding before each bf16 rounding. workspace: oudjat_patch_attention_prob_workspace_elems(B, N, H,
 * mode) fp32 (row statistics, then partial column sums). out [B, N] bf16 (row stride out_stride_b).
 * Dh in {64, 128}; 16-byte aligned rows. */
int oudjat_patch_attention_prob(const uint16_t* q, int64_t q_row_stride, int64_t B, int64_t N, int64_t H,
                                int64_t Dh, const uint16_t* kv, int64_t kv_stride_b, int64_t kv_stride_n,
                                int64_t kv_stride_h, float scale, int mode, float* workspace, uint16_t* out,
                                int64_t out_stride_b, oudjat_stream_t stream);

/* fp32 elements of the workspace oudjat_patch_attention_prob needs for this shape and mode (the same
 * call site, attention.py:241-253): 2*B*H*N, plus B*ceil(N/128)*N in mode 0. */
int64_t oudjat_patch_attention_prob_workspace_elems(int64_t B, int64_t N, int64_t H, int mode);

/* Mode 1 of oudjat_patch_attention_prob given the attention's row log-sum-exp instead of computing it
 * (the key-side kernel of attention_pscore.py:20-98 after cuDNN's LSE, :172-241): one pass over the
 * scores, out[b, n] = bf16(fl(sum_{t,h} exp2(s log2e - lse[(b*H + h)*N + t] log2e)) * fl(1/(H N))),
 * the sum in fp32 over head groups added in a fixed order (the reference's atomics have none).
 * lse: B*H*N fp32 as oudjat_sparse_query_attention_lse writes it (T = N); workspace: B*H*N fp32
 * (partial column sums); other arguments as oudjat_patch_attention_prob. */
int oudjat_patch_attention_prob_lse(const uint16_t* q, int64_t q_row_stride, int64_t B, int64_t N, int64_t H,
                                    int64_t Dh, const uint16_t* kv, int64_t kv_stride_b, int64_t kv_stride_n,
                                    int64_t kv_stride_h, float scale, const float* lse, float* workspace,
                                    uint16_t* out, int64_t out_stride_b, oudjat_stream_t stream);

/* Introspection, no counterpart in the reference: writes to buf (NUL-terminated) the demangled name,
 * as rocprofv3 prints it, of the kernel oudjat_linear_bf16 launches for an M x N x K product with
 * epilogue epi (16-byte aligned operands); epi = 5 names the oudjat_linear_qkv_rope_kv kernel
 * (N = 3 H Dh, Dh = 64). Lets benchmark and profile tooling check that a stored
 * per-kernel measurement belongs to the kernel the build runs. */
int oudjat_linear_kernel_name(int64_t M, int64_t N, int64_t K, int epi, char* buf, int64_t buflen);

/* Row 17 -- NVFP4 quantize: x [M, K] bf16 (row stride stride_m) with fp32 tensor scale at
 * *tensor_scale (device) -> qdata [M, K/2] (two e2m1 codes per byte, even element in the low
 * nibble) and e4m3 block scales in the swizzled layout of 32x16 bytes per 128x64 tile
 * (ceil(M/128) * ceil(K/64) * 512 bytes; padding scales are 0).
 * Replaces quantize_nvfp4_swizzled (appcorr/models/dinov3/layers/triton_kernels/nvfp4_fused.py:119-145). K % 16 == 0;
 * x 16-byte aligned with stride_m % 8 == 0, qdata 8-byte and scales 4-byte aligned. */
int oudjat_nvfp4_quantize(const uint16_t* x, int64_t M, int64_t K, int64_t stride_m,
                          const float* tensor_scale, uint8_t* qdata, uint8_t* scales,
                          oudjat_stream_t stream);

/* Row 18 -- NVFP4 dequantize: out[m, k] = bf16(fp32(e2m1(q) * e4m3(s)) * tensor_scale).
 * Inverse of oudjat_nvfp4_quantize; the dequant side of FastFP4Linear
 * (offload/server/model/fp4_fast_linear.py:221-283). K % 16 == 0; qdata 8-byte aligned, out
 * 16-byte aligned with out_stride % 8 == 0. */
int oudjat_nvfp4_dequantize(const uint8_t* qdata, const uint8_t* scales, const float* tensor_scale,
                            int64_t M, int64_t K, uint16_t* out, int64_t out_stride,
                            oudjat_stream_t stream);

/* NVFP4 activation operand of the FP4 correction linears -- FastFP4Linear._quantize
 * (offload/server/model/fp4_fast_linear.py:171-219) with the same arithmetic as oudjat_nvfp4_quantize,
 * additionally writing xhat[m, k] = e2m1(q) * e4m3(s) (bf16, exact: the block-scaled value without
 * the tensor scale, which is what a block-scaled FP4 GEMM multiplies). qdata and scales may both be
 * NULL (only xhat written). Same shape / alignment rules as oudjat_nvfp4_quantize; xhat 16-byte
 * aligned with xhat_stride % 8 == 0. */
int oudjat_nvfp4_quantize_dequantize(const uint16_t* x, int64_t M, int64_t K, int64_t stride_m,
                                     const float* tensor_scale, uint8_t* qdata, uint8_t* scales,
                                     uint16_t* xhat, int64_t xhat_stride, oudjat_stream_t stream);

/* FP8 (e4m3fn, per-tensor scale) operand of FastFP8Linear (fp8_fast_linear.py), written as its exact
 * bf16 value: mode 0 (activations, fp8_fast_linear.py:71-73, 183-186): out = e4m3(clamp(x * s, +-448))
 * with the fp32 product, *scale = the bf16 inverse activation scale; mode 1 (the weight,
 * fp8_fast_linear.py:123-125): out = e4m3(clamp(bf16(x / bf16(*scale)), +-448)). e4m3 rounding is to
 * nearest even. K % 8 == 0, 16-byte aligned rows. */
int oudjat_fp8_quantize_dequantize(const uint16_t* x, int64_t M, int64_t K, int64_t stride_m,
                                   const float* scale, int mode, uint16_t* out, int64_t out_stride,
                                   oudjat_stream_t stream);

/* The FP8 operand as its e4m3fn codes, one byte per element (the operands of oudjat_linear_fp8):
 * the same quantizer as oudjat_fp8_quantize_dequantize (mode 0 activations, mode 1 the weight;
 * fp8_fast_linear.py:71-73, 123-125, 183-186), out[m, k] = sign << 7 | magnitude code (NaN: 0x7f with
 * its sign). K % 8 == 0, 16-byte aligned input rows, 8-byte aligned output rows. */
int oudjat_fp8_quantize(const uint16_t* x, int64_t M, int64_t K, int64_t stride_m, const float* scale, int mode,
                        uint8_t* out, int64_t out_stride, oudjat_stream_t stream);

/* torch._scaled_mm of FastFP8Linear (fp8_fast_linear.py:174-196; the reference's FP8 correction
 * linears) on gfx950's FP8 MFMA: acc = A . W^T over e4m3fn codes A [M, K], W [N, K] (one byte per
 * element, row strides lda, ldw in elements), exact products accumulated in fp32, then the epilogue
 * of oudjat_linear_bf16 with acc_scale = scale_a * scale_b (OUDJAT_EPI_BIAS, _BIAS_LS_RESID, _BIAS_LS,
 * _BIAS_SILU_MUL). The result equals oudjat_linear_bf16 on the codes' exact bf16 values up to the
 * order of the fp32 additions. K % 128 == 0, N % 256 == 0, lda % 16 == 0, ldw % 16 == 0, 16-byte
 * aligned operands, output, residual and gamma rows (OUDJAT_ERR_UNSUPPORTED_SHAPE / _LAYOUT
 * otherwise). */
int oudjat_linear_fp8(const uint8_t* A, int64_t M, int64_t K, int64_t lda, const uint8_t* W, int64_t N, int64_t ldw,
                      const uint16_t* bias, int epilogue, const uint16_t* gamma, const uint16_t* resid, int64_t ldr,
                      uint16_t* C, int64_t ldc, float acc_scale, oudjat_stream_t stream);

/* oudjat_linear_qkv_rope_kv with e4m3fn code operands on the FP8 MFMA (the FP8 qkv linear of a
 * correction block, fp8_fast_linear.py:174-196 into attention.py:415-454): same outputs and epilogue
 * arithmetic, acc_scale = scale_a * scale_b. K % 128 == 0, 3 * H * Dh % 256 == 0, Dh in {16, 32, 64,
 * 128}, lda % 16 == 0, ldw % 16 == 0. */
int oudjat_linear_qkv_rope_kv_fp8(const uint8_t* A, int64_t M, int64_t K, int64_t lda, const uint8_t* W, int64_t ldw,
                                  const uint16_t* bias, int64_t H, int64_t Dh, const float* sin_table,
                                  const float* cos_table, int64_t table_stride, const uint8_t* patch_mask,
                                  const int64_t* rope_idx, const int64_t* batch_idx, const int64_t* token_idx,
                                  uint16_t* kv, int64_t kv_stride_b, int64_t kv_stride_n, uint16_t* q_out,
                                  float acc_scale, oudjat_stream_t stream);

/* Producers of the NVFP4 operand (fp4_fast_linear.py:171-219 folded into the kernel that makes the
 * linear's input; no separate quantize pass): each writes x_hat = e2m1 * e4m3-scale (bf16, exactly what
 * oudjat_nvfp4_quantize_dequantize gives on the bf16 tensor it would otherwise write) with tensor
 * scale *tensor_scale, 16-element blocks along the row (C or N % 16 == 0).
 *   oudjat_layernorm_rows_nvfp4: of LayerNorm(x) (norm1 -> the NVFP4 qkv linear, norm2 -> w1 / w2,
 *     block.py:1114, 1141); other arguments as oudjat_layernorm_rows.
 *   oudjat_packed_residual_persist_ln_nvfp4: of the next block's LayerNorm(x_new); x_new and the
 *     blocks_out_sum rows as oudjat_packed_residual_persist_ln.
 *   oudjat_swiglu_scaled_nvfp4: of the SwiGLU output (the NVFP4 w3 linear's input, ffn_layers.py:106-115
 *     with token_update.py:620-669); other arguments as oudjat_swiglu_scaled. */
int oudjat_layernorm_rows_nvfp4(const uint16_t* x, int64_t rows, int64_t C, int64_t x_stride, const uint16_t* weight,
                                const uint16_t* bias, float eps, const float* tensor_scale, uint16_t* xhat,
                                int64_t xhat_stride, oudjat_stream_t stream);

/* Rows 4 and 5 fused for the first block of a packed run (the gather of the selected rows,
 * token_update.py:455-473, then norm1, block.py:1114): packed row i = x[batch_idx[i], token_idx[i]]
 * (x with element strides stride_b, stride_n, rows of C contiguous bf16) is copied to x_out [rows, C]
 * byte for byte, and its LayerNorm goes to ln_out [rows, C] -- bit-identical to oudjat_gather_rows
 * followed by oudjat_layernorm_rows, or with tensor_scale non-NULL to oudjat_layernorm_rows_nvfp4
 * (the NVFP4 operand of the LayerNorm output). int64 indices; 16-byte aligned rows, C % 8 == 0
 * (C % 16 == 0 for the NVFP4 output), C <= 8192. */
int oudjat_gather_rows_ln(const uint16_t* x, int64_t stride_b, int64_t stride_n, int64_t C,
                          const int64_t* batch_idx, const int64_t* token_idx, int64_t rows, const uint16_t* w,
                          const uint16_t* b, float eps, const float* tensor_scale, uint16_t* x_out,
                          uint16_t* ln_out, oudjat_stream_t stream);
int oudjat_packed_residual_persist_ln_nvfp4(const uint16_t* x_act, const uint16_t* x_attn, const uint16_t* mlp,
                                            int64_t rows, int64_t C, const int64_t* batch_idx,
                                            const int64_t* token_idx, uint16_t* bos, int64_t bos_stride_b,
                                            int64_t bos_stride_n, uint16_t* x_new, const uint16_t* ln_w,
                                            const uint16_t* ln_b, float eps, const float* tensor_scale,
                                            uint16_t* xhat, oudjat_stream_t stream);
int oudjat_swiglu_scaled_nvfp4(const uint16_t* x1, float s1, const uint16_t* b1, const uint16_t* x2, float s2,
                               const uint16_t* b2, int64_t M, int64_t N, const float* tensor_scale, uint16_t* xhat,
                               oudjat_stream_t stream);

/* oudjat_qkv_rope_kv_scatter on the raw product of an NVFP4 qkv linear: every value first goes through
 * the linear's scale-and-bias epilogue bf16(raw * scale + bias[col]) (bf16(raw * scale) for a NULL
 * bias; scale_bias_inplace_triton, token_update.py:571-617), then RoPE and the K/V / q writes
 * (attention.py:415-454). 16-byte aligned bias. */
int oudjat_qkv_rope_kv_scatter_scaled(const uint16_t* qkv_raw, int64_t M, int64_t H, int64_t Dh, float scale,
                                      const uint16_t* bias, const float* sin_table, const float* cos_table,
                                      int64_t table_stride, const uint8_t* patch_mask, const int64_t* rope_idx,
                                      const int64_t* batch_idx, const int64_t* token_idx, uint16_t* kv,
                                      int64_t kv_stride_b, int64_t kv_stride_n, uint16_t* q_out,
                                      oudjat_stream_t stream);

/* Introspection, no counterpart in the reference: the kernel oudjat_linear_fp8 launches for an
 * M x N x K product with epilogue epi (5: oudjat_linear_qkv_rope_kv_fp8), as rocprofv3 prints it. */
int oudjat_linear_fp8_kernel_name(int64_t M, int64_t N, int64_t K, int epi, char* buf, int64_t buflen);

/* The NVFP4 linears' output epilogue, scale_bias_inplace_triton (token_update.py:571-617):
 * out = bf16(x * scale + bias[col]) over [M, N] (bias may be NULL: bf16(x * scale)); with gamma
 * (may be NULL) out = bf16(that * gamma[col]), the block's LayerScale (layer_scale.py:28-29). out may
 * alias x. N % 8 == 0, 16-byte aligned rows. */
int oudjat_scale_bias_rows(const uint16_t* x, int64_t M, int64_t N, int64_t x_stride, float scale,
                           const uint16_t* bias, const uint16_t* gamma, uint16_t* out, int64_t out_stride,
                           oudjat_stream_t stream);

/* The SwiGLU pair's fused NVFP4 epilogue, fused_swiglu_epilogue_triton (token_update.py:620-669):
 * a = x1 * s1 + b1, b = x2 * s2 + b2 (fp32), out = bf16(silu(a) * b) over contiguous [M, N]; b1 and b2
 * are both NULL or both given. out may alias x1. N % 8 == 0, 16-byte aligned. */
int oudjat_swiglu_scaled(const uint16_t* x1, float s1, const uint16_t* b1, const uint16_t* x2, float s2,
                         const uint16_t* b2, int64_t M, int64_t N, uint16_t* out, oudjat_stream_t stream);

/* Calibration observer of the low-precision linears (fp4_fast_linear.py:256-259,
 * fp8_fast_linear.py:176-179): *amax = max(*amax, max |x|) over rows [M, K] (NaN propagates).
 * K % 8 == 0, 16-byte aligned rows. */
int oudjat_amax_update(const uint16_t* x, int64_t M, int64_t K, int64_t stride_m, float* amax,
                       oudjat_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* OUDJAT_H */
