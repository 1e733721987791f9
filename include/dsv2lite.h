/*
 * dsv2lite.h -- C ABI of the MI355X (gfx950) DeepSeek-V2-Lite decode-step library
 * (libdsv2lite_hip.so).
 *
 * Conventions (every entry point):
 *   - device pointers are plain `void*` / typed pointers to HBM buffers owned by
 *     the caller; bf16 tensors are passed as `void*` (2 bytes per element);
 *   - `stream` is a hipStream_t passed as `void*` (the caller's current stream);
 *   - no entry point allocates, synchronises or reads device memory on the host,
 *     so every one of them may be recorded into a hipGraph;
 *   - return 0 on success, a negative DSV2_E* code for a rejected argument, or a
 *     positive hipError_t from the launch.  dsv2_last_error_message() gives the
 *     text of the last failure on the calling thread.
 *
 * The reference (heiheiha798/Flash-DeepSeeek-V2-Lite) has no native FFI: its
 * operator boundary is the Python `triton_kernels` package patched into the HF
 * model by src/run.py:256-502.  Each entry point below cites the Python
 * function (file:line in that repository) whose role it takes.
 */
#ifndef DSV2LITE_H_
#define DSV2LITE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DSV2_ABI_VERSION 2

#define DSV2_OK 0
#define DSV2_E_NULL (-1)      /* a required pointer is null            */
#define DSV2_E_SHAPE (-2)     /* a size is out of the supported range  */
#define DSV2_E_ALIGN (-3)     /* a pointer/stride is not 16B-aligned   */
#define DSV2_E_FLAGS (-4)     /* unsupported flag combination          */

/* bits a kernel ORs into the caller's device status word (int32, optional) */
#define DSV2_DEVERR_CACHE_FULL 1  /* a cache write at or past a row's capacity was skipped */

/* flags of dsv2_gemv_bf16 / dsv2_gemm_bf16 */
#define DSV2_LINEAR_SWIGLU 1  /* W holds [gate; up] (2N rows): y = bf16(silu(bf16 g)) * bf16 u */
#define DSV2_LINEAR_OUT_F32 2 /* store fp32(bf16(acc)) instead of bf16 (logits)               */
#define DSV2_LINEAR_OUT_F32_EXACT 4 /* dsv2_gemm_bf16: store the fp32 accumulator unrounded
                                       (router logits: HF's fp32 gate product); no SwiGLU or residual */

int dsv2_abi_version(void);
const char* dsv2_last_error_message(void);

/* ---- elementwise -------------------------------------------------------- */

/* y[r,:] = w * bf16(x[r,:] * rsqrt(mean(x^2) + eps)), fp32 math, bf16 out.
 * Replaces rmsnorm_triton (triton_kernels/rmsnorm.py:60-95). cols % 8 == 0, cols <= 8192. */
int dsv2_rmsnorm_bf16(const void* x, int64_t x_stride, const void* w, void* y, int64_t y_stride,
                      int rows, int cols, float eps, void* stream);

/* out = bf16(fp32(a) + fp32(b)).  Replaces residual_add_triton
 * (triton_kernels/attention_prepost.py:191-223).  n % 8 == 0. */
int dsv2_residual_add_bf16(const void* a, const void* b, void* out, int64_t n, void* stream);

/* fp16 form of dsv2_residual_add_bf16: out = fp16(fp32(a) + fp32(b)), the fp16 inputs
 * residual_add_triton also accepts (triton_kernels/attention_prepost.py:196). */
int dsv2_residual_add_f16(const void* a, const void* b, void* out, int64_t n, void* stream);

/* out = bf16(g * sigmoid(g) * u) in fp32.  Replaces silu_mul_triton
 * (triton_kernels/mlp_elementwise.py:24-45).  n % 8 == 0. */
int dsv2_silu_mul_bf16(const void* gate, const void* up, void* out, int64_t n, void* stream);

/* mask[b,j] = (index[j] <= pos), position_ids[b] = pos with pos = cache_position[0], int64
 * (index = attention_mask_index [max_len]; NULL means index[j] = j).
 * Replaces prepare_decode_inputs_triton (triton_kernels/attention_prepost.py:152-188). */
int dsv2_prepare_decode_inputs(const int64_t* cache_position, const int64_t* attention_mask_index,
                               int64_t* attention_mask, int64_t* position_ids, int batch, int max_len, void* stream);

/* dst[b, pos, :] = src[b, :] for b < batch, pos = cache_position[0]; row_bytes % 16 == 0.
 * dst row b starts at dst + b*dst_batch_stride bytes, token rows are row_bytes apart.
 * A pos outside [0, max_tokens) writes nothing and ORs DSV2_DEVERR_CACHE_FULL into *status
 * (when status != NULL).  Replaces copy_single_token_to_cache
 * (triton_kernels/attention_prepost.py:113-149); the reference's GraphCache raises on
 * overflow instead (src/run.py:131-134). */
int dsv2_copy_token_rows(const void* src, int64_t src_batch_stride, void* dst, int64_t dst_batch_stride,
                         int64_t row_bytes, const int64_t* cache_position, int64_t max_tokens, int batch,
                         int32_t* status, void* stream);

/* pos32[b] = cache_position[0]; base[b] = b * per_row_capacity (int64, if base != NULL);
 * cap[b] = per_row_capacity (int32, if cap != NULL).  Turns the reference's shared scalar
 * cache_position (src/run.py:196-202) into the per-row arrays of the MLA entry points. */
int dsv2_fill_positions(const int64_t* cache_position, int32_t* pos, int64_t* base, int32_t* cap,
                        int64_t per_row_capacity, int batch, void* stream);

/* out[r,:] = table[ids[r], :] (bf16 rows of `hidden`).  The embed_tokens gather of the
 * HF model (run.py:577-584 feeds input_ids into the model). */
int dsv2_embed_gather_bf16(const int64_t* ids, const void* table, int hidden, void* out, int rows,
                           void* stream);

/* next_ids[r] = first index of the max of logits[r, :vocab] (fp32); if pos != NULL,
 * pos[r] += 1.  Replaces _greedy_decode + cache_position.add_(1) (src/run.py:252-253,585-588). */
int dsv2_argmax_f32(const float* logits, int rows, int vocab, int64_t* next_ids, int32_t* pos,
                    void* stream);

/* dst[0, nbytes) = src[0, nbytes): a streaming device copy (16-byte aligned, nbytes % 16 == 0).
 * No reference counterpart: the measured copy bandwidth the benchmark quotes each step's
 * byte rate against, beside the HBM peak. */
int dsv2_stream_copy(const void* src, void* dst, int64_t nbytes, void* stream);

/* ---- linears -------------------------------------------------------------- */

/* y[r, n] = bf16( x'[r,:] . W[n,:] ) for r < rows, n < N, fp32 accumulation, where
 * x' = x, or RMSNorm(x; norm_w, eps) when norm_w != NULL (fused prologue).  With
 * residual != NULL: y = bf16(residual + bf16(acc)).  flags: DSV2_LINEAR_*.
 * VALU GEMV for few rows (weights streamed once per 8 rows).  K % 8 == 0, N % 8 == 0.
 * Replaces the small-family GEMVs (attention_decode_small.py:55-137, :858-929) and the
 * torch F.linear calls of the dense / shared MLP and lm_head (src/run.py:341-352). */
int dsv2_gemv_bf16(const void* x, int64_t x_stride, int rows, int K, const void* W, int N,
                   const void* norm_w, float eps, const void* residual, int64_t res_stride, void* y,
                   int64_t y_stride, int flags, void* stream);

/* Final RMSNorm + lm_head + greedy argmax for 1..8 rows (hidden 2048):
 *   logits[r, v] = fp32(bf16(RMSNorm(x[r]; norm_w) . W[v, :]))   (W [vocab, 2048], vocab even)
 *   next_ids[r] = first index of the row maximum;  pos[r] += 1 when pos != NULL.
 * The GEMV leaves each wave's (max, first index) in `partials` (caller-owned, at least
 * dsv2_lm_head_argmax_workspace_size(rows) bytes) and a one-workgroup-per-row kernel
 * reduces them.  Replaces lm_head + .float() + _greedy_decode + cache_position.add_(1)
 * (src/run.py:252-253, 585-588). */
int64_t dsv2_lm_head_argmax_workspace_size(int rows);
int dsv2_lm_head_argmax_bf16(const void* x, int64_t x_stride, int rows, const void* W, int vocab, const void* norm_w,
                             float eps, float* logits, void* partials, int64_t partials_bytes, int64_t* next_ids,
                             int32_t* pos, void* stream);

/* dsv2_lm_head_argmax_bf16 without the caller's workspace, for callers that cannot
 * allocate (code under hipGraph capture, serving loops that forbid hipMalloc).  No
 * counterpart in the reference.  The argmax partials live in a library-owned device array
 * (one per GPU, 256 KiB, kept until the process ends): rows <= 8 (larger requests are
 * rejected with DSV2_E_SHAPE).  Nothing is allocated; the array's per-device address is
 * looked up (hipGetSymbolAddress) on the first call made with that device current, so make
 * that first call outside graph capture.  Every call on one GPU shares the array: calls
 * that overlap in time on one GPU (other streams, other threads) race and must be ordered
 * by the caller.  The partials need no clearing: each call writes every one it reads. */
int dsv2_lm_head_argmax_bf16_noalloc(const void* x, int64_t x_stride, int rows, const void* W, int vocab,
                                     const void* norm_w, float eps, float* logits, int64_t* next_ids, int32_t* pos,
                                     void* stream);

/* Grouped bf16 MFMA GEMM (v_mfma_f32_16x16x32_bf16), fp32 accumulation:
 *   for group g < n_groups, row r < rows:
 *     Y[g*y_gstride + r*y_stride + n] = x[g*x_gstride + r*x_stride, :] . W[g*w_gstride + n*K, :]
 * Same flags/residual semantics as dsv2_gemv_bf16 (residual only with n_groups == 1).
 * K % 64 == 0, N % 16 == 0.  Replaces _batched_linear_kernel
 * (triton_kernels/attention_decode_batch.py:421-468) and cuBLAS F.linear at batch sizes. */
int dsv2_gemm_bf16(const void* x, int64_t x_stride, int64_t x_gstride, int rows, int K, const void* W,
                   int64_t w_gstride, int N, int n_groups, const void* residual, int64_t res_stride, void* y,
                   int64_t y_stride, int64_t y_gstride, int flags, void* stream);

/* ---- absorbed MLA -------------------------------------------------------- */

/* Per-row cache bounds (every MLA entry point): row r owns cache rows
 * [base[r], base[r] + cap[r]) (int32 cap).  The new token of row r is stored only when
 * 0 <= pos[r] < cap[r]; otherwise nothing is written, DSV2_DEVERR_CACHE_FULL is ORed into
 * *status (when status != NULL) and the row attends its cap[r] cached rows, so no launch
 * reads or writes outside the row's own slots.  The reference raises on overflow
 * (GraphCacheLayer.update, src/run.py:131-134); here the host reads status after the step.
 *
 * Per row r (new token at cache slot base[r] + pos[r]):
 *   c = RMSNorm(qkva[r, 3072:3584]; kv_norm_w) -> cache[slot, 0:512]
 *   k_pe = RoPE(qkva[r, 3584:3648], pos)      -> cache[slot, 512:576]
 *   q_out[r, h, 512:576] = RoPE(q_pe_h);  q_out[r, h, 0:512] = W_UK_h^T q_nope_h
 *     (only when w_ukt != NULL: W_UK transposed, [16, 512, 128], as a per-row GEMV; the batch
 *     family runs the absorption on MFMA in dsv2_mla_prepare_qlat).
 * RoPE rotates de-interleaved pairs with bf16 cos/sin tables [max_pos, 64].
 * Replaces kv-norm + _batched_build_qkv_rope_kernel + _cache_write_q1_dual_kernel
 * (attention_decode_batch.py:719-813; attention_decode_small.py:141-339). */
int dsv2_mla_prepare(const void* qkva, int64_t qkva_stride, int rows, const int32_t* pos,
                     const int64_t* base, const int32_t* cap, const void* kv_norm_w, float eps, const void* rope_cos,
                     const void* rope_sin, int max_pos, const void* w_ukt, void* cache, void* q_out,
                     int32_t* status, void* stream);

/* dsv2_mla_prepare with w_ukt (required here) in one launch for the batch family: the same
 * outputs, bit for bit, as dsv2_mla_prepare(..., w_ukt = NULL, ...) followed by the grouped
 * absorption dsv2_gemm_bf16(qkva, qkva_stride, 192, rows, 128, w_ukt, 512 * 128, 512, 16,
 * NULL, 0, q_out, 16 * 576, 576, 0) -- the absorption's MFMA workgroups and the per-row
 * RoPE / cache workgroups run side by side (they read only qkva and write disjoint outputs).
 * Replaces the q absorption of attention_decode_batch.py:726-745 together with the kv-norm,
 * RoPE and cache write of :719-813. */
int dsv2_mla_prepare_qlat(const void* qkva, int64_t qkva_stride, int rows, const int32_t* pos,
                          const int64_t* base, const int32_t* cap, const void* kv_norm_w, float eps,
                          const void* rope_cos, const void* rope_sin, int max_pos, const void* w_ukt, void* cache,
                          void* q_out, int32_t* status, void* stream);

/* Split-KV absorbed-MLA decode over the compressed cache [*, 576] bf16.
 * Row r attends cache rows base[r] .. base[r]+min(pos[r], cap[r]-1) (inclusive); split s covers
 * tokens [s*split_tokens, (s+1)*split_tokens).  Writes unnormalised partial
 * o_lat [rows, max_splits, 16, 512] fp32 and (m, l) [rows, max_splits, 16, 2]
 * (m in log2 units).  split_tokens % 32 == 0.  Replaces _batched_decode_attention_q1_kernel
 * (attention_decode_batch.py:241-342) / _decode_attention_q1_kernel (attention_decode_small.py:343-423). */
int dsv2_mla_decode(const void* q, const void* cache, const int64_t* base, const int32_t* pos, const int32_t* cap,
                    int rows, int split_tokens, int max_splits, float softmax_scale, float* part_o, float* part_ml,
                    void* stream);

/* dsv2_mla_decode with one split per row (a workgroup attends the whole row) and the
 * normalisation done in the same launch: olat[r, h*512 + j] = bf16 o_lat [rows, 16, 512]
 * (row stride olat_stride >= 8192), equal bit for bit to dsv2_mla_decode + dsv2_mla_combine
 * (w_uv == NULL) with max_splits = 1; no partials.  For rows >= ~256, where one workgroup per
 * row already fills the GPU.  Replaces the same reference functions as the pair. */
int dsv2_mla_decode_rows(const void* q, const void* cache, const int64_t* base, const int32_t* pos,
                         const int32_t* cap, int rows, float softmax_scale, void* olat, int64_t olat_stride,
                         void* stream);

/* Merge the splits of dsv2_mla_decode (same pos / cap).  With w_uv != NULL: out[r, h*128 + i] =
 * bf16(sum_j W_UV[h, i, j] o_lat[r, h, j]) (bf16 [rows, 2048], row stride out_stride);
 * with w_uv == NULL: out = bf16 o_lat [rows, 16, 512] for a grouped GEMM.
 * Together with dsv2_mla_decode this replaces the attention core + v-combine
 * (attention_decode_batch.py:240-401). */
int dsv2_mla_combine(const float* part_o, const float* part_ml, const int32_t* pos, const int32_t* cap, int rows,
                     int split_tokens, int max_splits, const void* w_uv, void* out, int64_t out_stride,
                     void* stream);

/* Absorbed-MLA decode for a few rows in one launch: per row 64 workgroups, one per (head,
 * quarter of W_UV_h's 128 outputs); each absorbs q_h = W_UK_h^T q_nope_h itself, builds the
 * new token's kv-norm + RoPE(k_pe) row (stored to cache[base+pos] by one workgroup), applies
 * RoPE(q_pe), attends the row's pos cached tokens plus the new one and applies its 32 W_UV
 * rows:
 *   out[r, h*128 + i] = bf16(W_UV_h softmax(scale * q_h . C^T) C[:, :512]).
 * w_ukt is W_UK transposed [16, 512, 128].  Together with dsv2_gemv_bf16 for the q/kv and
 * o projections this replaces attention_decode_only_triton / attention_decode_small_batch_triton
 * (triton_kernels/attention_decode_small.py:553-674, :932-1070) for the small family. */
int dsv2_mla_fused(const void* qkva, int64_t qkva_stride, int rows, const int32_t* pos, const int64_t* base,
                   const int32_t* cap, const void* kv_norm_w, float eps, const void* rope_cos, const void* rope_sin,
                   int max_pos, const void* w_ukt, const void* w_uv, void* cache, float softmax_scale, void* out,
                   int64_t out_stride, int32_t* status, void* stream);

/* The same result as dsv2_mla_fused after dsv2_mla_prepare(..., w_ukt, ...) has written the
 * absorbed, rotated q [rows, 16, 576] and the new cache rows: per row 64 workgroups, one per
 * (head, quarter of W_UV_h's 128 outputs), each attending the row's min(pos+1, cap) cached
 * tokens and applying its 32 W_UV rows:
 *   out[r, h*128 + i] = bf16(W_UV_h softmax(scale * q_h . C^T) C[:, :512])   (row stride out_stride).
 * Same reference functions as dsv2_mla_fused (attention_decode_small.py:553-674, :932-1070). */
int dsv2_mla_attend(const void* q, const void* cache, const int64_t* base, const int32_t* pos, const int32_t* cap,
                    int rows, const void* w_uv, float softmax_scale, void* out, int64_t out_stride, void* stream);

/* dsv2_mla_prepare (with W_UK absorption into q_buf [rows, 16, 576] bf16, a caller-owned
 * buffer) followed by dsv2_mla_attend, as two launches: the same inputs and result as
 * dsv2_mla_fused.  The absorbing workgroups also bring the attention's W_UV rows and the
 * first 256 cached rows into L2 ahead of it.  Same reference functions as dsv2_mla_fused. */
int dsv2_mla_spread(const void* qkva, int64_t qkva_stride, int rows, const int32_t* pos, const int64_t* base,
                    const int32_t* cap, const void* kv_norm_w, float eps, const void* rope_cos, const void* rope_sin,
                    int max_pos, const void* w_ukt, const void* w_uv, void* cache, void* q_buf, float softmax_scale,
                    void* out, int64_t out_stride, int32_t* status, void* stream);

/* The q | kv_a projection of rows x [rows, 2048] (row stride x_stride) with the RMSNorm
 * prologue (norm_w, eps; norm_w == NULL: x is used as it is), as
 * dsv2_gemv_bf16(x, ..., w_qkva [3648, 2048], 3648, norm_w, eps, ...)
 * writes it into qkva [rows, 3648] (row stride qkva_stride), plus the W_UK absorption of its
 * q_nope in partial sums: for head h and block i of its q_nope rows 16i .. 16i+15,
 *   qlat_part[r, h, i, c] = sum_{d in block i} w_uk[h, d, c] * qkva[r, h*192 + d]   (fp32),
 * with w_uk [16, 128, 512] (kv_b's k_nope rows).  The projection's workgroups also bring the
 * first 256 cached rows of each row (cache / base / pos / cap as dsv2_mla_fused) into L2 for
 * the attention that follows.  qlat_part holds rows * 16 * 8 * 512 floats.  Replaces the
 * q+kv_a linear (attention_decode_small.py:55-96) and, with dsv2_mla_attend_parts, the small
 * family's q/k build (attention_decode_small.py:141-264) and attention
 * (attention_decode_small.py:553-674, :932-1070). */
int dsv2_qkva_absorb_bf16(const void* x, int64_t x_stride, int rows, const void* w_qkva, const void* norm_w, float eps,
                          const void* w_uk, void* qkva, int64_t qkva_stride, float* qlat_part, const void* cache,
                          const int64_t* base, const int32_t* pos, const int32_t* cap, void* stream);

/* dsv2_mla_fused with the absorbed query taken from dsv2_qkva_absorb_bf16's partial sums:
 * q_lat[r, h, c] = bf16(sum over the 8 blocks of qlat_part[r, h, i, c]) instead of each head
 * workgroup absorbing q_nope itself; otherwise the same inputs (qkva: q_pe, latent and k_pe
 * are read from it), cache write, capacity rule and result.  Same reference functions as
 * dsv2_qkva_absorb_bf16. */
int dsv2_mla_attend_parts(const void* qkva, int64_t qkva_stride, int rows, const int32_t* pos, const int64_t* base,
                          const int32_t* cap, const void* kv_norm_w, float eps, const void* rope_cos,
                          const void* rope_sin, int max_pos, const float* qlat_part, const void* w_uv, void* cache,
                          float softmax_scale, void* out, int64_t out_stride, int32_t* status, void* stream);

/* q_len = 1 attention over an EXPANDED per-head cache (keys [B, H, L, q_dim], values
 * [B, H, L, v_dim], bf16, last dim contiguous, element strides as given):
 *   out[b, h, :] = bf16( softmax_n(scale * k[b,h,n,:] . q[b,h,:]) . v[b,h,n,:] ),  n = 0..pos
 * with pos = cache_position[0] (int64, device).  pos outside [0, seq_len) attends
 * min(max(pos, 0), seq_len - 1) + 1 rows and ORs DSV2_DEVERR_CACHE_FULL into *status.
 * q_dim, v_dim <= 256 and % 8.  Replaces batched_attention_decode_q1_triton
 * (triton_kernels/attention_decode_batch.py:345-401, attention_decode_small.py:782-840);
 * the decode step itself reads the compressed cache instead. */
int dsv2_attention_decode_expanded(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k,
                                   int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_s, const void* v,
                                   int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_s, void* out,
                                   int64_t out_stride_b, int64_t out_stride_h, int batch, int heads, int q_dim,
                                   int v_dim, int seq_len, const int64_t* cache_position, float softmax_scale,
                                   int32_t* status, void* stream);

/* Prefill attention (the prompt's tokens, before the decode path) in MLA's expanded form,
 * per head h and query row r (position p, in the sequence whose position 0 is cache row sb):
 *   out[r, h*128 + i] = bf16( softmax_{n <= p}(scale * q_rh . k_nh) . v_nh[i] )
 *   q_rh = [qkva[r, h*192 .. +128] | q_rope[r, h*576 + 512 .. +64]]   (mla_prepare's RoPE(q_pe))
 *   k_nh = [k_nope[sb + n - exp_lo, h, :128] | cache[sb + n, 512 .. 576]],
 *   v_nh = v[sb + n - exp_lo, h, :128]
 * k_nope / v [exp_rows, 16, 128] bf16 are W_UK / W_UV applied to cache rows exp_lo .. (the
 * kv_b projection of every cached token: one dsv2_gemm_bf16 over the heads side by side).
 * tiles [n_tiles <= 2^27 - 1] int32x4 {first row, rows (1..128), position of the first row,
 * sb}: <= 128 consecutive query rows of one sequence each, a sequence's tiles consecutive
 * (the XCD placement assumes it; any order gives the same result).  Indices derived from the table are clamped into rows /
 * cache_rows / exp_rows.  Replaces the prefill attention of the HF model the reference runs
 * eagerly (src/run.py:526-544; remote DeepseekV2Attention.forward over the expanded K/V). */
int dsv2_mla_prefill_attention(const void* qkva, int64_t qkva_stride, const void* q_rope, int64_t q_rope_stride,
                               int rows, const void* cache, int64_t cache_rows, const void* k_nope, const void* v,
                               int64_t exp_lo, int64_t exp_rows, const int32_t* tiles, int n_tiles,
                               float softmax_scale, void* out, int64_t out_stride, void* stream);

/* ---- MoE ------------------------------------------------------------------ */

/* Router logits only, spread over 16 workgroups per token: xn = RMSNorm(h) (written by the
 * first workgroup of each row to xn_out), logits[r, e] = fp32(xn) . fp32(W_r[e]) (fp32 [rows, 64]).
 * The softmax/top-6 then runs inside dsv2_moe_route_gateup_logits.  Replaces the router
 * GEMV of _graph_gate_forward (src/run.py:268-272). */
int dsv2_router_logits(const void* h, int64_t h_stride, const void* norm_w, float eps, const void* w_router,
                       int rows, void* xn_out, float* logits, void* stream);

/* dsv2_moe_route_gateup with the router's softmax + top-6 (triton_kernels/moe_router.py:9-60)
 * done inside every routed workgroup from the fp32 logits; ids [rows, 6] (int32) and weights
 * [rows, 6] (score * scaling) are written once per row for the down projection.  hbuf is
 * [rows, 8, inter]: routes 0..5 (and the shared halves 6, 7 when sh_gate_up != NULL). */
int dsv2_moe_route_gateup_logits(const void* xn, int rows, const float* logits, float scaling, int32_t* ids,
                                 float* weights, const void* w_gate_up, const void* sh_gate_up, int inter,
                                 void* hbuf, void* stream);

/* Router: xn = RMSNorm(h; norm_w) (written to xn_out), logits = fp32(xn) . fp32(W_r)^T
 * [64], softmax, top-6 by repeated max (ties -> lower index), weights = score * scaling.
 * ids as int32 (ids32) and/or int64 (ids64).  Replaces _graph_gate_forward + the router
 * kernel (src/run.py:257-275; triton_kernels/moe_router.py:9-86). */
int dsv2_router_topk6(const void* h, int64_t h_stride, const void* norm_w, float eps, const void* w_router,
                      float scaling, int rows, void* xn_out, int32_t* ids32, int64_t* ids64, float* weights,
                      void* stream);

/* Softmax + top-6 from given fp32 logits [rows, 64]: router_softmax_topk6_triton
 * (triton_kernels/moe_router.py:63-86). */
int dsv2_router_topk6_from_logits(const float* logits, int rows, float scaling, int32_t* ids32,
                                  int64_t* ids64, float* weights, void* stream);

/* Small family, route-local gate_up + SwiGLU: for row r, route s < n_routes:
 *   hbuf[r, s, :inter] = bf16(silu(bf16 g)) * bf16 u  with expert e = ids[r, s] (s < 6) or
 *   the shared expert half s-6 (s = 6, 7 when sh_gate_up != NULL: rows [(s-6)*inter, ...)
 *   of gate and of up).  w_gate_up [64, 2*inter, 2048]; sh_gate_up [2*2*inter, 2048].
 * Replaces _fused_gate_up_swiglu_kernel / _batched_fused_gate_up_swiglu_kernel
 * (triton_kernels/moe_small_gemv.py:53-105, :195-253) with the gate/up rows paired correctly. */
int dsv2_moe_route_gateup(const void* xn, int rows, const int32_t* ids, const void* w_gate_up,
                          const void* sh_gate_up, int inter, void* hbuf, void* stream);

/* Small family, route-local down + top-6 combine (+ shared, + residual):
 *   d_s = bf16(hbuf[r,s,:] . Wd_s[j,:]);  routed = bf16(sum_{s<6} w[r,s] d_s)  (fp32, slot order)
 *   shared = bf16(d_6 + d_7) when sh_down != NULL, or shared_y[r, j] (a precomputed shared-expert
 *   output) when shared_y != NULL;  y = bf16(routed + shared)
 *   out[r, j] = residual ? bf16(residual[r, j] + y) : y.
 * hbuf is [rows, hbuf_routes, inter] (6 or 8).  w_down [64, 2048, inter]; sh_down [2048, 2*inter].
 * Replaces _down_partial_kernel + _down_reduce_topk6_kernel (moe_small_gemv.py:109-191, :257-347). */
int dsv2_moe_route_down(const void* hbuf, int rows, const int32_t* ids, const float* weights,
                        const void* w_down, const void* sh_down, int inter, int hbuf_routes, const void* shared_y,
                        const void* residual, void* out, void* stream);

/* FP8 expert weights (small family): dsv2_moe_route_gateup_logits / dsv2_moe_route_down with
 * every routed and shared expert row in OCP e4m3 (1 byte per weight, same row layouts) and one
 * fp32 scale per row: weight = e4m3 value * scale (gate_up_scale [64, 2*inter], sh_gate_up_scale
 * [2*2*inter], down_scale [64, 2048], sh_down_scale [2048]).  Each row's dot product is taken
 * in fp32 over the e4m3 values (converted by v_cvt_pk_f32_fp8) and multiplied by the row's
 * scale; the rounding points are those of the bf16 entry points.  No counterpart in the
 * reference (bf16 only): the low-precision weights of the build's next steps.  inter % 4 == 0
 * (gate_up), inter % 16 == 0 and <= 2048 (down). */
int dsv2_moe_route_gateup_logits_fp8(const void* xn, int rows, const float* logits, float scaling, int32_t* ids,
                                     float* weights, const uint8_t* w_gate_up, const float* gate_up_scale,
                                     const uint8_t* sh_gate_up, const float* sh_gate_up_scale, int inter, void* hbuf,
                                     void* stream);
int dsv2_moe_route_down_fp8(const void* hbuf, int rows, const int32_t* ids, const float* weights,
                            const uint8_t* w_down, const float* down_scale, const uint8_t* sh_down,
                            const float* sh_down_scale, int inter, int hbuf_routes, const void* residual, void* out,
                            void* stream);

/* Batch family bucketing (one workgroup, deterministic counting sort by expert):
 *   sorted_routes[p] = route index r*6+s in expert order, stable in r;
 *   route_pos[r*6+s] = p;  tiles[t] = {expert, first slot, count<=tile_tokens, 0} (int32x4);
 *   num_tiles[0] = number of tiles (<= rows*6/tile_tokens + 64).  rows*6 <= 49152 (8192 rows),
 *   1 <= tile_tokens <= 256.
 * Replaces _build_route_indices_kernel + _build_route_blocks_kernel (moe_batch.py:95-148). */
int dsv2_moe_bucket(const int32_t* ids, int rows, int tile_tokens, int32_t* sorted_routes, int32_t* route_pos,
                    int32_t* tiles, int32_t* num_tiles, void* stream);

/* dsv2_moe_bucket over many workgroups, for the route counts of prefill chunks: the same
 * outputs bit for bit, in three launches (per-chunk histograms, the exclusive prefix over
 * chunks with the tile table, the stable scatter), the per-chunk histograms in the caller's
 * workspace of dsv2_moe_bucket_workspace_size(rows) bytes (16-byte aligned); rows*6 <= 49152
 * as for dsv2_moe_bucket.  Replaces _build_route_indices_kernel + _build_route_blocks_kernel
 * (moe_batch.py:95-148). */
int64_t dsv2_moe_bucket_workspace_size(int rows);
int dsv2_moe_bucket_wide(const int32_t* ids, int rows, int tile_tokens, int32_t* sorted_routes, int32_t* route_pos,
                         int32_t* tiles, int32_t* num_tiles, void* workspace, int64_t workspace_bytes, void* stream);

/* Expert-grouped gate_up + SwiGLU on bf16 MFMA over the tiles of dsv2_moe_bucket:
 *   hsorted[p, :inter] for p in tile = SwiGLU(xn[sorted_routes[p]/6] . W_e^T).
 * tile_tokens 16, 32, 64 or 256 (256: inter % 128 == 0).
 * Grid is sized by max_tiles; tiles >= num_tiles[0] exit.  Replaces
 * _grouped_gate_up_swiglu_kernel (moe_batch.py:152-234). */
int dsv2_moe_grouped_gateup(const void* xn, const int32_t* sorted_routes, const int32_t* tiles,
                            const int32_t* num_tiles, int max_tiles, int tile_tokens, const void* w_gate_up,
                            int inter, void* hsorted, void* stream);

/* dsv2_moe_grouped_gateup plus the two shared-expert halves in the same launch:
 * shared_out[t, h*inter + i] = SwiGLU(xn[t] . gate/up rows h*inter + i of sh_gate_up)
 * for t < rows, h = 0, 1 (sh_gate_up [2*2*inter, 2048]: gate rows, then up rows), i.e. the
 * dense shared gate_up of dsv2_gemm_bf16 with DSV2_LINEAR_SWIGLU.  The tile table must come
 * from dsv2_moe_bucket with the same tile_tokens (16, 32, 64 or 256).  Replaces _grouped_gate_up_swiglu_kernel
 * (moe_batch.py:152-234) and the shared MLP's gate_proj / up_proj + SiLU-mul (src/run.py:341-351). */
int dsv2_moe_grouped_gateup_shared(const void* xn, int rows, const int32_t* sorted_routes, const int32_t* tiles,
                                   const int32_t* num_tiles, int max_tiles, int tile_tokens, const void* w_gate_up,
                                   const void* sh_gate_up, int inter, void* hsorted, void* shared_out, void* stream);

/* Expert-grouped down projection: ysorted[p, :] = bf16(hsorted[p, :] . Wd_e^T).
 * Replaces _grouped_down_partial_kernel (moe_batch.py:238-307) with a bf16 result
 * (the expert output's own rounding point) instead of an fp32 partial. */
int dsv2_moe_grouped_down(const void* hsorted, const int32_t* tiles, const int32_t* num_tiles, int max_tiles,
                          int tile_tokens, const void* w_down, int inter, void* ysorted, void* stream);

/* dsv2_moe_grouped_down plus the two shared-expert halves in the same launch: shared_parts[h, t, :] = fp32 shared_mid[t, h*inter : (h+1)*inter] . sh_down[:, same]^T
 * for t < rows, h = 0, 1 (shared_mid [rows, 2*inter] from dsv2_moe_grouped_gateup_shared,
 * sh_down [2048, 2*inter]); dsv2_moe_combine_parts adds bf16(half 0 + half 1), the shared
 * MLP's down_proj output (src/run.py:351).  Replaces _grouped_down_partial_kernel
 * (moe_batch.py:238-307) and the shared experts' down projection. */
int dsv2_moe_grouped_down_shared(const void* hsorted, int rows, const int32_t* tiles, const int32_t* num_tiles,
                                 int max_tiles, int tile_tokens, const void* w_down, const void* shared_mid,
                                 const void* sh_down, int inter, void* ysorted, float* shared_parts, void* stream);

/* dsv2_moe_grouped_gateup_shared / dsv2_moe_grouped_down_shared on e4m3 (OCP float8_e4m3fn)
 * expert weights with one fp32 power-of-two scale per weight row (gu_scale [E, 2*inter],
 * sh_gu_scale [2*2816], down_scale [E, 2048], sh_down_scale [2048]; the layouts of
 * quantize_experts_fp8): every product is that of the dequantized bf16 weight (w8 * scale,
 * exact), decoded in the kernel (bf16 MFMA on the activations; the scale multiplies the fp32
 * accumulator).  Same outputs, rounding points and tile table as the bf16 launches; tile_tokens
 * 32 or 64.  The reference's grouped MoE is bf16 only (moe_batch.py:152-307): these replace
 * the same functions with half the weight bytes. */
int dsv2_moe_grouped_gateup_shared_fp8(const void* xn, int rows, const int32_t* sorted_routes, const int32_t* tiles,
                                       const int32_t* num_tiles, int max_tiles, int tile_tokens,
                                       const void* w_gate_up8, const float* gu_scale, const void* sh_gate_up8,
                                       const float* sh_gu_scale, int inter, void* hsorted, void* shared_out,
                                       void* stream);
int dsv2_moe_grouped_down_shared_fp8(const void* hsorted, int rows, const int32_t* tiles, const int32_t* num_tiles,
                                     int max_tiles, int tile_tokens, const void* w_down8, const float* down_scale,
                                     const void* shared_mid, const void* sh_down8, const float* sh_down_scale, int inter,
                                     void* ysorted, float* shared_parts, void* stream);

/* Combine: routed = bf16(sum_s w[r,s] ysorted[route_pos[r*6+s]]) (fp32, slot order);
 * y = shared ? bf16(routed + shared[r]) : routed;  out[r] = residual ? bf16(residual[r] + y) : y.
 * If next_norm_w != NULL also xn_out[r] = RMSNorm(out[r]; next_norm_w).
 * Replaces _batched_down_reduce_topk6_kernel (moe_batch.py:56-92) + the shared add and
 * residual add of the MoE layer (src/run.py:486). */
int dsv2_moe_combine(const void* ysorted, const int32_t* route_pos, const float* weights, int rows,
                     const void* shared, const void* residual, void* out, const void* next_norm_w, float eps,
                     void* xn_out, void* stream);

/* dsv2_moe_combine with the shared output given as the two fp32 halves of
 * dsv2_moe_grouped_down_shared (shared_parts [2, rows, 2048]): shared = bf16(half 0 + half 1). */
int dsv2_moe_combine_parts(const void* ysorted, const int32_t* route_pos, const float* weights, int rows,
                           const float* shared_parts, const void* residual, void* out, const void* next_norm_w,
                           float eps, void* xn_out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSV2LITE_H_ */
