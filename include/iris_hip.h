/* C ABI of libiris_hip.so: the Iris-3B denoiser forward step on one MI355X (gfx950).
 *
 * Conventions shared by every entry point:
 *  - all pointers are caller-owned device memory; nothing here allocates, frees or
 *    synchronises the host, and the work is enqueued on `stream` (0 = null stream);
 *  - return IRIS_OK (0) or a negative IRIS_E_* code; iris_last_error() returns the
 *    message of the calling thread's last failure. Arguments are validated on the
 *    host before anything is launched, as the reference wrappers do with ValueError
 *    (src/iris_metal/kernels.py:299-306);
 *  - dtype codes: IRIS_F32, IRIS_BF16; FP32 is required where the reference requires it
 *    (norm gains, rotary tables, modulation vectors, src/iris_metal/kernels.py:20-21);
 *  - matrices are row-major; "rows" are tokens (or pixels); widths are in elements.
 *
 * The reference's kernel-level FFI is torch.mps.compile_shader + getattr(lib, name)(...)
 * (src/iris_metal/kernels.py:309-311); each entry below names the kernel or the
 * PyTorch op of the reference forward (src/iris_metal/model.py:177-345) it replaces.
 */
#ifndef IRIS_HIP_H
#define IRIS_HIP_H

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { IRIS_OK = 0, IRIS_E_INVALID = -1, IRIS_E_LAUNCH = -2, IRIS_E_UNSUPPORTED = -3 };
enum { IRIS_F32 = 0, IRIS_BF16 = 1 };
/* GEMM epilogues (bias is a separate optional pointer and is added first). */
enum { IRIS_EPI_NONE = 0, IRIS_EPI_SILU_MUL = 1, IRIS_EPI_SILU = 2 };
/* Activations of the GEMV input / output. */
enum { IRIS_ACT_NONE = 0, IRIS_ACT_SILU = 1 };

const char* iris_last_error(void);
/* Library ABI version (bumped on any signature change). */
int iris_abi_version(void);

/* rms_norm_modulate (src/iris_metal/kernels.py:116-146, wrapper 413-452):
 * out[r] = (rmsnorm(x[r]) * weight * (1 + scale[b]) + shift[b]) cast to out_dtype,
 * b = r / rows_per_batch, shift/scale rows mod_stride floats apart. width % 128 == 0, <= 8192. */
int iris_rms_norm_modulate(const void* x, int x_dtype, void* out, int out_dtype, const float* weight,
                           const float* shift, const float* scale, long rows, long rows_per_batch, int width,
                           long mod_stride, float eps, hipStream_t stream);

/* gated_residual_rms_norm_ (src/iris_metal/kernels.py:148-175, wrapper 455-480):
 * residual[r] += gate[b] * rmsnorm(branch[r]) * weight, in place on the FP32 residual. */
int iris_gated_residual_rms_norm(float* residual, const void* branch, int branch_dtype, const float* weight,
                                 const float* gate, long rows, long rows_per_batch, int width, long mod_stride,
                                 float eps, hipStream_t stream);

/* iris_gated_residual_rms_norm followed by iris_rms_norm_modulate of the updated residual in one
 * pass (the post-norm residual of one branch and the input norm of the next, model.py:286-289,
 * 311-313): next_out[r] = (rmsnorm(residual[r]) * next_weight * (1 + next_scale[b]) + next_shift[b])
 * in next_out_dtype, modulation rows next_mod_stride floats apart. */
int iris_gated_residual_norm_modulate(float* residual, const void* branch, int branch_dtype, const float* weight,
                                      const float* gate, long rows, long rows_per_batch, int width, long mod_stride,
                                      float eps, const float* next_weight, const float* next_shift,
                                      const float* next_scale, long next_mod_stride, void* next_out,
                                      int next_out_dtype, hipStream_t stream);

/* The image- and text-stream calls of a dual-stream block in one launch (no reference
 * counterpart; the reference calls gated_residual_rms_norm_ once per stream,
 * model.py:286-289, 311-313): group i is iris_gated_residual_rms_norm (next_out == NULL) or
 * iris_gated_residual_norm_modulate on its own tensors, with the same results; groups = 1 or 2,
 * one branch dtype, one width, one next_out dtype. */
int iris_gated_residual_grouped(int groups, float* const* residual, const void* const* branch, int branch_dtype,
                                const float* const* weight, const float* const* gate, const long* rows,
                                const long* rows_per_batch, int width, const long* mod_stride, float eps,
                                const float* const* next_weight, const float* const* next_shift,
                                const float* const* next_scale, const long* next_mod_stride, void* const* next_out,
                                int next_out_dtype, hipStream_t stream);

/* qk_norm_rope (src/iris_metal/kernels.py:37-84, wrapper 334-397): per (batch, token, head)
 * RMSNorm over 128 values with an FP32 gain, then rotation of pairs (2j, 2j+1) by
 * (cos, sin)[dst_offset + token, j]; reads heads at col_offset of a [batch, n_src, row_stride]
 * projection and writes [batch, heads, n_dst, 128] rows dst_offset + token.
 * cos/sin: FP32 [table_rows, 64]. */
int iris_qk_norm_rope(const void* src, int src_dtype, void* dst, int dst_dtype, const float* weight,
                      const float* cos_table, const float* sin_table, long table_rows, int batch, long n_src,
                      long n_dst, int heads, long dst_offset, long row_stride, long col_offset, float eps,
                      hipStream_t stream);

/* The V half of the attention input (src/iris_metal/model.py:243-250 builds [B,Hkv,N,128]):
 * heads at col_offset of a BF16 [batch, n_src, row_stride] projection are written transposed
 * into a BF16 [batch, heads, 128, n_dst] buffer (n_dst % 64 == 0): token dst_offset + t goes to
 * position s(dst_offset + t), where s swaps the 4-position quads 1 and 2 of every group of 16
 * (positions 4..7 <-> 8..11), the layout iris_flash_attn reads. Other positions are untouched. */
int iris_v_heads_t(const void* src, void* dst, int batch, long n_src, long n_dst, int heads, long dst_offset,
                   long row_stride, long col_offset, hipStream_t stream);

/* The three attention-input calls of one BF16 projection in one launch (the reference makes
 * them separately: qk_norm_rope on Q and on K, src/iris_metal/model.py:236-250, and the V
 * layout): iris_qk_norm_rope of the `heads` Q heads at q_col into q and of the `kv_heads` K
 * heads at k_col into k (gains q_weight / k_weight, rows at dst_offset + t of n_dst), and
 * iris_v_heads_t of the `kv_heads` V heads at v_col into vt (n_vt positions). Same results as
 * the three calls, all BF16. */
int iris_qkv_prepare(const void* src, void* q, void* k, void* vt, const float* q_weight, const float* k_weight,
                     const float* cos_table, const float* sin_table, long table_rows, int batch, long n_src,
                     long n_dst, long n_vt, int heads, int kv_heads, long dst_offset, long row_stride, long q_col,
                     long k_col, long v_col, float eps, hipStream_t stream);

/* softmax(q k^T * scale) v over a joint sequence of n tokens (F.scaled_dot_product_attention
 * with GQA, src/iris_metal/model.py:243-250; src/iris3b/nn/attention.py:61-91).
 * q: BF16 [batch, heads, n_pad, 128]; k: BF16 [batch, kv_heads, n_pad, 128];
 * vt: BF16 [batch, kv_heads, 128, n_pad] as written by iris_v_heads_t (V transposed, the two middle
 * 4-token quads of every 16 positions swapped), zero at the positions of tokens >= n;
 * n_pad = n rounded up to 64.
 * Output row r of batch b goes to out0 row (b*out_batch_rows0 + r) when r < n_split, else to out1
 * row (b*out_batch_rows1 + r - n_split), column h*128 + d, BF16, row stride ld_out; a null out
 * pointer skips its rows. With gate0/gate1 (rows b*gate_batch_rows{0,1} + r or r - n_split,
 * stride ld_gate) the stored value is multiplied by sigmoid(gate) (the attention gate of
 * src/iris_metal/model.py:282-283, 309). Operands are addressed with 32-bit byte offsets:
 * n_pad < 2^23 (IRIS_E_INVALID otherwise). */
int iris_flash_attn(const void* q, const void* k, const void* vt, int batch, int heads, int kv_heads, long n,
                    long n_pad, long n_split, float scale, void* out0, void* out1, long ld_out,
                    long out_batch_rows0, long out_batch_rows1, const void* gate0, const void* gate1, long ld_gate,
                    long gate_batch_rows0, long gate_batch_rows1, hipStream_t stream);

/* Tuning hook for the benchmark sweep and the variant tests: force the attention variant of
 * later iris_flash_attn calls made by the calling thread (32 query rows per wave in all;
 * 0: 64-key tiles staged through registers, 1: 32-key tiles staged through registers,
 * 2: 64-key tiles in a 2-stage global_load_lds ring, 3: 32-key tiles in a 3-stage ring,
 * 4: 32-key tiles in a 3-stage ring shared by twelve waves, four query heads by three 32-row
 * blocks, 5: variant 4 on v_mfma_f32_16x16x32_bf16 instead of v_mfma_f32_32x32x16_bf16) or
 * restore the automatic choice (-1: with four or more query heads per K/V head, variant 5 when
 * one batch item's grid of kv_heads * ceil(n / 96) workgroups fills at least 80% of its rounds
 * over the CUs, else variant 1, so that a row's result never depends on the batch; with fewer,
 * variant 2). Variants 1, 3 and 4 give the same bits;
 * variant 5 sums each score's 128 products and each output's keys in other blocks (to FP32
 * rounding). The setting is per thread. No counterpart in the reference. */
int iris_flash_attn_force_variant(int variant);

/* The text refiner's masked attention (SelfAttention.forward with attn_mask = mask | eye,
 * src/iris3b/nn/attention.py:117-132, src/iris3b/nn/embeddings.py:196-205): as iris_flash_attn
 * with n_split = 0 and no gate, except that query q of batch b attends key j < n only where
 * key_mask[b * n_pad + j] != 0 or j == q. key_mask: [batch, n_pad] bytes, 4-byte aligned (as
 * written by iris_text_key_mask). Output row r of batch b goes to out row b*out_batch_rows + r.
 * n_pad < 2^23, as for iris_flash_attn. */
int iris_flash_attn_masked(const void* q, const void* k, const void* vt, int batch, int heads, int kv_heads, long n,
                           long n_pad, float scale, const void* key_mask, void* out, long ld_out, long out_batch_rows,
                           hipStream_t stream);

/* mask.bool() of the encoder's [batch, >= n] attention mask (row stride ld elements) as the
 * [batch, n_pad] 0/1 bytes iris_flash_attn_masked reads (src/iris3b/nn/embeddings.py:199);
 * elem_kind: 0 bool / uint8, 1 int32, 2 float32, 3 int64; bytes n .. n_pad - 1 are 0. */
int iris_text_key_mask(const void* mask, int elem_kind, long ld, int batch, long n, long n_pad, void* out,
                       hipStream_t stream);

/* Self-attention of each text token over its encoder-layer states (LayerwiseAttentionBlock's
 * SelfAttention without QK norm or RoPE, src/iris3b/nn/embeddings.py:110-141,
 * src/iris3b/nn/attention.py:117-132): qkv BF16 [seqs * seq_len, 3 * heads * head_dim] (q | k |
 * v, head-major inside each) -> out BF16 [seqs * seq_len, heads * head_dim], FP32 softmax with
 * the given scale. seq_len <= 16, head_dim <= 128. */
int iris_layer_attention(const void* qkv, void* out, long seqs, int seq_len, int heads, int head_dim, float scale,
                         hipStream_t stream);

/* The learned pool over encoder layers (LayerwiseTextEmbedder.layer_pool, embeddings.py:262):
 * out[r, c] = sum_l weight[l] * (h[r*layers + l, c] + branch[r*layers + l, c]) + bias[0], with h
 * FP32 [rows * layers, width], branch BF16 of the same shape or null (the last block's residual
 * add, fused), bias null or one value; out FP32 or BF16 [rows, width]. width % 4 == 0. */
int iris_layer_pool(const float* h, const void* branch, const float* weight, const float* bias, long rows, int layers,
                    int width, void* out, int out_dtype, hipStream_t stream);

/* F.linear on bf16 MFMA (src/iris_metal/model.py:46-52): C[m, n] = sum_k A[m, k] B[n, k] + bias[n]
 * with A BF16 [m, lda], B (the weight) BF16 [n, ldb], C in c_dtype with row stride ldc.
 * k % 64 == 0. IRIS_EPI_SILU_MUL: B holds w1 / w3 rows interleaved in 32-row groups
 * (rows 64p..64p+31 = w1 rows 32p.., rows 64p+32..64p+63 = w3 rows 32p..) and
 * C[m, j] = silu(a_j) * b_j is n/2 wide (SwiGLU, src/iris3b/nn/mlp.py:24-40).
 * IRIS_EPI_SILU: C = silu(A B^T + bias) (the Linear + SiLU of the layer-wise text adapter's
 * MLP, src/iris3b/nn/embeddings.py:131-135). Operands are addressed with 32-bit byte offsets:
 * m * lda and n * ldb below 2^30 elements (2 GiB), else IRIS_E_INVALID before any launch.
 * Every output element is the FP32 sum over k in increasing order whatever m and the tile
 * choice, so a row's result does not depend on the other rows. Stateless: no allocation, no
 * host synchronisation, safe to record in a graph. */
int iris_gemm_bf16(const void* a, const void* b, const float* bias, void* c, int c_dtype, int m, int n, int k,
                   long lda, long ldb, long ldc, int epilogue, hipStream_t stream);

/* Tuning hook for the benchmark sweep and the tile tests: force the GEMM tile of later
 * iris_gemm_bf16* calls made by the calling thread (an index into the tile table of gemm.hip:
 * 0-10 tiles of 256x256, 256x192, 192x256 and 128x128 for the eight-wave 32x32x16-MFMA kernel
 * with direct-to-LDS refills, the SiLU epilogue's; 11 and 12 the four-wave 32x32x16 kernel at
 * 256x256 and 192x256; 13-17 the four-wave 16x16x32 kernel at 288x160, 256x160, 128x160,
 * 256x256 and 192x256, the automatic choice for plain, bias and SwiGLU outputs) or restore the
 * automatic choice (-1). A forced tile of the other MFMA shape rounds differently from the
 * automatic one. The setting is per thread. No counterpart in the reference. */
int iris_gemm_force_tile(int tile);

/* Up to two GEMMs of equal n, k and strides in one launch (the image and text streams of a
 * dual-stream block, src/iris_metal/model.py:273-289); each group's operands below 2 GiB, as
 * for iris_gemm_bf16. */
int iris_gemm_bf16_grouped(int groups, const void* const* a, const void* const* b, const float* const* bias,
                           void* const* c, const int* m, int c_dtype, int n, int k, long lda, long ldb, long ldc,
                           int epilogue, hipStream_t stream);

/* The q | k | v projection of an attention block with the per-head RMSNorm + RoPE of its Q and K
 * heads done in the GEMM's store (the reference runs F.linear, then qk_norm_rope on Q and on K,
 * src/iris_metal/model.py:236-250; src/iris_metal/kernels.py:37-84): up to two groups of equal n,
 * k and strides as for iris_gemm_bf16_grouped, no bias. Output columns [0, 128 heads) are the Q
 * heads and the next 128 kv_heads the K heads: they are written as iris_qk_norm_rope writes them
 * (same results) to q BF16 [batch, heads, n_dst, 128] and k_out BF16 [batch, kv_heads, n_dst, 128],
 * row m of group g being token t = m % rows_per_batch[g] of batch item m / rows_per_batch[g], at
 * row dst_offset[g] + t with gains q_weight[g] / k_weight[g] and (cos, sin)[dst_offset[g] + t]
 * (FP32 [table_rows, 64]). The remaining columns go to c (BF16, row stride ldc) as iris_gemm_bf16
 * writes them, and c's Q and K columns are not written; with vt non-null, the kv_heads V heads
 * after the K heads go instead transposed to vt as iris_v_heads_t writes them (BF16 [batch,
 * kv_heads, 128, n_vt], n_vt % 64 == 0; same results), which needs n >= (heads + 2 kv_heads) 128,
 * every group's rows_per_batch % 256 == 0 and dst_offset % 16 == 0, and c then receives only the
 * columns after the V heads. Columns after the V heads (the attention gate of a q | k | v | gate
 * weight, src/iris_metal/model.py:282-283, 309) run as a plain product beside the store, in the
 * same launch for the step's shapes. n % 128 == 0; operands below 2 GiB as for iris_gemm_bf16. */
int iris_gemm_bf16_qk_rope(int groups, const void* const* a, const void* const* b, void* const* c, const int* m,
                           int n, int k, long lda, long ldb, long ldc, const float* const* q_weight,
                           const float* const* k_weight, const int* rows_per_batch, const int* dst_offset,
                           const float* cos_table, const float* sin_table, long table_rows, void* q, void* k_out,
                           int heads, int kv_heads, long n_dst, void* vt, long n_vt, float eps, hipStream_t stream);

/* Matrix-vector products for the timestep MLP and the shared adaLN cores
 * (src/iris_metal/model.py:190-192; src/iris3b/nn/modulation.py:258-285):
 * y[b, n] = act_out(sum_k W[n, k] act_in(x[b, k]) + bias[n]), W BF16 [n, k];
 * with n_extra > 0, out[j, b, n] = y[b, n] + extra_bias[j, n] for j < n_extra
 * (the per-block adaLN biases added to a shared core). */
int iris_gemv_bf16(const void* w, const float* x, int batch, int n, int k, const float* bias,
                   const float* extra_bias, int n_extra, float* out, int in_act, int out_act, hipStream_t stream);

/* Sinusoidal timestep features [cos | sin] (src/iris3b/nn/embeddings.py:41-45):
 * out[b, j] = cos(t[b] * freqs[j]), out[b, half + j] = sin(t[b] * freqs[j]). */
int iris_timestep_features(const float* t, const float* freqs, int batch, int half, float* out,
                           hipStream_t stream);

/* Patchify + pixel embedding (src/iris_metal/model.py:188-189, 208-210; PixelEmbedder,
 * src/iris3b/nn/embeddings.py:291-328; pixel_rms_norm, src/iris_metal/kernels.py:217-232):
 * x FP32 [batch, channels, H, W], channels 3, or 4 for the depth fine-tune's widened embedders
 * (src/iris3b/downstream/depth.py:30-39); patches BF16 [batch, L, patch_stride] (first
 * channels*p*p columns) in (channel, row, column) order; pixels [batch*L, p*p, 16] = x W^T + b +
 * sincos position (W [16, channels], pos_x [W, 8], pos_y [H, 8]); normed BF16 =
 * rmsnorm(pixels) * norm_weight. */
int iris_patchify_embed(const float* x, int batch, int channels, int height, int width, int patch, void* patches,
                        long patch_stride, const float* pix_w, const float* pix_b, const float* pos_x, const float* pos_y,
                        const float* norm_weight, float eps, void* pixels, int pixels_dtype, void* normed,
                        hipStream_t stream);

/* pixel_rms_norm (src/iris_metal/kernels.py:217-232): out = rmsnorm(pixels) * weight, 16 channels. */
int iris_pixel_rms_norm(const void* pixels, int pixels_dtype, void* out, const float* weight, long n_pixels,
                        float eps, hipStream_t stream);

/* pixel_mlp_ (src/iris_metal/kernels.py:235-293, wrapper 527-584), per pixel of 16 channels:
 * x = pixels + branch*(1+scale1)+shift1; h = bf16(rmsnorm(x)*norm_weight);
 * a = bf16(fc1(h)); g = bf16(gelu(a)) (exact-erf GELU, correctly rounded);
 * x += fc2(g)*(1+scale2)+shift2; pixels = x; next_input = rmsnorm(x)*next_norm_weight.
 * The BF16 points (h, a, g and both weights) are the reference kernel's; fc1 / fc2 run on BF16 MFMA
 * with FP32 sums, the stream and the modulation stay FP32 (pixels_dtype F32) or round on store (BF16).
 * mods BF16 [n_pixels, 64] = (scale1, shift1, scale2, shift2); fc1 [64,16], fc2 [16,64] FP32 in memory. */
int iris_pixel_mlp(void* pixels, int pixels_dtype, const void* branch, const void* mods, const float* norm_weight,
                   const float* fc1_w, const float* fc1_b, const float* fc2_w, const float* fc2_b,
                   const float* next_norm_weight, void* next_input, long n_pixels, float eps, hipStream_t stream);

/* Head + unpatchify (src/iris_metal/model.py:214-217): out[b, c, y, x] = h[pixel] . w[c] + bias[c]
 * for h BF16 [batch*L, p*p, 16] (pixels row-major in each patch), w FP32 [out_channels, 16];
 * out_channels 3, or 1 for the depth head (the 1x1 reducer of src/iris3b/downstream/depth.py:37,
 * 47 folded into w and bias by the caller). */
int iris_unpatchify_head(const void* h, const float* w, const float* bias, float* out, int out_channels, int batch,
                         int height, int width, int patch, hipStream_t stream);

/* s_cond = silu(t_emb + image) (src/iris_metal/model.py:207): out[r] = silu(x[r] + t[r / rows_per_batch]). */
int iris_silu_add_rows(const float* x, const float* t, long rows, long rows_per_batch, int width, void* out,
                       int out_dtype, hipStream_t stream);

/* Pre-norm residual step of the text adapter's blocks (src/iris3b/nn/embeddings.py:105-107,
 * 139-141, 205): residual += branch (FP32 residual [rows, width], branch BF16/FP32 or null),
 * then out = rmsnorm(residual) * weight (+ add_rows[row % add_period] when add_rows is given:
 * the position table y_pos_embedding after the refiner's final norm, dit.py:278-279).
 * width % 8 == 0, <= 8192; out BF16 or FP32, not aliasing residual or branch. */
int iris_residual_rms_norm(float* residual, const void* branch, int branch_dtype, const float* weight,
                           const float* add_rows, long add_period, long rows, int width, float eps, void* out,
                           int out_dtype, hipStream_t stream);

/* Row-block copy, dst[b*dst_batch_rows + dst_row_offset + r] = src[b*src_batch_rows + src_row_offset + r]
 * for r < rows: the [text | image] join (src/iris_metal/model.py:201-202) and the image-only
 * slice of the last block (model.py:307-308). FP32 rows of `width`. */
int iris_copy_rows(const float* src, float* dst, int batch, long rows, int width, long src_batch_rows,
                   long src_row_offset, long dst_batch_rows, long dst_row_offset, hipStream_t stream);

/* Turbo flow-Euler update in FP32, in the reference's operation order
 * (src/iris3b/sampling.py:129-135): clean = x - sigma*v; x_next = (1-sigma_next)*clean
 * + sigma_next*((x - (1-sigma)*clean)/sigma). x_next may be null (last step). */
int iris_flow_euler(const float* x, const float* v, long n, float sigma, float sigma_next, float* x_next,
                    float* clean, hipStream_t stream);

/* First-order DPM-Solver++ step (src/iris3b/flow/solver.py:90-94 with x0 = x - s*v):
 * x_next = c_x * x - c_x0 * (x - s * v). */
int iris_dpm1_update(const float* x, const float* v, long n, float s, float c_x, float c_x0, float* x_next,
                     hipStream_t stream);

/* One step of the multistep FlowDPMSolver (src/iris3b/flow/solver.py:90-109, 130-139), FP32, in
 * the reference's operation order: x0 = x - s*v, stored to x0_out when non-null (the next
 * step's history); with x0_prev null the first-order step x_next = c_x*x - c_x0*x0, else the
 * second-order one x_next = (c_x*x - c_x0*x0) - c_d*((x0 - x0_prev)/r0), where c_x = t/s0,
 * c_x0 = (1-t)*expm1(-h), c_d = 0.5*(1-t)*expm1(-h) and r0 = h0/h. Outputs must not alias
 * inputs. */
int iris_dpm_update(const float* x, const float* v, const float* x0_prev, long n, float s, float c_x, float c_x0,
                    float c_d, float r0, float* x_next, float* x0_out, hipStream_t stream);

/* Classifier-free guidance combine (src/iris3b/flow/solver.py:72-74): out = u + scale*(c - u). */
int iris_cfg_combine(const float* v_uncond, const float* v_cond, long n, float scale, float* out,
                     hipStream_t stream);

/* out = clamp(x, lo, hi) (src/iris3b/sampling.py:138). */
int iris_clamp(const float* x, long n, float lo, float hi, float* out, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* IRIS_HIP_H */
