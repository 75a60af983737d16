/*
 * ltx_hip.h -- C ABI of libltx_hip.so, the gfx950 (MI355X) kernels of the
 * LTX-2.3 audio+video DiT denoise step.
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers.  bf16 tensors are passed as `void*`
 *     (2-byte IEEE bfloat16 elements), fp32 tensors as `float*`.
 *   - `stream` is a hipStream_t passed as `void*` (NULL = the null stream).
 *     Every call only enqueues work on that stream; nothing synchronises the
 *     host, allocates or frees memory, or keeps state between calls (the one
 *     exception, ltx_flash_attn_splitkv_noalloc_bf16, keeps a fixed scratch
 *     array per GPU instead of taking a workspace).
 *   - Row-major 2-D tensors carry an explicit row stride in ELEMENTS.
 *   - The return value is an LTX_* status code.  LTX_ERR_UNSUPPORTED means the
 *     shape is outside what the kernel implements; the caller decides whether
 *     a fallback expression applies (the reference's shape gates do exactly
 *     that, see LTX_2_MLX/kernels/fused_ops.py:204-234, :369-395).
 *
 * Reference interfaces replaced (paths relative to the LTX-2-MLX tree):
 *   ltx_adaln_norm_fused_bf16   <- kernels/fused_ops.py:237 adaln_norm_fused
 *                                  (Metal kernel :104-180; inline forms
 *                                  model/transformer/transformer.py:21-37,
 *                                  :374-375, :535-580)
 *   ltx_gated_add_fused_bf16    <- kernels/fused_ops.py:398 gated_add_fused
 *                                  (Metal kernel :314-353; inline forms
 *                                  transformer.py:40-50, :387, :484, :598, :625)
 *   ltx_qknorm_rope_bf16        <- model/transformer/attention.py:578-584
 *                                  (RMSNorm :320-329 + rope.py:16-89)
 *   ltx_output_norm_modulate_bf16 <- model/transformer/model.py:1312-1342
 *   ltx_euler_x0_step_bf16      <- model.py:1519-1525 (X0Model.denoise) +
 *                                  components/diffusion_steps.py:19-69
 *   ltx_timestep_embedding_f32  <- model/transformer/timestep_embedding.py:9-59
 *   ltx_gemv_f32_bf16w          <- timestep_embedding.py:88-201 (AdaLN MLPs)
 */
#ifndef LTX_HIP_H_
#define LTX_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LTX_OK 0
#define LTX_ERR_INVALID_ARG (-1)
#define LTX_ERR_UNSUPPORTED (-2)
#define LTX_ERR_HIP (-3)
#define LTX_ERR_ALIGNMENT (-4)
/* The request needs more than the fixed scratch of a no-allocation entry point. */
#define LTX_ERR_SCRATCH_LIMIT (-5)

/* Human-readable name of a status code (static storage). */
const char* ltx_status_string(int status);

/* Library version, encoded as major*10000 + minor*100 + patch. */
int ltx_version(void);

/* Measurement aid with no counterpart in the reference: writes the GPU's
 * constant-rate real-time counter (s_memrealtime) to dst[0] (device memory,
 * 8-byte aligned) when the stream reaches the call; under graph capture it
 * becomes a kernel node, so a pair of stamps times the work between them
 * inside a replayed graph (HIP events cannot be recorded there).  Ticks per
 * second are found by comparing two stamps with the host clock. */
int ltx_device_clock_stamp(uint64_t* dst, void* stream);

/* ---- flags for ltx_adaln_norm_fused_bf16 ---------------------------------- */
/* Round the normalised row to bf16 before modulating: the reference's
 * `mx.fast.rms_norm(x)` (bf16 output) followed by the fp32 modulation, i.e.
 * transformer.py:36-37 / :374 / :535-580.  Without it the single-rounding
 * fused-kernel semantics of fused_ops.py:172-175 apply. */
#define LTX_ADALN_ROUND_NORM 1
/* Skip the RMS normalisation: out = bf16(x*(1+scale)+shift), the text-context
 * KV modulation of transformer.py:375. */
#define LTX_ADALN_NO_NORM 2

/*
 * out[r, c] = bf16( rms(x[r,:]) * (1 + scale[c]) + shift[c] ),
 *   rms(x) = x * rsqrt(mean(x^2) + eps), sum of squares in fp32.
 * x: (rows, C) bf16 with row stride x_stride; out: (rows, C) bf16 with row
 * stride out_stride (out may alias x).  scale/shift: fp32 (C).  C must be a
 * multiple of 512 and at most 4096.  Replaces adaln_norm_fused
 * (kernels/fused_ops.py:237-287).
 */
int ltx_adaln_norm_fused_bf16(const void* x, int64_t x_stride, const float* scale,
                              const float* shift, void* out, int64_t out_stride,
                              int64_t rows, int64_t C, float eps, int flags,
                              void* stream);

/*
 * Two modulations of one row norm: out as ltx_adaln_norm_fused_bf16 with
 * (scale, shift), out2 with (scale2, shift2), each row read once.  The
 * reference's block modulates the same pre-cross-attention norm of a stream
 * twice, for its A2V and its V2A input (transformer.py:535-564); bit-identical
 * to two ltx_adaln_norm_fused_bf16 calls.  out2 row stride out2_stride.
 */
int ltx_adaln_norm_fused2_bf16(const void* x, int64_t x_stride, const float* scale,
                               const float* shift, void* out, int64_t out_stride,
                               const float* scale2, const float* shift2, void* out2,
                               int64_t out2_stride, int64_t rows, int64_t C, float eps,
                               int flags, void* stream);

/* ---- flags for ltx_gated_add_fused_bf16 ----------------------------------- */
/* Round branch*gate to bf16 before the add: `x + (attn_out*gate).astype(bf16)`
 * of the text cross-attention (transformer.py:387, :484). */
#define LTX_GATED_ROUND_PRODUCT 1

/*
 * out[r, c] = bf16( gate[c] * branch[r, c] + residual[r, c] ) in fp32.
 * residual/branch/out: (rows, C) bf16, each with its own row stride; out may
 * alias residual.  gate: fp32 (C).  C must be a multiple of 512 and at most
 * 4096.  Replaces gated_add_fused (kernels/fused_ops.py:398-442).
 */
int ltx_gated_add_fused_bf16(const void* residual, int64_t residual_stride,
                             const void* branch, int64_t branch_stride,
                             const float* gate, void* out, int64_t out_stride,
                             int64_t rows, int64_t C, int flags, void* stream);

/*
 * In-place QK-RMSNorm + split RoPE for one attention call
 * (attention.py:578-584):
 *   q[t,:] = bf16( rope( bf16( rms(q[t,:]) * wq ), cos_q[t], sin_q[t] ) )
 *   k[t,:] = likewise with wk, cos_k, sin_k.
 * The norm spans the whole inner dim D (= heads*head_dim), as the reference's
 * RMSNorm(inner_dim) does.  Split RoPE (rope.py:37-50): within each head the
 * first half of the channels rotates with the second half,
 *   [x1*c - x2*s, x1*s + x2*c], evaluated in fp32.
 * Tables are fp32, row-major (rows, D/2): entry [t, h*head_dim/2 + i] is the
 * angle's cos/sin for head h, pair i -- the reference's (1, H, T, dh/2)
 * tensor transposed to token-major.  Pass NULL tables to skip RoPE (text
 * cross-attention).  q/k rows have strides q_stride/k_stride (elements), so
 * they can live inside a fused QKV projection output.  D must be a multiple of
 * 1024 and at most 4096; head_dim in {64, 128}.  rows_q or rows_k may be 0.
 */
int ltx_qknorm_rope_bf16(void* q, int64_t q_stride, int64_t rows_q, const float* wq,
                         const float* cos_q, const float* sin_q, void* k,
                         int64_t k_stride, int64_t rows_k, const float* wk,
                         const float* cos_k, const float* sin_k, int64_t D,
                         int64_t head_dim, float eps, void* stream);

/*
 * ltx_qknorm_rope_bf16 with tables factored over the position axes (same
 * reference call site; the reference builds its per-token tables from
 * per-axis frequencies, rope.py:92-336).  Each table column depends on one
 * position axis only, so cos_q / sin_q hold tab_rows_q stacked rows -- a few
 * per axis -- and idx_q (rows_q, axes_q) int32 selects the token's row of
 * every axis; the kernel combines them as
 *   cos = cos_q[idx[t,0]] * cos_q[idx[t,1]] * ...,
 *   sin = sin_q[idx[t,0]] + sin_q[idx[t,1]] + ...   (fp32, axis order),
 * a column's foreign-axis rows holding exactly 1 and -0, which reproduces the
 * per-token table bit for bit while its bytes stay in cache.  idx NULL means
 * row t of a per-token table (as ltx_qknorm_rope_bf16); 1 <= axes <= 3;
 * indices outside [0, tab_rows) are clamped.  Same for the k side.
 */
int ltx_qknorm_rope_axes_bf16(void* q, int64_t q_stride, int64_t rows_q, const float* wq,
                              const float* cos_q, const float* sin_q, const int32_t* idx_q,
                              int64_t axes_q, int64_t tab_rows_q, void* k, int64_t k_stride,
                              int64_t rows_k, const float* wk, const float* cos_k,
                              const float* sin_k, const int32_t* idx_k, int64_t axes_k,
                              int64_t tab_rows_k, int64_t D, int64_t head_dim, float eps,
                              void* stream);

/*
 * Output head modulation (model.py:1312-1342):
 *   ss     = bf16(table[0:2, :] + emb[:])           (shift row 0, scale row 1)
 *   n      = bf16(LayerNorm(x, no affine, eps))
 *   out    = bf16(bf16(n * bf16(1 + scale)) + shift)  (bf16 arithmetic)
 * x/out: (rows, C) bf16 with row strides; table: fp32 (2, C); emb: fp32 (C).
 * C must be a multiple of 512 and at most 4096.
 */
int ltx_output_norm_modulate_bf16(const void* x, int64_t x_stride, const float* table,
                                  const float* emb, void* out, int64_t out_stride,
                                  int64_t rows, int64_t C, float eps, void* stream);

/*
 * One distilled Euler step fused with the X0 conversion
 * (model.py:1519-1525, diffusion_steps.py:58-69), elementwise over n values:
 *   x0  = fp32(latent) - sigma * fp32(velocity)
 *   out = bf16( x0 + ratio * (fp32(latent) - x0) ),  ratio = fp32(sigma_next/sigma)
 * Every product and sum is rounded separately, as in the reference.  out may
 * alias latent.
 */
int ltx_euler_x0_step_bf16(const void* latent, const void* velocity, float sigma,
                           float ratio, void* out, int64_t n, void* stream);

/*
 * Sinusoidal timestep embedding with flip_sin_to_cos=True, shift 0,
 * max_period 10000 (timestep_embedding.py:9-59, :140-144):
 *   out[i]        = cos(t * exp(-ln(10000) * i / half)),  i < half
 *   out[half + i] = sin(...)
 * for `count` timesteps t[j] = values[j] * multiplier; out is (count, dim).
 */
int ltx_timestep_embedding_f32(const float* values, int64_t count, float multiplier,
                               float* out, int64_t dim, void* stream);

/* ---- flags for ltx_gemv_f32_bf16w ----------------------------------------- */
#define LTX_GEMV_SILU_INPUT 1  /* apply SiLU to x before the product */
#define LTX_GEMV_SILU_OUTPUT 2 /* apply SiLU to y after the bias */

/*
 * y[b, n] = act( sum_k W[n, k] * act(x[b, k]) + bias[n] ), fp32 accumulation.
 * x: fp32 (batch, K); W: bf16 (N, K) row-major; bias: fp32 (N) or NULL;
 * y: fp32 (batch, N).  batch <= 8.  The AdaLN MLP layers run on a
 * per-step scalar timestep (timestep_embedding.py:111-123, :186-201).
 */
int ltx_gemv_f32_bf16w(const float* x, int64_t batch, int64_t K, const void* W,
                       const float* bias, float* y, int64_t N, int flags,
                       void* stream);

/*
 * out[b, i] = table[b, i] + vec[i] for b < nb, i < n (fp32): the AdaLN
 * modulation rows of every block, `scale_shift_table + timestep`
 * (transformer.py:286-342), computed for all blocks in one launch per step.
 */
int ltx_broadcast_add_f32(const float* table, const float* vec, float* out, int64_t nb,
                          int64_t n, void* stream);

/* ---- projection GEMMs ------------------------------------------------------
 * C[m, n] = epilogue( sum_k A[m, k] * W[n, k] + bias[n] ),
 * fp32 accumulation on bf16 matrix cores (v_mfma_f32_32x32x16_bf16).
 * A: bf16 (M, K) row stride lda.  W in nn.Linear layout (N, K), row stride ldw,
 * as bf16, int8 (+ fp32 per-row scale) or MXFP8 (E4M3 codes + E8M0 scale per
 * 32 consecutive k, scale row stride ld_scale bytes).  Quantised weights are
 * dequantised to bf16 exactly per their definition before the bf16 MFMA:
 *   int8 : w = bf16(fp32(q) * s[n])
 *   MXFP8: w = bf16(e4m3(q) * 2^(e - 127))
 * bias: fp32 (N) or NULL.  C: bf16 (M, N) row stride ldc.
 * Requirements: K % 64 == 0, N % 8 == 0, 16-byte aligned pointers and row
 * strides; MXFP8 scales 4-byte aligned with ld_scale % 4 == 0.  `epilogue` is
 * one of LTX_GEMM_EPI_* optionally OR-ed with a tile override
 * (LTX_GEMM_TILE_256 / _128 / _256_DMA / _256x128 / _G8; default: by problem size;
 * the default may run the product as two launches on `stream`, 256-row tiles
 * for the first rows and 128-row tiles for the rest, bit-identical to one).
 * With LTX_GEMM_EPI_BIAS, output columns n >= sigmoid_from get the head-gate
 * epilogue of LTX_GEMM_EPI_SIGMOID2 instead (pass N for none): the per-head
 * gate logits ride along with the Q / QKV projection in one GEMM.
 * Replaces mx.addmm / nn.Linear (attention.py:425-437, feed_forward.py:91-112)
 * and mx.quantized_matmul(mode="mxfp8") (loader/transformer_cache.py:177-193).
 */
#define LTX_GEMM_EPI_BIAS 0           /* C = bf16(acc + bias) */
#define LTX_GEMM_EPI_GELU 1           /* C = bf16(gelu_tanh(bf16(acc + bias))) (feed_forward.py:101-102) */
#define LTX_GEMM_EPI_RESIDUAL 2       /* C = bf16(R + gate * bf16(acc + bias)) (fused_ops.py:345-348) */
#define LTX_GEMM_EPI_RESIDUAL_ROUND 3 /* C = bf16(R + bf16(gate * bf16(acc + bias))) (transformer.py:387, :484) */
#define LTX_GEMM_EPI_SIGMOID2 4       /* C = bf16(2 * bf16(sigmoid(bf16(acc + bias)))) (attention.py:563-569) */
#define LTX_GEMM_TILE_256 (1 << 8)
#define LTX_GEMM_TILE_128 (2 << 8)
#define LTX_GEMM_TILE_256_DMA (3 << 8) /* 256x256, LDS-DMA loader */
#define LTX_GEMM_TILE_256x128 (4 << 8) /* 256 rows x 128 columns */
/* 256x256, eight waves in two groups that alternate between global->LDS
 * loads / fragment reads and MFMAs; every weight format (MXFP8 needs
 * K % 512 == 0 and 16-byte aligned scale rows, else LTX_ERR_UNSUPPORTED).
 * The automatic choice for int8 and MXFP8 weights when 256x256 tiles are
 * chosen, and for bf16 weights on products at least as wide as deep
 * (N >= K) or of 100-159 tiles. */
#define LTX_GEMM_TILE_G8 (5 << 8)
/* The eight-wave kernel with 128 x 256 tiles (same conditions as
 * LTX_GEMM_TILE_G8), for products whose 256 x 256 tiles fill only part of
 * one round; never the automatic choice. */
#define LTX_GEMM_TILE_G8_128 (6 << 8)
/* OR-ed into `epilogue`: the bias is added to the bf16-rounded product,
 * acc' = bf16(acc) + bias, before the epilogue's own steps -- the
 * quantised-linear form `quantized_matmul(x, w) + bias` of nn.QuantizedLinear
 * (loader/transformer_cache.py:177-193), which rounds the product to the
 * activation dtype before the bias add.  Without it the bias is added to the
 * fp32 accumulator (mx.addmm, one rounding). */
#define LTX_GEMM_ROUND_THEN_BIAS (1 << 12)

int ltx_gemm_bf16(const void* A, int64_t lda, const void* W, int64_t ldw, const float* bias,
                  void* C, int64_t ldc, int64_t M, int64_t N, int64_t K, int epilogue,
                  const void* residual, int64_t ldr, const float* gate, int64_t sigmoid_from,
                  void* stream);

int ltx_gemm_w8a16_bf16(const void* A, int64_t lda, const int8_t* Wq, int64_t ldw,
                        const float* w_scale, const float* bias, void* C, int64_t ldc,
                        int64_t M, int64_t N, int64_t K, int epilogue, const void* residual,
                        int64_t ldr, const float* gate, int64_t sigmoid_from, void* stream);

int ltx_gemm_mxfp8_bf16(const void* A, int64_t lda, const uint8_t* Wq, int64_t ldw,
                        const uint8_t* w_scale, int64_t ld_scale, const float* bias, void* C,
                        int64_t ldc, int64_t M, int64_t N, int64_t K, int epilogue,
                        const void* residual, int64_t ldr, const float* gate, int64_t sigmoid_from,
                        void* stream);

/* The bias-epilogue product (LTX_GEMM_EPI_BIAS, optionally OR-ed with
 * LTX_GEMM_ROUND_THEN_BIAS and LTX_GEMM_TILE_G8 / _G8_128) of one weight
 * format -- wformat 0: bf16 W as ltx_gemm_bf16, 1: int8 W + fp32 w_scale as
 * ltx_gemm_w8a16_bf16, 2: MXFP8 W + E8M0 w_scale (ld_scale) as
 * ltx_gemm_mxfp8_bf16 -- plus the per-row sums of squares of its bf16
 * outputs in columns [0, ss_cols):
 *   rowss[m * ld_rowss + j] = sum_{n in [64 j, 64 j + 64)} C[m, n]^2 (fp32).
 * ss_cols % 64 == 0, ss_cols <= min(N, sigmoid_from), ld_rowss >= ss_cols / 64,
 * rowss 4-byte aligned.  Always the eight-wave kernel (LTX_ERR_UNSUPPORTED
 * where it does not apply); C equals the plain entry point's result on that
 * kernel bit for bit.  No counterpart in the reference: the row statistics of
 * the query RMS norm (attention.py:578-580) for ltx_flash_attn_qnorm_v_bf16,
 * which then needs no separate pass over Q. */
int ltx_gemm_rowss_bf16(int wformat, const void* A, int64_t lda, const void* W, int64_t ldw,
                        const void* w_scale, int64_t ld_scale, const float* bias, void* C, int64_t ldc,
                        int64_t M, int64_t N, int64_t K, int epilogue, int64_t sigmoid_from,
                        float* rowss, int64_t ld_rowss, int64_t ss_cols, void* stream);

/* MXFP8 activations x MXFP8 weights on the gfx950 scaled fp8 MFMA
 * (v_mfma_scale_f32_32x32x64_f8f6f4), an opt-in path.  No counterpart in the
 * reference: its MXFP8 weights (loader/transformer_cache.py:177-193) are
 * dequantised and multiplied with bf16 activations, as ltx_gemm_mxfp8_bf16
 * does; here the activations are quantised too (E4M3 codes (M, K), row stride
 * lda bytes, E8M0 scales (M, K/32), row stride ld_ascale -- the layout
 * ltx_quantize_mxfp8_bf16 writes for any rows), so results differ from the
 * bf16-activation path by the activations' E4M3 rounding.  W / w_scale as in
 * ltx_gemm_mxfp8_bf16; same epilogue codes and LTX_GEMM_ROUND_THEN_BIAS.
 * Needs K % 512 == 0, N % 8 == 0, 16-byte aligned pointers and byte strides. */
int ltx_gemm_mx_bf16(const uint8_t* A, int64_t lda, const uint8_t* a_scale, int64_t ld_ascale,
                     const uint8_t* Wq, int64_t ldw, const uint8_t* w_scale, int64_t ld_scale,
                     const float* bias, void* C, int64_t ldc, int64_t M, int64_t N, int64_t K,
                     int epilogue, const void* residual, int64_t ldr, const float* gate,
                     int64_t sigmoid_from, void* stream);

/* The opt-in MX path's feed-forward up-projection (no counterpart in the
 * reference): ltx_gemm_mx_bf16 with the GELU epilogue
 * (feed_forward.py:101-102) whose bf16 result is written as MXFP8 rows --
 * E4M3 codes (M, N) with row stride ldcq bytes and E8M0 scales (M, N/32) --
 * exactly what ltx_quantize_mxfp8_bf16 makes of the bf16 GELU output, i.e.
 * the down-projection's quantised input.  flags: 0 or LTX_GEMM_ROUND_THEN_BIAS.
 * Needs N % 32 == 0 besides ltx_gemm_mx_bf16's conditions. */
int ltx_gemm_mx_gelu_mxfp8(const uint8_t* A, int64_t lda, const uint8_t* a_scale, int64_t ld_ascale,
                           const uint8_t* Wq, int64_t ldw, const uint8_t* w_scale, int64_t ld_scale,
                           const float* bias, uint8_t* Cq, int64_t ldcq, uint8_t* c_scale, int64_t ld_cscale,
                           int64_t M, int64_t N, int64_t K, int flags, void* stream);

/* Split-K forms of the three GEMMs for few-row products (the 68-token audio
 * stream, 256-token contexts): `splits` blocks per 128x128 output tile each
 * accumulate K / splits of the product into an fp32 partial tile in
 * `workspace` (ltx_gemm_splitk_workspace_bytes(M, N, splits) bytes, 16-byte
 * aligned, caller-owned), then one pass sums the partials in split order and
 * applies the epilogue of the single-pass kernel (same flags, same rounding
 * points; the fp32 sum order differs).  K % (64 * splits) == 0 (MXFP8:
 * K % (128 * splits) == 0), 1 <= splits <= 64, tile override 0 or
 * LTX_GEMM_TILE_128.  Same operand rules as above.
 */
int64_t ltx_gemm_splitk_workspace_bytes(int64_t M, int64_t N, int64_t splits);
int ltx_gemm_splitk_bf16(const void* A, int64_t lda, const void* W, int64_t ldw, const float* bias,
                         void* C, int64_t ldc, int64_t M, int64_t N, int64_t K, int epilogue,
                         const void* residual, int64_t ldr, const float* gate, int64_t sigmoid_from,
                         int splits, float* workspace, int64_t workspace_bytes, void* stream);
int ltx_gemm_splitk_w8a16_bf16(const void* A, int64_t lda, const int8_t* Wq, int64_t ldw,
                               const float* w_scale, const float* bias, void* C, int64_t ldc,
                               int64_t M, int64_t N, int64_t K, int epilogue, const void* residual,
                               int64_t ldr, const float* gate, int64_t sigmoid_from, int splits,
                               float* workspace, int64_t workspace_bytes, void* stream);
int ltx_gemm_splitk_mxfp8_bf16(const void* A, int64_t lda, const uint8_t* Wq, int64_t ldw,
                               const uint8_t* w_scale, int64_t ld_scale, const float* bias, void* C,
                               int64_t ldc, int64_t M, int64_t N, int64_t K, int epilogue,
                               const void* residual, int64_t ldr, const float* gate,
                               int64_t sigmoid_from, int splits, float* workspace,
                               int64_t workspace_bytes, void* stream);

/* Few-row forms of the three GEMMs, in one launch: the same products as
 * ltx_gemm_bf16 / ltx_gemm_w8a16_bf16 / ltx_gemm_mxfp8_bf16 (the reference's
 * nn.Linear / nn.QuantizedLinear calls, attention.py:425-437,
 * feed_forward.py:91-112, loader/transformer_cache.py:177-193) for products
 * with few rows -- the 68- or 121-token audio stream -- which these kernels
 * bind by their weight bytes rather than their flops.  Workgroups of 128
 * columns x up to 128 rows each accumulate K / splits of the product into an
 * fp32 partial tile in `workspace` (ltx_gemm_rows_workspace_bytes(M, N,
 * splits) bytes, 16-byte aligned); the last split of each tile to finish sums
 * the partials in split order and applies the epilogue, with the flags and
 * rounding points of ltx_gemm_* (the fp32 sum order differs).  `counters`
 * (ltx_gemm_rows_counter_words(M, N) uint32 words, 4-byte aligned; needed
 * when splits > 1) must be zero on the first call and every call leaves them
 * zero, so one zeroed array serves every later call on a stream; calls that
 * may run at the same time need their own workspace and counters.
 * K % (128 * splits) == 0 for 8-bit weights, K % (64 * splits) == 0 for bf16;
 * 1 <= splits <= 64; MXFP8 scale rows 4-byte aligned with ld_scale % 4 == 0.
 * Operand rules as for ltx_gemm_*. */
int64_t ltx_gemm_rows_workspace_bytes(int64_t M, int64_t N, int64_t splits);
int64_t ltx_gemm_rows_counter_words(int64_t M, int64_t N);
int ltx_gemm_rows_bf16(const void* A, int64_t lda, const void* W, int64_t ldw, const float* bias,
                       void* C, int64_t ldc, int64_t M, int64_t N, int64_t K, int epilogue,
                       const void* residual, int64_t ldr, const float* gate, int64_t sigmoid_from,
                       int splits, float* workspace, int64_t workspace_bytes, uint32_t* counters,
                       int64_t counter_words, void* stream);
int ltx_gemm_rows_w8a16_bf16(const void* A, int64_t lda, const int8_t* Wq, int64_t ldw,
                             const float* w_scale, const float* bias, void* C, int64_t ldc,
                             int64_t M, int64_t N, int64_t K, int epilogue, const void* residual,
                             int64_t ldr, const float* gate, int64_t sigmoid_from, int splits,
                             float* workspace, int64_t workspace_bytes, uint32_t* counters,
                             int64_t counter_words, void* stream);
int ltx_gemm_rows_mxfp8_bf16(const void* A, int64_t lda, const uint8_t* Wq, int64_t ldw,
                             const uint8_t* w_scale, int64_t ld_scale, const float* bias, void* C,
                             int64_t ldc, int64_t M, int64_t N, int64_t K, int epilogue,
                             const void* residual, int64_t ldr, const float* gate,
                             int64_t sigmoid_from, int splits, float* workspace,
                             int64_t workspace_bytes, uint32_t* counters, int64_t counter_words,
                             void* stream);

/* ---- weight formats (load-time) --------------------------------------------
 * MXFP8, OCP Microscaling v1.0 with E4M3 elements, blocks of 32 along K and an
 * E8M0 scale (the storage of loader/transformer_cache.py:1255-1267; codes (N,K)
 * uint8 are byte-identical to the reference's (N, K/4) uint32 words):
 *   X = floor(log2(max|w|)) - 8 clamped to [-127, 127] (-127 for a zero block),
 *   scale = X + 127, code = E4M3(w / 2^X), round-to-nearest-even, saturated to
 *   +-448.  The reference's own encoder is MLX-internal; this is the OCP rule.
 * int8 W8A16, symmetric per output channel (defined for the W8A16 GEMMs):
 *   s[n] = max|w[n,:]| / 127 (fp32), q = clamp(rint(w / s), -127, 127),
 *   q = 0 for a zero row.  Decode: bf16(fp32(q) * s[n]).
 * W: bf16 (N, K) row stride ldw.  Decoders write bf16 (N, K) row stride ldo.
 */
int ltx_quantize_mxfp8_bf16(const void* W, int64_t ldw, int64_t N, int64_t K, uint8_t* q,
                            int64_t ldq, uint8_t* scales, int64_t ld_scale, void* stream);
int ltx_dequantize_mxfp8_bf16(const uint8_t* q, int64_t ldq, const uint8_t* scales,
                              int64_t ld_scale, int64_t N, int64_t K, void* out, int64_t ldo,
                              void* stream);
int ltx_quantize_w8_bf16(const void* W, int64_t ldw, int64_t N, int64_t K, int8_t* q,
                         int64_t ldq, float* scale, void* stream);
int ltx_dequantize_w8_bf16(const int8_t* q, int64_t ldq, const float* scale, int64_t N,
                           int64_t K, void* out, int64_t ldo, void* stream);

/* FP8 checkpoint tensor dequantisation -- the numeric step of
 * loader/transformer_cache.py:658-708 (_iter_fp8_checkpoint_weights):
 *   out[i] = OUT(from_fp8(codes[i]) * weight_scale)
 * with the E4M3 decode exact (0x7F / 0xFF NaN), the product in fp32 and one
 * round-to-nearest-even into OUT = bf16 (out_dtype 0) or fp32 (out_dtype 1).
 * scale: device pointer to the tensor's fp32 weight_scale, or NULL for an
 * unscaled tensor (exact decode).  codes and out 16-byte aligned, n elements
 * (any n >= 0), flat.  E5M2 is not decoded (the reference rejects it too).
 */
int ltx_dequantize_fp8_e4m3(const uint8_t* codes, int64_t n, const float* scale, void* out,
                            int out_dtype, void* stream);

/* ---- guided sampling ----------------------------------------------------------
 * The elementwise math around the transformer passes of the guided loops
 * (pipelines/av_pipeline.py:625-757, two_stage.py:306-388).  Every operation
 * is one IEEE fp32 operation in the reference's order; scalars are the fp32
 * values of the reference's python floats (MLX casts weak scalars to fp32).
 *
 * ltx_x0_from_velocity_f32  <- X0Model.denoise (model/transformer/model.py:1519-1525)
 *   out = latent - sigma * velocity            (bf16 latent / velocity, fp32 out)
 * ltx_guidance_f32          <- CFGGuider / CFGStarRescalingGuider / STGGuider .guide
 *                              and .delta, MultiModalGuider.calculate
 *                              (components/guiders.py:10-172)
 *   u0  = coef0 ? coef0[0] * term0 : term0
 *   out = base + c0*(base - u0) + c1*(base - term1) + c2*(base - term2)
 *         (terms added left to right, absent (NULL) terms skipped), then
 *         * factor[0] if factor is given;  LTX_GUIDE_DELTA_ONLY: out = c0*(base - u0).
 *   CFG guide: base=cond, term0=uncond, c0=scale-1; CFG-star: coef0 from the
 *   projection statistic; STG: base=guided, term0=perturbed, c0=scale;
 *   MultiModalGuider: base=cond, terms (uncond, perturbed, modality).
 * ltx_guidance_stats_f32    <- projection_coef (guiders.py:175-190) and the
 *                              MultiModalGuider std rescale (:155-161); one
 *                              workgroup, fp64 accumulation of fp32 products:
 *   LTX_GUIDE_STATS_PROJECTION: out[0] = sum(a*b) / (sum(b*b) + 1e-8)
 *   LTX_GUIDE_STATS_STD_RATIO:  out[0] = rescale * std(a)/std(b) + one_minus_rescale,
 *                               std(x) = sqrt(var(x) + 1e-8)
 * ltx_ge_correct_f32        <- GE velocity correction (av_pipeline.py:722-728), in place:
 *   cur = (latent - denoised) / sigma; if prev_valid:
 *   denoised = latent - (gamma*(cur - prev) + prev) * sigma;  prev = cur
 * ltx_euler_step_bf16       <- EulerDiffusionStep.step (components/diffusion_steps.py:19-69)
 *   out = bf16(denoised + ratio * (sample - denoised)), ratio = fp32(sigma_next / sigma)
 * fp32 arrays 16-byte aligned (scalars 4-byte), n elements, flat.
 */
#define LTX_GUIDE_DELTA_ONLY 1
#define LTX_GUIDE_STATS_PROJECTION 1
#define LTX_GUIDE_STATS_STD_RATIO 2

int ltx_x0_from_velocity_f32(const void* latent, const void* velocity, float sigma, float* out,
                             int64_t n, void* stream);
int ltx_guidance_f32(const float* base, const float* term0, const float* term1, const float* term2,
                     float c0, float c1, float c2, const float* coef0, const float* factor,
                     float* out, int64_t n, int flags, void* stream);
int ltx_guidance_stats_f32(const float* a, const float* b, int64_t n, int mode, float rescale,
                           float one_minus_rescale, float* out, void* stream);
int ltx_ge_correct_f32(const void* latent, float* denoised, float* prev_velocity, int prev_valid,
                       float sigma, float gamma, int64_t n, void* stream);
int ltx_euler_step_bf16(const void* sample, const float* denoised, float ratio, void* out, int64_t n,
                        void* stream);

/* ---- text-conditioning features ------------------------------------------------
 * GemmaFeaturesExtractorV2 normalisation (model/text_encoder/feature_extractor.py:
 * 9-79) for `layers` Gemma hidden states of `tokens` x `dim` bf16 (layer l,
 * token t at hidden + l*layer_stride + t*row_stride), in the reference's bf16
 * arithmetic:  y = mask[t] ? bf16(x * bf16(1/sqrt(bf16(bf16(mean(bf16(x*x))) + eps)))) : 0,
 *   out_video[t, l*dim + d] = bf16(y * scale_video),  out_audio likewise,
 * eps / scales given as their bf16 values (python floats meeting bf16 arrays).
 * Output rows (tokens, layers*dim) are layer-major; the aggregate-embedding
 * weights are permuted to match (the reference's feature index is d*layers + l).
 * mask: int32 (tokens), nonzero keeps the token; NULL keeps all.
 */
int ltx_gemma_features_bf16(const void* hidden, int64_t layers, int64_t tokens, int64_t dim,
                            int64_t layer_stride, int64_t row_stride, const int32_t* mask, float eps,
                            float scale_video, float scale_audio, void* out_video, void* out_audio,
                            int64_t out_stride, void* stream);

/* ---- latent layouts ------------------------------------------------------------
 * Swap of the two outer axes of an (A, B, R) array, out[b, a, r] = in[a, b, r],
 * for 2- or 4-byte elements; out must not alias in.  The reference's
 * patchifiers at batch 1 (components/patchifiers.py:52-124, :327-374):
 *   video patchify   (C, F*H*W, 1) -> (F*H*W, C, 1)   unpatchify: the inverse swap
 *   audio patchify   (C, T, M)     -> (T, C, M)       unpatchify: the inverse swap
 */
int ltx_swap_axes(const void* in, int64_t A, int64_t B, int64_t R, int elem_bytes, void* out,
                  void* stream);

/* ---- attention ---------------------------------------------------------------
 * Flash attention with the per-head output gate fused (replaces
 * attention.py:283-302 -> kernels/steel_attention.py:251-280 and the gate of
 * attention.py:594-598):
 *   O[q, h*dh + :] = bf16( bf16( softmax_k(Q_h[q] . K_h[k] * scale) V_h ) * gate[q, h] )
 * bf16 inputs, fp32 scores, online softmax and accumulation, bf16 P for the
 * second product; no mask (the reference's T2V calls pass none,
 * pipelines/common.py:242-252).
 * Q (Tq, H*head_dim), K (Tk, H*head_dim), O (Tq, H*head_dim): token-major
 * rows with row strides q_rs/k_rs/o_rs (elements), head h at columns
 * [h*head_dim, (h+1)*head_dim).  gate: bf16 (Tq, H) with row stride gate_rs,
 * or NULL.  head_dim in {64, 128}.
 * ltx_flash_attn_v_bf16 reads V (Tk, H*head_dim) token-major with row stride
 * v_rs, like Q and K (the projection output as written; the kernel transposes
 * V fragments on their way out of LDS).  ltx_flash_attn_bf16 takes V
 * pre-transposed as Vt (H, head_dim, tk_pad), produced by
 * ltx_attn_transpose_v_bf16; both give bit-identical results.
 */
int ltx_flash_attn_v_bf16(const void* Q, int64_t q_rs, const void* K, int64_t k_rs,
                          const void* V, int64_t v_rs, void* O, int64_t o_rs,
                          const void* gate, int64_t gate_rs, int64_t Tq, int64_t Tk,
                          int64_t H, int64_t head_dim, float scale, void* stream);
int64_t ltx_attn_vt_padded_len(int64_t Tk);
int ltx_attn_transpose_v_bf16(const void* V, int64_t v_rs, int64_t Tk, int64_t H,
                              int64_t head_dim, void* Vt, int64_t tk_pad, void* stream);
int ltx_flash_attn_bf16(const void* Q, int64_t q_rs, const void* K, int64_t k_rs,
                        const void* Vt, int64_t tk_pad, void* O, int64_t o_rs,
                        const void* gate, int64_t gate_rs, int64_t Tq, int64_t Tk,
                        int64_t H, int64_t head_dim, float scale, void* stream);

/* ltx_flash_attn_v_bf16 on the raw query projection: the kernel applies the
 * query RMS norm and split RoPE of ltx_qknorm_rope_bf16 / _axes_bf16 as it
 * loads Q (attention.py:578-584 fused into the attention core,
 * attention.py:283-302), from ss (Tq, ss_parts) fp32 per-row partial sums of
 * squares over the whole inner dim H*head_dim (ss_parts a multiple of 4 in
 * [4, 64], row stride ld_ss a multiple of 4, 16-byte aligned; e.g. the rowss
 * of ltx_gemm_rowss_bf16 for the Q columns), the norm weights wq (fp32,
 * H*head_dim, 16-byte aligned) and eps:
 *   x = bf16(q * rsqrt(sum(ss[q, :]) / (H*head_dim) + eps) * wq)
 * then the pair (d, d + head_dim/2) of each head rotated by the fp32 tables
 * cos / sin of H*head_dim/2 columns (16-byte aligned): one row per query
 * (idx NULL, tab_rows >= Tq) or `axes` (1-3) factored rows per query at
 * idx[q * axes + a] (int32, clamped to [0, tab_rows)), combined as for
 * ltx_qknorm_rope_axes_bf16; cos = sin = NULL: no RoPE.  Single pass (no
 * split-KV form), token-major V. */
int ltx_flash_attn_qnorm_v_bf16(const void* Q, int64_t q_rs, const void* K, int64_t k_rs,
                                const void* V, int64_t v_rs, void* O, int64_t o_rs, const void* gate,
                                int64_t gate_rs, int64_t Tq, int64_t Tk, int64_t H, int64_t head_dim,
                                float scale, const float* ss, int64_t ld_ss, int64_t ss_parts,
                                const float* wq, float eps, const float* cos, const float* sin,
                                const int* idx, int64_t axes, int64_t tab_rows, void* stream);

/* Split-KV form of ltx_flash_attn_bf16 for few queries over many keys (the
 * audio-query V2A cross-attention: 68-121 queries x 3456-6144 video keys):
 * the keys are cut into `splits` ranges processed by separate workgroups,
 * whose partial (O, max, sum) go to `workspace` and are merged by a second
 * kernel; same result contract as ltx_flash_attn_bf16 (the merge reorders the
 * fp32 sums only).  workspace: device memory of at least
 * ltx_attn_splitkv_workspace_bytes(Tq, H, head_dim, splits) bytes, 16-byte
 * aligned, owned by the caller; concurrent calls need separate workspaces.
 * 1 <= splits <= 256.  Same reference call site as ltx_flash_attn_bf16; the
 * _v_ form reads token-major V as ltx_flash_attn_v_bf16 does.
 */
int64_t ltx_attn_splitkv_workspace_bytes(int64_t Tq, int64_t H, int64_t head_dim, int64_t splits);
int ltx_flash_attn_splitkv_v_bf16(const void* Q, int64_t q_rs, const void* K, int64_t k_rs,
                                  const void* V, int64_t v_rs, void* O, int64_t o_rs,
                                  const void* gate, int64_t gate_rs, int64_t Tq, int64_t Tk,
                                  int64_t H, int64_t head_dim, float scale, int64_t splits,
                                  void* workspace, int64_t workspace_bytes, void* stream);
int ltx_flash_attn_splitkv_bf16(const void* Q, int64_t q_rs, const void* K, int64_t k_rs,
                                const void* Vt, int64_t tk_pad, void* O, int64_t o_rs,
                                const void* gate, int64_t gate_rs, int64_t Tq, int64_t Tk,
                                int64_t H, int64_t head_dim, float scale, int64_t splits,
                                void* workspace, int64_t workspace_bytes, void* stream);

/* ltx_flash_attn_splitkv_bf16 without the workspace argument and without any
 * allocation: the partials go to a scratch array of
 * LTX_ATTN_NOALLOC_SCRATCH_BYTES that the library holds in device memory, one
 * per GPU, for the life of the process (its address is resolved once per
 * device, on the first call whose stream is on that device; make that first
 * call outside HIP graph capture -- later calls only enqueue kernels and can
 * be captured).  No counterpart
 * in the reference: it exists for callers that cannot allocate device memory
 * (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc).  Same arguments and result contract as
 * ltx_flash_attn_splitkv_bf16; a request with
 * ltx_attn_splitkv_workspace_bytes(Tq, H, head_dim, splits) above the limit
 * returns LTX_ERR_SCRATCH_LIMIT and enqueues nothing.  Nothing in the scratch
 * needs to start at zero.  Every call on one GPU uses that GPU's one array,
 * so calls that may overlap on a GPU (different streams, or several host
 * threads) race: serialise them. */
#define LTX_ATTN_NOALLOC_SCRATCH_BYTES (32ll << 20)
int ltx_flash_attn_splitkv_noalloc_bf16(const void* Q, int64_t q_rs, const void* K, int64_t k_rs,
                                        const void* Vt, int64_t tk_pad, void* O, int64_t o_rs,
                                        const void* gate, int64_t gate_rs, int64_t Tq, int64_t Tk,
                                        int64_t H, int64_t head_dim, float scale, int64_t splits,
                                        void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LTX_HIP_H_ */
