/*
 * qdiy/decode.h -- C ABI of the rest of one decode step on MI355X (gfx950):
 * the launches of the reference engine's QwenEngine::step around attention
 * (SeaTheDestiny/LLM-inference-DIY, framework_src/qwen_infer.cu:700-731).
 *
 *   gemm(d_attn_proj, d_qkv_out, attn_proj_w, 1, H, H)        (:701)
 *   add_bias_kernel(d_x, d_attn_proj, H)                      (:704)
 *       -> qd_proj_residual(d_qkv_out, attn_proj_w, d_x, d_x, H, H)
 *   rmsnorm_kernel(d_norm_x, d_x, ln_2, H, eps)               (:708)
 *   gemm(d_ffn_w1, ...) ; gemm(d_ffn_w2, ...)                 (:711-712)
 *   swiglu_kernel(d_ffn_act, d_ffn_w1, d_ffn_w2, IM)          (:715)
 *       -> qd_ffn_up_swiglu(d_x, ln_2, eps, ffn_w1, ffn_w2, d_ffn_act, H, IM)
 *   gemm(d_ffn_proj, d_ffn_act, ffn_proj_w, 1, H, IM)         (:718)
 *   add_bias_kernel(d_x, d_ffn_proj, H)                       (:721)
 *       -> qd_proj_residual(d_ffn_act, ffn_proj_w, d_x, d_x, H, IM)
 *   rmsnorm_kernel(d_norm_x, d_x, ln_f, H, eps)               (:725)
 *   gemm(d_logits, d_norm_x, lm_head, 1, V, H)                (:728)
 *   argmax_kernel(d_next_token, d_logits, V)                  (:731)
 *       -> qd_lm_head_argmax(d_x, ln_f, eps, lm_head, d_logits, V, H, ws, ...)
 *
 * Conventions are those of qdiy/attn.h: fp16 as uint16_t bit patterns in
 * device memory, asynchronous on `stream`, status codes, no host sync.
 * Weight matrices stay in the .bin file's [out][in] layout
 * (model_weights/convert_weights.py:135-172); the reference engine transposes
 * them at load (qwen_infer.cu:230-241) for its hgemv_kernel, this library
 * reads them as stored.
 *
 * Numerics: every GEMV output is the fp32 sum of exact fp16 x fp16 products in
 * one fixed order -- lane l of a 64-lane wave owns elements
 * k = 512*j + 8*l + e and adds them sequentially (j, then e ascending), then
 * the 64 lane sums are added in a fixed tree -- rounded once to fp16 where the
 * reference stores a half.  RMSNorm uses the same order for its sum of
 * squares.  Results are therefore bit-for-bit reproducible on the host.
 */
#ifndef QDIY_DECODE_H
#define QDIY_DECODE_H

#include <stddef.h>
#include <stdint.h>

#include "qdiy/attn.h"
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* out[n] = half(residual[n] + half(sum_k W[n][k] * x[k])) for n < n_out.
 * W is [n_out][k_in] fp16; k_in a multiple of 8, at most 8192; x, w 16-byte
 * aligned.
 * residual and out may be the same buffer (the reference adds in place into
 * d_x); otherwise they must not overlap, and out must not overlap x or w
 * (QD_EINVAL).  Replaces hgemv_kernel + add_bias_kernel (hgemm_final.cuh:274-295,
 * bias.cuh:6-11; qwen_infer.cu:701-704 and :718-721). */
int qd_proj_residual(const uint16_t* x, const uint16_t* w, const uint16_t* residual,
                     uint16_t* out, int n_out, int k_in, hipStream_t stream);

/* act[i] = half(g_i * (u_i / (1 + exp(-u_i)))), g_i = half(W1[i] . xn),
 * u_i = half(W2[i] . xn), xn = half(x * (1/sqrt(mean(x^2) + eps)) * norm_w),
 * for i < inter.  W1 (gate, ffn_w1) and W2 (up, ffn_w2) are [inter][hidden];
 * hidden a multiple of 512, at most 4096.  exp(-u) is computed as
 * 2^(-u * log2 e) by a polynomial the host can repeat exactly.  act must
 * not overlap x, norm_w, w1 or w2 (QD_EINVAL).  Replaces
 * rmsnorm_kernel + 2 x hgemv_kernel + swiglu_kernel (rmsnorm.cuh:6-57,
 * swiglu.cuh:6-15; qwen_infer.cu:708-715). */
int qd_ffn_up_swiglu(const uint16_t* x, const uint16_t* norm_w, float eps, const uint16_t* w1,
                     const uint16_t* w2, uint16_t* act, int hidden, int inter,
                     hipStream_t stream);

/* Batched projection of m rows (prompt tokens at once):
 *   y[i][j] = half(sum_k x[i][k] * w[j][k])                        residual == NULL
 *   y[i][j] = half(float(residual[i][j]) + float(half(sum)))       otherwise
 * for i < m, j < n.  x rows are ldx elements apart, y and residual rows ldy
 * apart; w is [n][k], the .bin file's layout (the reference transposes its
 * weights at load and multiplies [k][n]).  Replaces QwenEngine::gemm for m > 1
 * (qwen_infer.cu:359-367: hgemm_swizzle_nn) in prefill (:462, :542, :573-574,
 * :593).
 *   mode QD_GEMM_EXACT: every output is the decode step's sum for that row --
 *     lane l of a wave adds k = 512j + 8l + e in order, then the fixed wave64
 *     tree -- so a prompt's rows are bit-identical to qd_proj_residual and the
 *     decode GEMVs token by token.  k a multiple of 8, at most 8192.
 *   mode QD_GEMM_MFMA: the matrix cores (v_mfma_f32_16x16x32_f16); products
 *     are exact and summed in fp32 in the hardware's order, so results are not
 *     reproducible on the host.  k a multiple of 64.
 * x and w 16-byte aligned, ldx a multiple of 8 and >= k, ldy >= n; y and
 * residual 2-byte aligned.  residual may be y (in place); y must not overlap x
 * or w (QD_EINVAL). */
#define QD_GEMM_EXACT 0
#define QD_GEMM_MFMA 1
int qd_gemm_nt(const uint16_t* x, long long ldx, const uint16_t* w, const uint16_t* residual,
               uint16_t* y, long long ldy, int m, int n, int k, int mode, hipStream_t stream);

/* Batched FFN up-projection of m prompt rows on the matrix cores, gate and up
 * GEMMs in one pass with the SwiGLU in the epilogue:
 *   act[i][j] = half(g * (u / (1 + exp(-u)))),  g = half(x[i] . w1[j]),
 *                                              u = half(x[i] . w2[j])
 * for i < m, j < n (x rows ldx apart, act rows ldy apart; w1 and w2 [n][k]).
 * Replaces the prompt's w1 and w2 gemms and swiglu_kernel
 * (qwen_infer.cu:573-586).  exp(-u) is this library's exp2 of -u * log2(e)
 * (as qd_ffn_up_swiglu); the sums are fp32 in the hardware's order, as in
 * QD_GEMM_MFMA.  k a positive multiple of 64; x, w1 and w2 16-byte aligned,
 * ldx a multiple of 8 and >= k, ldy >= n, act 2-byte aligned and not
 * overlapping x, w1 or w2. */
int qd_gemm_swiglu(const uint16_t* x, long long ldx, const uint16_t* w1, const uint16_t* w2,
                   uint16_t* act, long long ldy, int m, int n, int k, hipStream_t stream);

/* Causal attention of `tokens` prompt queries at positions pos0 .. pos0 +
 * tokens - 1 of one layer, all heads: query t attends over cache rows
 * [0, pos0 + t] (rows written beforehand, K rotated).  Query t's row is
 * q + t*q_stride (head h at + h*128: the rotated Q third of the prefill's QKV
 * rows); its output row is out + t*out_stride.  Replaces the reference's
 * prompt attention, qwen_infer.cu:484-527 (gather_q_from_qkv and
 * gather_kv_from_cache into per-head buffers, flash_attn_tuned_A_kernel with
 * the causal mask of flash_attn_causal.cuh once per head, then
 * scatter_interleaved_kernel), reading Q and the cache in place.
 *   mode QD_GEMM_EXACT: every query with the arithmetic qd_decode_attention
 *     uses at its length, batched (one fused launch for the queries of up to
 *     224 rows, scan + merge pairs for the others): outputs are bit-identical
 *     to decoding the prompt token by token.  The first call with queries
 *     beyond 224 rows allocates the context's prefill scratch.
 *   mode QD_GEMM_MFMA: one causal FlashAttention launch on the matrix cores
 *     (v_mfma_f32_16x16x32_f16, softmax weights rounded to fp16 for the
 *     product, hardware exp2): within 2e-3 of the exact outputs for
 *     N(0,1)-scale inputs, not reproducible on the host.
 * Requires tokens >= 1, 0 <= pos0, pos0 + tokens <= max_seqlen; q, out,
 * k_layer and v_layer 16-byte aligned; q_stride and out_stride multiples of 8
 * and >= num_heads*128; out must not overlap q or the cache rows read. */
int qd_prefill_attention(qd_ctx* ctx, const uint16_t* q, long long q_stride, const uint16_t* k_layer,
                         const uint16_t* v_layer, uint16_t* out, long long out_stride, int pos0,
                         int tokens, int num_heads, int head_dim, int mode, hipStream_t stream);

/* Device workspace (bytes) qd_lm_head_argmax needs for a vocabulary size. */
size_t qd_lm_head_workspace_bytes(int vocab);

/* logits[v] = half(W[v] . xn) for v < vocab with xn the RMSNorm of x by
 * norm_w (as above), then *token (device int) = the index of the largest
 * logit.  Ties go to the lowest index; -0 equals +0; NaN never wins.  (The
 * reference's argmax_kernel breaks ties by its thread and lane order,
 * argmax.cuh:19-66.)  W is [vocab][hidden].  workspace: device memory of
 * qd_lm_head_workspace_bytes(vocab) bytes, 8-byte aligned.  logits,
 * workspace and token must not overlap each other or x, norm_w, w
 * (QD_EINVAL).  Replaces
 * rmsnorm_kernel + hgemv_kernel + argmax_kernel (qwen_infer.cu:725-731). */
int qd_lm_head_argmax(const uint16_t* x, const uint16_t* norm_w, float eps, const uint16_t* w,
                      uint16_t* logits, int vocab, int hidden, void* workspace,
                      size_t workspace_bytes, int* token, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* QDIY_DECODE_H */
