/*
 * qd_oracle.h -- CPU restatement of the reference's decode-attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links or calls this
 * code; it is the checker used by tests/, by __graft_entry__.smoke() and by the
 * cpu_baseline leg of bench.py.
 *
 * Every function restates, in plain C with IEEE fp32 arithmetic and no FP
 * contraction (built with -ffp-contract=off), the exact operation order of the
 * reference CUDA kernel it cites.  fp16 values travel as raw IEEE binary16 bit
 * patterns (uint16_t).
 *
 * Reference files (SeaTheDestiny/LLM-inference-DIY):
 *   kernels/flash_decode_q1_opt.cuh:434-537  fd_v5_fused_kernel
 *   kernels/flash_decode_q1_opt.cuh:548-656  fd_v5_split_stage1_kernel
 *   kernels/flash_decode_q1_opt.cuh:666-724  fd_opt_stage2_kernel
 *   framework_src/qwen_infer.cu:644-678      per-layer fused/split dispatch
 *   kernels/fused_qkv_rope_cache.cuh:6-55    fused_qkv_rope_cache_kernel
 *   kernels/bias.cuh:6-11                    add_bias_kernel (QKV bias use)
 *
 * Deviations that no run of the reference here can pin (documented, not gaps):
 *   - the reference builds with --use_fast_math (__expf/__logf/__sinf...); the
 *     oracle calls glibc expf/logf/powf/cosf/sinf;
 *   - where the reference source writes `a*b + c` without __fmaf_rn, nvcc may
 *     contract it; the oracle rounds the product and the sum separately.
 */
#ifndef QD_ORACLE_H
#define QD_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE binary16 <-> binary32 (round-to-nearest-even), as cuda_fp16's
 * __half2float / __float2half. */
float qd_oracle_h2f(uint16_t h);
uint16_t qd_oracle_f2h(float f);
void qd_oracle_h2f_array(const uint16_t* in, float* out, long long n);
void qd_oracle_f2h_array(const float* in, uint16_t* out, long long n);

/* Variants of the decode-attention restatement. */
enum {
  QD_ORACLE_ENGINE = 0, /* qwen_infer.cu:646-678: C=ceil(L/256); fused<128,8,32> if C==1 else split */
  QD_ORACLE_FUSED = 1,  /* fd_v5_fused_kernel<128,32,32>, min(32,ceil(L/32)) warps (bench_fd_opt.cu:303-317); L <= 1024 */
  QD_ORACLE_SPLIT = 2   /* fd_v5_split_stage1_kernel<128,256,8> + fd_opt_stage2_kernel<128>, any L >= 1 */
};

/* One head of fd_v5_fused_kernel<128, *, rows_per_warp> launched with
 * num_warps warps.  q[128]; K/V row r at k + r*row_stride.  Rows beyond
 * num_warps*rows_per_warp are not visited (as in the reference). */
void qd_oracle_fd_fused_head(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                             uint16_t* out, int seqlen, long long row_stride,
                             int rows_per_warp, int num_warps);

/* One head of the split path: stage 1 over ceil(L/chunk) chunks of `chunk`
 * rows with `warps` warps each, then stage 2.  partial (ceil(L/chunk)*128 fp16)
 * and lse (ceil(L/chunk) floats) receive the stage-1 intermediates when non-NULL. */
void qd_oracle_fd_split_head(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                             uint16_t* out, int seqlen, long long row_stride,
                             int chunk, int warps, uint16_t* partial, float* lse);

/* All heads.  q/out are [H][128] contiguous.  Head h's K/V rows live at
 * k + h*head_stride + r*row_stride (elements).  nthreads >= 1 worker threads
 * split the (head, chunk) tasks.  Returns 0, or -1 on invalid arguments. */
int qd_oracle_decode_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                               uint16_t* out, int seqlen, int num_heads,
                               long long row_stride, long long head_stride,
                               int variant, int nthreads);

/* add_bias_kernel on qkv[3*H*D] (when bias != NULL) followed by
 * fused_qkv_rope_cache_kernel at position pos: Q rotated in place, rotated K and
 * raw V written to cache row pos at k_cache/v_cache + pos*row_stride +
 * h*head_stride + d.  Returns 0, or -1 on invalid arguments. */
int qd_oracle_qkv_bias_rope_cache(uint16_t* qkv, const uint16_t* bias,
                                  uint16_t* k_cache, uint16_t* v_cache, int pos,
                                  int num_heads, int head_dim,
                                  long long row_stride, long long head_stride,
                                  float rope_base);

/* cos/sin of fused_qkv_rope_cache.cuh:36-38 for one (pos, i). */
void qd_oracle_rope_cos_sin(int pos, int i, int head_dim, float rope_base,
                            float* cos_out, float* sin_out);

/* Reduction orders of the adjacent decode-step ops.
 *   QD_ORDER_REF:    the reference kernels' order (rmsnorm.cuh:15-45 per-thread
 *                    blocks + 32-lane butterflies; hgemm_final.cuh:278-294
 *                    sequential k per output column);
 *   QD_ORDER_WAVE64: the fixed order of this build's gfx950 kernels: lane l of
 *                    a 64-lane wave owns elements k = 512*j + 8*l + e (j outer,
 *                    e inner, summed sequentially), then the 64 lane sums are
 *                    added in the tree of qd_oracle_wave64_sum. */
enum { QD_ORDER_REF = 0, QD_ORDER_WAVE64 = 1 };

/* The gfx950 wave reduction: within each 16-lane row ((a0+a1)+(a2+a3)) +
 * ((a4+a5)+(a6+a7)) ..., then (row0+row1) + (row2+row3). */
float qd_oracle_wave64_sum(const float* lanes);

/* RMSNorm (rmsnorm.cuh:6-57): out = half(x * r * w), r = 1/sqrt(mean(x^2)+eps).
 * ORDER_REF follows the reference's 512-thread reduction (n must be a multiple
 * of 512); both orders take r = 1.0f / sqrtf(.) where the reference calls
 * rsqrtf. */
void qd_oracle_rmsnorm(const uint16_t* x, const uint16_t* w, int n, float eps,
                       uint16_t* out, int order);

/* out[n] = half(sum_k x[k] * W(n, k)), n < N.  layout 0: W(n,k) = W[n*K + k]
 * (the .bin file's [out][in]); layout 1: W(n,k) = W[k*N + n] (the reference
 * engine's transposed [in][out], transpose.cuh:17-30). */
void qd_oracle_gemv(const uint16_t* x, const uint16_t* W, int N, int K, int layout,
                    int order, uint16_t* out);

/* Attention front end of one decode layer (qwen_infer.cu:626-642):
 * [RMSNorm of x with norm_w when norm_w != NULL] -> QKV GEMV with
 * w_qkv [3*H*D][H*D] ([out][in]) -> half -> + bias -> half -> rotate-half RoPE
 * at pos -> K/V cache append.  qkv_out receives the rotated Q and the biased
 * K and V, as the reference's d_qkv after its three launches. */
int qd_oracle_qkv_front(const uint16_t* x, const uint16_t* norm_w, float eps,
                        const uint16_t* w_qkv, const uint16_t* bias, uint16_t* qkv_out,
                        uint16_t* k_cache, uint16_t* v_cache, int pos, int num_heads,
                        int head_dim, long long row_stride, long long head_stride,
                        float rope_base, int order);

/* ---- the gfx950 kernels' own arithmetic (llm-inference-diy_amd/csrc) ----
 * These restate this build's kernels step for step, so the GPU results can be
 * compared bit for bit.  They are pinned independently (float64, the
 * reference-order functions above, closed forms) by tests/test_oracle_gfx.py. */

/* exp2_rep (qd_device.h): n = rint(x), f = x - n, 2^f = 1 + f*q(f) with q
 * in Estrin form (c1 + c2 f) + f^2((c3 + c4 f) + f^2 (c5 + c6 f)), every
 * bracket and the final 1 + f*q one fmaf, ldexp by n; 0 for x <= -125 or
 * NaN, +inf for x >= 128. */
float qd_oracle_exp2(float x);
void qd_oracle_exp2_array(const float* x, float* out, long long n);

/* A decode-attention launch plan (qd_attn_plan of include/qdiy/attn.h). */
typedef struct {
  int variant;        /* 0: one workgroup per head (fused), 1: split + merge */
  int num_splits;     /* split workgroups per head */
  int rows_per_split; /* KV rows per split workgroup */
  int rows_per_tile;  /* rows each 16-lane group takes per tile (template U) */
  int waves;          /* wavefronts per scan workgroup */
  int block_rows;     /* split plans: 0 for contiguous ranges [c * rows_per_split,
                         ...); else the rows form blocks of block_rows (waves * 4 *
                         rows_per_tile) dealt to the splits in turn, split c taking
                         blocks c, c + num_splits, ... */
} qd_oracle_plan;

/* decode_attention_scan_kernel (+ decode_attention_merge_kernel for split
 * plans) of qd_attention.hip for all heads under `plan`: scores by 8-term
 * fmaf chains per lane and the 16-lane tree, exp2 by qd_oracle_exp2, the
 * tile-wise online softmax, the lane-shuffle and LDS folds, and the 8-slice
 * merge.  Same argument meaning as qd_oracle_decode_attention.  Returns 0, or
 * -1 on invalid arguments (including a split plan that does not cover
 * [0, seqlen) with non-empty workgroups, and interleaved blocks other than
 * one load round of a workgroup). */
int qd_oracle_attention_planned(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                uint16_t* out, int seqlen, int num_heads, long long row_stride,
                                long long head_stride, const qd_oracle_plan* plan, int nthreads);

/* ---- the rest of the decode step and the model (qd_oracle_model.c) ----
 * GEMVs in the wave64 order (QD_ORDER_WAVE64), fp16 roundings where the
 * reference stores halves; nthreads >= 1 host threads split GEMV rows (results
 * do not depend on it). */

/* out[n] = half(residual[n] + half(W[n] . x)), W [n_out][k_in] (out may alias
 * residual): qwen_infer.cu:701-704, :718-721. */
void qd_oracle_proj_residual(const uint16_t* x, const uint16_t* W, const uint16_t* residual,
                             uint16_t* out, int n_out, int k_in, int nthreads);

/* half(g * (u / (1 + exp2(-u * log2 e)))) of two fp16 values (swiglu.cuh:6-15
 * with exp(-u) as qd_oracle_exp2). */
uint16_t qd_oracle_swiglu(uint16_t g, uint16_t u);

/* act[i] = swiglu(half(W1[i] . xn), half(W2[i] . xn)), xn = RMSNorm(x) * norm_w:
 * qwen_infer.cu:708-715. */
void qd_oracle_ffn_up_swiglu(const uint16_t* x, const uint16_t* norm_w, float eps,
                             const uint16_t* w1, const uint16_t* w2, uint16_t* act, int hidden,
                             int inter, int nthreads);

/* The reference's SwiGLU of two fp16 values, half(g * (u / (1 + expf(-u))))
 * (swiglu.cuh:11-13 with glibc expf for __expf). */
uint16_t qd_oracle_swiglu_ref(uint16_t g, uint16_t u);

/* argmax_kernel<<<1, 512>>> over vocab fp16 logits (argmax.cuh:7-72), its tie
 * order included; -1 when no value exceeds -inf. */
int qd_oracle_argmax_ref(const uint16_t* logits, int vocab);

/* logits[v] = half(W[v] . xn) (logits may be NULL); returns the argmax, ties
 * to the lowest index, -0 == +0, NaN never wins: qwen_infer.cu:725-731. */
int qd_oracle_lm_head_argmax(const uint16_t* x, const uint16_t* norm_w, float eps,
                             const uint16_t* W, uint16_t* logits, int vocab, int hidden,
                             int nthreads);

/* A model over a .bin image (include/qdiy/engine.h's format; the image is
 * referenced, not copied, and must outlive the model) with a KV cache of
 * max_pos positions.  NULL on invalid arguments. */
typedef struct qd_oracle_model qd_oracle_model;
qd_oracle_model* qd_oracle_model_new(const void* image, long long bytes, int max_pos, int nthreads);

/* The same with the arithmetic `order` of every op: QD_ORDER_WAVE64 (as
 * qd_oracle_model_new: this build's kernels) or QD_ORDER_REF (the reference
 * kernels' own: 512-thread RMSNorm, GEMV sums with k ascending, the engine's
 * attention dispatch of qd_oracle_decode_attention, SwiGLU with expf, and
 * argmax_kernel's tie order).  Forward then ignores `plan` (may be NULL). */
qd_oracle_model* qd_oracle_model_new_order(const void* image, long long bytes, int max_pos,
                                           int nthreads, int order);
void qd_oracle_model_free(qd_oracle_model* m);

/* One token through all layers at `pos` (KV rows written), attention under
 * `plan` (the plan at length pos + 1).  With want_logits, also the final norm,
 * lm_head and argmax: returns the next token and copies the vocab fp16
 * logits to logits_out (may be NULL); otherwise returns 0.  -1 on invalid
 * arguments. */
int qd_oracle_model_forward(qd_oracle_model* m, int token, int pos, const qd_oracle_plan* plan,
                            int want_logits, uint16_t* logits_out);

/* Greedy generation from a .bin image (include/qdiy/engine.h's format): the
 * prompt's first n_prompt - 1 tokens fill the KV cache, then n_new steps from
 * the last prompt token, each token produced by the full layer stack and
 * lm_head argmax (qwen_infer.cu:780-817, prompts through the decode step).
 * plans[L - 1] is the attention launch plan at length L for L = 1 ..
 * n_prompt + n_new.  out_tokens receives *n_out tokens (fewer than n_new only
 * when stop_at_eos hits 151645 or 151643); last_logits (vocab fp16, may be
 * NULL) the logits of the last step.  Returns 0, or -1 on invalid
 * arguments. */
int qd_oracle_generate(const void* image, long long bytes, const int* prompt, int n_prompt,
                       int n_new, int stop_at_eos, const qd_oracle_plan* plans, int n_plans,
                       int* out_tokens, int* n_out, uint16_t* last_logits, int nthreads);

#ifdef __cplusplus
}
#endif
#endif /* QD_ORACLE_H */
