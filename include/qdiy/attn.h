/*
 * qdiy/attn.h -- C ABI of the MI355X (gfx950) q=1 decode-attention hot path.
 *
 * Drop-in replacement for the decode-attention section of the reference
 * engine's per-layer step (SeaTheDestiny/LLM-inference-DIY,
 * framework_src/qwen_infer.cu:629-678):
 *
 *   add_bias_kernel<<<24,256>>>(d_qkv, qkv_b, 3H)                  (:631)
 *   fused_qkv_rope_cache_kernel<<<16,64>>>(d_qkv, Kc_l, Vc_l, pos)   (:634-642)
 *   for h in 0..15: fd_v5_fused_kernel | fd_v5_split_stage1_kernel +
 *                   fd_opt_stage2_kernel on head h                   (:646-678)
 *
 * becomes two calls per layer:
 *
 *   qd_qkv_bias_rope_cache(ctx, d_qkv, qkv_b, Kc_l, Vc_l, pos, ...)
 *   qd_decode_attention(ctx, d_qkv, Kc_l, Vc_l, d_qkv_out, pos + 1, ...)
 *
 * Conventions
 *   - fp16 buffers are IEEE binary16 bit patterns (uint16_t), device memory.
 *   - KV cache element (pos, head, d) of one layer lives at
 *       base + pos*kv_row_stride + head*kv_head_stride + d      (elements)
 *     The reference engine layout [max_seqlen][num_heads*128] is
 *     kv_row_stride = num_heads*128, kv_head_stride = 128 (qwen_infer.cu:75-76,
 *     :636-637, :654-661).
 *   - q and out are [num_heads][128] contiguous (the Q third of d_qkv and
 *     d_qkv_out, qwen_infer.cu:659,662).
 *   - Every call is asynchronous on `stream` and never synchronises the host.
 *     Launch errors are returned at once; execution errors surface on the
 *     caller's next synchronisation.
 *   - Status codes replace the reference's print-and-continue
 *     (qwen_infer.cu:679-683).  No call ever exits the process.
 *   - A context owns device scratch (split partials, RoPE table).  Calls that
 *     share a context must be ordered on one stream, the way the reference's
 *     per-head launches share d_fd_partial on the default stream
 *     (qwen_infer.cu:672-676).
 */
#ifndef QDIY_ATTN_H
#define QDIY_ATTN_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QD_HEAD_DIM 128

enum qd_status {
  QD_OK = 0,
  QD_EINVAL = 1,   /* an argument is out of range, misaligned or NULL */
  QD_EHIP = 2,     /* a HIP runtime call failed; see qd_last_error() */
  QD_ENOMEM = 3    /* device or host allocation failed */
};

typedef struct qd_cfg {
  int num_heads;            /* heads per layer (16 for Qwen-1.8B)            */
  int head_dim;             /* must be 128 (qwen_infer.cu:641,649)           */
  int max_seqlen;           /* cache rows per layer; bounds pos and seqlen   */
  long long kv_row_stride;  /* elements between positions (num_heads*128)    */
  long long kv_head_stride; /* elements between heads in a position (128)    */
  float rope_base;          /* 10000.0f (fused_qkv_rope_cache.cuh:36)        */
} qd_cfg;

typedef struct qd_ctx qd_ctx;

/* Creates a context on the current HIP device: validates cfg, allocates the
 * split scratch and builds the [max_seqlen][64] RoPE cos/sin table on the host
 * (fp32 powf/cosf/sinf, the formula of fused_qkv_rope_cache.cuh:36-38) and
 * uploads it.  Mirrors the engine-owned d_fd_partial/d_fd_lse allocation
 * (qwen_infer.cu:264-266).  Synchronous. */
int qd_ctx_create(const qd_cfg* cfg, qd_ctx** out_ctx);

/* Frees everything qd_ctx_create allocated.  NULL is accepted. */
int qd_ctx_destroy(qd_ctx* ctx);

/* QKV bias + rotate-half RoPE + KV-cache append for one token at `pos`.
 * Replaces add_bias_kernel (bias.cuh:6-11, call qwen_infer.cu:631) followed by
 * fused_qkv_rope_cache_kernel (fused_qkv_rope_cache.cuh:6-55, call
 * qwen_infer.cu:634-642) in one launch, with the same double rounding:
 *   qkv[j] = half(float(qkv[j]) + float(bias[j]))   for all 3*H*128 j
 *   Q part of qkv rotated in place; rotated K and biased V written to cache
 *   row pos of k_layer / v_layer.  The K/V thirds of qkv keep the biased,
 *   unrotated values, exactly as after the reference's two launches.
 * bias == NULL skips the add (the caller already added it).
 * qkv: [3*num_heads*128]; k_layer/v_layer: this layer's cache base.
 * Requires 0 <= pos < max_seqlen, num_heads/head_dim equal to the cfg's. */
int qd_qkv_bias_rope_cache(qd_ctx* ctx, uint16_t* qkv, const uint16_t* bias,
                           uint16_t* k_layer, uint16_t* v_layer, int pos,
                           int max_seqlen, int num_heads, int head_dim,
                           hipStream_t stream);

/* Attention front end of one decode layer in one launch: RMSNorm of x (when
 * norm_w != NULL; rmsnorm.cuh:6-57, call qwen_infer.cu:626) -> QKV GEMV
 * (hgemv_kernel, hgemm_final.cuh:274-295, call :629) -> + qkv_bias (:631) ->
 * rotate-half RoPE and K/V append at pos (:634-642).  Each intermediate is
 * rounded to fp16 where the reference stores one (normalised x, GEMV output,
 * biased QKV).
 *   x:      [H*128] layer input (d_x), 16-byte aligned
 *   norm_w: [H*128] RMSNorm weight (ln_1) or NULL to use x as given
 *   w_qkv:  [3*H*128][H*128] QKV weight in the .bin file's [out][in] layout
 *           (c_attn.weight, convert_weights.py:133-137), 16-byte aligned
 *   qkv:    [3*H*128] out: rotated Q, biased K and V (the reference's d_qkv);
 *           must not overlap x, norm_w, w_qkv or qkv_bias (QD_EINVAL)
 * H*128 must be a multiple of 512, at most 4096.  The GEMV sums each row in a
 * fixed order (per-lane sequential, then a fixed 64-lane tree), so results
 * are deterministic and reproducible on the host. */
int qd_qkv_proj_rope_cache(qd_ctx* ctx, const uint16_t* x, const uint16_t* norm_w, float eps,
                           const uint16_t* w_qkv, const uint16_t* qkv_bias, uint16_t* qkv,
                           uint16_t* k_layer, uint16_t* v_layer, int pos, int max_seqlen,
                           int num_heads, int head_dim, hipStream_t stream);

/* q=1 attention of all heads over cache rows [0, seqlen):
 *   out[h] = half( softmax_j( q[h].K[j,h] / sqrt(128) ) . V[j,h] )
 * in fp32 with fp16 inputs and output.  Picks the single-workgroup-per-head
 * (fused) or the split-KV path and its split count from seqlen.  Replaces
 * the 16-32 per-head launches of qwen_infer.cu:646-678 with one launch
 * (fused) or two (split: stage 1 + merge), covering all heads.
 * Requires 1 <= seqlen <= max_seqlen; q, out, k_layer, v_layer 16-byte
 * aligned; kv strides multiples of 8 elements.  out may be q itself but must
 * not overlap the cache rows read (QD_EINVAL). */
int qd_decode_attention(qd_ctx* ctx, const uint16_t* q, const uint16_t* k_layer,
                        const uint16_t* v_layer, uint16_t* out, int seqlen,
                        int num_heads, int head_dim, hipStream_t stream);

/* Explicit single-workgroup-per-head variant (fd_v5_fused_kernel,
 * flash_decode_q1_opt.cuh:434-537): one workgroup scans all seqlen rows of a
 * head and merges its wavefront partials in LDS.  Any seqlen. */
int qd_decode_attention_fused(qd_ctx* ctx, const uint16_t* q, const uint16_t* k_layer,
                              const uint16_t* v_layer, uint16_t* out, int seqlen,
                              int num_heads, int head_dim, hipStream_t stream);

/* Explicit split-KV variant (fd_v5_split_stage1_kernel + fd_opt_stage2_kernel,
 * flash_decode_q1_opt.cuh:548-724): num_splits workgroups per head write fp32
 * partials (m, l, O[128]); a one-workgroup-per-head merge kernel on the same
 * stream folds them with the log-sum-exp rule.  num_splits <= 0 picks the
 * count; otherwise 1 <= num_splits <= qd_max_splits(). */
int qd_decode_attention_split(qd_ctx* ctx, const uint16_t* q, const uint16_t* k_layer,
                              const uint16_t* v_layer, uint16_t* out, int seqlen,
                              int num_heads, int head_dim, int num_splits,
                              hipStream_t stream);

/* The attention front end and decode attention of one decode layer, the
 * reference's chain rmsnorm (qwen_infer.cu:626) -> QKV hgemv (:629) -> bias
 * (:631) -> RoPE + K/V append at pos (:634-642) -> Flash-Decoding over
 * pos + 1 rows (:646-678): qd_qkv_proj_rope_cache followed by
 * qd_decode_attention(q = qkv, seqlen = pos + 1), with those two calls'
 * outputs (qkv, the cache row at pos, out) bit for bit.  Where the attention
 * plan merges its splits inside the scan kernel with one workgroup per CU
 * (qd_attn_plan.merge_in_kernel; 129 to 3072 rows at 16 heads on MI355X),
 * num_heads is 8 or 16 and out is apart from qkv, it is one launch: each
 * workgroup computes four rotation pairs of the front end, then its split of
 * the attention, which reads its head's rotated Q (and the appended row's K
 * and V) from the producers of the same XCD without waiting for a kernel
 * boundary, its first K/V loads issued behind its front end's weight rows.
 * Elsewhere it makes the two launches.  Arguments as the two calls; out must not
 * overlap x or w_qkv (QD_EINVAL). */
int qd_qkv_proj_rope_cache_attention(qd_ctx* ctx, const uint16_t* x, const uint16_t* norm_w,
                                     float eps, const uint16_t* w_qkv, const uint16_t* qkv_bias,
                                     uint16_t* qkv, uint16_t* k_layer, uint16_t* v_layer,
                                     uint16_t* out, int pos, int max_seqlen, int num_heads,
                                     int head_dim, hipStream_t stream);

/* Allocation-free qd_decode_attention.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc), since
 * qd_ctx_create allocates.  Same outputs, bit for bit, as qd_decode_attention
 * with a default context (QD_MERGE_AUTO) of these strides on the current
 * device: the same plan, with its partials folded by the merge kernel, whose
 * fold is the in-kernel merge's, operation for operation; the KV strides are
 * passed here instead of through a qd_cfg.  The plan depends on the device's
 * workgroup placement over its XCDs, which the first call on a device probes
 * (unless a context was created on it before): one small kernel on the null
 * stream and a synchronous 1 KiB device-to-host copy, so make that first
 * call outside graph capture.
 * The split partials live in a static device array (520 KiB per GPU, held
 * until the process ends) instead of context scratch, so the call makes no
 * hipMalloc/hipFree and no other allocating call.  Limit: the plan's
 * num_heads * splits partial slots must fit its 1024 slots, which every
 * automatic plan does on devices of up to 512 compute units at any head
 * count up to 1024 (QD_EINVAL otherwise).  Every call on one GPU shares that
 * GPU's array: calls that overlap on one GPU (two streams, two threads) race;
 * order them on one stream.  Requirements on the pointers and strides are
 * qd_decode_attention's; seqlen * kv_row_stride * 2 must stay below 4 GiB. */
int qd_decode_attention_noalloc(const uint16_t* q, const uint16_t* k_layer,
                                const uint16_t* v_layer, uint16_t* out, int seqlen,
                                int num_heads, int head_dim, long long kv_row_stride,
                                long long kv_head_stride, hipStream_t stream);

/* Launch plan qd_decode_attention would use for seqlen: *variant is 0 for
 * fused, 1 for split; *num_splits the split count (1 for fused). */
int qd_decode_attention_plan(const qd_ctx* ctx, int seqlen, int* variant, int* num_splits);

/* Complete launch plan of one decode-attention call. */
typedef struct qd_attn_plan {
  int variant;        /* 0: one workgroup per head (fused), 1: split + merge */
  int num_splits;     /* workgroups per head (1 when fused) */
  int rows_per_split; /* KV rows each workgroup scans (seqlen when fused) */
  int rows_per_tile;  /* rows each 16-lane group loads per tile */
  int waves;          /* wavefronts per scan workgroup */
  int merge_in_kernel;/* split plans: 1 if the last split workgroup of each head
                         merges inside the scan kernel (one launch), 0 if a
                         merge kernel follows (two launches); same bits */
  int loads_per_round;/* tiles whose loads a wave issues before consuming them
                         in order (1 or 2; same bits) */
  int block_rows;     /* split plans: 0 if split c scans the contiguous rows
                         [c * rows_per_split, ...); else the rows form blocks
                         of block_rows (waves * 4 * rows_per_tile) dealt to the
                         splits in turn, split c scanning blocks c,
                         c + num_splits, ... (rows_per_split is then split 0's
                         row count, the largest) */
} qd_attn_plan;

/* Plan of the call selected by `entry` (0: qd_decode_attention,
 * 1: qd_decode_attention_fused, 2: qd_decode_attention_split with num_splits)
 * at seqlen.  For a given plan and inputs the outputs are bit-for-bit
 * deterministic; the plan depends on seqlen, num_heads and the device's CU
 * count.  No counterpart in the reference (its launch shape is fixed at the
 * call site, qwen_infer.cu:648-678); it lets a host-side checker restate a
 * call exactly. */
int qd_decode_attention_plan_detail(const qd_ctx* ctx, int seqlen, int entry, int num_splits,
                                    qd_attn_plan* plan);

/* Largest split count a context supports. */
int qd_max_splits(void);

/* Message of the last failing call on this host thread ("" if none). */
const char* qd_last_error(void);

/* Library version, e.g. "0.1.0". */
const char* qd_version(void);

#ifdef __cplusplus
}
#endif
#endif /* QDIY_ATTN_H */
