// Benchmark driver for the decode-attention entry points (libqdiy_bench.so).
//
// Issues `iters` calls of the public C ABI back to back on one stream, cycling
// over `n_layers` layers of a multi-layer KV cache, the way the engine's
// per-token loop visits layers (framework_src/qwen_infer.cu:623-678).  Cycling
// over layers whose total size exceeds the 256 MB Infinity Cache makes every
// call stream its KV rows from HBM.  The caller brackets the loop with events
// on the same stream; this function never synchronises.
#include <cstdint>

#include "qdiy/bench.h"

extern "C" {

// variant: 0 auto (qd_decode_attention), 1 fused, 2 split with num_splits,
// 3 the scan kernel of qd_decode_attention only, 4 its merge kernel only
// (qd_decode_attention_stage).
int qd_bench_decode_attention(qd_ctx* ctx, const uint16_t* q, const uint16_t* k,
                              const uint16_t* v, uint16_t* out, long long q_layer_stride,
                              long long kv_layer_stride, int n_layers, int seqlen, int num_heads,
                              int iters, int variant, int num_splits, hipStream_t stream) {
  if (n_layers < 1 || iters < 0) return QD_EINVAL;
  for (int it = 0; it < iters; ++it) {
    const int layer = it % n_layers;
    const uint16_t* ql = q + layer * q_layer_stride;
    uint16_t* ol = out + layer * q_layer_stride;
    const uint16_t* kl = k + layer * kv_layer_stride;
    const uint16_t* vl = v + layer * kv_layer_stride;
    int rc;
    if (variant == 1)
      rc = qd_decode_attention_fused(ctx, ql, kl, vl, ol, seqlen, num_heads, QD_HEAD_DIM, stream);
    else if (variant == 2)
      rc = qd_decode_attention_split(ctx, ql, kl, vl, ol, seqlen, num_heads, QD_HEAD_DIM,
                                     num_splits, stream);
    else if (variant == 3 || variant == 4)
      rc = qd_decode_attention_stage(ctx, ql, kl, vl, ol, seqlen, num_heads, QD_HEAD_DIM,
                                     variant == 3 ? QD_STAGE_SCAN : QD_STAGE_MERGE, stream);
    else
      rc = qd_decode_attention(ctx, ql, kl, vl, ol, seqlen, num_heads, QD_HEAD_DIM, stream);
    if (rc != QD_OK) return rc;
  }
  return QD_OK;
}

// One decode step's attention section for `n_layers` layers: feeder at `pos`
// then attention over pos + 1 rows, per layer (qwen_infer.cu:631-678).
int qd_bench_decode_step(qd_ctx* ctx, uint16_t* qkv, const uint16_t* bias, uint16_t* k,
                         uint16_t* v, uint16_t* out, long long qkv_layer_stride,
                         long long bias_layer_stride, long long kv_layer_stride, int n_layers,
                         int pos, int max_seqlen, int num_heads, int iters, hipStream_t stream) {
  if (n_layers < 1 || iters < 0) return QD_EINVAL;
  for (int it = 0; it < iters; ++it) {
    const int layer = it % n_layers;
    uint16_t* ql = qkv + layer * qkv_layer_stride;
    uint16_t* kl = k + layer * kv_layer_stride;
    uint16_t* vl = v + layer * kv_layer_stride;
    int rc = qd_qkv_bias_rope_cache(ctx, ql, bias ? bias + layer * bias_layer_stride : nullptr, kl,
                                    vl, pos, max_seqlen, num_heads, QD_HEAD_DIM, stream);
    if (rc != QD_OK) return rc;
    rc = qd_decode_attention(ctx, ql, kl, vl, out + layer * (long long)num_heads * QD_HEAD_DIM,
                             pos + 1, num_heads, QD_HEAD_DIM, stream);
    if (rc != QD_OK) return rc;
  }
  return QD_OK;
}

// Config-4 loop: per layer, qd_qkv_proj_rope_cache (GEMV [3*hid][hid] + bias +
// RoPE + append at pos) and, with with_attention 1, qd_decode_attention over
// pos + 1 rows; with with_attention 2, both in qd_qkv_proj_rope_cache_attention.
// Layer l's buffers sit at the given strides from the bases.
int qd_bench_attn_front(qd_ctx* ctx, const uint16_t* x, const uint16_t* w_qkv, const uint16_t* bias,
                        uint16_t* qkv, uint16_t* k, uint16_t* v, uint16_t* out,
                        long long w_layer_stride, long long kv_layer_stride, int n_layers, int pos,
                        int max_seqlen, int num_heads, int iters, int with_attention,
                        hipStream_t stream) {
  if (n_layers < 1 || iters < 0) return QD_EINVAL;
  const long long hid = (long long)num_heads * QD_HEAD_DIM;
  for (int it = 0; it < iters; ++it) {
    const int layer = it % n_layers;
    uint16_t* ql = qkv + layer * 3 * hid;
    uint16_t* kl = k + layer * kv_layer_stride;
    uint16_t* vl = v + layer * kv_layer_stride;
    int rc;
    if (with_attention == 2) {
      rc = qd_qkv_proj_rope_cache_attention(ctx, x + layer * hid, nullptr, 1e-6f,
                                            w_qkv + layer * w_layer_stride, bias + layer * 3 * hid, ql,
                                            kl, vl, out + layer * hid, pos, max_seqlen, num_heads,
                                            QD_HEAD_DIM, stream);
      if (rc != QD_OK) return rc;
      continue;
    }
    rc = qd_qkv_proj_rope_cache(ctx, x + layer * hid, nullptr, 1e-6f, w_qkv + layer * w_layer_stride,
                                bias + layer * 3 * hid, ql, kl, vl, pos, max_seqlen, num_heads,
                                QD_HEAD_DIM, stream);
    if (rc != QD_OK) return rc;
    if (with_attention) {
      rc = qd_decode_attention(ctx, ql, kl, vl, out + layer * hid, pos + 1, num_heads, QD_HEAD_DIM,
                               stream);
      if (rc != QD_OK) return rc;
    }
  }
  return QD_OK;
}

}  // extern "C"
