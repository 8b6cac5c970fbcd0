// Internal declarations shared by the C-ABI layer and the HIP kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "qdiy/attn.h"

namespace qd {

// Largest split count (workgroups per head).  Scratch per context:
// num_heads * kMaxSplits * (128 + 2) floats (2.1 MB at 16 heads).
constexpr int kMaxSplits = 256;

// Per-launch arguments of the decode-attention kernels.  Offsets are in fp16
// elements.
struct AttnParams {
  const uint16_t* q;      // [H][128]
  const uint16_t* k;      // layer base; (pos, h, d) at pos*row_stride + h*head_stride + d
  const uint16_t* v;
  uint16_t* out;          // [H][128]
  float* part_o;          // [H][splits][128] unnormalised fp32 partial outputs
  float2* part_ml;        // [H][splits] (running max in log2 units, running sum)
  long long row_stride;
  long long head_stride;
  int seqlen;
  int num_heads;
  int splits;             // workgroups per head
  int rows_per_split;
  float scale_log2;       // log2(e) / sqrt(128)
};

struct RopeParams {
  uint16_t* qkv;          // [3][H][128]
  const uint16_t* bias;   // [3][H][128] or null
  uint16_t* k_layer;
  uint16_t* v_layer;
  const float2* rope_cs;  // [max_seqlen][64] (cos, sin)
  long long row_stride;
  long long head_stride;
  int pos;
  int num_heads;
};

// Attention front end of one decode layer: [RMSNorm] -> QKV GEMV -> bias ->
// RoPE -> KV append.  hidden = num_heads * 128, a multiple of 512 up to 4096.
struct QkvFrontParams {
  const uint16_t* x;      // [hidden] layer input
  const uint16_t* norm_w; // [hidden] RMSNorm weight, or null for no norm
  float eps;
  const uint16_t* w;      // [3*hidden][hidden] QKV weight, [out][in]
  const uint16_t* bias;   // [3*hidden] or null
  uint16_t* qkv;          // [3*hidden] out: rotated Q, biased K and V
  uint16_t* k_layer;
  uint16_t* v_layer;
  const float2* rope_cs;  // [max_seqlen][64] (cos, sin)
  long long row_stride;
  long long head_stride;
  int pos;
  int num_heads;
};

// out[n] = half(res[n] + half(W[n] . x)) for n < n_out; W is [n_out][k_in]
// ([out][in]), k_in a multiple of 8.  res and out may alias.
struct ProjResidualParams {
  const uint16_t* x;
  const uint16_t* w;
  const uint16_t* res;
  uint16_t* out;
  int n_out;
  int k_in;
};

// act[i] = half(g * (u / (1 + exp(-u)))) with g = half(W1[i] . xn),
// u = half(W2[i] . xn), xn = RMSNorm(x) * norm_w; W1/W2 are [inter][hidden].
struct FfnUpParams {
  const uint16_t* x;
  const uint16_t* norm_w;
  float eps;
  const uint16_t* w1;
  const uint16_t* w2;
  uint16_t* act;
  int hidden;
  int inter;
};

// logits[v] = half(W[v] . xn) for v < vocab, xn = RMSNorm(x) * norm_w; each
// workgroup also writes its best (logit, lowest index) as a packed key.
struct LmHeadParams {
  const uint16_t* x;
  const uint16_t* norm_w;
  float eps;
  const uint16_t* w;
  uint16_t* logits;
  unsigned long long* part;
  int vocab;
  int hidden;
};

// Rows per wave and waves per workgroup of the lm_head kernel; the number of
// per-workgroup keys for a vocabulary follows from them.
constexpr int kLmRowsPerWave = 8;
constexpr int kLmWaves = 4;
inline int lm_head_parts(int vocab) {
  const int rows = kLmRowsPerWave * kLmWaves;
  return (vocab + rows - 1) / rows;
}

// Launch plan of one decode-attention call.
struct AttnPlan {
  int variant;            // 0 fused, 1 split
  int splits;             // workgroups per head
  int rows_per_split;     // rows each workgroup scans
  int rows_per_tile;      // rows per group per tile (template U)
  int waves;              // waves per split workgroup (4, 8 or 16)
};

// Error reporting of the C ABI: records a printf-style message for
// qd_last_error() on this host thread and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_fail(hipError_t e, const char* what);
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

hipError_t launch_decode_attention(const AttnParams& p, const AttnPlan& plan, hipStream_t stream);
hipError_t launch_qkv_bias_rope_cache(const RopeParams& p, hipStream_t stream);
hipError_t launch_qkv_front(const QkvFrontParams& p, hipStream_t stream);
hipError_t launch_proj_residual(const ProjResidualParams& p, hipStream_t stream);
hipError_t launch_ffn_up(const FfnUpParams& p, hipStream_t stream);
// lm_head kernel, then the one-workgroup reduction of its keys into *token.
hipError_t launch_lm_head_argmax(const LmHeadParams& p, int* token, hipStream_t stream);

}  // namespace qd

struct qd_ctx {
  qd_cfg cfg;
  int device;
  int num_cus;            // compute units of the device (256 on MI355X)
  float2* rope_cs;        // [max_seqlen][64]
  float* part_o;          // [H][kMaxSplits][128]
  float2* part_ml;        // [H][kMaxSplits]
};
