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

// Launch plan of one decode-attention call.
struct AttnPlan {
  int variant;            // 0 fused, 1 split
  int splits;             // workgroups per head
  int rows_per_split;     // rows each workgroup scans
  int rows_per_tile;      // rows per group per tile (template U)
  int waves;              // waves per split workgroup (4, 8 or 16)
};

hipError_t launch_decode_attention(const AttnParams& p, const AttnPlan& plan, hipStream_t stream);
hipError_t launch_qkv_bias_rope_cache(const RopeParams& p, hipStream_t stream);
hipError_t launch_qkv_front(const QkvFrontParams& p, hipStream_t stream);

}  // namespace qd

struct qd_ctx {
  qd_cfg cfg;
  int device;
  int num_cus;            // compute units of the device (256 on MI355X)
  float2* rope_cs;        // [max_seqlen][64]
  float* part_o;          // [H][kMaxSplits][128]
  float2* part_ml;        // [H][kMaxSplits]
};
