// QKV bias + rotate-half RoPE + KV-cache append for one decode token (gfx950).
//
// Replaces add_bias_kernel (kernels/bias.cuh:6-11, engine call
// framework_src/qwen_infer.cu:631) followed by fused_qkv_rope_cache_kernel
// (kernels/fused_qkv_rope_cache.cuh:6-55, call qwen_infer.cu:634-642) with one
// launch.  One thread per (head, i < 64) rotation pair, as in the reference.
//
// Bit-exactness: the bias add is one fp32 add rounded to fp16 (the reference's
// double rounding half(gemv) -> half(+bias) is kept).  cos/sin come from the
// context's [max_seqlen][64] table built on the host with fp32
// powf/cosf/sinf of theta = float(pos) * powf(base, -2i/128), and the rotation
// is evaluated as written -- mul, mul, add/sub, each rounded (FP contraction
// is disabled in this kernel) -- so results equal a host fp32 evaluation of
// the reference formula bit for bit.
#include "qd_device.h"
#include "qd_internal.h"

namespace qd {
namespace {

__global__ __launch_bounds__(256) void qkv_bias_rope_cache_kernel(RopeParams p) {
#pragma clang fp contract(off)
  const int gid = blockIdx.x * 256 + threadIdx.x;
  if (gid >= p.num_heads * 64) return;
  const int h = gid >> 6;
  const int i = gid & 63;
  const int hid = p.num_heads * 128;
  const int idx1 = h * 128 + i;
  const int idx2 = idx1 + 64;

  _Float16* qkv = reinterpret_cast<_Float16*>(p.qkv);
  _Float16 hq1 = qkv[idx1], hq2 = qkv[idx2];
  _Float16 hk1 = qkv[hid + idx1], hk2 = qkv[hid + idx2];
  _Float16 hv1 = qkv[2 * hid + idx1], hv2 = qkv[2 * hid + idx2];
  if (p.bias) {
    const _Float16* b = reinterpret_cast<const _Float16*>(p.bias);
    hq1 = (_Float16)((float)hq1 + (float)b[idx1]);
    hq2 = (_Float16)((float)hq2 + (float)b[idx2]);
    hk1 = (_Float16)((float)hk1 + (float)b[hid + idx1]);
    hk2 = (_Float16)((float)hk2 + (float)b[hid + idx2]);
    hv1 = (_Float16)((float)hv1 + (float)b[2 * hid + idx1]);
    hv2 = (_Float16)((float)hv2 + (float)b[2 * hid + idx2]);
    // the reference's add_bias_kernel leaves the biased K and V in d_qkv
    qkv[hid + idx1] = hk1;
    qkv[hid + idx2] = hk2;
    qkv[2 * hid + idx1] = hv1;
    qkv[2 * hid + idx2] = hv2;
  }
  const float2 cs = p.rope_cs[p.pos * 64 + i];
  const float q1 = (float)hq1, q2 = (float)hq2, k1 = (float)hk1, k2 = (float)hk2;
  const float q1c = q1 * cs.x, q2s = q2 * cs.y, q2c = q2 * cs.x, q1s = q1 * cs.y;
  const float k1c = k1 * cs.x, k2s = k2 * cs.y, k2c = k2 * cs.x, k1s = k1 * cs.y;
  qkv[idx1] = to_f16(q1c - q2s);
  qkv[idx2] = to_f16(q2c + q1s);

  const long long base = (long long)p.pos * p.row_stride + (long long)h * p.head_stride;
  _Float16* kc = reinterpret_cast<_Float16*>(p.k_layer) + base;
  _Float16* vc = reinterpret_cast<_Float16*>(p.v_layer) + base;
  kc[i] = to_f16(k1c - k2s);
  kc[64 + i] = to_f16(k2c + k1s);
  vc[i] = hv1;
  vc[64 + i] = hv2;
}

}  // namespace

hipError_t launch_qkv_bias_rope_cache(const RopeParams& p, hipStream_t stream) {
  const int threads = p.num_heads * 64;
  hipLaunchKernelGGL(qkv_bias_rope_cache_kernel, dim3((threads + 255) / 256), dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace qd
