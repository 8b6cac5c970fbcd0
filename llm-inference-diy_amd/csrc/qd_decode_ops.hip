// Decode-step kernels around attention for gfx950: the fused attention front
// end (RMSNorm -> QKV GEMV -> bias -> RoPE -> KV-cache append).
//
// Replaces, for one decode token of one layer, the reference's
//   rmsnorm_kernel<<<1,512>>>            (kernels/rmsnorm.cuh:6-57, qwen_infer.cu:626)
//   hgemv_kernel<<<24,256>>>             (kernels/hgemm_final.cuh:274-295, :629)
//   add_bias_kernel<<<24,256>>>          (kernels/bias.cuh:6-11, :631)
//   fused_qkv_rope_cache_kernel<<<16,64>>> (kernels/fused_qkv_rope_cache.cuh:6-55, :634-642)
// with one launch.
//
// GEMV mapping: the weight is read in the .bin file's [out][in] layout, one
// wave per output row.  Lane l holds elements k = 512*j + 8*l + e of the
// row (16-byte loads, one 1 KB contiguous segment per wave instruction), sums
// its products sequentially (j outer, e inner) and the 64 lane sums are added
// in the fixed wave64 tree (qd_device.h).  fp16 x fp16 products are exact in
// fp32, so the result depends only on that order, which the CPU oracle
// restates (QD_ORDER_WAVE64) -- outputs are bit-identical to it.
//
// Work split: one workgroup per (head h, rotation pair i < 64): six waves
// compute rows q1 = h*128+i, q2 = q1+64 and the matching K and V rows; one
// thread then adds the bias, rotates and appends, so no value crosses
// workgroups.  The RMSNorm of x (when requested) is recomputed by every wave
// from its own 32 elements and one wave64 reduction.
#include "qd_device.h"
#include "qd_internal.h"

namespace qd {
namespace {

// x (optionally RMS-normalised) for this lane's elements k = 512*j + 8*l + e.
template <int NJ>
__device__ __forceinline__ void load_input(const QkvFrontParams& p, int lane, f16x8 (&xv)[NJ]) {
  const int hidden = NJ * 512;
#pragma unroll
  for (int j = 0; j < NJ; ++j)
    xv[j] = *reinterpret_cast<const f16x8*>(p.x + 512 * j + 8 * lane);
  if (p.norm_w == nullptr) return;
  f16x8 wv[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
    wv[j] = *reinterpret_cast<const f16x8*>(p.norm_w + 512 * j + 8 * lane);
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = (float)xv[j][e];
      acc = __builtin_fmaf(v, v, acc);   // exact square: rounds only the sum
    }
  const float var = wave64_sum(acc) / (float)hidden;
  const float r = __fdiv_rn(1.0f, __fsqrt_rn(var + p.eps));
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
#pragma clang fp contract(off)
      xv[j][e] = (_Float16)(((float)xv[j][e] * r) * (float)wv[j][e]);
    }
}

template <int NJ>
__device__ __forceinline__ float row_dot(const uint16_t* __restrict__ w_row, int lane,
                                         const f16x8 (&xv)[NJ]) {
  f16x8 wv[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
    wv[j] = __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(w_row + 512 * j + 8 * lane));
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e)   // exact product: the fmaf rounds only the sum
      acc = __builtin_fmaf((float)wv[j][e], (float)xv[j][e], acc);
  return wave64_sum(acc);
}

// Bias, rotate-half RoPE and cache append for pair (h, i), evaluated as
// written (each product and sum rounded; no contraction), on the six GEMV
// outputs y = {q1, q2, k1, k2, v1, v2}.
__device__ __forceinline__ void qkv_front_epilogue(const QkvFrontParams& p, int h, int i,
                                                   int hidden, const _Float16* y) {
#pragma clang fp contract(off)
  _Float16 v6[6];
#pragma unroll
  for (int r = 0; r < 6; ++r) {
    const int n = (r >> 1) * hidden + h * 128 + i + (r & 1) * 64;
    v6[r] = p.bias ? (_Float16)((float)y[r] + (float)reinterpret_cast<const _Float16*>(p.bias)[n])
                   : y[r];
  }
  const float2 cs = p.rope_cs[p.pos * 64 + i];
  const float q1 = (float)v6[0], q2 = (float)v6[1], k1 = (float)v6[2], k2 = (float)v6[3];
  const float q1c = q1 * cs.x, q2s = q2 * cs.y, q2c = q2 * cs.x, q1s = q1 * cs.y;
  const float k1c = k1 * cs.x, k2s = k2 * cs.y, k2c = k2 * cs.x, k1s = k1 * cs.y;
  _Float16* qkv = reinterpret_cast<_Float16*>(p.qkv);
  const int idx1 = h * 128 + i;
  qkv[idx1] = (_Float16)(q1c - q2s);
  qkv[idx1 + 64] = (_Float16)(q2c + q1s);
  qkv[hidden + idx1] = v6[2];
  qkv[hidden + idx1 + 64] = v6[3];
  qkv[2 * hidden + idx1] = v6[4];
  qkv[2 * hidden + idx1 + 64] = v6[5];
  const long long base = (long long)p.pos * p.row_stride + (long long)h * p.head_stride;
  _Float16* kc = reinterpret_cast<_Float16*>(p.k_layer) + base;
  _Float16* vc = reinterpret_cast<_Float16*>(p.v_layer) + base;
  kc[i] = (_Float16)(k1c - k2s);
  kc[64 + i] = (_Float16)(k2c + k1s);
  vc[i] = v6[4];
  vc[64 + i] = v6[5];
}

template <int NJ>
__global__ __launch_bounds__(384) void qkv_front_kernel(QkvFrontParams p) {
  __shared__ _Float16 y[6];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;          // 0..5: q1 q2 k1 k2 v1 v2
  const int h = blockIdx.x >> 6;
  const int i = blockIdx.x & 63;
  const int hidden = NJ * 512;
  const int row = (wave >> 1) * hidden + h * 128 + i + (wave & 1) * 64;

  f16x8 xv[NJ];
  load_input<NJ>(p, lane, xv);
  const float acc = row_dot<NJ>(p.w + (long long)row * hidden, lane, xv);
  if (lane == 0) y[wave] = (_Float16)acc;     // hgemv's half output
  __syncthreads();
  if (threadIdx.x == 0) qkv_front_epilogue(p, h, i, hidden, y);
}

}  // namespace

hipError_t launch_qkv_front(const QkvFrontParams& p, hipStream_t stream) {
  const dim3 grid(p.num_heads * 64), block(384);
  switch (p.num_heads * 128 / 512) {
    case 1: hipLaunchKernelGGL(qkv_front_kernel<1>, grid, block, 0, stream, p); break;
    case 2: hipLaunchKernelGGL(qkv_front_kernel<2>, grid, block, 0, stream, p); break;
    case 3: hipLaunchKernelGGL(qkv_front_kernel<3>, grid, block, 0, stream, p); break;
    case 4: hipLaunchKernelGGL(qkv_front_kernel<4>, grid, block, 0, stream, p); break;
    case 5: hipLaunchKernelGGL(qkv_front_kernel<5>, grid, block, 0, stream, p); break;
    case 6: hipLaunchKernelGGL(qkv_front_kernel<6>, grid, block, 0, stream, p); break;
    case 7: hipLaunchKernelGGL(qkv_front_kernel<7>, grid, block, 0, stream, p); break;
    case 8: hipLaunchKernelGGL(qkv_front_kernel<8>, grid, block, 0, stream, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace qd
