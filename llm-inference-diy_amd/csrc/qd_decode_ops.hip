// Decode-step kernels around attention for gfx950: the fused attention front
// end (RMSNorm -> QKV GEMV -> bias -> RoPE -> KV-cache append), the output
// projections with their residual adds, the SwiGLU FFN input side, and the
// lm_head GEMV with greedy argmax.
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
// Work split: one wave per (head h, rotation pair i < 64), four pairs per
// workgroup.  The wave computes rows q1 = h*128+i, q2 = q1+64 and the matching
// K and V rows, then its lane 0 adds the bias, rotates and appends, so no
// value leaves the wave.  The RMSNorm of x (when requested) is computed once
// per wave from its lanes' elements and one wave64 reduction.  (Six waves per
// pair with an LDS hand-off measured ~1 us slower per launch at hidden 2048:
// the per-wave normalisation and the barrier, not the weight stream.)
#include "qd_device.h"
#include "qd_front_device.h"
#include "qd_internal.h"

namespace qd {
namespace {


// kBiasWords: the bias pointer is 4-byte aligned (checked by the launcher),
// so each bias value is read with a scalar load of its 32-bit word.
template <int NJ, bool kBiasWords>
__global__ __launch_bounds__(kQkvPairsPerBlock * 64) void qkv_front_kernel(QkvFrontParams p) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform
  const int pair = blockIdx.x * kQkvPairsPerBlock + wave;              // grid covers num_heads*64 exactly
  (void)qkv_front_pair<NJ, kBiasWords>(p, pair >> 6, pair & 63, lane);
}

// Output projection + residual add (qwen_infer.cu:701-704 and :718-721:
// hgemv into a half buffer, then add_bias_kernel onto d_x).  One wave per
// output row, four waves per workgroup.  NJ = ceil(k_in / 512) chunks per lane
// are all in flight at once; in the last chunk only lanes with 8*lane <
// k_in - 512*(NJ-1) hold elements (the others skip it, they do not add zeros).
template <int NJ>
__global__ __launch_bounds__(256) void proj_residual_kernel(ProjResidualParams p) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= p.n_out) return;                    // whole wave
  const int K = p.k_in;
  const bool tail = 8 * lane < K - 512 * (NJ - 1);
  const uint16_t* w_row = p.w + (long long)n * K;
  f16x8 xv[NJ], wv[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    if (j < NJ - 1 || tail) {
      xv[j] = *reinterpret_cast<const f16x8*>(p.x + 512 * j + 8 * lane);
      wv[j] = __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(w_row + 512 * j + 8 * lane));
    }
  }
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < NJ; ++j)
    if (j < NJ - 1 || tail)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc = __builtin_fmaf((float)wv[j][e], (float)xv[j][e], acc);
  const float s = wave64_sum(acc);
  if (lane == 0) {
    const _Float16 y = to_f16(s);              // hgemv's half output
    reinterpret_cast<_Float16*>(p.out)[n] =
        (_Float16)((float)reinterpret_cast<const _Float16*>(p.res)[n] + (float)y);
  }
}

// SwiGLU input side (qwen_infer.cu:708-715): RMSNorm(x) with ln_2, the W1
// (gate) and W2 (up) GEMVs, and act = half(g * (u / (1 + exp(-u)))) as in
// swiglu.cuh:6-15, with exp(-u) = exp2_rep(-u * log2(e)).  One wave per
// intermediate index: both rows' loads are issued before either sum.
template <int NJ>
__global__ __launch_bounds__(256) void ffn_up_kernel(FfnUpParams p) {
  const int lane = threadIdx.x & 63;
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= p.inter) return;                    // whole wave
  constexpr int hidden = NJ * 512;
  f16x8 xv[NJ], nv[NJ], a[NJ], b[NJ];
  issue_input<NJ>(p.x, p.norm_w, lane, xv, nv);
  issue_row<NJ>(p.w1 + (long long)i * hidden, lane, a);
  issue_row<NJ>(p.w2 + (long long)i * hidden, lane, b);
  __builtin_amdgcn_sched_barrier(0);
  normalise<NJ>(xv, nv, p.eps);
  float ga = 0.0f, ua = 0.0f;
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      ga = __builtin_fmaf((float)a[j][e], (float)xv[j][e], ga);
      ua = __builtin_fmaf((float)b[j][e], (float)xv[j][e], ua);
    }
  const float g = wave64_sum(ga);
  const float u = wave64_sum(ua);
  if (lane == 0) {
    const float gh = (float)to_f16(g);
    const float uh = (float)to_f16(u);
    const float e = exp2_rep(-uh * kLog2e);
    const float silu = uh / (1.0f + e);
    reinterpret_cast<_Float16*>(p.act)[i] = to_f16(gh * silu);
  }
}

// Packed argmax key of an fp16 logit at index `row`: the upper half orders the
// values (-0 counts as +0, NaN below everything), the lower half is
// 0xFFFFFFFF - row, so the largest key is the largest value at its lowest
// index.
__device__ __forceinline__ unsigned long long argmax_key(_Float16 h, int row) {
  unsigned int b = __builtin_bit_cast(unsigned short, h);
  if (b == 0x8000u) b = 0u;
  unsigned int k;
  if ((b & 0x7FFFu) > 0x7C00u) k = 0u;
  else k = (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
  return ((unsigned long long)k << 32) | (unsigned long long)(0xFFFFFFFFu - (unsigned int)row);
}

// Final RMSNorm with ln_f, lm_head GEMV and the first half of the greedy
// argmax (qwen_infer.cu:725-731).  Each wave normalises x once and takes
// kLmRowsPerWave consecutive rows, two at a time; every logit is written (the
// reference's d_logits) and each workgroup stores its best key.
template <int NJ>
__global__ __launch_bounds__(kLmWaves * 64) void lm_head_kernel(LmHeadParams p) {
  __shared__ unsigned long long best[kLmWaves];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  constexpr int hidden = NJ * 512;
  const int row0 = (blockIdx.x * kLmWaves + wave) * kLmRowsPerWave;
  unsigned long long key = 0ull;
  if (row0 < p.vocab) {
    f16x8 xv[NJ], nv[NJ];
    issue_input<NJ>(p.x, p.norm_w, lane, xv, nv);
#pragma unroll
    for (int r = 0; r < kLmRowsPerWave; r += 2) {
      const int ra = min(row0 + r, p.vocab - 1);
      const int rb = min(row0 + r + 1, p.vocab - 1);
      f16x8 a[NJ], b[NJ];
      issue_row<NJ>(p.w + (long long)ra * hidden, lane, a);
      issue_row<NJ>(p.w + (long long)rb * hidden, lane, b);
      if (r == 0) {
        __builtin_amdgcn_sched_barrier(0);
        normalise<NJ>(xv, nv, p.eps);
      }
      float sa = 0.0f, sb = 0.0f;
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          sa = __builtin_fmaf((float)a[j][e], (float)xv[j][e], sa);
          sb = __builtin_fmaf((float)b[j][e], (float)xv[j][e], sb);
        }
      const _Float16 ha = to_f16(wave64_sum(sa));
      const _Float16 hb = to_f16(wave64_sum(sb));
      if (row0 + r < p.vocab) {
        if (lane == 0) reinterpret_cast<_Float16*>(p.logits)[row0 + r] = ha;
        const unsigned long long k = argmax_key(ha, row0 + r);
        key = k > key ? k : key;
      }
      if (row0 + r + 1 < p.vocab) {
        if (lane == 0) reinterpret_cast<_Float16*>(p.logits)[row0 + r + 1] = hb;
        const unsigned long long k = argmax_key(hb, row0 + r + 1);
        key = k > key ? k : key;
      }
    }
  }
  if (lane == 0) best[wave] = key;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long k = best[0];
#pragma unroll
    for (int w = 1; w < kLmWaves; ++w) k = best[w] > k ? best[w] : k;
    p.part[blockIdx.x] = k;
  }
}

// Second half of the argmax: one workgroup folds the per-workgroup keys and
// writes the winning row as the next token id.
__global__ __launch_bounds__(1024) void argmax_reduce_kernel(const unsigned long long* part,
                                                             int nparts, int* token) {
  __shared__ unsigned long long best[16];
  unsigned long long k = 0ull;
  for (int i = threadIdx.x; i < nparts; i += 1024) k = part[i] > k ? part[i] : k;
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const unsigned long long o = __shfl_xor(k, m);
    k = o > k ? o : k;
  }
  if ((threadIdx.x & 63) == 0) best[threadIdx.x >> 6] = k;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long b = best[0];
#pragma unroll
    for (int w = 1; w < 16; ++w) b = best[w] > b ? best[w] : b;
    *token = (int)(0xFFFFFFFFu - (unsigned int)(b & 0xFFFFFFFFull));
  }
}

}  // namespace

template <bool kBiasWords>
static hipError_t launch_qkv_front_t(const QkvFrontParams& p, hipStream_t stream) {
  const dim3 grid(p.num_heads * 64 / kQkvPairsPerBlock), block(kQkvPairsPerBlock * 64);
  switch (p.num_heads * 128 / 512) {
#define QD_QKV_CASE(n) \
    case n: hipLaunchKernelGGL((qkv_front_kernel<n, kBiasWords>), grid, block, 0, stream, p); break;
    QD_QKV_CASE(1) QD_QKV_CASE(2) QD_QKV_CASE(3) QD_QKV_CASE(4)
    QD_QKV_CASE(5) QD_QKV_CASE(6) QD_QKV_CASE(7) QD_QKV_CASE(8)
#undef QD_QKV_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_qkv_front(const QkvFrontParams& p, hipStream_t stream) {
  const bool words = (reinterpret_cast<uintptr_t>(p.bias) & 3u) == 0;   // also true for no bias
  return words ? launch_qkv_front_t<true>(p, stream) : launch_qkv_front_t<false>(p, stream);
}

}  // namespace qd

namespace qd {

hipError_t launch_proj_residual(const ProjResidualParams& p, hipStream_t stream) {
  const dim3 grid((p.n_out + 3) / 4), block(256);
  switch ((p.k_in + 511) / 512) {
#define QD_PROJ_CASE(n) \
    case n: hipLaunchKernelGGL(proj_residual_kernel<n>, grid, block, 0, stream, p); break;
    QD_PROJ_CASE(1) QD_PROJ_CASE(2) QD_PROJ_CASE(3) QD_PROJ_CASE(4) QD_PROJ_CASE(5) QD_PROJ_CASE(6)
    QD_PROJ_CASE(7) QD_PROJ_CASE(8) QD_PROJ_CASE(9) QD_PROJ_CASE(10) QD_PROJ_CASE(11)
    QD_PROJ_CASE(12) QD_PROJ_CASE(13) QD_PROJ_CASE(14) QD_PROJ_CASE(15) QD_PROJ_CASE(16)
#undef QD_PROJ_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_ffn_up(const FfnUpParams& p, hipStream_t stream) {
  const dim3 grid((p.inter + 3) / 4), block(256);
  switch (p.hidden / 512) {
    case 1: hipLaunchKernelGGL(ffn_up_kernel<1>, grid, block, 0, stream, p); break;
    case 2: hipLaunchKernelGGL(ffn_up_kernel<2>, grid, block, 0, stream, p); break;
    case 3: hipLaunchKernelGGL(ffn_up_kernel<3>, grid, block, 0, stream, p); break;
    case 4: hipLaunchKernelGGL(ffn_up_kernel<4>, grid, block, 0, stream, p); break;
    case 5: hipLaunchKernelGGL(ffn_up_kernel<5>, grid, block, 0, stream, p); break;
    case 6: hipLaunchKernelGGL(ffn_up_kernel<6>, grid, block, 0, stream, p); break;
    case 7: hipLaunchKernelGGL(ffn_up_kernel<7>, grid, block, 0, stream, p); break;
    case 8: hipLaunchKernelGGL(ffn_up_kernel<8>, grid, block, 0, stream, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_lm_head_argmax(const LmHeadParams& p, int* token, hipStream_t stream) {
  const int parts = lm_head_parts(p.vocab);
  const dim3 grid(parts), block(kLmWaves * 64);
  switch (p.hidden / 512) {
    case 1: hipLaunchKernelGGL(lm_head_kernel<1>, grid, block, 0, stream, p); break;
    case 2: hipLaunchKernelGGL(lm_head_kernel<2>, grid, block, 0, stream, p); break;
    case 3: hipLaunchKernelGGL(lm_head_kernel<3>, grid, block, 0, stream, p); break;
    case 4: hipLaunchKernelGGL(lm_head_kernel<4>, grid, block, 0, stream, p); break;
    case 5: hipLaunchKernelGGL(lm_head_kernel<5>, grid, block, 0, stream, p); break;
    case 6: hipLaunchKernelGGL(lm_head_kernel<6>, grid, block, 0, stream, p); break;
    case 7: hipLaunchKernelGGL(lm_head_kernel<7>, grid, block, 0, stream, p); break;
    case 8: hipLaunchKernelGGL(lm_head_kernel<8>, grid, block, 0, stream, p); break;
    default: return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(argmax_reduce_kernel, dim3(1), dim3(1024), 0, stream,
                     (const unsigned long long*)p.part, parts, token);
  return hipGetLastError();
}

}  // namespace qd
