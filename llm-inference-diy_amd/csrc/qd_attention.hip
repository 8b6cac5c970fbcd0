// q=1 decode attention over an fp16 KV cache for gfx950 (MI355X).
//
// Replaces the reference's Flash-Decoding v5 kernels
// (kernels/flash_decode_q1_opt.cuh:434-537 fused, :548-656 split stage 1,
// :666-724 stage 2) and their 16-launches-per-layer dispatch
// (framework_src/qwen_infer.cu:646-678) with ONE launch per layer.
//
// Mapping (wave64):
//   * A 128-dim fp16 row is 256 B = 16 lanes x 16 B, so a wavefront holds four
//     16-lane "groups", each owning one KV row per load instruction.  A group's
//     row-dot is 4 v_dot2 (fp16 x fp16 -> fp32) per lane plus a 4-step DPP
//     butterfly inside the 16-lane DPP row; every lane of the group ends with
//     the same score.
//   * Each group keeps its own online-softmax state (m, l, 8 dims of O) in
//     fp32.  It consumes rows in tiles of U: all 2U 16-byte loads of a tile are
//     issued first, then one max/rescale per tile, then U exp2 + 8U fp16*fp32
//     FMAs (v_fma_mix_f32, no conversions).
//   * Scores live in log2 units (scale_log2 = log2(e)/sqrt(128)) so the
//     exponentials are single v_exp_f32 instructions.
//   * Groups of a workgroup are merged in LDS.  The split kernel writes each
//     workgroup's unnormalised (m, l, O[128]) partial in fp32 (the reference
//     keeps fp16 partials); the last workgroup of a head to finish -- found with
//     an agent-scope counter -- merges that head's partials with the
//     log-sum-exp rule and writes the fp16 output.  No second launch.
//   * No MFMA: at q=1 the work is a bandwidth-bound GEMV-like reduction.
#include "qd_internal.h"

namespace qd {
namespace {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kD = 128;

// DPP row-local permutations (gfx9 encodings).
constexpr int kDppQuadSwap1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kDppQuadSwap2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // row_half_mirror: lane i <-> 7-i within 8
constexpr int kDppMirror = 0x140;     // row_mirror: lane i <-> 15-i within 16

template <int Ctrl>
__device__ __forceinline__ float dpp_mov(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), Ctrl, 0xF, 0xF, true));
}

// Sum over the 16 lanes of a DPP row; all 16 lanes receive the same value
// (each step adds a partner whose value is the mirror image of its own).
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_mov<kDppQuadSwap1>(x);
  x += dpp_mov<kDppQuadSwap2>(x);
  x += dpp_mov<kDppHalfMirror>(x);
  x += dpp_mov<kDppMirror>(x);
  return x;
}

__device__ __forceinline__ float dot8(const f16x8 k, const f16x8 q) {
  float d = __builtin_amdgcn_fdot2(f16x2{k[0], k[1]}, f16x2{q[0], q[1]}, 0.0f, false);
  d = __builtin_amdgcn_fdot2(f16x2{k[2], k[3]}, f16x2{q[2], q[3]}, d, false);
  d = __builtin_amdgcn_fdot2(f16x2{k[4], k[5]}, f16x2{q[4], q[5]}, d, false);
  d = __builtin_amdgcn_fdot2(f16x2{k[6], k[7]}, f16x2{q[6], q[7]}, d, false);
  return d;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Base of a running max that may still be -inf (no rows seen): exp2(x - base)
// then maps -inf inputs to 0 without producing NaN.
__device__ __forceinline__ float safe_base(float m) { return m == -__builtin_inff() ? 0.0f : m; }

// Online-softmax state of one 16-lane group: each lane owns dims [8t, 8t+8).
struct GroupState {
  float m;
  float l;
  float o[8];
};

// Scan rows [0, nrows) of one head starting at kbase/vbase (already offset to
// the workgroup's first row and to this lane's 8 dims).  Wave `wave` of NW
// takes blocks of 4U consecutive rows round-robin; row blk + 4u + g goes to
// group g.
template <int NW, int U>
__device__ __forceinline__ void scan_rows(GroupState& st, const _Float16* __restrict__ kbase,
                                          const _Float16* __restrict__ vbase, long long row_stride,
                                          int nrows, int wave, int g, const f16x8 qv,
                                          float scale_log2) {
  for (int blk = wave * 4 * U; blk < nrows; blk += NW * 4 * U) {
    f16x8 kt[U], vt[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int r = min(blk + 4 * u + g, nrows - 1);
      kt[u] = *reinterpret_cast<const f16x8*>(kbase + r * row_stride);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int r = min(blk + 4 * u + g, nrows - 1);
      vt[u] = *reinterpret_cast<const f16x8*>(vbase + r * row_stride);
    }
    float s[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float d = row16_sum(dot8(kt[u], qv));
      s[u] = (blk + 4 * u + g < nrows) ? d * scale_log2 : -__builtin_inff();
    }
    float mt = s[0];
#pragma unroll
    for (int u = 1; u < U; ++u) mt = fmaxf(mt, s[u]);
    const float mn = fmaxf(st.m, mt);
    const float base = safe_base(mn);
    const float alpha = fast_exp2(st.m - base);
    st.l *= alpha;
#pragma unroll
    for (int j = 0; j < 8; ++j) st.o[j] *= alpha;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float p = fast_exp2(s[u] - base);
      st.l += p;
#pragma unroll
      for (int j = 0; j < 8; ++j) st.o[j] = __builtin_fmaf((float)vt[u][j], p, st.o[j]);
    }
    st.m = mn;
  }
}

// Merge the 4*NW group states of a workgroup in LDS.  Two levels: thread
// (d = tid % 128, slice = tid / 128) folds 8 groups, then threads < 128 fold
// the NW/2 slices.  Returns (for tid < 128) the merged m, l and O[d].
template <int NW>
struct WgMergeSmem {
  static constexpr int kGroups = NW * 4;
  static constexpr int kSlices = NW / 2;
  float o[kGroups][kD];
  float m[kGroups];
  float l[kGroups];
  float so[kSlices][kD];
  float sm[kSlices];
  float sl[kSlices];
};

template <int NW>
__device__ __forceinline__ void wg_merge(WgMergeSmem<NW>& sh, const GroupState& st, int tid,
                                         float& m_out, float& l_out, float& o_out) {
  static_assert(NW % 2 == 0, "need an even number of waves");
  constexpr int kGroups = WgMergeSmem<NW>::kGroups;
  constexpr int kSlices = WgMergeSmem<NW>::kSlices;
  const int lane = tid & 63;
  const int gid = (tid >> 6) * 4 + (lane >> 4);
  const int t = lane & 15;
  *reinterpret_cast<f32x4*>(&sh.o[gid][t * 8]) = f32x4{st.o[0], st.o[1], st.o[2], st.o[3]};
  *reinterpret_cast<f32x4*>(&sh.o[gid][t * 8 + 4]) = f32x4{st.o[4], st.o[5], st.o[6], st.o[7]};
  if (t == 0) {
    sh.m[gid] = st.m;
    sh.l[gid] = st.l;
  }
  __syncthreads();
  {
    const int d = tid & (kD - 1);
    const int slice = tid >> 7;
    float mm = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < kGroups / kSlices; ++j) mm = fmaxf(mm, sh.m[slice + j * kSlices]);
    const float base = safe_base(mm);
    float ll = 0.0f, oo = 0.0f;
#pragma unroll
    for (int j = 0; j < kGroups / kSlices; ++j) {
      const int gg = slice + j * kSlices;
      const float w = fast_exp2(sh.m[gg] - base);
      ll = __builtin_fmaf(w, sh.l[gg], ll);
      oo = __builtin_fmaf(w, sh.o[gg][d], oo);
    }
    sh.so[slice][d] = oo;
    if (d == 0) {
      sh.sm[slice] = mm;
      sh.sl[slice] = ll;
    }
  }
  __syncthreads();
  if (tid < kD) {
    float mm = -__builtin_inff();
#pragma unroll
    for (int s = 0; s < kSlices; ++s) mm = fmaxf(mm, sh.sm[s]);
    const float base = safe_base(mm);
    float ll = 0.0f, oo = 0.0f;
#pragma unroll
    for (int s = 0; s < kSlices; ++s) {
      const float w = fast_exp2(sh.sm[s] - base);
      ll = __builtin_fmaf(w, sh.sl[s], ll);
      oo = __builtin_fmaf(w, sh.so[s][tid], oo);
    }
    m_out = mm;
    l_out = ll;
    o_out = oo;
  }
}

// One workgroup per head scans every row (fd_v5_fused_kernel's role).
template <int NW, int U>
__global__ __launch_bounds__(NW * 64) void decode_attention_fused_kernel(AttnParams p) {
  __shared__ WgMergeSmem<NW> sh;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 4;
  const int t = lane & 15;
  const int h = blockIdx.x;

  const f16x8 qv = *reinterpret_cast<const f16x8*>(p.q + h * kD + t * 8);
  const _Float16* kb = reinterpret_cast<const _Float16*>(p.k) + h * p.head_stride + t * 8;
  const _Float16* vb = reinterpret_cast<const _Float16*>(p.v) + h * p.head_stride + t * 8;

  GroupState st;
  st.m = -__builtin_inff();
  st.l = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) st.o[j] = 0.0f;
  scan_rows<NW, U>(st, kb, vb, p.row_stride, p.seqlen, wave, g, qv, p.scale_log2);

  float m, l, o;
  wg_merge<NW>(sh, st, tid, m, l, o);
  if (tid < kD) {
    reinterpret_cast<_Float16*>(p.out)[h * kD + tid] = (_Float16)(o / l);
  }
}

// splits workgroups per head; blockIdx.x = split * num_heads + head, so the
// workgroups resident together cover all heads of neighbouring positions.
template <int NW, int U>
__global__ __launch_bounds__(NW * 64) void decode_attention_split_kernel(AttnParams p) {
  __shared__ WgMergeSmem<NW> sh;
  __shared__ float fo[NW * 2][kD];
  __shared__ float fm[NW * 2];
  __shared__ float fl[NW * 2];
  __shared__ unsigned is_last;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 4;
  const int t = lane & 15;
  const int h = blockIdx.x % p.num_heads;
  const int c = blockIdx.x / p.num_heads;
  const int r0 = c * p.rows_per_split;
  const int nrows = min(p.seqlen - r0, p.rows_per_split);

  const f16x8 qv = *reinterpret_cast<const f16x8*>(p.q + h * kD + t * 8);
  const long long off = h * p.head_stride + (long long)r0 * p.row_stride + t * 8;
  const _Float16* kb = reinterpret_cast<const _Float16*>(p.k) + off;
  const _Float16* vb = reinterpret_cast<const _Float16*>(p.v) + off;

  GroupState st;
  st.m = -__builtin_inff();
  st.l = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) st.o[j] = 0.0f;
  scan_rows<NW, U>(st, kb, vb, p.row_stride, nrows, wave, g, qv, p.scale_log2);

  float m, l, o;
  wg_merge<NW>(sh, st, tid, m, l, o);
  const long long pidx = (long long)h * p.splits + c;
  if (tid < kD) {
    p.part_o[pidx * kD + tid] = o;
    if (tid == 0) p.part_ml[pidx] = float2{m, l};
  }

  // Publish the partial, count it, and let the head's last workgroup merge.
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = atomicAdd(&p.counters[h], 1u);
    is_last = (prev == (unsigned)(p.splits - 1)) ? 1u : 0u;
  }
  __syncthreads();
  if (!is_last) return;
  __threadfence();

  // Thread (dq = tid % 32 -> dims 4dq..4dq+3, slice = tid / 32) folds splits
  // slice, slice + P, ... with its own running max; slices are folded in LDS.
  constexpr int P = NW * 2;
  const int dq = tid & 31;
  const int slice = tid >> 5;
  const float* po = p.part_o + (long long)h * p.splits * kD + dq * 4;
  const float2* pml = p.part_ml + (long long)h * p.splits;
  float mm = -__builtin_inff(), ll = 0.0f;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int c0 = slice; c0 < p.splits; c0 += 4 * P) {
    float2 ml[4];
    f32x4 ov[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int cc = c0 + j * P;
      if (cc < p.splits) {
        ml[j] = pml[cc];
        ov[j] = *reinterpret_cast<const f32x4*>(po + (long long)cc * kD);
      } else {
        ml[j] = float2{-__builtin_inff(), 0.0f};
        ov[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float mn = fmaxf(mm, ml[j].x);
      const float base = safe_base(mn);
      const float a = fast_exp2(mm - base);
      const float b = fast_exp2(ml[j].x - base);
      ll = ll * a + ml[j].y * b;
      acc = acc * a + ov[j] * b;
      mm = mn;
    }
  }
  *reinterpret_cast<f32x4*>(&fo[slice][dq * 4]) = acc;
  if (dq == 0) {
    fm[slice] = mm;
    fl[slice] = ll;
  }
  __syncthreads();
  if (tid < kD) {
    float M = -__builtin_inff();
#pragma unroll
    for (int s = 0; s < P; ++s) M = fmaxf(M, fm[s]);
    const float base = safe_base(M);
    float L = 0.0f, O = 0.0f;
#pragma unroll
    for (int s = 0; s < P; ++s) {
      const float w = fast_exp2(fm[s] - base);
      L = __builtin_fmaf(w, fl[s], L);
      O = __builtin_fmaf(w, fo[s][tid], O);
    }
    reinterpret_cast<_Float16*>(p.out)[h * kD + tid] = (_Float16)(O / L);
    if (tid == 0) p.counters[h] = 0u;   // every other split of this head has counted
  }
}

}  // namespace

hipError_t launch_decode_attention(const AttnParams& p, const AttnPlan& plan, hipStream_t stream) {
  if (plan.variant == 0) {
    constexpr int NW = 16;
    hipLaunchKernelGGL((decode_attention_fused_kernel<NW, 4>), dim3(p.num_heads), dim3(NW * 64), 0,
                       stream, p);
  } else {
    constexpr int NW = 4;
    const dim3 grid(p.num_heads * plan.splits);
    switch (plan.rows_per_tile) {
      case 8:
        hipLaunchKernelGGL((decode_attention_split_kernel<NW, 8>), grid, dim3(NW * 64), 0, stream, p);
        break;
      case 4:
        hipLaunchKernelGGL((decode_attention_split_kernel<NW, 4>), grid, dim3(NW * 64), 0, stream, p);
        break;
      default:
        hipLaunchKernelGGL((decode_attention_split_kernel<NW, 2>), grid, dim3(NW * 64), 0, stream, p);
        break;
    }
  }
  return hipGetLastError();
}

}  // namespace qd
