// q=1 decode attention over an fp16 KV cache for gfx950 (MI355X).
//
// Replaces the reference's Flash-Decoding v5 kernels
// (kernels/flash_decode_q1_opt.cuh:434-537 fused, :548-656 split stage 1,
// :666-724 stage 2) and their 16-32 launches per layer
// (framework_src/qwen_infer.cu:646-678) with one or two launches covering all
// heads.
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
//   * The four groups of a wave are merged with lane shuffles, the waves of a
//     workgroup in LDS.  A split workgroup writes one fp32 partial
//     (m, l, O[128]); the reference keeps fp16 partials.
//   * Partials are folded with the log-sum-exp rule by a second,
//     one-workgroup-per-head kernel.  Cross-workgroup hand-off goes through the
//     kernel boundary: an agent-scope release inside the kernel lowers to a
//     whole-L2 writeback per workgroup on gfx950 (buffer_wbl2 sc1, measured
//     ~1 us each and serialised per XCD), far more than a second launch.
//   * No MFMA: at q=1 the work is a bandwidth-bound GEMV-like reduction.
#include "qd_device.h"
#include "qd_internal.h"

namespace qd {
namespace {

constexpr int kD = 128;

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

__device__ __forceinline__ void init_state(GroupState& st) {
  st.m = -__builtin_inff();
  st.l = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) st.o[j] = 0.0f;
}

// Scan rows [0, nrows) of one head.  kbase/vbase are workgroup-uniform (the
// head's first row of this workgroup); lane t of group g reads the 16 bytes at
// byte offset row*row_bytes + 16t, a 32-bit offset added to a scalar base
// (global_load ... saddr form).  Wave `wave` of NW takes blocks of 4U
// consecutive rows round-robin; row blk + 4u + g goes to group g.  All 2U
// loads of a block are issued before any of them is consumed.  KV rows are
// read once, so the loads carry the non-temporal hint: streamed lines do not
// displace L2 contents (measured ~15% faster per call at L=32768).
template <int NW, int U>
__device__ __forceinline__ void scan_rows(GroupState& st, const char* __restrict__ kbase,
                                          const char* __restrict__ vbase, unsigned row_bytes,
                                          int nrows, int wave, int g, int t, const f16x8 qv,
                                          float scale_log2) {
  for (int blk = wave * 4 * U; blk < nrows; blk += NW * 4 * U) {
    f16x8 kt[U], vt[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const unsigned r = (unsigned)min(blk + 4 * u + g, nrows - 1);
      kt[u] = __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(kbase + (r * row_bytes + t * 16u)));
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const unsigned r = (unsigned)min(blk + 4 * u + g, nrows - 1);
      vt[u] = __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(vbase + (r * row_bytes + t * 16u)));
    }
    // keep the scheduler from sinking loads next to their uses
    __builtin_amdgcn_sched_barrier(0);
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

// Fold the four groups of a wave (lanes t, t+16, t+32, t+48 hold the same
// dims) with a two-step xor butterfly over lane ^ 16 and lane ^ 32.  Afterwards
// lanes 0..15 hold the wave's merged state.
__device__ __forceinline__ void wave_merge(GroupState& st) {
#pragma unroll
  for (int mask = 16; mask <= 32; mask <<= 1) {
    const float om = __shfl_xor(st.m, mask);
    const float ol = __shfl_xor(st.l, mask);
    float oo[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) oo[j] = __shfl_xor(st.o[j], mask);
    const float mn = fmaxf(st.m, om);
    const float base = safe_base(mn);
    const float a = fast_exp2(st.m - base);
    const float b = fast_exp2(om - base);
    st.l = st.l * a + ol * b;
#pragma unroll
    for (int j = 0; j < 8; ++j) st.o[j] = st.o[j] * a + oo[j] * b;
    st.m = mn;
  }
}

// Scan kernel.  Workgroup (split c, head h) with blockIdx.x = c * num_heads + h
// (so the workgroups resident together cover all heads of neighbouring
// positions) scans rows [c * rows_per_split, ...) of head h with NW waves.
// Each wave folds its four groups with lane shuffles; the NW wave states are
// folded in LDS by threads 0..127, one dim each.  kSplit = false is the
// single-workgroup-per-head path (fd_v5_fused_kernel's role): it writes the
// normalised fp16 output.  kSplit = true writes the workgroup's unnormalised
// fp32 partial (m, l, O[128]) to slot h * splits + c.
template <int NW, int U, bool kSplit>
__global__ __launch_bounds__(NW * 64) void decode_attention_scan_kernel(AttnParams p) {
  __shared__ float so[NW][kD];
  __shared__ float sm[NW];
  __shared__ float sl[NW];
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
  const long long off = h * p.head_stride + (long long)r0 * p.row_stride;
  GroupState st;
  init_state(st);
  scan_rows<NW, U>(st, reinterpret_cast<const char*>(p.k + off),
                   reinterpret_cast<const char*>(p.v + off), (unsigned)(p.row_stride * 2), nrows,
                   wave, g, t, qv, p.scale_log2);
  wave_merge(st);
  if (lane < 16) {
    *reinterpret_cast<f32x4*>(&so[wave][t * 8]) = f32x4{st.o[0], st.o[1], st.o[2], st.o[3]};
    *reinterpret_cast<f32x4*>(&so[wave][t * 8 + 4]) = f32x4{st.o[4], st.o[5], st.o[6], st.o[7]};
    if (t == 0) {
      sm[wave] = st.m;
      sl[wave] = st.l;
    }
  }
  __syncthreads();
  if (tid < kD) {
    float M = -__builtin_inff();
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, sm[w]);
    const float base = safe_base(M);
    float L = 0.0f, O = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float wt = fast_exp2(sm[w] - base);
      L = __builtin_fmaf(wt, sl[w], L);
      O = __builtin_fmaf(wt, so[w][tid], O);
    }
    if constexpr (kSplit) {
      const long long slot = (long long)h * p.splits + c;
      p.part_o[slot * kD + tid] = O;
      if (tid == 0) p.part_ml[slot] = float2{M, L};
    } else {
      reinterpret_cast<_Float16*>(p.out)[h * kD + tid] = (_Float16)(O / L);
    }
  }
}

// Stage 2: one workgroup per head folds the head's p.splits partials with the
// log-sum-exp rule (fd_opt_stage2_kernel's role) and writes the fp16 output.
// Thread (dq = tid % 32 -> dims 4dq..4dq+3, slice = tid / 32) folds splits
// slice, slice + P, ... with its own running max, issuing eight splits' loads
// at a time; the P slices are then folded in LDS.  The kernel boundary after
// stage 1 makes every partial visible on every XCD.
template <int NT>
__global__ __launch_bounds__(NT) void decode_attention_merge_kernel(AttnParams p) {
  constexpr int P = NT / 32;
  constexpr int B = 8;
  __shared__ float so[P][kD];
  __shared__ float sm[P];
  __shared__ float sl[P];
  const int tid = threadIdx.x;
  const int h = blockIdx.x;
  const int dq = tid & 31;
  const int slice = tid >> 5;
  const float* po = p.part_o + (long long)h * p.splits * kD + dq * 4;
  const float2* pml = p.part_ml + (long long)h * p.splits;
  float mm = -__builtin_inff(), ll = 0.0f;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int c0 = slice; c0 < p.splits; c0 += B * P) {
    float2 ml[B];
    f32x4 ov[B];
#pragma unroll
    for (int j = 0; j < B; ++j) {
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
    for (int j = 0; j < B; ++j) {
      const float mn = fmaxf(mm, ml[j].x);
      const float base = safe_base(mn);
      const float a = fast_exp2(mm - base);
      const float b = fast_exp2(ml[j].x - base);
      ll = ll * a + ml[j].y * b;
      acc = acc * a + ov[j] * b;
      mm = mn;
    }
  }
  *reinterpret_cast<f32x4*>(&so[slice][dq * 4]) = acc;
  if (dq == 0) {
    sm[slice] = mm;
    sl[slice] = ll;
  }
  __syncthreads();
  if (tid < kD) {
    float M = -__builtin_inff();
#pragma unroll
    for (int s = 0; s < P; ++s) M = fmaxf(M, sm[s]);
    const float base = safe_base(M);
    float L = 0.0f, O = 0.0f;
#pragma unroll
    for (int s = 0; s < P; ++s) {
      const float w = fast_exp2(sm[s] - base);
      L = __builtin_fmaf(w, sl[s], L);
      O = __builtin_fmaf(w, so[s][tid], O);
    }
    reinterpret_cast<_Float16*>(p.out)[h * kD + tid] = (_Float16)(O / L);
  }
}

}  // namespace

template <int NW, bool kSplit>
static void launch_scan(const AttnParams& p, int rows_per_tile, dim3 grid, hipStream_t stream) {
  switch (rows_per_tile) {
    case 8:
      hipLaunchKernelGGL((decode_attention_scan_kernel<NW, 8, kSplit>), grid, dim3(NW * 64), 0, stream, p);
      break;
    case 4:
      hipLaunchKernelGGL((decode_attention_scan_kernel<NW, 4, kSplit>), grid, dim3(NW * 64), 0, stream, p);
      break;
    default:
      hipLaunchKernelGGL((decode_attention_scan_kernel<NW, 2, kSplit>), grid, dim3(NW * 64), 0, stream, p);
      break;
  }
}

hipError_t launch_decode_attention(const AttnParams& p, const AttnPlan& plan, hipStream_t stream) {
  if (plan.variant == 0) {
    launch_scan<16, false>(p, plan.rows_per_tile, dim3(p.num_heads), stream);
    return hipGetLastError();
  }
  const dim3 grid(p.num_heads * p.splits);
  switch (plan.waves) {
    case 16: launch_scan<16, true>(p, plan.rows_per_tile, grid, stream); break;
    case 8: launch_scan<8, true>(p, plan.rows_per_tile, grid, stream); break;
    default: launch_scan<4, true>(p, plan.rows_per_tile, grid, stream); break;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(decode_attention_merge_kernel<256>, dim3(p.num_heads), dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace qd
