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
//     16-lane "groups", each owning one KV row per load instruction.  A lane's
//     share of a row-dot is a chain of fused multiply-adds over its 8 fp16
//     pairs (v_fma_mix_f32 takes the fp16 key directly); a 4-step DPP
//     butterfly inside the 16-lane DPP row adds the lanes, and every lane of
//     the group ends with the same score.
//   * Each group keeps its own online-softmax state (m, l, 8 dims of O) in
//     fp32.  It consumes rows in tiles of U: one max/rescale per tile, then U
//     exp2 + 8U fp16*fp32 FMAs (v_fma_mix_f32, no conversions).
//   * A launch has about one wave per SIMD, so no other wave hides a tile's
//     compute latency: the arithmetic is kept short (Estrin exp2, one FMA per
//     key element, one exponential per lane per tile shared across the
//     group by DPP, max-first merges whose exponentials are independent).
//     Every instruction of the tile loop costs four cycles of the one wave a
//     SIMD runs, so instruction count is time: the FMA chain and the shared
//     exponentials took the loop from 281 to 217 instructions per 16-row tile
//     (15.45 -> 14.87 us per call at L=8192).
//   * Scores live in log2 units (scale_log2 = log2(e)/sqrt(128)); the
//     exponentials are exp2_rep (qd_device.h), a polynomial whose every step a
//     host implementation can repeat.
//   * Every floating-point operation is explicit (the library is built with
//     -ffp-contract=off; fused operations are written as fmaf) and every
//     reduction has a fixed order, so for a given launch plan the outputs are
//     a deterministic function of the inputs that the host oracle restates
//     bit for bit.
//   * Merges are max-first: the common maximum is found before any
//     exponential, so the rescaling exponentials are independent of each
//     other and the sums that follow are plain fmaf / add chains.  The four
//     groups of a wave merge with lane shuffles, the waves of a workgroup in
//     LDS.  A split workgroup writes one fp32 partial (m, l, O[128]); the
//     reference keeps fp16 partials.
//   * Partials are folded by a second, one-workgroup-per-head kernel.
//     Cross-workgroup hand-off goes through the kernel boundary: an
//     agent-scope release inside the kernel lowers to a whole-L2 writeback per
//     workgroup on gfx950 (buffer_wbl2 sc1, measured ~1 us each and
//     serialised per XCD), far more than a second launch.
//   * No MFMA: at q=1 the work is a bandwidth-bound GEMV-like reduction.
#include <atomic>
#include <mutex>

#include "qd_device.h"
#include "qd_internal.h"

namespace qd {

// Split partials of qd_decode_attention_noalloc: a static device array, so
// that entry point allocates nothing.  Every GPU the library runs on holds its
// own copy until the process ends, and every call on a GPU shares it, so calls
// that overlap on one GPU (e.g. on two streams) race.  Nothing in it must
// start at zero: each scan workgroup writes its whole slot before the merge
// kernel reads it.  In host code the name `scratch` is a host-side stand-in,
// not a device address; host code uses only the per-device address that
// static_scratch() looks up.
static __device__ __align__(256) float scratch[kStaticScratchSlots * (128 + 2)];

namespace {
constexpr int kMaxDevices = 64;
std::atomic<float*> g_scratch_addr[kMaxDevices];
std::mutex g_scratch_mu;
}  // namespace

int static_scratch(float** part_o, float2** part_ml) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices)
    return fail(QD_EINVAL, "device %d above the static scratch's %d devices", dev, kMaxDevices);
  float* base = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (!base) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    base = g_scratch_addr[dev].load(std::memory_order_relaxed);
    if (!base) {
      void* addr = nullptr;
      e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));   // this device's copy
      if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
      if (!addr) return fail(QD_EHIP, "hipGetSymbolAddress(scratch) returned NULL");
      base = static_cast<float*>(addr);
      g_scratch_addr[dev].store(base, std::memory_order_release);
    }
  }
  *part_o = base;
  *part_ml = reinterpret_cast<float2*>(base + (size_t)kStaticScratchSlots * 128);
  return QD_OK;
}

namespace {

constexpr int kD = 128;

// One lane's share of a row-dot: acc = k0*q0 (exact in fp32), then
// acc = fmaf(k_e, q_e, acc) for e = 1..7, each rounding once.  (fmaf with a
// -0 addend is the exact product, signed zeros included.)
__device__ __forceinline__ float dot8(const f16x8 k, const f16x8 q) {
  float acc = __builtin_fmaf((float)k[0], (float)q[0], -0.0f);
#pragma unroll
  for (int e = 1; e < 8; ++e) acc = __builtin_fmaf((float)k[e], (float)q[e], acc);
  return acc;
}

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

template <int U>
struct KvTile {
  f16x8 k[U];
  f16x8 v[U];
};

// Issue the loads of the tile starting at row blk: lane t of group g reads the
// 16 bytes at byte offset r*row_bytes + 16t for rows r = blk + 4u + g, clamped
// to nrows - 1 (a clamped row is loaded but masked out of the softmax).
// kbase/vbase are workgroup-uniform, so the loads take the saddr form (scalar
// base + 32-bit lane offset).  KV rows are read once, so the loads carry the
// non-temporal hint: streamed lines do not displace L2 contents (measured ~15%
// faster per call at L=32768).
template <int U>
__device__ __forceinline__ void load_tile(KvTile<U>& tl, const char* __restrict__ kbase,
                                          const char* __restrict__ vbase, unsigned row_bytes,
                                          int blk, int nrows, int g, int t) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const unsigned r = (unsigned)min(blk + 4 * u + g, nrows - 1);
    tl.k[u] = __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(kbase + (r * row_bytes + t * 16u)));
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const unsigned r = (unsigned)min(blk + 4 * u + g, nrows - 1);
    tl.v[u] = __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(vbase + (r * row_bytes + t * 16u)));
  }
}

// Online-softmax update of a group with one tile: scores s_u (rows >= nrows
// get -inf), tile max mt = max_u s_u (u ascending), mn = max(m, mt),
// alpha = exp2(m - mn), l = l*alpha, o = o*alpha, then for u ascending
// p = exp2(s_u - mn), l = l + p, o = fmaf(v_u, p, o).  Every exponent here
// and in the merges is <= 0, hence exp2_rep_nonpos.  All 16 lanes of a group
// hold the same scores, so lane j of each quad evaluates only p_{j mod U} and
// a quad broadcast (DPP quad_perm [u,u,u,u]) hands p_u to every lane.
template <int U>
__device__ __forceinline__ void consume_tile(GroupState& st, const KvTile<U>& tl, int blk,
                                             int nrows, int g, const f16x8 qv, float scale_log2) {
  static_assert(U == 2 || U == 4, "one exponential per lane covers at most 4 rows per group");
  float s[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const float d = row16_sum(dot8(tl.k[u], qv));
    s[u] = (blk + 4 * u + g < nrows) ? d * scale_log2 : -__builtin_inff();
  }
  float mt = s[0];
#pragma unroll
  for (int u = 1; u < U; ++u) mt = fmaxf(mt, s[u]);
  const float mn = fmaxf(st.m, mt);
  const float base = safe_base(mn);
  float p[U];
  {
    const int sel = (int)(threadIdx.x & (U - 1));   // this lane's row of the tile
    float sv = s[0];
#pragma unroll
    for (int u = 1; u < U; ++u) sv = sel == u ? s[u] : sv;
    const float pe = exp2_rep_nonpos(sv - base);
    p[0] = dpp_mov<0x00>(pe);                       // quad_perm [0,0,0,0]
    p[1] = dpp_mov<0x55>(pe);                       // quad_perm [1,1,1,1]
    if constexpr (U == 4) {
      p[2] = dpp_mov<0xAA>(pe);
      p[3] = dpp_mov<0xFF>(pe);
    }
  }
  // The rescale is skipped when no group of the wave raised its maximum: alpha
  // would then be exp2(0) = 1 (or 0 on a state that is still empty and all
  // zero), so skipping it changes no bit.  The test is wave-uniform.
  if (__builtin_amdgcn_ballot_w64(mn != st.m)) {
    const float alpha = exp2_rep_nonpos(st.m - base);
    st.l *= alpha;
#pragma unroll
    for (int j = 0; j < 8; ++j) st.o[j] *= alpha;
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    st.l += p[u];
#pragma unroll
    for (int j = 0; j < 8; ++j) st.o[j] = __builtin_fmaf((float)tl.v[u][j], p[u], st.o[j]);
  }
  st.m = mn;
}

// Scan rows [0, nrows) of one head.  Wave `wave` of NW takes the tiles of 4U
// consecutive rows starting at wave*4U, (wave+NW)*4U, ...; row blk + 4u + g of
// a tile goes to group g.  All 2U loads of a tile are issued before any of
// them is consumed.  (Double-buffering the tiles was measured: it was slower
// at L = 8192-32768, where the launch already streams at the box's read
// ceiling, by 4-8%.)
template <int NW, int U>
__device__ __forceinline__ void scan_rows(GroupState& st, const char* __restrict__ kbase,
                                          const char* __restrict__ vbase, unsigned row_bytes,
                                          int nrows, int wave, int g, int t, const f16x8 qv,
                                          float scale_log2) {
  for (int blk = wave * 4 * U; blk < nrows; blk += NW * 4 * U) {
    KvTile<U> tl;
    load_tile<U>(tl, kbase, vbase, row_bytes, blk, nrows, g, t);
    // keep the scheduler from sinking loads next to their uses
    __builtin_amdgcn_sched_barrier(0);
    consume_tile<U>(st, tl, blk, nrows, g, qv, scale_log2);
  }
}

// Fold the four groups of a wave (lanes t, t+16, t+32, t+48 hold the same
// dims), max-first: M = max of the four m (xor 16, then xor 32), each group
// scales its l and o by exp2(m - M), and the scaled values are summed as
// (g0 + g1) + (g2 + g3) with xor-16 then xor-32 shuffles.  Afterwards every
// lane holds the wave's state for its dims.
__device__ __forceinline__ void wave_merge(GroupState& st) {
  float M = fmaxf(st.m, __shfl_xor(st.m, 16));
  M = fmaxf(M, __shfl_xor(M, 32));
  const float sc = exp2_rep_nonpos(st.m - safe_base(M));
  float l = st.l * sc;
  float o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = st.o[j] * sc;
  l += __shfl_xor(l, 16);
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] += __shfl_xor(o[j], 16);
  l += __shfl_xor(l, 32);
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] += __shfl_xor(o[j], 32);
  st.m = M;
  st.l = l;
#pragma unroll
  for (int j = 0; j < 8; ++j) st.o[j] = o[j];
}

// Scan kernel.  Workgroup (split c, head h) with blockIdx.x = c * num_heads + h
// (so the workgroups resident together cover all heads of neighbouring
// positions) scans rows [c * rows_per_split, ...) of head h with NW waves.
// Each wave folds its four groups with lane shuffles; the NW wave states are
// folded in LDS by threads 0..127, one dim each.  kSplit = false is the
// single-workgroup-per-head path (fd_v5_fused_kernel's role): it writes the
// normalised fp16 output.  kSplit = true writes the workgroup's unnormalised
// fp32 partial (m, l, O[128]) to slot h * splits + c.  kBatch (with kSplit):
// query b = blockIdx.y over seqlen + b rows plans itself (auto_split), the
// workgroups past its split count exit, and its partials go to slots
// (b * num_heads + h) * split_stride + c; every workgroup that runs does
// exactly the work of the same workgroup of that query's single call.
template <int NW, int U, bool kSplit, bool kBatch = false>
__global__ __launch_bounds__(NW * 64) void decode_attention_scan_kernel(AttnParams p) {
  __shared__ float so[NW][kD];
  __shared__ float sm[NW];
  __shared__ float sl[NW];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: scalar loop control
  const int g = lane >> 4;
  const int t = lane & 15;
  const int h = blockIdx.x % p.num_heads;
  const int c = blockIdx.x / p.num_heads;
  const int b = blockIdx.y;                   // query of a batched call, else 0
  const int seqlen = p.seqlen + b;
  int rows_per_split = kSplit ? p.rows_per_split : seqlen;
  int splits = p.splits;
  if constexpr (kBatch) {
    auto_split(seqlen, p.num_cus, p.num_heads, &splits, &rows_per_split);
    if (c >= splits) return;                  // workgroup-uniform: this query has fewer splits
  }
  const int r0 = c * rows_per_split;
  const int nrows = min(seqlen - r0, rows_per_split);

  const f16x8 qv = *reinterpret_cast<const f16x8*>(p.q + b * p.q_batch_stride + h * kD + t * 8);
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
      const float wt = exp2_rep_nonpos(sm[w] - base);
      L = __builtin_fmaf(wt, sl[w], L);
      O = __builtin_fmaf(wt, so[w][tid], O);
    }
    if constexpr (kSplit) {
      const long long slot = kBatch ? ((long long)b * p.num_heads + h) * p.split_stride + c
                                    : (long long)h * splits + c;
      p.part_o[slot * kD + tid] = O;
      if (tid == 0) p.part_ml[slot] = float2{M, L};
    } else {
      reinterpret_cast<_Float16*>(p.out + b * p.out_batch_stride)[h * kD + tid] = to_f16(O / L);
    }
  }
}

// Stage 2: one workgroup per head folds the head's p.splits partials with the
// log-sum-exp rule (fd_opt_stage2_kernel's role) and writes the fp16 output.
// kBatch: workgroup (h, b = blockIdx.y) folds query b's auto_split partials
// from its slots (see the scan kernel) into out + b * out_batch_stride.
// Max-first: thread (dq = tid % 32 -> dims 4dq..4dq+3, slice = tid / 32)
// takes splits slice, slice + P, ...; the slices' maxima meet in LDS, so all
// threads share the head's maximum M before any exponential.  Each thread
// then sums w_c * l_c and w_c * O_c (w_c = exp2(m_c - M)) over its splits in
// ascending order with fmaf, issuing B splits' loads at a time, and the P
// slice sums are added in LDS (slice order).  The kernel boundary after
// stage 1 makes every partial visible on every XCD.
template <int NT, bool kBatch = false>
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
  int splits = p.splits;
  long long first = (long long)h * p.splits;  // this head's first partial slot
  _Float16* out = reinterpret_cast<_Float16*>(p.out);
  if constexpr (kBatch) {
    const int b = blockIdx.y;
    int rows;
    auto_split(p.seqlen + b, p.num_cus, p.num_heads, &splits, &rows);
    first = ((long long)b * p.num_heads + h) * p.split_stride;
    out += b * p.out_batch_stride;
  }
  const float* po = p.part_o + first * kD + dq * 4;
  const float2* pml = p.part_ml + first;
  // First batch of this thread's splits (slice, slice + P, ..., B of them),
  // loaded before the maximum is known so one memory round trip serves both.
  float2 ml[B];
  f32x4 ov[B];
#pragma unroll
  for (int j = 0; j < B; ++j) {
    const int cc = min(slice + j * P, splits - 1);
    ml[j] = pml[cc];
    ov[j] = *reinterpret_cast<const f32x4*>(po + (long long)cc * kD);
  }
  float mm = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < B; ++j)
    if (slice + j * P < splits) mm = fmaxf(mm, ml[j].x);
  for (int c = slice + B * P; c < splits; c += P) mm = fmaxf(mm, pml[c].x);
  if (dq == 0) sm[slice] = mm;
  __syncthreads();
  float M = sm[0];
#pragma unroll
  for (int s = 1; s < P; ++s) M = fmaxf(M, sm[s]);
  const float base = safe_base(M);
  float ll = 0.0f;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int c0 = slice;;) {
#pragma unroll
    for (int j = 0; j < B; ++j) {
      if (c0 + j * P < splits) {
        const float w = exp2_rep_nonpos(ml[j].x - base);
        ll = __builtin_fmaf(w, ml[j].y, ll);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf(w, ov[j][e], acc[e]);
      }
    }
    c0 += B * P;
    if (c0 >= splits) break;
#pragma unroll
    for (int j = 0; j < B; ++j) {
      const int cc = min(c0 + j * P, splits - 1);
      ml[j] = pml[cc];
      ov[j] = *reinterpret_cast<const f32x4*>(po + (long long)cc * kD);
    }
  }
  *reinterpret_cast<f32x4*>(&so[slice][dq * 4]) = acc;
  if (dq == 0) sl[slice] = ll;
  __syncthreads();
  if (tid < kD) {
    float L = sl[0], O = so[0][tid];
#pragma unroll
    for (int s = 1; s < P; ++s) {
      L += sl[s];
      O += so[s][tid];
    }
    out[h * kD + tid] = to_f16(O / L);
  }
}

}  // namespace

template <int NW, bool kSplit>
static void launch_scan(const AttnParams& p, int rows_per_tile, dim3 grid, hipStream_t stream) {
  switch (rows_per_tile) {
    case 4:
      hipLaunchKernelGGL((decode_attention_scan_kernel<NW, 4, kSplit>), grid, dim3(NW * 64), 0, stream, p);
      break;
    default:
      hipLaunchKernelGGL((decode_attention_scan_kernel<NW, 2, kSplit>), grid, dim3(NW * 64), 0, stream, p);
      break;
  }
}

hipError_t launch_decode_attention_fused_batch(const AttnParams& p, int tokens, hipStream_t stream) {
  hipLaunchKernelGGL((decode_attention_scan_kernel<16, 4, false>), dim3(p.num_heads, tokens),
                     dim3(16 * 64), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_decode_attention_split_batch(const AttnParams& p, int rows_per_tile, int tokens,
                                               hipStream_t stream) {
  const dim3 scan_grid(p.num_heads * p.split_stride, tokens);
  if (rows_per_tile == 4)
    hipLaunchKernelGGL((decode_attention_scan_kernel<4, 4, true, true>), scan_grid, dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((decode_attention_scan_kernel<4, 2, true, true>), scan_grid, dim3(256), 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((decode_attention_merge_kernel<256, true>), dim3(p.num_heads, tokens), dim3(256), 0,
                     stream, p);
  return hipGetLastError();
}

hipError_t launch_decode_attention(const AttnParams& p, const AttnPlan& plan, hipStream_t stream,
                                   int stages) {
  if (plan.variant == 0) {
    if (stages & kStageScan) launch_scan<16, false>(p, plan.rows_per_tile, dim3(p.num_heads), stream);
    return hipGetLastError();
  }
  if (stages & kStageScan) {
    const dim3 grid(p.num_heads * p.splits);
    switch (plan.waves) {
      case 16: launch_scan<16, true>(p, plan.rows_per_tile, grid, stream); break;
      case 8: launch_scan<8, true>(p, plan.rows_per_tile, grid, stream); break;
      default: launch_scan<4, true>(p, plan.rows_per_tile, grid, stream); break;
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (stages & kStageMerge)
    hipLaunchKernelGGL(decode_attention_merge_kernel<256>, dim3(p.num_heads), dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace qd
