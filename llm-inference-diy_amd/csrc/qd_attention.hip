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
//   * Split partials are folded either by a second, one-workgroup-per-head
//     kernel or, where every split of a head runs on one XCD, by the head's
//     last split workgroup inside the scan kernel (one launch), which reads
//     the other splits' tagged partials through its XCD's L2 with no fence:
//     an agent-scope release inside the kernel lowers to a whole-L2 writeback
//     per workgroup on gfx950 (buffer_wbl2 sc1, measured ~1 us each and
//     serialised per XCD), more than a second launch.  Both folds perform the
//     same operations in the same order.
//   * No MFMA: at q=1 the work is a bandwidth-bound GEMV-like reduction.
#include <algorithm>
#include <atomic>
#include <mutex>

#include "qd_device.h"
#include "qd_front_device.h"
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
// Layer row of a split's row j: j itself for a contiguous range (the range's
// first row is in the base), or, for interleaved blocks of kBlock rows (a power
// of two), row ((j / kBlock) * splits + c) * kBlock + j % kBlock.
template <int kBlock>
__device__ __forceinline__ unsigned split_row(int j, int c, int splits) {
  if constexpr (kBlock == 0) {
    return (unsigned)j;
  } else {
    static_assert((kBlock & (kBlock - 1)) == 0, "interleaved blocks of a power-of-two row count");
    return (unsigned)(((j / kBlock) * splits + c) * kBlock + (j & (kBlock - 1)));
  }
}

template <int U, int kBlock = 0>
__device__ __forceinline__ void load_tile(KvTile<U>& tl, const char* __restrict__ kbase,
                                          const char* __restrict__ vbase, unsigned row_bytes,
                                          int blk, int nrows, int g, int t, int c = 0, int splits = 1) {
  unsigned r[U];
#pragma unroll
  for (int u = 0; u < U; ++u) r[u] = split_row<kBlock>(min(blk + 4 * u + g, nrows - 1), c, splits);
#pragma unroll
  for (int u = 0; u < U; ++u)
    tl.k[u] = __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(kbase + (r[u] * row_bytes + t * 16u)));
#pragma unroll
  for (int u = 0; u < U; ++u)
    tl.v[u] = __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(vbase + (r[u] * row_bytes + t * 16u)));
}

// load_tile for a tile all of whose rows are valid, at byte offsets from a
// wave-uniform tile base: lane t of group g reads tbase + off[u], off[u] =
// (first + 4u + g) * row_bytes + 16 t, the same addresses load_tile forms for
// such a tile (rows first + 4u + g of the tile's first block row), with the
// per-row arithmetic moved out of the loop.
// (The empty asm keeps each offset a 32-bit lane value at its use, so the
// loads take the saddr form -- scalar tile base + lane offset -- instead of a
// 64-bit lane address the compiler would otherwise hoist and add per load.)
template <int U>
__device__ __forceinline__ void load_tile_at(KvTile<U>& tl, const char* __restrict__ kt,
                                             const char* __restrict__ vt, const unsigned (&off)[U]) {
  unsigned o[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    o[u] = off[u];
    asm volatile("" : "+v"(o[u]));
  }
#pragma unroll
  for (int u = 0; u < U; ++u)
    tl.k[u] = __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(kt + o[u]));
#pragma unroll
  for (int u = 0; u < U; ++u)
    tl.v[u] = __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(vt + o[u]));
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
// a tile goes to group g.  The loads of D consecutive tiles of the wave (all
// 2U loads of each) are issued before any of them is consumed, then the tiles
// are consumed in order: D changes how many memory round trips a wave waits
// for, not the arithmetic.  (Prefetching tile i+1 while consuming tile i was
// measured: it was slower at L = 8192-32768, where the launch already streams
// at the box's read ceiling, by 4-8%.)
// D = 0 is a rolling pipeline instead: the loads of tile i + 1 are issued
// before tile i is consumed, so a wave's next loads are in flight while it
// computes (the same tiles consumed in the same order: the same bits).
template <int NW, int U, int D = 1, bool kInter = false>
__device__ __forceinline__ void scan_rows(GroupState& st, const char* __restrict__ kbase,
                                          const char* __restrict__ vbase, unsigned row_bytes,
                                          int nrows, int wave, int g, int t, const f16x8 qv,
                                          float scale_log2, int c = 0, int splits = 1) {
  constexpr int kStep = NW * 4 * U;   // rows from one of a wave's tiles to its next
  constexpr int kBlock = kInter ? kStep : 0;
  if constexpr (D == 0) {
    const int blk0 = wave * 4 * U;
    if (blk0 >= nrows) return;
    // Tiles blk0 + i * kStep, i < n.  Tile i's rows are rows blk0 + 4u + g
    // past layer row first_row + i * step_rows (interleaved: split c's i-th
    // block, kStep == kBlock; contiguous: kStep rows on), so every tile loads
    // from a wave-uniform base with lane offsets fixed for the whole scan: the
    // saddr form with no per-row arithmetic.  Only the last tile can hold rows
    // past nrows - 1 (every earlier one ends at blk0 + i * kStep + 4U <=
    // nrows), and a clamped row lies in its block, so the last tile's offsets
    // are load_tile's clamp taken once, in the same base: load_tile's
    // addresses, so the same rows and bits.  (8192 rows: 13.82-13.93 against
    // 14.03-14.06 us per call with load_tile's per-row addresses; the
    // one-round-at-a-time loop below ran slower in this form, 8.9 against 8.4
    // us at 3072 rows and 41.6 against 41.0 at 32768, and keeps load_tile.)
    const int n = (nrows - blk0 + kStep - 1) / kStep;
    const unsigned step_bytes = (unsigned)(kBlock ? splits * kBlock : kStep) * row_bytes;
    const unsigned first_bytes = (unsigned)(kBlock ? c * kBlock : 0) * row_bytes;
    const int lim = nrows - 1 - (n - 1) * kStep;   // the last tile's last valid row
    unsigned off[U], offl[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      off[u] = (unsigned)(blk0 + 4 * u + g) * row_bytes + (unsigned)t * 16u;
      offl[u] = (unsigned)min(blk0 + 4 * u + g, lim) * row_bytes + (unsigned)t * 16u;
    }
    auto load = [&](KvTile<U>& tl, int i) {
      const size_t tb = first_bytes + (size_t)i * step_bytes;
      unsigned o[U];
#pragma unroll
      for (int u = 0; u < U; ++u) o[u] = i + 1 < n ? off[u] : offl[u];
      load_tile_at<U>(tl, kbase + tb, vbase + tb, o);
    };
    // The loop runs whole pairs with one exit, so on every edge into it
    // exactly the loads of tile i are pending.
    KvTile<U> a, b;   // ping-pong buffers: no register copies between tiles
    load(a, 0);
    int i = 0;
    for (; i + 2 < n; i += 2) {
      const int blk = blk0 + i * kStep;
      load(b, i + 1);
      __builtin_amdgcn_sched_barrier(0);
      consume_tile<U>(st, a, blk, nrows, g, qv, scale_log2);
      load(a, i + 2);
      __builtin_amdgcn_sched_barrier(0);
      consume_tile<U>(st, b, blk + kStep, nrows, g, qv, scale_log2);
    }
    const int blk = blk0 + i * kStep;
    if (i + 1 < n) {
      load(b, i + 1);
      __builtin_amdgcn_sched_barrier(0);
      consume_tile<U>(st, a, blk, nrows, g, qv, scale_log2);
      consume_tile<U>(st, b, blk + kStep, nrows, g, qv, scale_log2);
    } else {
      consume_tile<U>(st, a, blk, nrows, g, qv, scale_log2);
    }
  } else {
    for (int blk = wave * 4 * U; blk < nrows; blk += kStep * D) {
      KvTile<U> tl[D];
#pragma unroll
      for (int d = 0; d < D; ++d)
        if (d == 0 || blk + d * kStep < nrows)
          load_tile<U, kBlock>(tl[d], kbase, vbase, row_bytes, blk + d * kStep, nrows, g, t, c, splits);
      // keep the scheduler from sinking loads next to their uses
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int d = 0; d < D; ++d)
        if (d == 0 || blk + d * kStep < nrows) consume_tile<U>(st, tl[d], blk + d * kStep, nrows, g, qv, scale_log2);
    }
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
// LDS of one workgroup's fold of its NW wave states.
template <int NW>
struct ScanLds {
  float so[NW][kD];
  float sm[NW];
  float sl[NW];
};

// Scan rows [r0, r0 + nrows) of head h for query row q (the whole workgroup,
// NW waves), fold each wave's four groups with lane shuffles and the NW wave
// states in LDS, max-first: for tid < 128, (M, L, O) is the workgroup's
// partial for dim tid (M and L the same in every thread).  Ends with the LDS
// reads of the fold; a caller that reuses `lds` synchronises first.
// Fold each wave's four groups with lane shuffles and the NW wave states in
// LDS, max-first: for tid < 128, (M, L, O) is the workgroup's partial for dim
// tid (M and L the same in every thread).  Ends with the LDS reads of the
// fold; a caller that reuses `lds` synchronises first.
template <int NW>
__device__ __forceinline__ void fold_waves(GroupState& st, ScanLds<NW>& lds, float& M, float& L,
                                           float& O);

template <int NW, int U, int D = 1, bool kInter = false>
__device__ __forceinline__ void scan_fold_q(const AttnParams& p, const f16x8 qv, int h, int r0,
                                            int nrows, ScanLds<NW>& lds, float& M, float& L,
                                            float& O, int c = 0) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: scalar loop control
  const int g = lane >> 4;
  const int t = lane & 15;
  const long long off = h * p.head_stride + (long long)r0 * p.row_stride;
  GroupState st;
  init_state(st);
  scan_rows<NW, U, D, kInter>(st, reinterpret_cast<const char*>(p.k + off),
                              reinterpret_cast<const char*>(p.v + off), (unsigned)(p.row_stride * 2),
                              nrows, wave, g, t, qv, p.scale_log2, c, p.splits);
  fold_waves<NW>(st, lds, M, L, O);
}

// scan_fold_q with Q read here, the fold written out (fold_waves' steps).
// Spelled out rather than calling scan_fold_q: built that way the split scan
// kernel at L=8192 compiled to a slightly different schedule and ran 0.6 us
// slower per launch (12.8 against 12.2 us, the same bits).
template <int NW, int U, int D = 1, bool kInter = false>
__device__ __forceinline__ void scan_fold(const AttnParams& p, const uint16_t* q, int h, int r0,
                                          int nrows, ScanLds<NW>& lds, float& M, float& L,
                                          float& O, int c, int splits) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: scalar loop control
  const int g = lane >> 4;
  const int t = lane & 15;
  const f16x8 qv = *reinterpret_cast<const f16x8*>(q + h * kD + t * 8);
  const long long off = h * p.head_stride + (long long)r0 * p.row_stride;
  GroupState st;
  init_state(st);
  scan_rows<NW, U, D, kInter>(st, reinterpret_cast<const char*>(p.k + off),
                              reinterpret_cast<const char*>(p.v + off), (unsigned)(p.row_stride * 2),
                              nrows, wave, g, t, qv, p.scale_log2, c, splits);
  wave_merge(st);
  if (lane < 16) {
    *reinterpret_cast<f32x4*>(&lds.so[wave][t * 8]) = f32x4{st.o[0], st.o[1], st.o[2], st.o[3]};
    *reinterpret_cast<f32x4*>(&lds.so[wave][t * 8 + 4]) = f32x4{st.o[4], st.o[5], st.o[6], st.o[7]};
    if (t == 0) {
      lds.sm[wave] = st.m;
      lds.sl[wave] = st.l;
    }
  }
  __syncthreads();
  M = -__builtin_inff();
  L = 0.0f;
  O = 0.0f;
  if (tid < kD) {
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, lds.sm[w]);
    const float base = safe_base(M);
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float wt = exp2_rep_nonpos(lds.sm[w] - base);
      L = __builtin_fmaf(wt, lds.sl[w], L);
      O = __builtin_fmaf(wt, lds.so[w][tid], O);
    }
  }
}

template <int NW>
__device__ __forceinline__ void fold_waves(GroupState& st, ScanLds<NW>& lds, float& M, float& L,
                                           float& O) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t = lane & 15;
  wave_merge(st);
  if (lane < 16) {
    *reinterpret_cast<f32x4*>(&lds.so[wave][t * 8]) = f32x4{st.o[0], st.o[1], st.o[2], st.o[3]};
    *reinterpret_cast<f32x4*>(&lds.so[wave][t * 8 + 4]) = f32x4{st.o[4], st.o[5], st.o[6], st.o[7]};
    if (t == 0) {
      lds.sm[wave] = st.m;
      lds.sl[wave] = st.l;
    }
  }
  __syncthreads();
  M = -__builtin_inff();
  L = 0.0f;
  O = 0.0f;
  if (tid < kD) {
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, lds.sm[w]);
    const float base = safe_base(M);
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float wt = exp2_rep_nonpos(lds.sm[w] - base);
      L = __builtin_fmaf(wt, lds.sl[w], L);
      O = __builtin_fmaf(wt, lds.so[w][tid], O);
    }
  }
}

template <int NW, int U, bool kSplit, bool kBatch = false, int D = 1, bool kInter = false>
__global__ __launch_bounds__(NW * 64) void decode_attention_scan_kernel(AttnParams p) {
  static_assert(!(kBatch && kInter), "batched queries choose their row mapping per query");
  __shared__ ScanLds<NW> lds;
  const int tid = threadIdx.x;
  const int h = blockIdx.x % p.num_heads;
  const int c = blockIdx.x / p.num_heads;
  const int b = blockIdx.y;                   // query of a batched call, else 0
  const int seqlen = p.seqlen + b;
  int rows_per_split = kSplit ? p.rows_per_split : seqlen;
  int splits = p.splits;
  float M, L, O;
  if constexpr (kBatch) {
    int block;
    auto_plan(seqlen, p.num_cus, p.num_heads, p.long_inter != 0, &splits, &rows_per_split, &block);
    if (c >= splits) return;                  // workgroup-uniform: this query has fewer splits
    // A long query deals its rows in interleaved blocks, as decode plans it;
    // the host launches each query with the tile its plan takes, so such a
    // query's block is this kernel's load round (NW * 4 * U rows).
    if (block != 0 && block == NW * 4 * U) {
      scan_fold<NW, U, D, true>(p, p.q + b * p.q_batch_stride, h, 0,
                                interleaved_rows(seqlen, block, splits, c), lds, M, L, O, c, splits);
    } else {
      const int r0 = c * rows_per_split;
      scan_fold<NW, U, D, false>(p, p.q + b * p.q_batch_stride, h, r0,
                                 min(seqlen - r0, rows_per_split), lds, M, L, O, c, splits);
    }
  } else {
    const int r0 = kInter ? 0 : c * rows_per_split;
    const int nrows = kInter ? interleaved_rows(seqlen, NW * 4 * U, splits, c)
                             : min(seqlen - r0, rows_per_split);
    scan_fold<NW, U, D, kInter>(p, p.q + b * p.q_batch_stride, h, r0, nrows, lds, M, L, O, c, splits);
  }
  if (tid < kD) {
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
constexpr int kMergeThreads = 256;
constexpr int kMergeSlices = kMergeThreads / 32;   // P
constexpr int kMergeBatch = 8;                     // B: splits per thread per round trip

struct MergeLds {
  float so[kMergeSlices][kD];
  float sm[kMergeSlices];
  float sl[kMergeSlices];
};

// Partials of one head as the merge reads them: (m, l) of split c, and dims
// 4dq..4dq+3 of its O.
struct PlainPartials {
  const float* po;     // + dq * 4 already applied
  const float2* pml;
  __device__ float2 ml(int c) const { return pml[c]; }
  __device__ f32x4 o4(int c) const { return *reinterpret_cast<const f32x4*>(po + (long long)c * kD); }
};

// Log-sum-exp fold of one head's `splits` partials by kMergeThreads threads,
// max-first: thread (dq = tid % 32 -> dims 4dq..4dq+3, slice = tid / 32) takes
// splits slice, slice + P, ...; the slices' maxima meet in LDS, so all threads
// share the head's maximum M before any exponential.  Each thread then sums
// w_c * l_c and w_c * O_c (w_c = exp2(m_c - M)) over its splits in ascending
// order with fmaf, B splits' loads at a time, and the P slice sums are added
// in LDS (slice order); out_head[d] = half(O_d / L).  ml / ov hold the
// thread's first batch (splits slice + j * P, clamped to splits - 1), loaded
// by the caller before the maximum is known so that one memory round trip
// serves both; src loads the splits beyond the first batch.
template <class Src>
__device__ __forceinline__ void merge_fold(float2 (&ml)[kMergeBatch], f32x4 (&ov)[kMergeBatch],
                                           int splits, const Src& src, MergeLds& lds,
                                           _Float16* out_head) {
  constexpr int P = kMergeSlices;
  constexpr int B = kMergeBatch;
  const int tid = threadIdx.x;
  const int dq = tid & 31;
  const int slice = tid >> 5;
  float mm = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < B; ++j)
    if (slice + j * P < splits) mm = fmaxf(mm, ml[j].x);
  for (int c = slice + B * P; c < splits; c += P) mm = fmaxf(mm, src.ml(c).x);
  if (dq == 0) lds.sm[slice] = mm;
  __syncthreads();
  float M = lds.sm[0];
#pragma unroll
  for (int s = 1; s < P; ++s) M = fmaxf(M, lds.sm[s]);
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
      ml[j] = src.ml(cc);
      ov[j] = src.o4(cc);
    }
  }
  *reinterpret_cast<f32x4*>(&lds.so[slice][dq * 4]) = acc;
  if (dq == 0) lds.sl[slice] = ll;
  __syncthreads();
  if (tid < kD) {
    float L = lds.sl[0], O = lds.so[0][tid];
#pragma unroll
    for (int s = 1; s < P; ++s) {
      L += lds.sl[s];
      O += lds.so[s][tid];
    }
    out_head[tid] = to_f16(O / L);
  }
}

template <bool kBatch = false>
__global__ __launch_bounds__(kMergeThreads) void decode_attention_merge_kernel(AttnParams p) {
  __shared__ MergeLds lds;
  const int tid = threadIdx.x;
  const int h = blockIdx.x;
  const int dq = tid & 31;
  const int slice = tid >> 5;
  int splits = p.splits;
  long long first = (long long)h * p.splits;  // this head's first partial slot
  _Float16* out = reinterpret_cast<_Float16*>(p.out);
  if constexpr (kBatch) {
    const int b = blockIdx.y;
    int rows, block;
    auto_plan(p.seqlen + b, p.num_cus, p.num_heads, p.long_inter != 0, &splits, &rows, &block);
    first = ((long long)b * p.num_heads + h) * p.split_stride;
    out += b * p.out_batch_stride;
  }
  const PlainPartials src{p.part_o + first * kD + dq * 4, p.part_ml + first};
  float2 ml[kMergeBatch];
  f32x4 ov[kMergeBatch];
#pragma unroll
  for (int j = 0; j < kMergeBatch; ++j) {
    const int cc = min(slice + j * kMergeSlices, splits - 1);
    ml[j] = src.ml(cc);
    ov[j] = src.o4(cc);
  }
  merge_fold(ml, ov, splits, src, lds, out + h * kD);
}

// ---------------------------------------------------------------------------
// Split attention with the merge inside the scan kernel (one launch).
//
// Every split workgroup but the head's last writes its partial as tagged
// words -- (value, tag) pairs, the tag being the call's sequence number --
// into its slot, waits for its stores to be acknowledged (s_waitcnt vmcnt(0):
// the L2 of its XCD holds them), then adds 1 to its head's arrival counter
// and ends.  The head's last split is its merger: it keeps its own partial in
// registers and reads the other splits' slots until every word it reads
// carries this call's tag, then folds.  (The counters are never reset: the
// host passes the value they hold when the call starts and adds the call's
// split count minus one.)  The fold performs exactly merge_fold's operations
// in merge_fold's order (below), one lane per dim, so a call gives the
// two-launch path's bits.
//
// Waves 0 and 1 of the merger each own 64 dims and poll on their own: a read
// is one 8-byte load per lane per slot (the lane's dim: value and tag) plus
// one slot record per lane (lane c: split c's m, l), the staleness test is a
// ballot per slot, the merge weights are computed in the lanes that hold the
// records and broadcast with readlane.  No LDS and no barrier stand between
// the last slot becoming visible and the output store.  The counter is read
// only to decide when a slot that stays stale may be scanned again (a slot
// still stale in a read issued after the counter showed every other split
// arrived was written where this workgroup cannot see it).  It is read with
// every kXCntPeriod-th read of the slots only, and consumed a round later: an
// agent-scope load is slower than the slot loads, which hit the XCD's L2, and
// a read lasts as long as its slowest load (reading it with every read cost
// 0.13-0.15 us per call at 160-3072 rows).
//
// The merger reads the slots through its XCD's L2.  With the launch's
// workgroup i on XCD (k + i) mod NX (round-robin dispatch, checked at context
// creation) and num_heads a multiple of NX, every split of head h runs on one
// XCD, so every slot the merger reads is in its own L2: no cache writeback or
// invalidation stands between the splits and the merge.  Correctness does not
// rest on that placement: every 8-byte word carries the tag and is written by
// one store, so a word the merger can see is either this call's or visibly
// stale.  A split whose words stay stale (written on another XCD, still in
// that XCD's L2) is scanned again by the whole merging workgroup from the KV
// cache -- the same arithmetic, so the same bits -- and the reads resume.
// The loads are non-temporal: they do not return a line the CU's L1 kept from
// an earlier read, which a later read of a slot must not see.  (In a dispatch
// that does not split workgroups across CUs, buffer_inv sc0 leaves L1 lines
// in place; measured on gfx950, a non-temporal load returned the line another
// CU of the XCD had written since, in 80-120 ns.)
// ---------------------------------------------------------------------------

// Words of one tagged slot: O[128] as (O_d, tag), then (m, tag), (l, tag).
constexpr int kXSlotWords = 144;   // 130 used; 1152 B, nine 128-B lines
constexpr int kXPolls = 1 << 14;   // reads of the slots before the stale ones are scanned again
constexpr int kXCntPeriod = 8;     // reads of the slots per read of the arrival counter
static_assert(kXMaxSplits <= 64 && kXMaxSplits <= kMergeSlices * kMergeBatch,
              "one wave holds a head's split weights; merge_fold reads them in one batch");

__device__ __forceinline__ bool tag_ok(float word_tag, unsigned tag) { return __float_as_uint(word_tag) == tag; }

// merge_fold's weights, one lane per split (lanes c < splits of one wave hold
// split c's m and l): M = max_c m_c (fmaxf, exact in any order), then
// s_w[c] = exp2(m_c - safe_base(M)) and s_l[c] = l_c.
template <int SMAX>
__device__ __forceinline__ void merge_weights(float m_c, float l_c, int lane, int splits,
                                              float* s_w, float* s_l) {
  float m = -__builtin_inff();
  if (lane < splits) m = fmaxf(m, m_c);
  const float M = SMAX <= 16 ? row16_max(m) : wave64_max(m);   // splits in lanes 0..SMAX-1
  if (lane < splits) {
    s_w[lane] = exp2_rep_nonpos(m - safe_base(M));
    s_l[lane] = l_c;
  }
}

// merge_fold's sums and output, one thread per dim d < 128: slice s (of
// kMergeSlices) adds w_c * l_c and w_c * O_c over its splits c = s, s + P, ...
// in ascending order with fmaf from 0, then the slice sums are added in slice
// order (empty slices add 0.0f, as merge_fold's do); out[d] = half(O / L).
// The LDS reads do not depend on splits, so they are all issued up front; the
// terms of absent splits are dropped by selects.
template <int SMAX>
__device__ __forceinline__ void fold_per_dim(const float* s_w, const float* s_l,
                                             const float (*s_o)[kD], int splits, _Float16* out) {
  const int tid = threadIdx.x;
  if (tid >= kD) return;
  float o[SMAX], w[SMAX], l[SMAX];
#pragma unroll
  for (int cc = 0; cc < SMAX; ++cc) {
    o[cc] = s_o[cc][tid];
    w[cc] = s_w[cc];
    l[cc] = s_l[cc];
  }
  float O = 0.0f, L = 0.0f;
#pragma unroll
  for (int s = 0; s < kMergeSlices; ++s) {
    float acc = 0.0f, ll = 0.0f;
#pragma unroll
    for (int cc = s; cc < SMAX; cc += kMergeSlices) {
      const bool on = cc < splits;
      const float nl = __builtin_fmaf(w[cc], l[cc], ll);
      const float na = __builtin_fmaf(w[cc], o[cc], acc);
      ll = on ? nl : ll;
      acc = on ? na : acc;
    }
    if (s == 0) {
      O = acc;
      L = ll;
    } else {
      O += acc;
      L += ll;
    }
  }
  out[tid] = to_f16(O / L);
}

// One read of the other splits' slots by a merging wave: lane l's dim
// (value, tag) of every slot, lane c's slot record (lanes c < others), and,
// issued last when `counter` is not null, the head's arrival counter (lane 0).
template <int SMAX>
struct SlotRead {
  f32x2 o[SMAX];
  f32x4 rec;
  unsigned cnt;
};

template <int SMAX>
__device__ __forceinline__ void issue_read(SlotRead<SMAX>& r, const char* head, unsigned dim_off,
                                           int last_slot, int lane, int others, float m_own,
                                           float l_own, const unsigned* counter) {
#pragma unroll
  for (int cc = 0; cc < SMAX; ++cc)
    r.o[cc] = __builtin_nontemporal_load(
        reinterpret_cast<const f32x2*>(head + (unsigned)(min(cc, last_slot) * kXSlotWords * 8) + dim_off));
  r.rec = f32x4{m_own, 0.0f, l_own, 0.0f};   // lane others (the merger's own split) keeps these
  if (lane < others)
    r.rec = __builtin_nontemporal_load(
        reinterpret_cast<const f32x4*>(head + (unsigned)(lane * kXSlotWords * 8 + kD * 8)));
  r.cnt = 0u;
  if (lane == 0 && counter) r.cnt = __hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Splits (< others) with a word in the read that is not this call's.
template <int SMAX>
__device__ __forceinline__ unsigned long long stale_splits(const SlotRead<SMAX>& r, int lane, int others,
                                                           unsigned tag) {
  unsigned long long stale =
      __builtin_amdgcn_ballot_w64(lane < others && (!tag_ok(r.rec[1], tag) || !tag_ok(r.rec[3], tag)));
#pragma unroll
  for (int cc = 0; cc < SMAX; ++cc)
    if (cc < others && __builtin_amdgcn_ballot_w64(!tag_ok(r.o[cc].y, tag))) stale |= 1ull << cc;
  return stale;
}

// merge_fold's weights in the record lanes (M = max_c m_c, w_c = exp2(m_c -
// safe_base(M))), broadcast with readlane, then its sums in its order: slice
// s (of kMergeSlices) adds w_c * l_c and w_c * O_c over c = s, s + P, ...
// ascending with fmaf from 0, the slice sums are added in slice order;
// out = half(O / L) for this lane's dim.  Split `others` is the merger's own
// (o_own).  Terms of absent splits are dropped by selects.
template <int SMAX>
__device__ __forceinline__ void fold_store(const SlotRead<SMAX>& r, int lane, int splits, float o_own,
                                           _Float16* dst) {
  const int others = splits - 1;
  const float m = lane < splits ? r.rec[0] : -__builtin_inff();
  const float M = SMAX <= 16 ? row16_max(m) : wave64_max(m);   // splits in lanes 0..SMAX-1
  const float wl = exp2_rep_nonpos(m - safe_base(M));
  const float lc_l = r.rec[2];
  float O = 0.0f, L = 0.0f;
#pragma unroll
  for (int s = 0; s < kMergeSlices; ++s) {
    float acc = 0.0f, ll = 0.0f;
#pragma unroll
    for (int cc = s; cc < SMAX; cc += kMergeSlices) {
      const bool on = cc < splits;
      const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wl), cc));
      const float lc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lc_l), cc));
      const float oc = cc == others ? o_own : r.o[cc].x;
      const float nl = __builtin_fmaf(w, lc, ll);
      const float na = __builtin_fmaf(w, oc, acc);
      ll = on ? nl : ll;
      acc = on ? na : acc;
    }
    if (s == 0) {
      O = acc;
      L = ll;
    } else {
      O += acc;
      L += ll;
    }
  }
  *dst = to_f16(O / L);
}

// One wave of the merger (wave 0 or 1: dims 64 * wave + lane): reads the
// other splits' slots until every word it needs is this call's, then folds
// and stores its 64 dims of the head's output and returns 0.  Returns the
// splits to scan again instead: those in `force`, or those still stale in a
// read issued after a completed counter read (one with every kXCntPeriod-th
// read) saw every other split arrived, or after kXPolls reads.  (m_own, l_own, o_own): the merger's own partial
// (o_own: this lane's dim).  One read is in flight at a time: a kernel ends
// only when its loads have returned, and a second read in flight when the
// first finds every slot measured 0.6 us slower per call at L=8192.
template <int SMAX>
__device__ __forceinline__ unsigned long long merge_wave(const AttnParams& p, const char* head, int wave,
                                                        int lane, int splits, float m_own, float l_own,
                                                        float o_own, unsigned long long force,
                                                        _Float16* out_head, unsigned& reads) {
  const int others = splits - 1;                               // slots 0 .. splits - 2
  const int last_slot = max(others - 1, 0);
  const unsigned dim_off = (unsigned)((wave * 64 + lane) * 8);
  const unsigned* counter = p.xcnt + (blockIdx.x % p.num_heads) * kXCounterStride;
  bool arrived = false;   // a completed counter read, before this read was issued, saw all arrived
  SlotRead<SMAX> r;
  for (int round = 0;; ++round) {
    const bool with_cnt = (round + 1) % kXCntPeriod == 0;
    issue_read<SMAX>(r, head, dim_off, last_slot, lane, others, m_own, l_own, with_cnt ? counter : nullptr);
    ++reads;
    const unsigned long long stale = stale_splits<SMAX>(r, lane, others, p.tag);
    if ((stale | force) == 0ull) {
      fold_store<SMAX>(r, lane, splits, o_own, out_head + wave * 64 + lane);
      return 0ull;
    }
    const unsigned long long rescan = force | (arrived || round >= kXPolls ? stale : 0ull);
    if (rescan) return rescan;
    // This read's counter value: complete now, so it covers the next read.
    if (with_cnt) arrived = (unsigned)__builtin_amdgcn_readfirstlane(r.cnt) - p.cnt_base >= (unsigned)others;
  }
}

// The end of a split workgroup of an in-kernel-merge plan, after its scan:
// (M, L, O) its partial (threads tid < 128).  Every split but the head's last
// publishes its partial as tagged words and ends; the last merges (see
// decode_attention_xmerge_kernel).  qv: this lane's Q chunk, for scanning
// splits again.
template <int U, int SMAX, int D, int NW, bool kInter>
__device__ __forceinline__ void xmerge_finish(const AttnParams& p, int h, int c, const f16x8 qv,
                                              float M, float L, float O, ScanLds<NW>& slds,
                                              unsigned long long (&s_need)[2]) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int splits = p.splits;
  const int merger = splits - 1;                             // the last split, often the shortest
  const float tagf = __uint_as_float(p.tag);
  float2* head_slots = p.xpart + (long long)h * kXMaxSplits * kXSlotWords;
  const char* head = reinterpret_cast<const char*>(head_slots);
  constexpr int kBlock = NW * 4 * U;
  if (c != merger) {
    // This split's partial, published as tagged words.
    float2* slot = head_slots + (long long)c * kXSlotWords;
    if (tid < kD) slot[tid] = float2{O, tagf};
    if (tid == 0) *reinterpret_cast<f32x4*>(slot + kD) = f32x4{M, tagf, L, tagf};
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // acknowledged: in its XCD's L2
    __syncthreads();
    // Arrival: read by the merger only to decide on scanning a split again;
    // no one waits for it here.
    if (tid == 0)
      __hip_atomic_fetch_add(p.xcnt + h * kXCounterStride, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }

  // The merger.  Waves 2 and up wait at the barrier below; they take part only
  // in scanning splits again.
  unsigned long long force = 0ull;   // test hook: splits treated as never visible
  if (p.recompute_mask)
    for (int cc = 0; cc < merger; ++cc)
      if ((p.recompute_mask >> (cc & 31)) & 1u) force |= 1ull << cc;
  bool done = wave >= 2;
  unsigned reads = 0u, rescanned = 0u;
  _Float16* out_head = reinterpret_cast<_Float16*>(p.out) + h * kD;
  for (;;) {
    unsigned long long need = 0ull;
    if (!done) {
      need = merge_wave<SMAX>(p, head, wave, lane, splits, M, L, O, force, out_head, reads);
      done = need == 0ull;
    }
    if (wave < 2 && lane == 0) s_need[wave] = need;
    __syncthreads();
    const unsigned long long all = s_need[0] | s_need[1];
    if (all == 0ull) break;
    // Scan those splits again (same plan, same arithmetic, same bits) and
    // publish them from this workgroup; the merging waves then read again.
    rescanned += (unsigned)__builtin_popcountll(all);
    for (int cc = 0; cc < merger; ++cc) {
      if (!((all >> cc) & 1ull)) continue;
      const int rr = kInter ? 0 : cc * p.rows_per_split;
      float Mc, Lc, Oc;
      scan_fold_q<NW, U, D, kInter>(p, qv, h, rr,
                                  kInter ? interleaved_rows(p.seqlen, kBlock, splits, cc)
                                         : min(p.seqlen - rr, p.rows_per_split),
                                  slds, Mc, Lc, Oc, cc);
      float2* slot = head_slots + (long long)cc * kXSlotWords;
      if (tid < kD) slot[tid] = float2{Oc, tagf};
      if (tid == 0) *reinterpret_cast<f32x4*>(slot + kD) = f32x4{Mc, tagf, Lc, tagf};
      __syncthreads();                                       // slds reuse
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    force = 0ull;
  }
  if (tid == 0) {   // statistics, after the output; not waited for
    unsigned* st = p.xcnt + h * kXCounterStride;
    if (p.count_merges) {
      __hip_atomic_fetch_add(st + kXStatMerges, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_fetch_add(st + kXStatReads, reads, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (rescanned)
      __hip_atomic_fetch_add(st + kXStatRescans, rescanned, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// SMAX: a bound on p.splits (16, 32 or 64): the slots each merging wave reads.
// NW scanning waves (4 or 8); kInter: interleaved blocks of NW * 4 * U rows.
template <int U, int SMAX, int D = 1, int NW = 4, bool kInter = false>
__global__ __launch_bounds__(NW * 64) void decode_attention_xmerge_kernel(AttnParams p) {
  static_assert(SMAX % 4 == 0 && SMAX <= kXMaxSplits, "SMAX: a multiple of 4, at most the slot count");
  static_assert(NW == 4 || NW == 8, "four or eight waves scan; waves 0 and 1 hold the 128 dims");
  __shared__ ScanLds<NW> slds;
  __shared__ unsigned long long s_need[2];   // splits to scan again, per merging wave
  const int lane = threadIdx.x & 63;
  const int h = blockIdx.x % p.num_heads;
  const int c = blockIdx.x / p.num_heads;
  const int splits = p.splits;
  constexpr int kBlock = NW * 4 * U;
  const int r0 = kInter ? 0 : c * p.rows_per_split;
  const f16x8 qv = *reinterpret_cast<const f16x8*>(p.q + h * kD + (lane & 15) * 8);
  float M, L, O;   // valid in threads tid < kD
  scan_fold_q<NW, U, D, kInter>(p, qv, h, r0,
                                kInter ? interleaved_rows(p.seqlen, kBlock, splits, c)
                                       : min(p.seqlen - r0, p.rows_per_split),
                                slds, M, L, O, c);
  xmerge_finish<U, SMAX, D, NW, kInter>(p, h, c, qv, M, L, O, slds, s_need);
}

// Stage 2 of the two-launch path for at most SMAX splits per head: merge_fold's
// arithmetic, mapped as the in-kernel merge maps it (fewer memory round trips
// and LDS steps than merge_fold's slices, the same bits).  One workgroup per
// head: wave w loads splits w, w + 4, ... (lane l: dims 2l, 2l + 1), wave 0's
// lane c split c's (m, l).
template <int SMAX>
__global__ __launch_bounds__(kMergeThreads) void decode_attention_merge_dim_kernel(AttnParams p) {
  static_assert(SMAX % 4 == 0 && SMAX <= 64, "one wave holds a head's split weights");
  __shared__ float s_o[SMAX][kD];
  __shared__ float s_w[SMAX];
  __shared__ float s_l[SMAX];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = blockIdx.x;
  const int splits = p.splits;
  const float* po = p.part_o + (long long)h * splits * kD;
  const float2* pml = p.part_ml + (long long)h * splits;
  float2 v[SMAX / 4];
#pragma unroll
  for (int j = 0; j < SMAX / 4; ++j)
    v[j] = *reinterpret_cast<const float2*>(po + (long long)min(wave + 4 * j, splits - 1) * kD + 2 * lane);
  float2 ml = {-__builtin_inff(), 0.0f};
  if (wave == 0) ml = pml[min(lane, splits - 1)];
#pragma unroll
  for (int j = 0; j < SMAX / 4; ++j)
    if (wave + 4 * j < splits) *reinterpret_cast<float2*>(&s_o[wave + 4 * j][2 * lane]) = v[j];
  if (wave == 0) merge_weights<SMAX>(ml.x, ml.y, lane, splits, s_w, s_l);
  __syncthreads();
  fold_per_dim<SMAX>(s_w, s_l, s_o, splits, reinterpret_cast<_Float16*>(p.out) + h * kD);
}

// ---------------------------------------------------------------------------
// The attention front end and attention in one launch (the decode step's
// qwen_infer.cu:626-678 chain: rmsnorm, QKV hgemv, bias, RoPE + cache append,
// then Flash-Decoding over pos + 1 rows), for in-kernel-merge split plans.
//
// Workgroup w is first a producer -- qkv_front_kernel's work for four
// rotation pairs of one head -- then a split workgroup of the attention plan
// (split c = w / H of head w % H).  With dispatch round-robin over the 8 XCDs
// (workgroup w on XCD w mod 8, probed at context creation) and H a multiple
// of 8, producer w takes head (w mod 8) + 8 ((w / 8) / 16), so head h's 16
// producers run on the XCD of its splits: every split reads its head's rotated
// Q, and the split holding the appended row that row's rotated K and V, from
// (value, tag) words the producers wrote into that XCD's L2 (as the in-kernel
// merge hands over partials).  No cache row this call writes is read from the
// cache: the appended row's loaded lanes are replaced by the tagged values,
// which are the values the producers store there, so each split's first load
// round of K and V is issued with its front-end work (behind the weight rows)
// and overlaps it.  The arithmetic is qkv_front_kernel's and the attention plan's, so every output
// (qkv, the cache row, out) has the bits of the two launches.  A split that
// still sees stale words after kFrontPolls reads (a producer ran on another
// XCD) computes its head's front end itself, in the same arithmetic; the test
// hook fh.force_local makes every split do so.
// ---------------------------------------------------------------------------
constexpr int kFrontPolls = 1 << 14;

// Replaces the appended row's K and V in tile blk (lanes whose loaded row --
// clamped to nrows - 1 -- is row `pos` of the layer).
template <int U>
__device__ __forceinline__ void patch_tile(KvTile<U>& tl, int blk, int nrows, int g, int r0, int pos,
                                           const f16x8 kpos, const f16x8 vpos) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const bool hit = r0 + min(blk + 4 * u + g, nrows - 1) == pos;
    tl.k[u] = hit ? kpos : tl.k[u];
    tl.v[u] = hit ? vpos : tl.v[u];
  }
}

template <int NJ, bool kBiasWords, int U, int SMAX, int D>
__global__ __launch_bounds__(256) void qkv_attention_kernel(QkvFrontParams f, AttnParams p, FrontHandoff fh) {
  constexpr int NW = 4;
  constexpr int kStep = NW * 4 * U;
  __shared__ ScanLds<NW> slds;
  __shared__ unsigned long long s_need[2];
  __shared__ float s_local[3][kD];   // the head's rotated Q, K and V values for the waves
  __shared__ int s_flag;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4;
  const int t = lane & 15;
  const int H = p.num_heads;
  const int w = blockIdx.x;
  const float tagf = __uint_as_float(p.tag);
  const int pos = p.seqlen - 1;
  if (tid == 0) s_flag = 0;

  // Attention role: split c of head ha.  Its first load round (rows below pos
  // are not written by this call) goes out behind the producer's weight rows,
  // so the front end's bytes are not queued behind the split's.
  const bool att = w < p.splits * H;
  const int ha = w % H, c = w / H;
  const int r0 = c * p.rows_per_split;
  const int nrows = att ? min(p.seqlen - r0, p.rows_per_split) : 0;
  const bool has_pos = r0 + nrows - 1 == pos;              // the head's last split
  const long long off = (long long)ha * p.head_stride + (long long)(att ? r0 : 0) * p.row_stride;
  const char* kbase = reinterpret_cast<const char*>(p.k + off);
  const char* vbase = reinterpret_cast<const char*>(p.v + off);
  const unsigned row_bytes = (unsigned)(p.row_stride * 2);
  const int blk0 = wave * 4 * U;
  KvTile<U> tl[D];
  // Every wave issues all D tiles, with rows clamped into its range (a
  // workgroup without a split reads row 0 of head ha): loads on both sides of
  // a branch would make the compiler's waits for the weight rows count only
  // the loads of the shorter side, and so also wait for these.  Tiles past the
  // range are not consumed.
  auto first_round = [&]() {
#pragma unroll
    for (int d = 0; d < D; ++d)
      load_tile<U>(tl[d], kbase, vbase, row_bytes, blk0 + d * kStep, max(nrows, 1), g, t);
  };

  // Producer role: four rotation pairs of head hp, then their tagged words.
  if (w >= H * 16) {
    first_round();
    __builtin_amdgcn_sched_barrier(0);
  } else {
    const int j = w >> 3;
    const int hp = (w & 7) + 8 * (j >> 4);
    const int i = 4 * (j & 15) + wave;
    const FrontPair o = qkv_front_pair<NJ, kBiasWords>(f, hp, i, lane, first_round);
    if (lane == 0) {
      float2* ft = fh.ftag + (long long)hp * 3 * kD;
      ft[i] = float2{(float)o.q1, tagf};
      ft[i + 64] = float2{(float)o.q2, tagf};
      ft[kD + i] = float2{(float)o.kr1, tagf};
      ft[kD + i + 64] = float2{(float)o.kr2, tagf};
      ft[2 * kD + i] = float2{(float)o.v1, tagf};
      ft[2 * kD + i + 64] = float2{(float)o.v2, tagf};
    }
  }
  if (!att) return;

  // The head's rotated Q and, in the split holding the appended row, that
  // row's rotated K and V, from the tagged words into s_local.  Wave 0 polls
  // (lane l: the words of dims 2l and 2l + 1); the other waves wait at the
  // barrier, so the workgroup goes on as soon as one read sees the words
  // (with every wave polling, the last of four reads in flight decided).
  if (wave == 0 && !fh.force_local) {
    const f32x4* fq = reinterpret_cast<const f32x4*>(fh.ftag + (long long)ha * 3 * kD) + lane;
    bool seen = false;
    for (int poll = 0; poll < kFrontPolls; ++poll) {
      // The loop stores nothing to memory, so without a compiler barrier the
      // loads would be hoisted out of it and read once.
      __asm__ volatile("" ::: "memory");
      f32x4 r[3];
      r[0] = __builtin_nontemporal_load(fq);
      if (has_pos) {
        r[1] = __builtin_nontemporal_load(fq + kD / 2);
        r[2] = __builtin_nontemporal_load(fq + kD);
      }
      bool ok = tag_ok(r[0][1], p.tag) && tag_ok(r[0][3], p.tag);
      if (has_pos)
        ok = ok && tag_ok(r[1][1], p.tag) && tag_ok(r[1][3], p.tag) && tag_ok(r[2][1], p.tag) &&
             tag_ok(r[2][3], p.tag);
      if (!__builtin_amdgcn_ballot_w64(!ok)) {
        s_local[0][2 * lane] = r[0][0];
        s_local[0][2 * lane + 1] = r[0][2];
        if (has_pos) {
#pragma unroll
          for (int j = 1; j < 3; ++j) {
            s_local[j][2 * lane] = r[j][0];
            s_local[j][2 * lane + 1] = r[j][2];
          }
        }
        seen = true;
        break;
      }
    }
    if (!seen && lane == 0) s_flag = 1;
  }
  if (fh.force_local && tid == 0) s_flag = 1;
  __syncthreads();
  if (s_flag && tid == 0 && !fh.force_local)   // a miss, counted (the hook's are not)
    __hip_atomic_fetch_add(p.xcnt + ha * kXCounterStride + kXStatFrontMisses, 1u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  if (s_flag) {
    // The head's front end here (every pair, no stores), wave w taking pairs
    // w, w + 4, ...; the same arithmetic, so the same values.
    for (int i = wave; i < 64; i += NW) {
      const FrontPair o = qkv_front_pair<NJ, kBiasWords, false>(f, ha, i, lane);
      if (lane == 0) {
        s_local[0][i] = (float)o.q1;
        s_local[0][i + 64] = (float)o.q2;
        s_local[1][i] = (float)o.kr1;
        s_local[1][i + 64] = (float)o.kr2;
        s_local[2][i] = (float)o.v1;
        s_local[2][i + 64] = (float)o.v2;
      }
    }
    __syncthreads();
  }
  // This lane's chunks (dims 8t .. 8t + 7).
  f16x8 qv, kpos, vpos;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    qv[e] = (_Float16)s_local[0][8 * t + e];
    kpos[e] = (_Float16)s_local[1][8 * t + e];
    vpos[e] = (_Float16)s_local[2][8 * t + e];
  }

  // The split's scan: scan_rows' tiles in its order, the first round already
  // loaded, the appended row's lanes replaced.
  GroupState st;
  init_state(st);
  if (blk0 < nrows) {
    for (int blk = blk0;; ) {
      if (has_pos) {
#pragma unroll
        for (int d = 0; d < D; ++d) patch_tile<U>(tl[d], blk + d * kStep, nrows, g, r0, pos, kpos, vpos);
      }
#pragma unroll
      for (int d = 0; d < D; ++d)
        if (d == 0 || blk + d * kStep < nrows) consume_tile<U>(st, tl[d], blk + d * kStep, nrows, g, qv, p.scale_log2);
      blk += kStep * D;
      if (blk >= nrows) break;
#pragma unroll
      for (int d = 0; d < D; ++d)
        if (d == 0 || blk + d * kStep < nrows) load_tile<U>(tl[d], kbase, vbase, row_bytes, blk + d * kStep, nrows, g, t);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  float M, L, O;
  fold_waves<NW>(st, slds, M, L, O);
  xmerge_finish<U, SMAX, D, NW, false>(p, ha, c, qv, M, L, O, slds, s_need);
}

}  // namespace

template <int NW, bool kSplit>
static void launch_scan(const AttnParams& p, int rows_per_tile, int depth, dim3 grid, hipStream_t stream) {
  if constexpr (NW == 4 && kSplit) {   // deeper load rounds: split plans of 4-wave workgroups
    if (depth == 0) {
      if (rows_per_tile == 4)
        hipLaunchKernelGGL((decode_attention_scan_kernel<4, 4, true, false, 0>), grid, dim3(256), 0, stream, p);
      else
        hipLaunchKernelGGL((decode_attention_scan_kernel<4, 2, true, false, 0>), grid, dim3(256), 0, stream, p);
      return;
    }
    if (depth == 4) {
      if (rows_per_tile == 4)
        hipLaunchKernelGGL((decode_attention_scan_kernel<4, 4, true, false, 4>), grid, dim3(256), 0, stream, p);
      else
        hipLaunchKernelGGL((decode_attention_scan_kernel<4, 2, true, false, 4>), grid, dim3(256), 0, stream, p);
      return;
    }
    if (depth == 2) {
      if (rows_per_tile == 4)
        hipLaunchKernelGGL((decode_attention_scan_kernel<4, 4, true, false, 2>), grid, dim3(256), 0, stream, p);
      else
        hipLaunchKernelGGL((decode_attention_scan_kernel<4, 2, true, false, 2>), grid, dim3(256), 0, stream, p);
      return;
    }
  }
  switch (rows_per_tile) {
    case 4:
      hipLaunchKernelGGL((decode_attention_scan_kernel<NW, 4, kSplit>), grid, dim3(NW * 64), 0, stream, p);
      break;
    default:
      hipLaunchKernelGGL((decode_attention_scan_kernel<NW, 2, kSplit>), grid, dim3(NW * 64), 0, stream, p);
      break;
  }
}

template <int SMAX, int D>
static void launch_xmerge_d(const AttnParams& p, int rows_per_tile, dim3 grid, hipStream_t stream) {
  if (rows_per_tile == 4)
    hipLaunchKernelGGL((decode_attention_xmerge_kernel<4, SMAX, D>), grid, dim3(kMergeThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((decode_attention_xmerge_kernel<2, SMAX, D>), grid, dim3(kMergeThreads), 0, stream, p);
}

// Interleaved-block split plans merged in the kernel: NW waves, U rows per tile
// (D: 1, or 0 for the rolling pipeline).
template <int SMAX, int D>
static void launch_xmerge_inter(const AttnParams& p, int waves, int rows_per_tile, dim3 grid,
                                hipStream_t stream) {
  if (waves == 8 && rows_per_tile == 2)
    hipLaunchKernelGGL((decode_attention_xmerge_kernel<2, SMAX, D, 8, true>), grid, dim3(512), 0, stream, p);
  else if (waves == 8)
    hipLaunchKernelGGL((decode_attention_xmerge_kernel<4, SMAX, D, 8, true>), grid, dim3(512), 0, stream, p);
  else if (rows_per_tile == 2)
    hipLaunchKernelGGL((decode_attention_xmerge_kernel<2, SMAX, D, 4, true>), grid, dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((decode_attention_xmerge_kernel<4, SMAX, D, 4, true>), grid, dim3(256), 0, stream, p);
}

template <int SMAX>
static void launch_xmerge(const AttnParams& p, const AttnPlan& plan, dim3 grid, hipStream_t stream) {
  if (plan.block_rows && plan.depth == 0)
    launch_xmerge_inter<SMAX, 0>(p, plan.waves, plan.rows_per_tile, grid, stream);
  else if (plan.block_rows)
    launch_xmerge_inter<SMAX, 1>(p, plan.waves, plan.rows_per_tile, grid, stream);
  else if (plan.depth == 0)
    launch_xmerge_d<SMAX, 0>(p, plan.rows_per_tile, grid, stream);
  else if (plan.depth == 4)
    launch_xmerge_d<SMAX, 4>(p, plan.rows_per_tile, grid, stream);
  else if (plan.depth == 2)
    launch_xmerge_d<SMAX, 2>(p, plan.rows_per_tile, grid, stream);
  else
    launch_xmerge_d<SMAX, 1>(p, plan.rows_per_tile, grid, stream);
}

// Scan-only launch of an interleaved-block split plan (D: 1, or 0 rolling).
template <int D>
static void launch_scan_inter(const AttnParams& p, int waves, int rows_per_tile, dim3 grid,
                              hipStream_t stream) {
  if (waves == 8 && rows_per_tile == 2)
    hipLaunchKernelGGL((decode_attention_scan_kernel<8, 2, true, false, D, true>), grid, dim3(512), 0, stream, p);
  else if (waves == 8)
    hipLaunchKernelGGL((decode_attention_scan_kernel<8, 4, true, false, D, true>), grid, dim3(512), 0, stream, p);
  else if (rows_per_tile == 2)
    hipLaunchKernelGGL((decode_attention_scan_kernel<4, 2, true, false, D, true>), grid, dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((decode_attention_scan_kernel<4, 4, true, false, D, true>), grid, dim3(256), 0, stream, p);
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
  hipLaunchKernelGGL((decode_attention_merge_kernel<true>), dim3(p.num_heads, tokens),
                     dim3(kMergeThreads), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_decode_attention(const AttnParams& p, const AttnPlan& plan, hipStream_t stream,
                                   int stages) {
  if (plan.variant == 0) {
    if (stages & kStageScan) launch_scan<16, false>(p, plan.rows_per_tile, 1, dim3(p.num_heads), stream);
    return hipGetLastError();
  }
  if (plan.block_rows && (plan.block_rows != plan.waves * 4 * plan.rows_per_tile ||
                          p.block_rows != plan.block_rows ||
                          !((plan.waves == 8 || plan.waves == 4) &&
                            (plan.rows_per_tile == 2 || plan.rows_per_tile == 4))))
    return hipErrorInvalidValue;
  if (plan.xmerge) {
    if ((plan.waves != 4 && !plan.block_rows) || p.splits > kXMaxSplits || !p.xpart || !p.xcnt)
      return hipErrorInvalidValue;
    if (stages & kStageScan) {
      const dim3 grid(p.num_heads * p.splits);
      if (p.splits <= 16)
        launch_xmerge<16>(p, plan, grid, stream);
      else if (p.splits <= 32)
        launch_xmerge<32>(p, plan, grid, stream);
      else
        launch_xmerge<64>(p, plan, grid, stream);
    }
    return hipGetLastError();
  }
  if ((stages & kStageScan) && plan.block_rows) {
    if (plan.depth == 0)
      launch_scan_inter<0>(p, plan.waves, plan.rows_per_tile, dim3(p.num_heads * p.splits), stream);
    else
      launch_scan_inter<1>(p, plan.waves, plan.rows_per_tile, dim3(p.num_heads * p.splits), stream);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  } else if (stages & kStageScan) {
    const dim3 grid(p.num_heads * p.splits);
    switch (plan.waves) {
      case 16: launch_scan<16, true>(p, plan.rows_per_tile, 1, grid, stream); break;
      case 8: launch_scan<8, true>(p, plan.rows_per_tile, 1, grid, stream); break;
      default: launch_scan<4, true>(p, plan.rows_per_tile, plan.depth, grid, stream); break;
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (stages & kStageMerge) {
    const dim3 grid(p.num_heads), block(kMergeThreads);
    if (p.splits <= 16)
      hipLaunchKernelGGL(decode_attention_merge_dim_kernel<16>, grid, block, 0, stream, p);
    else if (p.splits <= 32)
      hipLaunchKernelGGL(decode_attention_merge_dim_kernel<32>, grid, block, 0, stream, p);
    else if (p.splits <= 64)
      hipLaunchKernelGGL(decode_attention_merge_dim_kernel<64>, grid, block, 0, stream, p);
    else
      hipLaunchKernelGGL(decode_attention_merge_kernel<false>, grid, block, 0, stream, p);
  }
  return hipGetLastError();
}

template <int NJ, bool kBiasWords, int SMAX>
static void launch_qkv_attention_t(const QkvFrontParams& f, const AttnParams& p, const FrontHandoff& fh,
                                   const AttnPlan& plan,
                                   dim3 grid, hipStream_t stream) {
  if (plan.rows_per_tile == 4) {
    if (plan.depth == 2)
      hipLaunchKernelGGL((qkv_attention_kernel<NJ, kBiasWords, 4, SMAX, 2>), grid, dim3(256), 0, stream, f, p, fh);
    else
      hipLaunchKernelGGL((qkv_attention_kernel<NJ, kBiasWords, 4, SMAX, 1>), grid, dim3(256), 0, stream, f, p, fh);
  } else {
    if (plan.depth == 2)
      hipLaunchKernelGGL((qkv_attention_kernel<NJ, kBiasWords, 2, SMAX, 2>), grid, dim3(256), 0, stream, f, p, fh);
    else
      hipLaunchKernelGGL((qkv_attention_kernel<NJ, kBiasWords, 2, SMAX, 1>), grid, dim3(256), 0, stream, f, p, fh);
  }
}

hipError_t launch_qkv_attention(const QkvFrontParams& f, const AttnParams& p, const FrontHandoff& fh,
                                const AttnPlan& plan,
                                hipStream_t stream) {
  const int H = p.num_heads;
  if (!plan.xmerge || plan.variant != 1 || plan.waves != 4 || plan.block_rows || !p.xpart ||
      !p.xcnt || !fh.ftag || (H != 8 && H != 16) || f.num_heads != H || f.pos != p.seqlen - 1 ||
      (plan.depth != 1 && plan.depth != 2) || p.splits > (H == 16 ? 16 : 32) ||
      std::max(H * 16, p.splits * H) > p.num_cus)
    return hipErrorInvalidValue;
  const dim3 grid(std::max(H * 16, p.splits * H));
  const bool words = (reinterpret_cast<uintptr_t>(f.bias) & 3u) == 0;
  if (H == 16) {
    if (words) launch_qkv_attention_t<4, true, 16>(f, p, fh, plan, grid, stream);
    else launch_qkv_attention_t<4, false, 16>(f, p, fh, plan, grid, stream);
  } else {
    if (words) launch_qkv_attention_t<2, true, 32>(f, p, fh, plan, grid, stream);
    else launch_qkv_attention_t<2, false, 32>(f, p, fh, plan, grid, stream);
  }
  return hipGetLastError();
}

namespace {
__global__ void xcd_probe_kernel(unsigned* out) {
  unsigned id;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(id));
  if (threadIdx.x == 0) out[blockIdx.x] = id;
}
}  // namespace

hipError_t launch_xcd_probe(unsigned* out, int grid, hipStream_t stream) {
  hipLaunchKernelGGL(xcd_probe_kernel, dim3(grid), dim3(64), 0, stream, out);
  return hipGetLastError();
}

}  // namespace qd
