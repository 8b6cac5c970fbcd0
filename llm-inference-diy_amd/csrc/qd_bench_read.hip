// Read ceiling of the decode-attention workload (libqdiy_bench.so): a kernel
// that only reads what a qd_decode_attention call must read -- one layer's K
// and V rows -- in the same launch shape as the split scan (256 workgroups of
// 256 threads at 16 heads on 256 CUs), with the same 16-byte non-temporal
// loads, rotating over the same layers.  It does no arithmetic beyond an XOR
// fold, so its time per launch is what the box gives one kernel streaming
// those bytes: the ceiling the attention call is measured against.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Workgroup w reads units [w * per_wg, (w + 1) * per_wg) of 16 bytes of K and
// of V; each thread keeps U units of each in flight, all issued before any is
// folded.  The fold feeds a store that never happens for real data (the
// sentinel would need an exact 128-bit XOR match), so no load is dead code.
template <int U>
__global__ __launch_bounds__(256) void read_ceiling_kernel(const u32x4* __restrict__ k,
                                                           const u32x4* __restrict__ v,
                                                           unsigned per_wg, u32x4* sink) {
  const size_t base = (size_t)blockIdx.x * per_wg;
  const u32x4* kb = k + base;
  const u32x4* vb = v + base;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (unsigned i = threadIdx.x; i < per_wg; i += 256u * U) {
    u32x4 a[U], b[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const unsigned j = min(i + 256u * u, per_wg - 1u);
      a[u] = __builtin_nontemporal_load(kb + j);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const unsigned j = min(i + 256u * u, per_wg - 1u);
      b[u] = __builtin_nontemporal_load(vb + j);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= a[u] ^ b[u];
  }
  if (acc.x == 0x9E3779B9u && acc.y == 0x7F4A7C15u && acc.z == 0x85EBCA6Bu && acc.w == 0xC2B2AE35u)
    sink[blockIdx.x] = acc;
}

// Read-ceiling sweep: the same bytes (one layer's K and V: `rows` rows of
// row_units 16-byte units each) read by kernels of other launch shapes, to find
// what any one-launch design reading them could reach.  NT threads per
// workgroup, U 16-byte loads per lane per stream (K and V) issued before any is
// folded (2 * U * 16 * 64 bytes in flight per wave), `grid` workgroups.
//   kPattern 0: workgroup w reads a contiguous 1/grid of each stream;
//   kPattern 1: the scan kernel's per-head slices -- workgroup (split c, head h)
//     with blockIdx.x = c * heads + h reads the 256-byte slice h of rows
//     [c * rows / splits, ...), four rows per wave instruction (lane l: row
//     4u + l / 16, bytes 16 (l % 16) of the slice);
//   kPattern 2: grid-strided chunks -- round i of workgroup w reads chunk
//     w + grid * i of NT * U units, so the whole grid reads one contiguous
//     region of each stream per round;
//   kPattern 3: per-head slices as in kPattern 1, but the rows in blocks of
//     B = 4 U NT / 64 (one load round of the workgroup) dealt to the splits in
//     turn: split c reads blocks c, c + splits, ..., so at any time the grid
//     reads one contiguous run of rows, as in kPattern 2;
//   kPattern 4, 5, 6: workgroups over groups of 4, 8 or 16 heads (HPW) --
//     workgroup (split c, head group g) with blockIdx.x = c * (heads / HPW) + g
//     reads the HPW * 256 contiguous bytes of group g in rows [c * rows /
//     splits, ...); every wave instruction reads 1 KB of one row (four heads'
//     slices), the workgroup's waves covering a row's HPW / 4 such pieces;
//   kPattern 7: kPattern 3's rows and slices, each wave's next tile in flight
//     while it folds one (the load order of the rolling attention plans).
// The loads of read_sweep_kernel: returns the XOR fold of every unit read.
template <int NT, int U, int kPattern>
__device__ __forceinline__ u32x4 sweep_body(const u32x4* __restrict__ k, const u32x4* __restrict__ v,
                                            unsigned total_units, unsigned row_units, int heads) {
  u32x4 acc = {0u, 0u, 0u, 0u};
  const unsigned tid = threadIdx.x;
  if constexpr (kPattern == 0) {
    const unsigned per_wg = total_units / gridDim.x;
    const unsigned base = blockIdx.x * per_wg;
    for (unsigned i = tid; i < per_wg; i += NT * U) {
      u32x4 a[U], b[U];
#pragma unroll
      for (int u = 0; u < U; ++u) a[u] = __builtin_nontemporal_load(k + base + min(i + NT * u, per_wg - 1u));
#pragma unroll
      for (int u = 0; u < U; ++u) b[u] = __builtin_nontemporal_load(v + base + min(i + NT * u, per_wg - 1u));
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < U; ++u) acc ^= a[u] ^ b[u];
    }
  } else if constexpr (kPattern == 1) {
    const unsigned splits = gridDim.x / heads;
    const unsigned h = blockIdx.x % heads, c = blockIdx.x / heads;
    const unsigned rows = total_units / row_units;
    const unsigned rps = rows / splits;
    const unsigned wave = tid >> 6, lane = tid & 63;
    const unsigned col = h * 16u + (lane & 15u);
    const unsigned r0 = c * rps;
    constexpr unsigned kWaves = NT / 64;
    for (unsigned blk = wave * 4u * U; blk < rps; blk += kWaves * 4u * U) {
      u32x4 a[U], b[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const unsigned r = r0 + min(blk + 4u * u + (lane >> 4), rps - 1u);
        a[u] = __builtin_nontemporal_load(k + r * row_units + col);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const unsigned r = r0 + min(blk + 4u * u + (lane >> 4), rps - 1u);
        b[u] = __builtin_nontemporal_load(v + r * row_units + col);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < U; ++u) acc ^= a[u] ^ b[u];
    }
  } else if constexpr (kPattern == 3) {
    const unsigned splits = gridDim.x / heads;
    const unsigned h = blockIdx.x % heads, c = blockIdx.x / heads;
    const unsigned rows = total_units / row_units;
    const unsigned wave = tid >> 6, lane = tid & 63;
    const unsigned col = h * 16u + (lane & 15u);
    constexpr unsigned kBlock = (NT / 64) * 4u * U;
    for (unsigned b0 = c * kBlock; b0 < rows; b0 += splits * kBlock) {
      const unsigned rb = b0 + wave * 4u * U + (lane >> 4);
      u32x4 a[U], b[U];
#pragma unroll
      for (int u = 0; u < U; ++u) a[u] = __builtin_nontemporal_load(k + min(rb + 4u * u, rows - 1u) * row_units + col);
#pragma unroll
      for (int u = 0; u < U; ++u) b[u] = __builtin_nontemporal_load(v + min(rb + 4u * u, rows - 1u) * row_units + col);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < U; ++u) acc ^= a[u] ^ b[u];
    }
  } else if constexpr (kPattern == 7) {
    // kPattern 3's rows and slices, each wave keeping its next tile's loads in
    // flight while it folds one (rolling, as the attention plans of 2-row
    // tiles load).  Tiles of a wave: rows b0 + wave * 4U + 4u + lane / 16 of
    // blocks b0 = (c + splits * i) * kBlock.
    const unsigned splits = gridDim.x / heads;
    const unsigned h = blockIdx.x % heads, c = blockIdx.x / heads;
    const unsigned rows = total_units / row_units;
    const unsigned wave = tid >> 6, lane = tid & 63;
    const unsigned col = h * 16u + (lane & 15u);
    constexpr unsigned kBlock = (NT / 64) * 4u * U;
    const unsigned nblk = (rows + kBlock - 1) / kBlock;
    const unsigned n = nblk > c ? (nblk - 1 - c) / splits + 1 : 0;   // this split's blocks
    auto load = [&](unsigned i, u32x4 (&a)[U], u32x4 (&b)[U]) {
      const unsigned rb = (c + splits * i) * kBlock + wave * 4u * U + (lane >> 4);
#pragma unroll
      for (int u = 0; u < U; ++u) a[u] = __builtin_nontemporal_load(k + min(rb + 4u * u, rows - 1u) * row_units + col);
#pragma unroll
      for (int u = 0; u < U; ++u) b[u] = __builtin_nontemporal_load(v + min(rb + 4u * u, rows - 1u) * row_units + col);
    };
    auto fold = [&](const u32x4 (&a)[U], const u32x4 (&b)[U]) {
#pragma unroll
      for (int u = 0; u < U; ++u) acc ^= a[u] ^ b[u];
    };
    if (n > 0) {
      u32x4 a0[U], b0[U], a1[U], b1[U];
      load(0, a0, b0);
      unsigned i = 0;
      for (; i + 2 < n; i += 2) {
        load(i + 1, a1, b1);
        __builtin_amdgcn_sched_barrier(0);
        fold(a0, b0);
        load(i + 2, a0, b0);
        __builtin_amdgcn_sched_barrier(0);
        fold(a1, b1);
      }
      if (i + 1 < n) {
        load(i + 1, a1, b1);
        __builtin_amdgcn_sched_barrier(0);
        fold(a0, b0);
        fold(a1, b1);
      } else {
        fold(a0, b0);
      }
    }
  } else if constexpr (kPattern >= 4) {
    constexpr unsigned kHpw = kPattern == 4 ? 4u : kPattern == 5 ? 8u : 16u;
    constexpr unsigned kPieces = kHpw / 4;                 // 1 KB pieces per row
    static_assert(NT / 64 >= kPieces, "a workgroup covers at least one row");
    constexpr unsigned kRowsPerLoad = (NT / 64) / kPieces;
    const unsigned groups = heads / kHpw;
    const unsigned splits = gridDim.x / groups;
    const unsigned g = blockIdx.x % groups, c = blockIdx.x / groups;
    const unsigned rows = total_units / row_units;
    const unsigned rps = rows / splits;
    const unsigned wave = tid >> 6, lane = tid & 63;
    const unsigned col = g * (kHpw * 16u) + (wave % kPieces) * 64u + lane;
    const unsigned r0 = c * rps;
    for (unsigned r = wave / kPieces; r < rps; r += kRowsPerLoad * U) {
      u32x4 a[U], b[U];
#pragma unroll
      for (int u = 0; u < U; ++u) a[u] = __builtin_nontemporal_load(k + (r0 + min(r + kRowsPerLoad * u, rps - 1u)) * row_units + col);
#pragma unroll
      for (int u = 0; u < U; ++u) b[u] = __builtin_nontemporal_load(v + (r0 + min(r + kRowsPerLoad * u, rps - 1u)) * row_units + col);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < U; ++u) acc ^= a[u] ^ b[u];
    }
  } else {
    constexpr unsigned kChunk = NT * U;
    const unsigned chunks = total_units / kChunk;
    for (unsigned ch = blockIdx.x; ch < chunks; ch += gridDim.x) {
      const unsigned base = ch * kChunk + tid;
      u32x4 a[U], b[U];
#pragma unroll
      for (int u = 0; u < U; ++u) a[u] = __builtin_nontemporal_load(k + base + NT * u);
#pragma unroll
      for (int u = 0; u < U; ++u) b[u] = __builtin_nontemporal_load(v + base + NT * u);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < U; ++u) acc ^= a[u] ^ b[u];
    }
  }
  return acc;
}

template <int NT, int U, int kPattern>
__global__ __launch_bounds__(NT) void read_sweep_kernel(const u32x4* __restrict__ k,
                                                        const u32x4* __restrict__ v,
                                                        unsigned total_units, unsigned row_units,
                                                        int heads, u32x4* sink) {
  const u32x4 acc = sweep_body<NT, U, kPattern>(k, v, total_units, row_units, heads);
  if (acc.x == 0x9E3779B9u && acc.y == 0x7F4A7C15u && acc.z == 0x85EBCA6Bu && acc.w == 0xC2B2AE35u)
    sink[blockIdx.x] = acc;
}

// Read-and-merge floor: a read-sweep kernel whose workgroups then hand a
// 130-word partial (a stand-in value per thread, derived from the loaded
// bytes) to one merging workgroup per group, as the in-kernel merge of a split
// plan does -- so its time per launch is what any design that reads the bytes
// once and folds split partials in the same launch could reach with that
// read pattern.  Workgroup w belongs to hand-off group w % 16 (with
// round-robin dispatch over 8 XCDs, one XCD per group) as split w / 16; the
// group's last split merges.  Each other split stores its words as (value,
// tag) 8-byte words, waits for the stores to be acknowledged and ends; the
// merger's waves 0 and 1 (dim = thread) read every other split's word of
// their dim with non-temporal loads until all carry this launch's tag (at
// most kFloorPolls reads; a merger that gives up counts itself in *stale),
// add them to their own value and store the sum.  No atomics and no fences on
// the path, as in the product's in-kernel merge.
constexpr int kFloorGroups = 16;
constexpr int kFloorMaxSplits = 64;
constexpr int kFloorSlotWords = 144;
constexpr int kFloorPolls = 1 << 14;

// The merging waves' read of one group's other splits (SMAX - 1 at most):
// lane tid's word of every slot, clamped loads issued before any is used (a
// clamped duplicate is loaded but not counted); returns whether every counted
// word carries `tag` in every lane of the wave, and the sum in *sum.
template <int SMAX>
__device__ __forceinline__ bool poll_slots(const f32x2* gw, unsigned tid, unsigned others, unsigned tag,
                                           float own, float* sum) {
  const unsigned last = others ? others - 1 : 0;
  f32x2 w[SMAX - 1];
#pragma unroll
  for (unsigned cc = 0; cc < SMAX - 1; ++cc)
    w[cc] = __builtin_nontemporal_load(gw + min(cc, last) * kFloorSlotWords + tid);
  bool ok = true;
  float s = own;
#pragma unroll
  for (unsigned cc = 0; cc < SMAX - 1; ++cc) {
    const bool on = cc < others;
    ok &= !on || __float_as_uint(w[cc][1]) == tag;
    s += on ? w[cc][0] : 0.0f;
  }
  *sum = s;
  return __builtin_amdgcn_ballot_w64(!ok) == 0ull;
}

template <int NT, int U, int kPattern, int SMAX>
__global__ __launch_bounds__(NT) void read_merge_kernel(const u32x4* __restrict__ k,
                                                        const u32x4* __restrict__ v,
                                                        unsigned total_units, unsigned row_units,
                                                        int heads, float2* slots, float* out,
                                                        unsigned tag, unsigned* stale) {
  const u32x4 acc = sweep_body<NT, U, kPattern>(k, v, total_units, row_units, heads);
  const unsigned tid = threadIdx.x;
  const unsigned g = blockIdx.x % kFloorGroups, c = blockIdx.x / kFloorGroups;
  const unsigned splits = gridDim.x / kFloorGroups;
  const float tagf = __uint_as_float(tag);
  const float val = (float)((acc.x ^ acc.y ^ acc.z ^ acc.w ^ tid) & 0xffffu);
  float2* gs = slots + (size_t)g * kFloorMaxSplits * kFloorSlotWords;
  if (c + 1 != splits) {
    if (tid < 130) gs[c * kFloorSlotWords + tid] = float2{val, tagf};
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    return;
  }
  if (tid >= 128) return;
  const f32x2* gw = reinterpret_cast<const f32x2*>(gs);
  float sum = val;
  bool fresh = splits == 1;
  for (int r = 0; r < kFloorPolls && !fresh; ++r) {
    asm volatile("" ::: "memory");   // the loads stay in the loop
    fresh = poll_slots<SMAX>(gw, tid, splits - 1, tag, val, &sum);
  }
  if (!fresh && (tid & 63) == 0) atomicAdd(stale, 1u);
  out[g * 128 + tid] = sum;
}

typedef void (*SweepKernel)(const u32x4*, const u32x4*, unsigned, unsigned, int, u32x4*);

// The sweep's shapes: (threads per workgroup, loads per lane per stream).
typedef void (*MergeKernel)(const u32x4*, const u32x4*, unsigned, unsigned, int, float2*, float*,
                            unsigned, unsigned*);

struct SweepShape {
  int nt, u;
  SweepKernel fn[8];
  MergeKernel merge[3][8];   // [SMAX 16, 32, 64][pattern]
};

#define QD_MERGE_ROW(NT, U, S)                                                                 \
  { read_merge_kernel<NT, U, 0, S>, read_merge_kernel<NT, U, 1, S>, read_merge_kernel<NT, U, 2, S>,   \
    read_merge_kernel<NT, U, 3, S>, read_merge_kernel<NT, U, 4, S>, read_merge_kernel<NT, U, 5, S>,   \
    read_merge_kernel<NT, U, 6, S>, read_merge_kernel<NT, U, 7, S> }

#define QD_SWEEP_SHAPE(NT, U)                                                               \
  SweepShape {                                                                              \
    NT, U, { read_sweep_kernel<NT, U, 0>, read_sweep_kernel<NT, U, 1>, read_sweep_kernel<NT, U, 2>, \
             read_sweep_kernel<NT, U, 3>, read_sweep_kernel<NT, U, 4>, read_sweep_kernel<NT, U, 5>, \
             read_sweep_kernel<NT, U, 6>, read_sweep_kernel<NT, U, 7> },                                                   \
    { QD_MERGE_ROW(NT, U, 16), QD_MERGE_ROW(NT, U, 32), QD_MERGE_ROW(NT, U, 64) }            \
  }

const SweepShape kSweepShapes[] = {
    QD_SWEEP_SHAPE(256, 2),  QD_SWEEP_SHAPE(256, 4),  QD_SWEEP_SHAPE(256, 8),
    QD_SWEEP_SHAPE(256, 16), QD_SWEEP_SHAPE(512, 2),  QD_SWEEP_SHAPE(512, 4),
    QD_SWEEP_SHAPE(512, 8),  QD_SWEEP_SHAPE(512, 16), QD_SWEEP_SHAPE(1024, 2),
    QD_SWEEP_SHAPE(1024, 4), QD_SWEEP_SHAPE(1024, 8),
};
#undef QD_SWEEP_SHAPE
#undef QD_MERGE_ROW

// Does nothing: back-to-back launches of it time the dispatch floor, the cost
// any dependent kernel (such as a separate merge launch) pays before its work.
__global__ __launch_bounds__(256) void empty_kernel() {}


// The sweep kernels' shape for (threads, loads), or null for arguments outside
// what read_sweep_kernel's pattern covers (see qd_bench_read_sweep).
const SweepShape* sweep_shape(int rows, int row_bytes, int heads, int n_layers, int threads,
                              int loads, int pattern, int grid, int iters) {
  if (rows < 1 || row_bytes < 16 || row_bytes % 16 || heads < 1 || n_layers < 1 || grid < 1 ||
      grid > 65536 || iters < 0 || pattern < 0 || pattern > 7)
    return nullptr;
  const long long units = (long long)rows * (row_bytes / 16);
  if (units > 0xFFFFFFFFLL) return nullptr;
  const SweepShape* shape = nullptr;
  for (const SweepShape& s : kSweepShapes)
    if (s.nt == threads && s.u == loads) shape = &s;
  if (!shape) return nullptr;
  if (pattern == 0 && units % grid) return nullptr;
  if (pattern == 1 && (grid % heads || rows % (grid / heads) || row_bytes / 16 != 16 * heads)) return nullptr;
  if (pattern == 2 && units % ((long long)threads * loads)) return nullptr;
  if ((pattern == 3 || pattern == 7) && (grid % heads || row_bytes / 16 != 16 * heads)) return nullptr;
  if (pattern >= 4) {
    const int hpw = pattern == 4 ? 4 : pattern == 5 ? 8 : 16;
    if (heads % hpw || threads / 64 < hpw / 4 || row_bytes / 16 != 16 * heads) return nullptr;
    const int groups = heads / hpw;
    if (grid % groups || rows % (grid / groups)) return nullptr;
  }
  return shape;
}

}  // namespace

extern "C" {

// `iters` launches, launch i reading layer i % n_layers: `bytes` of K at
// k + layer * layer_stride_bytes and the same of V.  bytes must be a multiple
// of 16 * grid; sink holds grid 16-byte slots.  Asynchronous on `stream`.
int qd_bench_read_ceiling(const void* k, const void* v, long long layer_stride_bytes,
                          long long bytes, int n_layers, int grid, int iters, void* sink,
                          hipStream_t stream) {
  if (!k || !v || !sink || n_layers < 1 || grid < 1 || iters < 0 || bytes <= 0 ||
      bytes % (16LL * grid) != 0 || bytes / 16 / grid > 0xFFFFFFFFLL)
    return 1;
  const unsigned per_wg = (unsigned)(bytes / 16 / grid);
  for (int it = 0; it < iters; ++it) {
    const long long off = (long long)(it % n_layers) * layer_stride_bytes;
    hipLaunchKernelGGL(read_ceiling_kernel<4>, dim3(grid), dim3(256), 0, stream,
                       reinterpret_cast<const u32x4*>(static_cast<const char*>(k) + off),
                       reinterpret_cast<const u32x4*>(static_cast<const char*>(v) + off), per_wg,
                       static_cast<u32x4*>(sink));
    if (hipGetLastError() != hipSuccess) return 2;
  }
  return 0;
}

// `iters` launches of an empty kernel of `grid` workgroups of 256 threads.
int qd_bench_empty(int grid, int iters, hipStream_t stream) {
  if (grid < 1 || iters < 0) return 1;
  for (int it = 0; it < iters; ++it) {
    hipLaunchKernelGGL(empty_kernel, dim3(grid), dim3(256), 0, stream);
    if (hipGetLastError() != hipSuccess) return 2;
  }
  return 0;
}


// `iters` launches of one read-sweep kernel, launch i reading layer
// i % n_layers (`rows` rows of row_bytes bytes of K at k + layer *
// layer_stride_bytes, and of V).  threads in {256, 512, 1024}, loads in
// {2, 4, 8, 16} (not 16 with 1024 threads), pattern 0-7 (read_sweep_kernel),
// grid workgroups; patterns 1, 3 and 7 need grid a multiple of heads and 16
// units per head in a row (pattern 1 also rows a multiple of grid / heads;
// patterns 4-6 heads a multiple of 4, 8, 16 and rows of grid / (heads / 4, 8,
// 16) splits),
// patterns 0 and 2 a whole number of units per workgroup or chunk.  Returns 0, or 1 for arguments outside those.
int qd_bench_read_sweep(const void* k, const void* v, long long layer_stride_bytes, int rows,
                        int row_bytes, int heads, int n_layers, int threads, int loads,
                        int pattern, int grid, int iters, void* sink, hipStream_t stream) {
  if (!k || !v || !sink) return 1;
  const SweepShape* shape = sweep_shape(rows, row_bytes, heads, n_layers, threads, loads, pattern, grid, iters);
  if (!shape) return 1;
  const long long units = (long long)rows * (row_bytes / 16);
  for (int it = 0; it < iters; ++it) {
    const long long off = (long long)(it % n_layers) * layer_stride_bytes;
    hipLaunchKernelGGL(shape->fn[pattern], dim3(grid), dim3(threads), 0, stream,
                       reinterpret_cast<const u32x4*>(static_cast<const char*>(k) + off),
                       reinterpret_cast<const u32x4*>(static_cast<const char*>(v) + off),
                       (unsigned)units, (unsigned)(row_bytes / 16), heads, static_cast<u32x4*>(sink));
    if (hipGetLastError() != hipSuccess) return 2;
  }
  return 0;
}

// `iters` launches of one read-and-merge floor kernel (read_merge_kernel):
// the read of qd_bench_read_sweep's (threads, loads, pattern, grid) shape,
// then every workgroup's 130-word partial handed to its group's merger, which
// stores 128 sums to out[16][128] (floats).  Launch i reads layer i %
// n_layers and tags its words tag0 + i (tag0 >= 1).  slots: 16 * 64 * 144
// 8-byte words, zero before the first call (no word carries a launch's tag
// before that launch writes it); stale: one counter, incremented by each
// merging wave that gave up waiting (0 when every group's splits ran on its
// merger's XCD).  grid a multiple of 16 with at most 64 workgroups per group,
// and the sweep's constraints.  Returns 0, or 1 for arguments outside those.
int qd_bench_read_merge(const void* k, const void* v, long long layer_stride_bytes, int rows,
                        int row_bytes, int heads, int n_layers, int threads, int loads,
                        int pattern, int grid, int iters, void* slots, void* out,
                        unsigned tag0, void* stale, hipStream_t stream) {
  if (!k || !v || !slots || !out || !stale || tag0 == 0u) return 1;
  if (grid % kFloorGroups || grid / kFloorGroups > kFloorMaxSplits) return 1;
  const SweepShape* shape = sweep_shape(rows, row_bytes, heads, n_layers, threads, loads, pattern, grid, iters);
  if (!shape) return 1;
  const long long units = (long long)rows * (row_bytes / 16);
  for (int it = 0; it < iters; ++it) {
    const long long off = (long long)(it % n_layers) * layer_stride_bytes;
    const int per_group = grid / kFloorGroups;
    const int row = per_group <= 16 ? 0 : per_group <= 32 ? 1 : 2;
    hipLaunchKernelGGL(shape->merge[row][pattern], dim3(grid), dim3(threads), 0, stream,
                       reinterpret_cast<const u32x4*>(static_cast<const char*>(k) + off),
                       reinterpret_cast<const u32x4*>(static_cast<const char*>(v) + off),
                       (unsigned)units, (unsigned)(row_bytes / 16), heads,
                       static_cast<float2*>(slots), static_cast<float*>(out), tag0 + (unsigned)it,
                       static_cast<unsigned*>(stale));
    if (hipGetLastError() != hipSuccess) return 2;
  }
  return 0;
}

}  // extern "C"
