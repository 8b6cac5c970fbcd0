// Causal prefill attention on the matrix cores (gfx950 v_mfma_f32_16x16x32_f16):
// the counterpart of the reference's prompt attention, qwen_infer.cu:484-527
// (gather_q_from_qkv / gather_kv_from_cache into per-head buffers,
// flash_attn_tuned_A_kernel with the causal mask of flash_attn_causal.cuh, one
// launch per head, then scatter_interleaved_kernel), as one launch that reads
// the rotated Q rows and the KV cache where they lie.
//
// Workgroup (h, tile) takes 64 consecutive queries of head h with eight waves
// (two per SIMD, so one wave's matrix-core products can run while the other
// computes its softmax).  The waves form four key groups of two: group k takes
// the 32-key blocks k, k + 4, ..., and within a group wave w takes queries
// 32 w .. 32 w + 31 as two 16-query MFMA tiles, so every K or V^T operand read
// from LDS feeds two products.  A group's two waves load each of its blocks
// once into LDS with direct loads (global_load_lds_dwordx4: no registers, no
// LDS store instructions), where both read it, so every K/V row read from
// memory serves 64 queries.  The next block's loads go out while the current
// block is computed; the buffers alternate per block, with one workgroup
// barrier per block.  The tile's Q rows come into LDS once, for all groups.  At
// the end the four groups' softmax states of each query are folded through LDS
// by all 512 threads.
//
// The two buffers are separate LDS variables and the loop is unrolled by two,
// so every LDS access names its buffer statically: the compiler then knows that
// the direct loads into one buffer do not touch the other and does not wait for
// them before the K reads.  The transposed V reads carry no such information,
// so each block's V^T operands are read before the next block's loads are
// issued.
//
// The grid is one-dimensional and its linear index is remapped so that, with
// workgroups dealt to the 8 XCDs in turn, the tiles of a head run on one XCD
// and share its L2 copy of the head's K/V rows; within a head the latest
// tiles (the longest key ranges) start first, and a CU that finishes a short
// tile takes a long one.  Per block a wave computes, for each query tile u,
//   S^T = K Q^T    (M = 16 keys per tile, two tiles; N = 16 queries; K = 128 dims)
//   O^T += V^T P^T (M = 16 dims per tile, eight tiles; N = 16 queries; K = 32 keys)
// Transposing both products puts the query in the MFMA's column, which is the
// lane's column l % 16 of every accumulator, so each lane's softmax state
// (running max m, denominator) belongs to query l % 16 of the tile in every
// product and rescaling O needs no lane exchange.  Operand lanes:
// A[l % 16][8 (l / 16) + e], B[8 (l / 16) + e][l % 16]; accumulator
// D[4 (l / 16) + r][l % 16].
//   - K rows feed A from LDS (a lane's 8 dims are 16 contiguous bytes).  Rows
//     are 256 bytes with their 16-byte chunks swizzled: chunk q of row r sits
//     at position q ^ (r % 16), so the 16 rows of one operand read fall on
//     distinct banks.
//   - S^T's accumulator gives lane (g = l / 16, c = l % 16) the keys
//     16 t + 4 g + r of query c, which become P^T's B operand as they are: the
//     P.V product sums over its 32 keys in any order, so element e of the lane
//     stands for key pi(8 g + e) = 16 (e / 4) + 4 g + e % 4 of the block, and
//     the V^T operand is read in the same order.
//   - V^T: per dims tile, the 4 + 4 keys pi(8 g ..) of dim 16 n + c, with two
//     transposed reads (gfx950's ds_read_b64_tr_b16) of the V block as it
//     lies in LDS, its chunks swizzled by 2 (r % 4): the 4 rows x 2 chunks of
//     one transposed read fall on distinct banks.
// P is rounded to fp16 for the product (as the reference's MMA kernel does)
// and the softmax denominator sums the rounded weights, on the matrix core (an
// all-ones A operand), so each output is a weighted mean of V rows.  A query's
// reference maximum moves only when a block's maximum passes it by more than
// 2^kLazy, so weights stay below 2^kLazy (fp16 holds them with the same
// relative precision) and O is rescaled in few blocks.  Exponentials are the
// hardware's exp2.  Nothing here is bit-reproducible on the host; the exact
// prefill path (the decode kernels batched) is.
#include "qd_device.h"
#include "qd_internal.h"

namespace qd {
namespace {

constexpr int kFpQueries = 64;             // queries per workgroup
constexpr int kFpKeys = 32;                // keys per block
constexpr int kQWaves = 2;                 // waves of a key group: 32 queries each
constexpr int kQTiles = 2;                 // 16-query MFMA tiles per wave
constexpr int kKeyGroups = 4;
constexpr int kXcds = 8;                   // MI355X: workgroups are dealt to 8 XCDs in turn
constexpr int kRow = 128;                  // K and V rows in LDS: 256 bytes, 16-byte chunks swizzled
constexpr int kBlk = kFpKeys * kRow;       // halves of one group's K (or V) block
// chunk q of row r sits at position q ^ swz(r): K by r % 16 (the 16 rows of one
// operand read), V by 2 (r % 4) (the 4 rows x 2 chunks of one transposed read)
__device__ __forceinline__ int kswz(int r) { return r & 15; }
__device__ __forceinline__ int vswz(int r) { return 2 * (r & 3); }
constexpr float kLazy = 8.0f;              // log2 of the largest softmax weight before a rescale
static_assert(kQWaves * kQTiles * 16 == kFpQueries, "a key group's waves cover the workgroup's queries");
static_assert(kQWaves * 16 == kFpKeys, "a group's waves load 16 rows of each block");
// The fold hands each group's fp32 O rows (64 queries x 128 dims, 32 KB) through
// one of the four block buffers and the (m, l) pairs through the Q rows' space.
static_assert((size_t)kFpQueries * 128 * 4 == (size_t)kKeyGroups * kBlk * 2, "an O tile fills one buffer");
static_assert((size_t)kKeyGroups * 2 * kFpQueries * 4 <= (size_t)kFpQueries * kRow * 2, "(m, l) fit in the Q rows");

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 Blk[kBlk];                // one group's K or V block in LDS

__global__ __launch_bounds__(kKeyGroups * kQWaves * 64) void flash_prefill_kernel(FlashPrefillParams p) {
  __shared__ __align__(16) Blk lk0[kKeyGroups];   // buffer 0: [group]
  __shared__ __align__(16) Blk lv0[kKeyGroups];
  __shared__ __align__(16) Blk lk1[kKeyGroups];   // buffer 1
  __shared__ __align__(16) Blk lv1[kKeyGroups];
  __shared__ __align__(16) _Float16 lq[kFpQueries * kRow];   // the tile's Q rows, chunks swizzled as K's
  const int lane = threadIdx.x & 63;
  const int wave8 = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int kg = wave8 / kQWaves;                // key group: blocks kg, kg + 4, ...
  const int wave = wave8 % kQWaves;              // queries 32 wave .. 32 wave + 31
  const int c = lane & 15;
  const int g = lane >> 4;
  const int ntile = (p.tokens + kFpQueries - 1) / kFpQueries;
  const int nwg = p.num_heads * ntile;
  int pi = blockIdx.x;                          // XCD-major order: XCD x runs pi in [x nwg/8, (x+1) nwg/8)
  if (nwg % kXcds == 0) pi = (pi % kXcds) * (nwg / kXcds) + pi / kXcds;
  const int h = pi / ntile;
  const int q0 = (ntile - 1 - pi % ntile) * kFpQueries;
  const int nq = min(kFpQueries, p.tokens - q0);
  const int nkeys = p.pos0 + q0 + nq;           // keys [0, nkeys) reach the last query
  const int nblk = (nkeys + kFpKeys - 1) / kFpKeys;
  const int wq0 = 32 * wave;
  const bool active = wq0 < nq;                 // wave-uniform: the wave has queries
  const int wpos = p.pos0 + q0 + wq0;           // the wave's first query position

  // B operand of S^T for tile u: Q[q0 + wq0 + 16 u + c][32 s + 8 g .. +8],
  // read from the tile's Q rows in LDS after the first barrier.  The rows come
  // in once per workgroup (direct loads, like K: wave w moves rows 8 w ..
  // 8 w + 7); rows past the last query repeat it and their outputs are not
  // stored.
  f16x8 qb[kQTiles][4];
  int qpos[kQTiles];                            // the lane's query position in tile u
#pragma unroll
  for (int u = 0; u < kQTiles; ++u) qpos[u] = wpos + 16 * u + c;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int row = 8 * wave8 + 4 * i + (lane >> 4);
    __builtin_amdgcn_global_load_lds(p.q + (long long)(q0 + min(row, nq - 1)) * p.q_stride + h * 128 +
                                         8 * ((lane & 15) ^ kswz(row)),
                                     (__attribute__((address_space(3))) void*)&lq[(8 * wave8 + 4 * i) * kRow], 16, 0, 0);
  }

  // A group's block: 32 rows of K and of V.  Rows past nkeys repeat row
  // nkeys - 1 and are masked.  Direct loads into LDS: wave w of the group moves
  // rows 16 w .. 16 w + 15, four rows (1 KB) per instruction; lane l fills
  // position l % 16 of row l / 16 of the four, i.e. the row's chunk
  // (l % 16) ^ swz(row).  The lane's source addresses for block 0 are formed
  // once; block j adds 32 j rows, a wave-uniform offset (the 64-bit address
  // arithmetic per load and block cost as much VALU time as the matrix-core
  // products).  Only a block that reaches past the last key clamps per lane.
  const uint16_t* kbase[4];
  const uint16_t* vbase[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 16 * wave + 4 * i + (lane >> 4);
    kbase[i] = p.k + (long long)h * p.head_stride + (long long)row * p.row_stride + 8 * ((lane & 15) ^ kswz(row));
    vbase[i] = p.v + (long long)h * p.head_stride + (long long)row * p.row_stride + 8 * ((lane & 15) ^ vswz(row));
  }
  auto dload = [&](int j, Blk* lk, Blk* lv) {
    const int kb = j * kFpKeys;
    if (kb + kFpKeys <= nkeys) {                // wave-uniform: every row of the block is a key
      const long long off = (long long)kb * p.row_stride;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        __builtin_amdgcn_global_load_lds(kbase[i] + off,
                                         (__attribute__((address_space(3))) void*)&lk[kg][(16 * wave + 4 * i) * kRow],
                                         16, 0, 0);
        __builtin_amdgcn_global_load_lds(vbase[i] + off,
                                         (__attribute__((address_space(3))) void*)&lv[kg][(16 * wave + 4 * i) * kRow],
                                         16, 0, 0);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 16 * wave + 4 * i + (lane >> 4);
        const long long off = (long long)(min(kb + row, nkeys - 1) - row) * p.row_stride;
        __builtin_amdgcn_global_load_lds(kbase[i] + off,
                                         (__attribute__((address_space(3))) void*)&lk[kg][(16 * wave + 4 * i) * kRow],
                                         16, 0, 0);
        __builtin_amdgcn_global_load_lds(vbase[i] + off,
                                         (__attribute__((address_space(3))) void*)&lv[kg][(16 * wave + 4 * i) * kRow],
                                         16, 0, 0);
      }
    }
  };

  float m[kQTiles];
  f32x4 ls[kQTiles];                            // the denominator, in every element
  f32x4 o[kQTiles][8];
#pragma unroll
  for (int u = 0; u < kQTiles; ++u) {
    m[u] = -__builtin_inff();
    ls[u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int n = 0; n < 8; ++n) o[u][n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  f16x8 ones;
#pragma unroll
  for (int e = 0; e < 8; ++e) ones[e] = (_Float16)1.0f;

  // V^T operands of a block.  Within a 16-lane group, lane i's element e of a
  // transposed read is element i % 4 of the four halves lane 4 e + i / 4
  // addresses.  Lane j of group g addresses key 4 g + j / 4 (+ 16 for the
  // second read), dims 16 n + 4 (j % 4) .. +4, so lane (c, g) receives dim
  // 16 n + c of keys 4 g + e and 16 + 4 g + e: the keys pi(8 g + e) its P^T
  // operand holds.
  auto vread = [&](const Blk* lv, f16x8 (&va)[8]) {
    const int vr = 4 * g + (c >> 2);                        // key of the low read; +16 for the high one
    const _Float16* vrow = &lv[kg][vr * kRow];
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      const int q = 2 * n + ((c >> 1) & 1);                // dims 16 n + 4 (c % 4) .. +4 lie in chunk q
      const int off = 8 * (q ^ vswz(vr)) + 4 * (c & 1);
      const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(vrow + off));
      const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(vrow + 16 * kRow + off));
      va[n] = __builtin_bit_cast(f16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
  };

  // Block j from K buffer lk and the V^T operands va: the wave's online-softmax update.
  auto compute = [&](int j, const Blk* lk, const f16x8 (&va)[8]) {
    const int kb = j * kFpKeys;
    f32x4 st[kQTiles][2];
#pragma unroll
    for (int u = 0; u < kQTiles; ++u)
#pragma unroll
      for (int t = 0; t < 2; ++t) st[u][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const f16x8 ka = *reinterpret_cast<const f16x8*>(&lk[kg][(16 * t + c) * kRow + 8 * ((4 * s + g) ^ kswz(16 * t + c))]);
#pragma unroll
        for (int u = 0; u < kQTiles; ++u) st[u][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qb[u][s], st[u][t], 0, 0, 0);
      }
    if (kb + kFpKeys - 1 > wpos) {              // wave-uniform: some key is past a query
#pragma unroll
      for (int u = 0; u < kQTiles; ++u)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) st[u][t][r] = kb + 16 * t + 4 * g + r <= qpos[u] ? st[u][t][r] : -__builtin_inff();
    }
    // Each lane tests its own 8 keys per tile against the lazy bound; only when
    // some lane's keys pass it are the block maxima formed across the lanes of
    // a query (the decisions a block-wide maximum gives).
    float lm[kQTiles];
    bool grow = false;
#pragma unroll
    for (int u = 0; u < kQTiles; ++u) {
      lm[u] = fmaxf(fmaxf(fmaxf(st[u][0][0], st[u][0][1]), fmaxf(st[u][0][2], st[u][0][3])),
                    fmaxf(fmaxf(st[u][1][0], st[u][1][1]), fmaxf(st[u][1][2], st[u][1][3])));
      grow |= lm[u] * p.scale_log2 > m[u] + kLazy;   // -inf + kLazy is -inf: a first finite block grows
    }
    if (__any(grow)) {
#pragma unroll
      for (int u = 0; u < kQTiles; ++u) {
        float bm = fmaxf(lm[u], __shfl_xor(lm[u], 16));
        bm = fmaxf(bm, __shfl_xor(bm, 32)) * p.scale_log2;   // log2 units (scale > 0)
        const float mn = bm > m[u] + kLazy ? bm : m[u];
        const float alpha = mn == m[u] ? 1.0f : __builtin_amdgcn_exp2f(m[u] - mn);
        ls[u] *= alpha;
#pragma unroll
        for (int n = 0; n < 8; ++n) o[u][n] *= alpha;
        m[u] = mn;
      }
    }
#pragma unroll
    for (int u = 0; u < kQTiles; ++u) {
      const float nref = m[u] == -__builtin_inff() ? 0.0f : -m[u];   // no key yet: every weight is 0
      f16x8 pb;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        pb[e] = (_Float16)__builtin_amdgcn_exp2f(__builtin_fmaf(st[u][e / 4][e % 4], p.scale_log2, nref));
      ls[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pb, ls[u], 0, 0, 0);
#pragma unroll
      for (int n = 0; n < 8; ++n) o[u][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[n], pb, o[u][n], 0, 0, 0);
    }
  };

  // One block of this group from buffers (ck, cv) while the group's next block
  // streams into (nk, nv), which were last read before the previous barrier.
  // Each wave waits for its own direct loads (vmcnt) before the barrier that
  // hands the buffers to the group.
  auto step = [&](int j, const Blk* ck, const Blk* cv, Blk* nk, Blk* nv) {
    const bool work = active && j < nblk && j * kFpKeys <= wpos + 31;   // wave-uniform: some key reaches a query
    f16x8 va[8];
    if (work) vread(cv, va);
    if (j + kKeyGroups < nblk) dload(j + kKeyGroups, nk, nv);
    if (work) compute(j, ck, va);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  };
  const int nit = (nblk + kKeyGroups - 1) / kKeyGroups;
  if (kg < nblk) dload(kg, lk0, lv0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kQTiles; ++u)
#pragma unroll
    for (int s = 0; s < 4; ++s)
      qb[u][s] = *reinterpret_cast<const f16x8*>(&lq[(wq0 + 16 * u + c) * kRow + 8 * ((4 * s + g) ^ kswz(c))]);
  for (int it = 0; it < nit; it += 2) {
    step(kKeyGroups * it + kg, lk0, lv0, lk1, lv1);
    if (it + 1 < nit) step(kKeyGroups * (it + 1) + kg, lk1, lv1, lk0, lv0);
  }

  // Fold the four key groups' states of each query through LDS (the buffers
  // are free after the last barrier): every group writes its O rows to one of
  // the four block buffers (128 floats per query, 16-byte chunks swizzled by
  // the query: chunk q of query r at q ^ (r % 16), so the 16 queries of a write
  // fall on distinct banks) and its (m, l) to the Q rows' space; then every
  // thread folds 16 dims of one query.
  float* const fo[4] = {reinterpret_cast<float*>(&lk0[0][0]), reinterpret_cast<float*>(&lv0[0][0]),
                        reinterpret_cast<float*>(&lk1[0][0]), reinterpret_cast<float*>(&lv1[0][0])};
  float* const fml = reinterpret_cast<float*>(&lq[0]);      // [group][m, l][query]
  {
    float* dst = kg == 0 ? fo[0] : kg == 1 ? fo[1] : kg == 2 ? fo[2] : fo[3];
#pragma unroll
    for (int u = 0; u < kQTiles; ++u) {
      const int qq = wq0 + 16 * u + c;
#pragma unroll
      for (int n = 0; n < 8; ++n) *reinterpret_cast<f32x4*>(dst + qq * 128 + 4 * ((4 * n + g) ^ c)) = o[u][n];
      if (g == 0) {
        fml[kg * 2 * kFpQueries + qq] = m[u];
        fml[kg * 2 * kFpQueries + kFpQueries + qq] = ls[u][0];
      }
    }
  }
  __syncthreads();
  {
    const int qq = (int)threadIdx.x >> 3;                    // the thread's query in the tile
    const int d4 = 4 * ((int)threadIdx.x & 7);               // its first 4-dim chunk: dims 4 d4 .. 4 d4 + 15
    if (qq < nq) {
      float mk[kKeyGroups], M = -__builtin_inff();
#pragma unroll
      for (int w = 0; w < kKeyGroups; ++w) {
        mk[w] = fml[w * 2 * kFpQueries + qq];
        M = fmaxf(M, mk[w]);                                 // finite: key 0 reaches every query
      }
      float a[kKeyGroups], l = 0.0f;
#pragma unroll
      for (int w = 0; w < kKeyGroups; ++w) {
        a[w] = mk[w] == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(mk[w] - M);
        l += a[w] * fml[w * 2 * kFpQueries + kFpQueries + qq];
      }
      const float inv = 1.0f / l;
      f16x8 v[2];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f32x4 acc = a[0] * *reinterpret_cast<const f32x4*>(fo[0] + qq * 128 + 4 * ((d4 + i) ^ (qq & 15)));
#pragma unroll
        for (int w = 1; w < kKeyGroups; ++w)
          acc += a[w] * *reinterpret_cast<const f32x4*>(fo[w] + qq * 128 + 4 * ((d4 + i) ^ (qq & 15)));
#pragma unroll
        for (int r = 0; r < 4; ++r) v[i / 2][4 * (i % 2) + r] = (_Float16)(acc[r] * inv);
      }
      _Float16* orow = reinterpret_cast<_Float16*>(p.out + (long long)(q0 + qq) * p.out_stride + h * 128 + 4 * d4);
      *reinterpret_cast<f16x8*>(orow) = v[0];
      *reinterpret_cast<f16x8*>(orow + 8) = v[1];
    }
  }
}

}  // namespace

hipError_t launch_flash_prefill(const FlashPrefillParams& p, hipStream_t stream) {
  const dim3 grid(p.num_heads * ((p.tokens + kFpQueries - 1) / kFpQueries));
  hipLaunchKernelGGL(flash_prefill_kernel, grid, dim3(kKeyGroups * kQWaves * 64), 0, stream, p);
  return hipGetLastError();
}

}  // namespace qd
