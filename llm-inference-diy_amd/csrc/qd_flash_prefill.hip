// Causal prefill attention on the matrix cores (gfx950 v_mfma_f32_16x16x32_f16):
// the counterpart of the reference's prompt attention, qwen_infer.cu:484-527
// (gather_q_from_qkv / gather_kv_from_cache into per-head buffers,
// flash_attn_tuned_A_kernel with the causal mask of flash_attn_causal.cuh, one
// launch per head, then scatter_interleaved_kernel), as one launch that reads
// the rotated Q rows and the KV cache where they lie.
//
// Workgroup (h, tile) takes 64 consecutive queries of head h with eight waves
// (two per SIMD, so one wave's matrix-core products can run while the other
// computes its softmax).  The waves form two key groups of four: group k takes
// the 64-key blocks k, k + 2, ..., and within a group wave w takes queries
// 16 w .. 16 w + 15 (the MFMA's N).  A group's four waves load each of its
// blocks once into LDS with direct loads (global_load_lds_dwordx4: no
// registers, no LDS store instructions), where all four read it, so every K/V
// row read from memory serves 64 queries.  The next block's loads go out while
// the current block is computed; the LDS buffers alternate per block, with one
// workgroup barrier per block.  At the end the two groups' softmax states of
// each query are folded through LDS.
//
// The grid is one-dimensional and its linear index is remapped so that, with
// workgroups dealt to the 8 XCDs in turn, the tiles of a head run on one XCD
// and share its L2 copy of the head's K/V rows; within a head the latest
// tiles (the longest key ranges) start first, and a CU that finishes a short
// tile takes a long one.  Per block a wave computes
//   S^T = K Q^T    (M = 16 keys per tile, four tiles; N = 16 queries; K = 128 dims)
//   O^T += V^T P^T (M = 16 dims per tile, eight tiles; N = 16 queries; K = 32 keys,
//                   two halves of the block)
// Transposing both products puts the query in the MFMA's column, which is the
// lane's column l % 16 of every accumulator, so each lane's softmax state
// (running max m, denominator) belongs to query l % 16 in every product and
// rescaling O needs no lane exchange.  Operand lanes: A[l % 16][8 (l / 16) + e],
// B[8 (l / 16) + e][l % 16]; accumulator D[4 (l / 16) + r][l % 16].
//   - K rows feed A from LDS (a lane's 8 dims are 16 contiguous bytes).  Rows
//     are 256 bytes with their 16-byte chunks swizzled: chunk q of row r sits
//     at position q ^ (r % 16), so the 16 rows of one operand read fall on
//     distinct banks.
//   - S^T's accumulator gives lane (g = l / 16, c = l % 16) the keys
//     16 t + 4 g + r of query c, which become P^T's B operand as they are: the
//     P.V product sums over its 32 keys in any order, so element e of the lane
//     stands for key pi(8 g + e) = 16 (e / 4) + 4 g + e % 4 of the half, and
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
constexpr int kFpKeys = 64;                // keys per block
constexpr int kQWaves = 4;                 // waves of a key group: 16 queries each
constexpr int kKeyGroups = 2;
constexpr int kXcds = 8;                   // MI355X: workgroups are dealt to 8 XCDs in turn
constexpr int kRow = 128;                  // K and V rows in LDS: 256 bytes, 16-byte chunks swizzled
constexpr int kKHalves = kFpKeys * kRow;
constexpr int kVHalves = kFpKeys * kRow;
// chunk q of row r sits at position q ^ swz(r): K by r % 16 (the 16 rows of one
// operand read), V by 2 (r % 4) (the 4 rows x 2 chunks of one transposed read)
__device__ __forceinline__ int kswz(int r) { return r & 15; }
__device__ __forceinline__ int vswz(int r) { return 2 * (r & 3); }
constexpr int kOLd = 128 + 4;              // fp32 O row in the fold
constexpr float kLazy = 8.0f;              // log2 of the largest softmax weight before a rescale
static_assert(kQWaves * 16 == kFpQueries, "a key group's waves cover the workgroup's queries");
static_assert((size_t)kFpQueries * kOLd * 4 <= (size_t)kKeyGroups * 2 * kKHalves * 2,
              "the fold's O rows fit in the K buffers");

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kKeyGroups * kQWaves * 64) void flash_prefill_kernel(FlashPrefillParams p) {
  __shared__ __align__(16) _Float16 lk[kKeyGroups][2][kKHalves];   // [group][buffer]
  __shared__ __align__(16) _Float16 lv[kKeyGroups][2][kVHalves];
  const int lane = threadIdx.x & 63;
  const int wave8 = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int kg = wave8 / kQWaves;                // key group: blocks kg, kg + 2, ...
  const int wave = wave8 % kQWaves;              // queries 16 wave .. 16 wave + 15
  const int tid = threadIdx.x & 255;             // thread within the key group
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
  const int wq0 = 16 * wave;
  const bool active = wq0 < nq;                 // wave-uniform: the wave has queries

  // B operand of S^T: Q[q0 + wq0 + c][32 s + 8 g .. +8] (rows past the last
  // query repeat it; their outputs are not stored)
  f16x8 qb[4];
  {
    const int qi = min(wq0 + c, nq - 1);
    const uint16_t* qrow = p.q + (long long)(q0 + qi) * p.q_stride + h * 128 + 8 * g;
#pragma unroll
    for (int s = 0; s < 4; ++s) qb[s] = *reinterpret_cast<const f16x8*>(qrow + 32 * s);
  }
  const int qpos = p.pos0 + q0 + wq0 + c;       // this lane's query position
  const int wpos = p.pos0 + q0 + wq0;           // the wave's first query position

  // A group's block: 64 rows of K and of V.  Rows past nkeys repeat row
  // nkeys - 1 and are masked.
  const uint16_t* khead = p.k + (long long)h * p.head_stride;
  const uint16_t* vhead = p.v + (long long)h * p.head_stride;
  // Direct loads into LDS: wave w of the group moves rows 16 w .. 16 w + 15 of
  // the block, four rows (1 KB) per instruction; lane l fills position l % 16 of
  // row l / 16 of the four, i.e. the row's chunk (l % 16) ^ swz(row).
  auto dload = [&](int j, int b) {
    const int kb = j * kFpKeys;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * wave + 4 * i + (lane >> 4);
      const long long grow = min(kb + row, nkeys - 1);
      const int kq = (lane & 15) ^ kswz(row), vq = (lane & 15) ^ vswz(row);
      __builtin_amdgcn_global_load_lds(khead + grow * p.row_stride + 8 * kq,
                                       (__attribute__((address_space(3))) void*)&lk[kg][b][(16 * wave + 4 * i) * kRow],
                                       16, 0, 0);
      __builtin_amdgcn_global_load_lds(vhead + grow * p.row_stride + 8 * vq,
                                       (__attribute__((address_space(3))) void*)&lv[kg][b][(16 * wave + 4 * i) * kRow],
                                       16, 0, 0);
    }
  };

  float m = -__builtin_inff();
  f32x4 ls = {0.0f, 0.0f, 0.0f, 0.0f};          // the denominator, in every element
  f32x4 o[8];
#pragma unroll
  for (int n = 0; n < 8; ++n) o[n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  f16x8 ones;
#pragma unroll
  for (int e = 0; e < 8; ++e) ones[e] = (_Float16)1.0f;

  // Block j of this group from LDS buffer b: the wave's online-softmax update.
  auto compute = [&](int j, int b) {
    const int kb = j * kFpKeys;
    if (!active || j >= nblk || kb > wpos + 15) return;   // wave-uniform: no key reaches a query
    f32x4 st[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      st[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      const _Float16* krow = &lk[kg][b][(16 * t + c) * kRow];
#pragma unroll
      for (int s = 0; s < 4; ++s)
        st[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
            *reinterpret_cast<const f16x8*>(krow + 8 * ((4 * s + g) ^ kswz(16 * t + c))), qb[s], st[t], 0, 0, 0);
    }
    if (kb + kFpKeys - 1 > wpos) {              // wave-uniform: some key is past a query
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) st[t][r] = kb + 16 * t + 4 * g + r <= qpos ? st[t][r] : -__builtin_inff();
    }
    // Each lane tests its own 16 keys against the lazy bound; only when some
    // lane's keys pass it are the block maxima formed across the lanes of a
    // query (the decisions a block-wide maximum gives).
    float lm = st[0][0];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) lm = fmaxf(lm, st[t][r]);
    if (__any(lm * p.scale_log2 > m + kLazy)) {   // -inf + kLazy is -inf: a first finite block grows
      float bm = fmaxf(lm, __shfl_xor(lm, 16));
      bm = fmaxf(bm, __shfl_xor(bm, 32)) * p.scale_log2;   // log2 units (scale > 0)
      const float mn = bm > m + kLazy ? bm : m;
      const float alpha = mn == m ? 1.0f : __builtin_amdgcn_exp2f(m - mn);
      ls *= alpha;
#pragma unroll
      for (int n = 0; n < 8; ++n) o[n] *= alpha;
      m = mn;
    }
    const float nref = m == -__builtin_inff() ? 0.0f : -m;   // no key yet: every weight is 0
    f16x8 pb[2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        pb[hh][e] = (_Float16)__builtin_amdgcn_exp2f(__builtin_fmaf(st[2 * hh + e / 4][e % 4], p.scale_log2, nref));
      ls = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pb[hh], ls, 0, 0, 0);
    }
    // O^T += V^T P^T per 32-key half.  Within a 16-lane group, lane i's element
    // e of a transposed read is element i % 4 of the four halves lane
    // 4 e + i / 4 addresses.  Lane j of group g addresses key 4 g + j / 4 (+ 16
    // for the second read), dims 16 n + 4 (j % 4) .. +4, so lane (c, g)
    // receives dim 16 n + c of keys 4 g + e and 16 + 4 g + e of the half: the
    // keys pi(8 g + e) its P^T operand holds.
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int vr = 32 * hh + 4 * g + (c >> 2);            // key of the low read; +16 for the high one
      const _Float16* vrow = &lv[kg][b][vr * kRow];
#pragma unroll
      for (int n = 0; n < 8; ++n) {
        const int q = 2 * n + ((c >> 1) & 1);              // dims 16 n + 4 (c % 4) .. +4 lie in chunk q
        const int off = 8 * (q ^ vswz(vr)) + 4 * (c & 1);
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(vrow + off));
        const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(vrow + 16 * kRow + off));
        const f16x8 va = __builtin_bit_cast(f16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        o[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[hh], o[n], 0, 0, 0);
      }
    }
  };

  // Iteration i computes the group's block 2 i + kg from LDS buffer i % 2 while
  // the block of iteration i + 1 streams into the other buffer.  The direct
  // loads are invisible to the compiler's waits: each wave waits for its own
  // (vmcnt) before the barrier that hands the buffer to the group.
  const int nit = (nblk + 1) / 2;
  if (kg < nblk) dload(kg, 0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  for (int it = 0; it < nit; ++it) {
    const int j = 2 * it + kg;
    const int b = it & 1;
    if (j + 2 < nblk) dload(j + 2, b ^ 1);     // buffer b ^ 1 was last read before the previous barrier
    compute(j, b);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }

  // Fold the two key groups' states of each query: group 1 hands (m, l, O) to
  // group 0 through LDS (the K/V buffers are free after the last barrier).
  float* fo = reinterpret_cast<float*>(&lk[0][0][0]);       // [query][dim]
  float* fm = reinterpret_cast<float*>(&lv[0][0][0]);       // [query][m, l]
  const int qq = wq0 + c;                                   // the lane's query in the tile
  if (kg == 1) {
#pragma unroll
    for (int n = 0; n < 8; ++n) *reinterpret_cast<f32x4*>(fo + qq * kOLd + 16 * n + 4 * g) = o[n];
    if (g == 0) {
      fm[2 * qq] = m;
      fm[2 * qq + 1] = ls[0];
    }
  }
  __syncthreads();
  if (kg == 0 && active && qq < nq) {
    const float m1 = fm[2 * qq], l1 = fm[2 * qq + 1];
    const float M = fmaxf(m, m1);                           // finite: key 0 reaches every query
    const float a0 = m == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(m - M);
    const float a1 = m1 == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(m1 - M);
    const float inv = 1.0f / (a0 * ls[0] + a1 * l1);
    _Float16* orow = reinterpret_cast<_Float16*>(p.out + (long long)(q0 + qq) * p.out_stride + h * 128);
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      const f32x4 o1 = *reinterpret_cast<const f32x4*>(fo + qq * kOLd + 16 * n + 4 * g);
      f16x4 v;
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = (_Float16)((a0 * o[n][r] + a1 * o1[r]) * inv);
      *reinterpret_cast<f16x4*>(orow + 16 * n + 4 * g) = v;
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

