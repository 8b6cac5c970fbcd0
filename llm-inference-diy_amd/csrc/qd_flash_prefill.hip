// Causal prefill attention on the matrix cores (gfx950 v_mfma_f32_16x16x32_f16):
// the counterpart of the reference's prompt attention, qwen_infer.cu:484-527
// (gather_q_from_qkv / gather_kv_from_cache into per-head buffers,
// flash_attn_tuned_A_kernel with the causal mask of flash_attn_causal.cuh, one
// launch per head, then scatter_interleaved_kernel), as one launch that reads
// the rotated Q rows and the KV cache where they lie.
//
// Workgroup (h, tile) takes 64 consecutive queries of head h, four tiles of
// 16 (the MFMA's N).  Its four waves all take the 64 queries and split the
// keys: wave w takes key blocks w, w + 4, ... of 32 keys each, so every K/V
// row a wave loads serves 64 queries; each wave keeps its own online-softmax
// state per query, and the four states are folded in LDS at the end.  The
// grid is one-dimensional and its linear index is remapped so that, with
// workgroups dealt to the 8 XCDs in turn, the tiles of a head run on one XCD
// and share its L2 copy of the head's K/V rows; within a head the latest
// tiles (the longest key ranges) start first.  Per block and query tile a
// wave computes
//   S^T = K Q^T   (M = 16 keys per tile, two tiles; N = 16 queries; K = 128 dims)
//   O^T += V^T P^T (M = 16 dims per tile, eight tiles; N = 16 queries; K = 32 keys)
// Transposing both products puts the query in the MFMA's column, which is the
// lane's column l % 16 of every accumulator, so each lane's softmax state
// (running max m, partial sum l) belongs to query l % 16 in every product and
// rescaling O needs no lane exchange.  Operand lanes: A[l % 16][8 (l / 16) + e],
// B[8 (l / 16) + e][l % 16]; accumulator D[4 (l / 16) + r][l % 16].
//   - K rows feed A directly (the 8 dims of a lane are 16 contiguous bytes).
//   - S^T's accumulator gives lane (g = l / 16, c = l % 16) the keys
//     16 t + 4 g + r of query c, which become P^T's B operand as they are: the
//     P.V product sums over its 32 keys in any order, so element e of the lane
//     stands for key pi(8 g + e) = 16 (e / 4) + 4 g + e % 4, and the V^T
//     operand is read in the same order.
//   - V^T comes from LDS: each wave writes its V block there as it lies
//     ([key][dim], 16-byte stores) and takes, per tile, the 4 + 4 keys
//     pi(8 g ..) of dim 16 n + c with two transposed reads (gfx950's
//     ds_read_b64_tr_b16).  (Writing the block transposed took 64 two-byte LDS
//     stores per lane and block.)
// P is rounded to fp16 for the product (as the reference's MMA kernel does)
// and the softmax denominator sums the rounded weights; exponentials are the
// hardware's exp2.  Nothing here is bit-reproducible on
// the host; the exact prefill path (the decode kernels batched) is.
#include "qd_device.h"
#include "qd_internal.h"

namespace qd {
namespace {

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

constexpr int kQt = 4;                     // 16-query tiles per workgroup
constexpr int kFpQueries = 16 * kQt;       // queries per workgroup
constexpr int kFpKeys = 32;                // keys per block: the P.V product's K
constexpr int kFpWaves = 4;
constexpr int kXcds = 8;                   // MI355X: workgroups are dealt to 8 XCDs in turn
// V block in LDS as it lies in memory, [key][dim], rows padded to 144 halves
// (288 bytes: the four rows one transposed read takes start 8 banks apart).
constexpr int kVPitch = 128 + 16;
constexpr int kVHalves = kFpKeys * kVPitch;  // per wave
constexpr int kOLd = 128 + 4;              // fp32 O row in the fold
constexpr float kLazy = 8.0f;              // log2 of the largest softmax weight before a rescale
static_assert((size_t)kFpWaves * 16 * kOLd * 4 <= (size_t)kFpWaves * kVHalves * 2,
              "one query tile's fold reuses the V buffers");

__device__ __forceinline__ void wave_lds_fence() {
  // Lanes of one wave hand data to each other through LDS: the wave's LDS
  // operations execute in order, and these fences keep the compiler from
  // moving the accesses across this point.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__global__ __launch_bounds__(kFpWaves * 64) void flash_prefill_kernel(FlashPrefillParams p) {
  __shared__ __align__(16) _Float16 lds[kFpWaves * kVHalves];
  __shared__ float fml[2][kFpWaves][kFpQueries];   // each wave's (m, l) per query
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
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

  // B operand of S^T per query tile u: Q[q0 + 16 u + c][32 s + 8 g .. +8]
  // (rows past the last query repeat it; their outputs are not stored)
  f16x8 qb[kQt][4];
  int qpos[kQt];                                // this lane's query position per tile
#pragma unroll
  for (int u = 0; u < kQt; ++u) {
    const uint16_t* qrow = p.q + (long long)(q0 + min(16 * u + c, nq - 1)) * p.q_stride + h * 128 + 8 * g;
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) qb[u][s4] = *reinterpret_cast<const f16x8*>(qrow + 32 * s4);
    qpos[u] = p.pos0 + q0 + 16 * u + c;
  }

  const uint16_t* kbase = p.k + (long long)h * p.head_stride + 8 * g;
  const uint16_t* vbase = p.v + (long long)h * p.head_stride + 8 * (lane >> 5);
  // K rows kb + 16 t + c (dims 32 s + 8 g .. +8) and V row kb + (l & 31)
  // (dims 16 i + 8 (l >> 5) .. +8) of block j, clamped into [0, nblk) so every
  // call issues them; keys past nkeys repeat key nkeys - 1 and are masked.
  f16x8 kr[2][4], vr[8];
  auto load = [&](int j) {
    j = min(j, nblk - 1);
    const int kb = j * kFpKeys;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const uint16_t* row = kbase + (long long)min(kb + 16 * t + c, nkeys - 1) * p.row_stride;
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) kr[t][s4] = *reinterpret_cast<const f16x8*>(row + 32 * s4);
    }
    const uint16_t* row = vbase + (long long)min(kb + (lane & 31), nkeys - 1) * p.row_stride;
#pragma unroll
    for (int i = 0; i < 8; ++i) vr[i] = *reinterpret_cast<const f16x8*>(row + 16 * i);
  };

  _Float16* vrow = lds + wave * kVHalves;
  float m[kQt], l[kQt];
  f32x4 o[kQt][8];
#pragma unroll
  for (int u = 0; u < kQt; ++u) {
    m[u] = -__builtin_inff();
    l[u] = 0.0f;
#pragma unroll
    for (int n = 0; n < 8; ++n) o[u][n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  int j = wave;
  if (j < nblk) load(j);
  for (; j < nblk; j += kFpWaves) {
    const int kb = j * kFpKeys;
    // V into LDS as it lies (key l & 31, dims 16 i + 8 (l >> 5) ..), then S^T
    // per tile; after that this block's K and V registers are free for the
    // next block.
    wave_lds_fence();                          // the previous block's V reads are done
    {
      _Float16* row = vrow + (lane & 31) * kVPitch + 8 * (lane >> 5);
#pragma unroll
      for (int i = 0; i < 8; ++i) *reinterpret_cast<f16x8*>(row + 16 * i) = vr[i];
    }
    f32x4 st[kQt][2];
#pragma unroll
    for (int u = 0; u < kQt; ++u)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        st[u][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4)
          st[u][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kr[t][s4], qb[u][s4], st[u][t], 0, 0, 0);
      }
    load(j + kFpWaves);
    __builtin_amdgcn_sched_barrier(0);         // keep the next block's loads here
    // Online softmax of query (u, c) over keys kb + 16 t + 4 g + r.  The
    // reference m (log2 units) moves only when a block's maximum passes it by
    // more than kLazy, so weights stay below 2^kLazy (fp16 holds them with the
    // same relative precision) and O and l are rescaled in few blocks; the
    // causal mask is applied only on blocks that reach past a query of the
    // tile; each exponent is one fma of the raw score.
    // The four query tiles go through each step together, with one
    // wave-uniform branch per block, so their dependency chains interleave.
    f16x8 pb[kQt];
    float sv[kQt][8], bm[kQt];
    bool grow = false;
#pragma unroll
    for (int u = 0; u < kQt; ++u) {
      const bool diag = kb + kFpKeys - 1 > p.pos0 + q0 + 16 * u;   // wave-uniform
      float bmax = -__builtin_inff();
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float s = st[u][t][r];
          if (diag) s = kb + 16 * t + 4 * g + r <= qpos[u] ? s : -__builtin_inff();
          sv[u][4 * t + r] = s;
          bmax = fmaxf(bmax, s);
        }
      bm[u] = bmax;
    }
#pragma unroll
    for (int u = 0; u < kQt; ++u) bm[u] = fmaxf(bm[u], __shfl_xor(bm[u], 16));
#pragma unroll
    for (int u = 0; u < kQt; ++u) {
      bm[u] = fmaxf(bm[u], __shfl_xor(bm[u], 32)) * p.scale_log2;   // log2 units (scale > 0)
      grow |= bm[u] > m[u] + kLazy;            // -inf + kLazy is -inf: a first finite block grows
    }
    if (__any(grow)) {
#pragma unroll
      for (int u = 0; u < kQt; ++u) {
        const float mn = bm[u] > m[u] + kLazy ? bm[u] : m[u];
        const float alpha = mn == m[u] ? 1.0f : __builtin_amdgcn_exp2f(m[u] - mn);
        l[u] *= alpha;
#pragma unroll
        for (int n = 0; n < 8; ++n) o[u][n] *= alpha;
        m[u] = mn;
      }
    }
#pragma unroll
    for (int u = 0; u < kQt; ++u) {
      const float nref = m[u] == -__builtin_inff() ? 0.0f : -m[u];   // no key yet: every weight is 0
      float ps = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        // the sum takes the rounded weights the product uses, so O / l stays
        // a weighted mean of V rows
        pb[u][e] = (_Float16)__builtin_amdgcn_exp2f(__builtin_fmaf(sv[u][e], p.scale_log2, nref));
        ps += (float)pb[u][e];
      }
      l[u] += ps;
    }
    wave_lds_fence();                          // V stores visible to the wave
    // The V^T operand of dims tile n by transposed reads (ds_read_b64_tr_b16):
    // within a 16-lane group, lane i's element e is element i % 4 of the four
    // halves lane 4 e + i / 4 addresses.  Lane j of group g addresses key
    // 4 g + j / 4 (+ 16 for the second read), dims 16 n + 4 (j % 4) .. +4, so
    // lane (c, g) receives dim 16 n + c of keys 4 g + e and 16 + 4 g + e: the
    // keys pi(8 g + e) its P^T operand holds.
    const _Float16* vtr = vrow + (4 * g + (c >> 2)) * kVPitch + 4 * (c & 3);
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      typedef short i16x4 __attribute__((ext_vector_type(4)));
      typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
      const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(vtr + 16 * n));
      const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(vtr + 16 * kVPitch + 16 * n));
      const f16x8 va = __builtin_bit_cast(f16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
      for (int u = 0; u < kQt; ++u) o[u][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[u], o[u][n], 0, 0, 0);
    }
  }
#pragma unroll
  for (int u = 0; u < kQt; ++u) {
    l[u] += __shfl_xor(l[u], 16);
    l[u] += __shfl_xor(l[u], 32);
    if (g == 0) {
      fml[0][wave][16 * u + c] = m[u];
      fml[1][wave][16 * u + c] = l[u];
    }
  }

  // Fold the four waves' states one query tile at a time: O rows
  // [wave][query][dim] in the V^T buffers, then each thread 8 dims of a query.
  float* fo = reinterpret_cast<float*>(lds);
  const int q = tid >> 4;
  const int d0 = (tid & 15) * 8;
#pragma unroll
  for (int u = 0; u < kQt; ++u) {
    __syncthreads();                           // V^T, or the previous tile's fold, is done
#pragma unroll
    for (int n = 0; n < 8; ++n)
      *reinterpret_cast<f32x4*>(fo + (wave * 16 + c) * kOLd + 16 * n + 4 * g) = o[u][n];
    __syncthreads();
    const int qq = 16 * u + q;
    if (qq < nq) {
      float mw[kFpWaves];
      float M = -__builtin_inff();
#pragma unroll
      for (int w = 0; w < kFpWaves; ++w) {
        mw[w] = fml[0][w][qq];
        M = fmaxf(M, mw[w]);
      }
      float L = 0.0f;
      float acc[8] = {};
#pragma unroll
      for (int w = 0; w < kFpWaves; ++w) {
        const float sc = mw[w] == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(mw[w] - M);
        L += sc * fml[1][w][qq];
        const float* row = fo + (w * 16 + q) * kOLd + d0;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += sc * row[e];
      }
      f16x8 outv;
#pragma unroll
      for (int e = 0; e < 8; ++e) outv[e] = (_Float16)(acc[e] / L);
      *reinterpret_cast<f16x8*>(p.out + (long long)(q0 + qq) * p.out_stride + h * 128 + d0) = outv;
    }
  }
}

}  // namespace

hipError_t launch_flash_prefill(const FlashPrefillParams& p, hipStream_t stream) {
  const dim3 grid(p.num_heads * ((p.tokens + kFpQueries - 1) / kFpQueries));
  hipLaunchKernelGGL(flash_prefill_kernel, grid, dim3(kFpWaves * 64), 0, stream, p);
  return hipGetLastError();
}

}  // namespace qd
