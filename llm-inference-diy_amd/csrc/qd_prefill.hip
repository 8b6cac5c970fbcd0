// Batched prompt processing (prefill) for gfx950 in the decode step's exact
// arithmetic.
//
// Role: QwenEngine::prefill (framework_src/qwen_infer.cu:372-611) runs the
// prompt's tokens 0..N-2 through the layers at once to fill the KV cache.  The
// reference does it with MMA GEMMs and FlashAttention, whose summation order
// differs from its own decode step.  Here every output of every token is the
// same fp32 sum, in the same order, as the single-token decode kernels compute
// (lane l of a 64-lane wave adds k = 512j + 8l + e sequentially, then the fixed
// wave64 tree), so the KV cache a prompt leaves is bit-identical to feeding the
// tokens one by one, and greedy decoding after a prompt stays reproducible on
// the host.  The GEMMs therefore run on the FMA pipes, not MFMA (whose internal
// summation order is not specified): each weight row is read from memory once
// per group of tokens and kept in registers while the tokens stream through LDS.
//
// Kernels (per layer, T tokens):
//   rmsnorm_batched_kernel     T waves: xn[t] = RMSNorm(x[t]) * w
//   gemv_batched_kernel        Y[t][n] = sum_k X[t][k] W[n][k], with an epilogue
//                              (store as half, or residual add into the stream)
//   rope_batched_kernel        bias + RoPE + KV append per token (qd_rope_cache)
//   swiglu_batched_kernel      act = half(g * (u / (1 + exp(-u))))
// Attention runs per token with qd_decode_attention's plan for that length.
#include <algorithm>
#include <atomic>

#include "qd_device.h"
#include "qd_internal.h"

namespace qd {
namespace {

constexpr float kLog2e = 1.44269504088896340736f;

// Tokens per workgroup of the batched GEMV; tokens per LDS tile (up to 8, so
// that a tile of NJ * 512 fp16 elements per token stays within 64 KB).  The
// tile is even: tokens are consumed in pairs, and an odd tile would end every
// tile on a half-used pair step.
constexpr int kTokPerWg = 32;
constexpr int tok_tile(int nj) { return nj <= 8 ? 8 : (64 / nj) & ~1; }
// Waves per workgroup, two rows each.  From NJ = 15 (K > 7168) the weights
// (16 * NJ VGPRs) and the unrolled sums no longer fit the 256 VGPRs a wave has
// at two waves per SIMD, so those workgroups have 4 waves (one per SIMD, whose
// wave may also use the accumulation registers): no scratch.  Which workgroup
// computes a row does not change its sums.
constexpr int gemv_waves(int nj) { return nj >= 15 ? 4 : 8; }

// One wave per token: the same normalisation as the decode kernels' normalise()
// (qd_decode_ops.hip), written out as fp16.
template <int NJ>
__global__ __launch_bounds__(256) void rmsnorm_batched_kernel(const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ w,
                                                             float eps, uint16_t* __restrict__ xn,
                                                             int T) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  constexpr int hidden = NJ * 512;
  const uint16_t* xr = x + (long long)t * hidden;
  f16x8 xv[NJ], nv[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    xv[j] = *reinterpret_cast<const f16x8*>(xr + 512 * j + 8 * lane);
    nv[j] = *reinterpret_cast<const f16x8*>(w + 512 * j + 8 * lane);
  }
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = (float)xv[j][e];
      acc = __builtin_fmaf(v, v, acc);
    }
  const float var = wave64_sum(acc) / (float)hidden;
  const float r = 1.0f / __builtin_sqrtf(var + eps);
  uint16_t* out = xn + (long long)t * hidden;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    f16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = to_f16(((float)xv[j][e] * r) * (float)nv[j][e]);
    *reinterpret_cast<f16x8*>(out + 512 * j + 8 * lane) = o;
  }
}

// 16-byte chunks of one token tile that each thread stages into LDS: a tile
// holds tok_tile(NJ) rows of at most NJ * 64 chunks, spread over the
// workgroup's threads.
constexpr int stage_chunks(int nj) {
  return (tok_tile(nj) * nj * 64 + gemv_waves(nj) * 64 - 1) / (gemv_waves(nj) * 64);
}

// DPP row rotations (gfx9 encodings): lane i of a 16-lane row reads lane
// (i - n) mod 16.
constexpr int kDppRowRor4 = 0x124;
constexpr int kDppRowRor8 = 0x128;

// The four sums of a 2-token x 2-row block, s0 = (t, na), s1 = (t+1, na),
// s2 = (t, nb), s3 = (t+1, nb), reduced over the wave in one transposed
// butterfly.  Afterwards lane 12 + q (q = token bit + 2 * row bit) of row 0
// holds block output q's total.  Every total is the sum wave64_sum forms,
// node for node, so the bits are the decode kernels':
//   lanes i, i^1  -- even lanes keep token t's two sums, odd lanes token t+1's;
//   lanes i, i^2  -- the quad's lanes with bit 1 clear keep row na, set row nb;
//                    every lane now holds a quad sum Q of its own output;
//   row_ror 4     -- lanes 4..7 and 12..15 add the quad before: Q1 + Q0 and
//                    Q3 + Q2 (wave64_sum pairs the same quads by a half-row
//                    mirror, whose lanes all hold the same quad sum);
//   row_ror 8     -- lanes 12..15 add lanes 4..7: the row sum (the mirror
//                    step of wave64_sum);
//   xor 16, xor 32 -- the rows, as in wave64_sum.
// IEEE addition is commutative, so the operand order inside a node does not
// change its bits.
__device__ __forceinline__ float block4_sum(float s0, float s1, float s2, float s3, int lane) {
  const bool odd = lane & 1;
  float k0 = odd ? s1 : s0;
  float k1 = odd ? s3 : s2;
  const float g0 = odd ? s0 : s1;
  const float g1 = odd ? s2 : s3;
  k0 += dpp_mov<kDppQuadSwap1>(g0);
  k1 += dpp_mov<kDppQuadSwap1>(g1);
  const bool hi = lane & 2;
  float k = hi ? k1 : k0;
  const float g = hi ? k0 : k1;
  k += dpp_mov<kDppQuadSwap2>(g);
  k += dpp_mov<kDppRowRor4>(k);
  k += dpp_mov<kDppRowRor8>(k);
  k += __shfl_xor(k, 16);
  k += __shfl_xor(k, 32);
  return k;
}

// Y[t][n] for n in this workgroup's 2W rows (W = gemv_waves(NJ)) and t in its
// kTokPerWg tokens.  Wave w holds rows n0 = 2W*bx + 2w and n0 + 1 (NJ chunks of 8 per lane, the
// last one masked when K is not a multiple of 512).  Token tiles of kTokTile
// rows of X are staged in LDS; each lane reads its 16-byte chunks from them
// (consecutive lanes, consecutive 16 B: conflict-free).  The next tile's
// global loads are issued into registers before the current tile is
// consumed, so their latency hides behind its arithmetic.  Two tokens and two
// rows are summed at a time: four independent sequential sums per lane, each
// in the decode order, then one transposed wave reduction (block4_sum) whose
// four totals four lanes store.
//   kEpi 0: Y[t][n] = half(sum)
//   kEpi 1: Y[t][n] = half(R[t][n] + half(sum))     (residual add; R may be Y)
template <int NJ, int kEpi>
__global__ __launch_bounds__(gemv_waves(NJ) * 64) void gemv_batched_kernel(BatchedGemvParams p) {
  constexpr int kGemvWaves = gemv_waves(NJ);
  extern __shared__ __align__(16) uint16_t xs[];        // [kTokTile][NJ * 512]
  constexpr int kTokTile = tok_tile(NJ);
  constexpr int kStage = stage_chunks(NJ);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int K = p.k;
  const int rem = K - 512 * (NJ - 1);                    // elements in the last chunk
  const bool tail = 8 * lane < rem;
  const int n0 = blockIdx.x * (2 * kGemvWaves) + 2 * wave;
  const int na = min(n0, p.n - 1), nb = min(n0 + 1, p.n - 1);
  f16x8 wa[NJ], wb[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    if (j < NJ - 1 || tail) {
      wa[j] = __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(p.w + (long long)na * K + 512 * j + 8 * lane));
      wb[j] = __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(p.w + (long long)nb * K + 512 * j + 8 * lane));
    }
  }
  const int tpw = p.tok_per_wg > 0 ? p.tok_per_wg : kTokPerWg;
  const int t_begin = blockIdx.y * tpw;
  const int t_end = min(p.t, t_begin + tpw);
  // This thread's staging chunks: chunk c = tid + 512 i is token c / chunks of
  // the tile, 16-byte chunk c % chunks of its row.  Up to NJ = 11 the map is
  // kept in registers and the next tile's loads are in flight while the
  // current tile is consumed.  Above that the registers are not there (the
  // weights alone take 16 * NJ), so each chunk is loaded and stored in turn.
  constexpr bool kPrefetch = NJ <= 11;
  const int chunks = K / 8;
  constexpr int kMap = kPrefetch ? kStage : 1;
  int st_tok[kMap], st_kc[kMap];
  f16x8 stage[kMap];
  if constexpr (kPrefetch) {
#pragma unroll
    for (int i = 0; i < kStage; ++i) {
      const int c = threadIdx.x + i * kGemvWaves * 64;
      st_tok[i] = c / chunks;
      st_kc[i] = c - st_tok[i] * chunks;
    }
  }
  // Loads are unconditional (a chunk past the tile reloads the tile's last
  // token), so they form one straight run with no wait between them; only the
  // LDS stores are predicated.
  auto fetch = [&](int t0, int nt) {
#pragma unroll
    for (int i = 0; i < kMap; ++i) {
      const int tk = min(st_tok[i], nt - 1);
      stage[i] = *reinterpret_cast<const f16x8*>(p.x + (long long)(t0 + tk) * p.ldx + st_kc[i] * 8);
    }
  };
  if (kPrefetch && t_begin < t_end) fetch(t_begin, min(kTokTile, t_end - t_begin));
  for (int t0 = t_begin; t0 < t_end; t0 += kTokTile) {
    const int nt = min(kTokTile, t_end - t0);
    __syncthreads();                                     // previous tile fully consumed
    if constexpr (kPrefetch) {
#pragma unroll
      for (int i = 0; i < kStage; ++i)
        if (st_tok[i] < nt) *reinterpret_cast<f16x8*>(xs + st_tok[i] * (NJ * 512) + st_kc[i] * 8) = stage[i];
    } else {
      for (int c = threadIdx.x; c < nt * chunks; c += kGemvWaves * 64) {
        const int tt = c / chunks, kc = c - tt * chunks;
        *reinterpret_cast<f16x8*>(xs + tt * (NJ * 512) + kc * 8) =
            *reinterpret_cast<const f16x8*>(p.x + (long long)(t0 + tt) * p.ldx + kc * 8);
      }
    }
    __syncthreads();
    if (kPrefetch && t0 + kTokTile < t_end) fetch(t0 + kTokTile, min(kTokTile, t_end - t0 - kTokTile));
    for (int tt = 0; tt < nt; tt += 2) {
      const bool two = tt + 1 < nt;
      const uint16_t* x0 = xs + tt * (NJ * 512);
      const uint16_t* x1 = xs + (two ? tt + 1 : tt) * (NJ * 512);
      float a0 = 0.0f, a1 = 0.0f, b0 = 0.0f, b1 = 0.0f;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        if (j < NJ - 1 || tail) {
          const f16x8 u0 = *reinterpret_cast<const f16x8*>(x0 + 512 * j + 8 * lane);
          const f16x8 u1 = *reinterpret_cast<const f16x8*>(x1 + 512 * j + 8 * lane);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            a0 = __builtin_fmaf((float)wa[j][e], (float)u0[e], a0);
            a1 = __builtin_fmaf((float)wa[j][e], (float)u1[e], a1);
            b0 = __builtin_fmaf((float)wb[j][e], (float)u0[e], b0);
            b1 = __builtin_fmaf((float)wb[j][e], (float)u1[e], b1);
          }
        }
      }
      const float sum = block4_sum(a0, a1, b0, b1, lane);
      const int q = lane - 12;                           // lanes 12..15 store
      if (q >= 0 && q < 4) {
        const int t = t0 + tt + (q & 1);
        const int n = n0 + (q >> 1);
        if ((two || (q & 1) == 0) && n < p.n) {
          const _Float16 y = to_f16(sum);
          _Float16* dst = reinterpret_cast<_Float16*>(p.y) + (long long)t * p.ldy + n;
          if constexpr (kEpi == 0) {
            *dst = y;
          } else {
            const float r = (float)reinterpret_cast<const _Float16*>(p.res)[(long long)t * p.ldy + n];
            *dst = (_Float16)(r + (float)y);
          }
        }
      }
    }
  }
}

// Four weight rows per wave, for K <= 2048 (NJ <= 4).  The fp16 x fp16 -> fp32
// FMA (v_fma_mix_f32) issues at ~0.6x the rate of the plain fp32 FMA on gfx950
// (35-37 against 52-59 T FMA/s in an ALU-only loop), so here both operands
// reach the FMA as fp32: the weights are converted once into registers and the
// token tile is staged in LDS as fp32.  That doubles the LDS bytes per token;
// four rows per wave (each token value feeds four FMAs) keep the LDS reads per
// FMA where two fp16 rows had them.  Each lane's sums and the wave reduction
// are the decode order, so the outputs are gemv_batched_kernel's bit for bit
// (an fp16 -> fp32 conversion is exact and the FMA rounds once either way).
// At 224 VGPRs only two waves share a SIMD, so LDS round trips and the
// per-tile barriers stay exposed: at 127 tokens it uses ~40% of the fp32 FMA
// issue rate and ~25% of the LDS read rate, 4.5-12% faster than the two-row
// kernel at n >= 4096.
constexpr int kR4Waves = 4;     // waves per workgroup: 16 rows
constexpr int kR4Tile = 8;      // tokens per LDS tile (64 KB at K = 2048)
constexpr int r4_stage(int nj) { return (kR4Tile * nj * 64 + kR4Waves * 64 - 1) / (kR4Waves * 64); }
constexpr int kDppRowRor12 = 0x12C;

// The eight sums of a 2-token x 4-row block, v[q] with q = token + 2 * row,
// reduced over the wave in one transposed butterfly.  Afterwards lane 8 + q of
// each 16-lane row holds block output q's total.  As in block4_sum, every total
// is the sum wave64_sum forms, node for node: lanes i, i^1 split the tokens;
// lanes i, i^2 the rows' low bit (each lane then holds a quad sum of its own
// output); lanes i, i^4 the rows' high bit while adding quad pairs (Q0 + Q1,
// Q2 + Q3: wave64_sum's half-row mirror step); row_ror 8 adds the half-rows
// (the mirror step); then xor 16 and xor 32 add the rows.
__device__ __forceinline__ float block8_sum(const float (&v)[8], int lane) {
  const bool b0 = lane & 1, b1 = lane & 2, b2 = lane & 4;
  float k[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float keep = b0 ? v[2 * r + 1] : v[2 * r];
    const float give = b0 ? v[2 * r] : v[2 * r + 1];
    k[r] = keep + dpp_mov<kDppQuadSwap1>(give);
  }
  float m[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float keep = b1 ? k[2 * i + 1] : k[2 * i];
    const float give = b1 ? k[2 * i] : k[2 * i + 1];
    m[i] = keep + dpp_mov<kDppQuadSwap2>(give);
  }
  const float keep = b2 ? m[1] : m[0];
  const float give = b2 ? m[0] : m[1];
  // lane i ^ 4 within the row: i - 4 for lanes with bit 2 set, i + 4 otherwise.
  // Both moves run in every lane before the select: under a branch a DPP move's
  // partner lanes would be inactive and read as zero.
  float up = dpp_mov<kDppRowRor4>(give), dn = dpp_mov<kDppRowRor12>(give);
  asm volatile("" : "+v"(up), "+v"(dn));
  float s = keep + (b2 ? up : dn);
  s += dpp_mov<kDppRowRor8>(s);
  s += __shfl_xor(s, 16);
  s += __shfl_xor(s, 32);
  return s;
}

// Y[t][n] for n in this workgroup's 16 rows and t in its kTokPerWg tokens;
// wave w holds rows n0 = 16 bx + 4 w .. n0 + 3.  The LDS tile is fp32, each
// token row split so that a lane's two 16-byte reads of a chunk are contiguous
// across the wave: chunk c = 64 j + l of a row keeps elements 0..3 at float4
// 128 j + l and 4..7 at float4 128 j + 64 + l.  Staging, prefetch of the next
// tile and the epilogues are gemv_batched_kernel's.
template <int NJ, int kEpi>
__global__ __launch_bounds__(kR4Waves * 64) void gemv_batched_r4_kernel(BatchedGemvParams p) {
  static_assert(NJ <= 4, "four fp32 rows per lane fit in registers up to K = 2048");
  extern __shared__ __align__(16) float xf[];           // [kR4Tile][NJ * 512]
  constexpr int kStage = r4_stage(NJ);
  constexpr int kRow = NJ * 512;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int K = p.k;
  const int rem = K - 512 * (NJ - 1);
  const bool tail = 8 * lane < rem;
  const int n0 = blockIdx.x * (4 * kR4Waves) + 4 * wave;
  float wf[4][NJ][8];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int n = min(n0 + r, p.n - 1);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      f16x8 h = {};
      if (j < NJ - 1 || tail)
        h = __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(p.w + (long long)n * K + 512 * j + 8 * lane));
#pragma unroll
      for (int e = 0; e < 8; ++e) wf[r][j][e] = (float)h[e];
    }
  }
  const int t_begin = blockIdx.y * kTokPerWg;
  const int t_end = min(p.t, t_begin + kTokPerWg);
  const int chunks = K / 8;
  int st_tok[kStage], st_kc[kStage];
  f16x8 stage[kStage];
#pragma unroll
  for (int i = 0; i < kStage; ++i) {
    const int c = threadIdx.x + i * kR4Waves * 64;
    st_tok[i] = c / chunks;
    st_kc[i] = c - st_tok[i] * chunks;
  }
  auto fetch = [&](int t0, int nt) {
#pragma unroll
    for (int i = 0; i < kStage; ++i) {
      const int tk = min(st_tok[i], nt - 1);
      stage[i] = *reinterpret_cast<const f16x8*>(p.x + (long long)(t0 + tk) * p.ldx + st_kc[i] * 8);
    }
  };
  if (t_begin < t_end) fetch(t_begin, min(kR4Tile, t_end - t_begin));
  for (int t0 = t_begin; t0 < t_end; t0 += kR4Tile) {
    const int nt = min(kR4Tile, t_end - t0);
    __syncthreads();                                     // previous tile fully consumed
#pragma unroll
    for (int i = 0; i < kStage; ++i)
      if (st_tok[i] < nt) {
        const int kc = st_kc[i];
        float* dst = xf + st_tok[i] * kRow + 4 * (128 * (kc >> 6) + (kc & 63));
        const f16x8 h = stage[i];
        *reinterpret_cast<float4*>(dst) = make_float4((float)h[0], (float)h[1], (float)h[2], (float)h[3]);
        *reinterpret_cast<float4*>(dst + 256) = make_float4((float)h[4], (float)h[5], (float)h[6], (float)h[7]);
      }
    __syncthreads();
    if (t0 + kR4Tile < t_end) fetch(t0 + kR4Tile, min(kR4Tile, t_end - t0 - kR4Tile));
    for (int tt = 0; tt < nt; tt += 2) {
      const bool two = tt + 1 < nt;
      const float* x0 = xf + tt * kRow;
      const float* x1 = xf + (two ? tt + 1 : tt) * kRow;
      float acc[8] = {};                                 // [row][token]
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        if (j < NJ - 1 || tail) {
          const float4 u0a = *reinterpret_cast<const float4*>(x0 + 4 * (128 * j + lane));
          const float4 u0b = *reinterpret_cast<const float4*>(x0 + 4 * (128 * j + 64 + lane));
          const float4 u1a = *reinterpret_cast<const float4*>(x1 + 4 * (128 * j + lane));
          const float4 u1b = *reinterpret_cast<const float4*>(x1 + 4 * (128 * j + 64 + lane));
          const float u0[8] = {u0a.x, u0a.y, u0a.z, u0a.w, u0b.x, u0b.y, u0b.z, u0b.w};
          const float u1[8] = {u1a.x, u1a.y, u1a.z, u1a.w, u1b.x, u1b.y, u1b.z, u1b.w};
#pragma unroll
          for (int e = 0; e < 8; ++e)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              acc[2 * r] = __builtin_fmaf(wf[r][j][e], u0[e], acc[2 * r]);
              acc[2 * r + 1] = __builtin_fmaf(wf[r][j][e], u1[e], acc[2 * r + 1]);
            }
        }
      }
      const float sum = block8_sum(acc, lane);
      const int q = lane - 8;                            // lanes 8..15 store
      if (q >= 0 && q < 8) {
        const int t = t0 + tt + (q & 1);
        const int n = n0 + (q >> 1);
        if ((two || (q & 1) == 0) && n < p.n) {
          const _Float16 y = to_f16(sum);
          _Float16* dst = reinterpret_cast<_Float16*>(p.y) + (long long)t * p.ldy + n;
          if constexpr (kEpi == 0) {
            *dst = y;
          } else {
            const float r = (float)reinterpret_cast<const _Float16*>(p.res)[(long long)t * p.ldy + n];
            *dst = (_Float16)(r + (float)y);
          }
        }
      }
    }
  }
}

// Bias, rotate-half RoPE and KV append for token t at position pos0 + t, with
// qkv_bias_rope_cache_kernel's arithmetic (qd_rope_cache.hip) element by
// element: one thread per (head, four consecutive rotation pairs), 16 threads
// per head, so Q, K, V and the cache rows move as 8-byte vectors.  One thread
// per pair with 2-byte accesses took twice as long (14 against 7 us per layer
// at 2048 tokens).  The bias is read element by element: it may sit at an odd
// element offset.
constexpr int kRopeHeads = 16;              // heads per workgroup (256 threads)
typedef _Float16 f16x4r __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(kRopeHeads * 16) void rope_batched_kernel(uint16_t* qkv, const uint16_t* bias,
                                                          uint16_t* k_layer, uint16_t* v_layer,
                                                          const float2* rope_cs, long long row_stride,
                                                          long long head_stride, int pos0,
                                                          int num_heads) {
  const int t = blockIdx.y;
  const int h = blockIdx.x * kRopeHeads + (threadIdx.x >> 4);
  if (h >= num_heads) return;
  const int i0 = 4 * (threadIdx.x & 15);      // rotation pairs i0 .. i0 + 3
  const int hid = num_heads * 128;
  const int pos = pos0 + t;
  _Float16* q = reinterpret_cast<_Float16*>(qkv) + (long long)t * 3 * hid;
  const _Float16* b = reinterpret_cast<const _Float16*>(bias);
  const int idx1 = h * 128 + i0, idx2 = idx1 + 64;
  f16x4r hq1 = *reinterpret_cast<const f16x4r*>(q + idx1), hq2 = *reinterpret_cast<const f16x4r*>(q + idx2);
  f16x4r hk1 = *reinterpret_cast<const f16x4r*>(q + hid + idx1), hk2 = *reinterpret_cast<const f16x4r*>(q + hid + idx2);
  f16x4r hv1 = *reinterpret_cast<const f16x4r*>(q + 2 * hid + idx1), hv2 = *reinterpret_cast<const f16x4r*>(q + 2 * hid + idx2);
  if (b) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      hq1[e] = (_Float16)((float)hq1[e] + (float)b[idx1 + e]);
      hq2[e] = (_Float16)((float)hq2[e] + (float)b[idx2 + e]);
      hk1[e] = (_Float16)((float)hk1[e] + (float)b[hid + idx1 + e]);
      hk2[e] = (_Float16)((float)hk2[e] + (float)b[hid + idx2 + e]);
      hv1[e] = (_Float16)((float)hv1[e] + (float)b[2 * hid + idx1 + e]);
      hv2[e] = (_Float16)((float)hv2[e] + (float)b[2 * hid + idx2 + e]);
    }
  }
  const float4 csa = *reinterpret_cast<const float4*>(rope_cs + pos * 64 + i0);       // pairs i0, i0 + 1
  const float4 csb = *reinterpret_cast<const float4*>(rope_cs + pos * 64 + i0 + 2);   // pairs i0 + 2, i0 + 3
  const float cx[4] = {csa.x, csa.z, csb.x, csb.z}, sy[4] = {csa.y, csa.w, csb.y, csb.w};
  f16x4r oq1, oq2, ok1, ok2;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float q1 = (float)hq1[e], q2 = (float)hq2[e], k1 = (float)hk1[e], k2 = (float)hk2[e];
    const float q1c = q1 * cx[e], q2s = q2 * sy[e], q2c = q2 * cx[e], q1s = q1 * sy[e];
    const float k1c = k1 * cx[e], k2s = k2 * sy[e], k2c = k2 * cx[e], k1s = k1 * sy[e];
    oq1[e] = to_f16(q1c - q2s);
    oq2[e] = to_f16(q2c + q1s);
    ok1[e] = to_f16(k1c - k2s);
    ok2[e] = to_f16(k2c + k1s);
  }
  *reinterpret_cast<f16x4r*>(q + idx1) = oq1;
  *reinterpret_cast<f16x4r*>(q + idx2) = oq2;
  *reinterpret_cast<f16x4r*>(q + hid + idx1) = hk1;
  *reinterpret_cast<f16x4r*>(q + hid + idx2) = hk2;
  *reinterpret_cast<f16x4r*>(q + 2 * hid + idx1) = hv1;
  *reinterpret_cast<f16x4r*>(q + 2 * hid + idx2) = hv2;
  const long long base = (long long)pos * row_stride + (long long)h * head_stride;
  _Float16* kc = reinterpret_cast<_Float16*>(k_layer) + base;
  _Float16* vc = reinterpret_cast<_Float16*>(v_layer) + base;
  *reinterpret_cast<f16x4r*>(kc + i0) = ok1;
  *reinterpret_cast<f16x4r*>(kc + 64 + i0) = ok2;
  *reinterpret_cast<f16x4r*>(vc + i0) = hv1;
  *reinterpret_cast<f16x4r*>(vc + 64 + i0) = hv2;
}

// act[r][c] = half(g * (u / (1 + exp2_rep(-u * log2 e)))) on fp16
// g = g[r * ld + c], u = u[r * ld + c]: the decode kernel's SwiGLU epilogue
// (qd_decode_ops.hip) over rows x cols, V consecutive columns per thread.
template <int V>
__global__ __launch_bounds__(256) void swiglu_batched_kernel(const uint16_t* __restrict__ g,
                                                            const uint16_t* __restrict__ u,
                                                            uint16_t* __restrict__ act, int rows,
                                                            int cols, long long ld) {
  const long long i = ((long long)blockIdx.x * 256 + threadIdx.x) * V;
  if (i >= (long long)rows * cols) return;
  const long long r = i / cols, c = i - r * cols;
  _Float16 gh[V], uh[V], out[V];
  if constexpr (V == 8) {
    *reinterpret_cast<f16x8*>(gh) = *reinterpret_cast<const f16x8*>(g + r * ld + c);
    *reinterpret_cast<f16x8*>(uh) = *reinterpret_cast<const f16x8*>(u + r * ld + c);
  } else {
    gh[0] = reinterpret_cast<const _Float16*>(g)[r * ld + c];
    uh[0] = reinterpret_cast<const _Float16*>(u)[r * ld + c];
  }
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const float uf = (float)uh[j];
    const float e = exp2_rep(-uf * kLog2e);
    const float silu = uf / (1.0f + e);
    out[j] = to_f16((float)gh[j] * silu);
  }
  if constexpr (V == 8)
    *reinterpret_cast<f16x8*>(act + i) = *reinterpret_cast<const f16x8*>(out);
  else
    reinterpret_cast<_Float16*>(act)[i] = out[0];
}

// Embedding rows: x[t] = wte[tokens[t]].
__global__ __launch_bounds__(256) void embed_kernel(const uint16_t* __restrict__ wte,
                                                    const int* __restrict__ tokens,
                                                    uint16_t* __restrict__ x, int hidden) {
  const int t = blockIdx.x;
  const uint16_t* src = wte + (long long)tokens[t] * hidden;
  uint16_t* dst = x + (long long)t * hidden;
  for (int c = threadIdx.x; c < hidden / 8; c += 256)
    *reinterpret_cast<f16x8*>(dst + 8 * c) = *reinterpret_cast<const f16x8*>(src + 8 * c);
}

// ---------------------------------------------------------------------------
// MFMA prefill GEMM (the fast, not bit-reproducible mode): Y[t][n] = sum_k
// X[t][k] W[n][k] on the matrix cores, fp16 x fp16 products accumulated in fp32
// by v_mfma_f32_16x16x32_f16 in the hardware's own order (the role of the
// reference's tensor-core hgemm_swizzle_nn in prefill, qwen_infer.cu:359-367).
//
// Operand layout of one 16x16x32 step (checked on gfx950): lane l holds
// A[l % 16][8 (l / 16) .. +8] and B[8 (l / 16) .. +8][l % 16], and receives
// D[4 (l / 16) + r][l % 16], r = 0..3.  With A = X (tokens x K) and B = W^T,
// both fragments are 16 contiguous bytes of one row of X or W.
//
// Workgroup: 4 waves, a 64-token x 64-row tile; wave w takes tokens
// 32 (w / 2) .. +32 and rows 32 (w % 2) .. +32 as 2 x 2 MFMA blocks.  K goes
// in tiles of 64 through a ring of 8 LDS stages (8 KB of X and 8 KB of W each),
// filled by direct loads (global_load_lds_dwordx4: each thread moves two 16-byte
// chunks of each operand per stage, no registers), with 7 tiles in flight: a
// short prompt's product is a chain of memory round trips, not of arithmetic,
// and one tile in flight per workgroup left each K tile waiting a full round
// trip (QKV at 127 tokens 17.9 -> 13.2 us, gate/up with the SwiGLU 28.6 -> 24.9
// us).  Rows are 128 bytes with their 16-byte chunks swizzled (chunk q of row r
// at q ^ ((r / 2) % 8)), so the 16 rows of one operand read fall on distinct
// banks.  Each stage is its own LDS variable and the loop is unrolled over the
// ring, so every access names its stage; the operand reads are inline assembly
// with their own waits, since the compiler, unable to tell eight stages apart,
// would wait for every load in flight before each read.  Tiles past the last
// repeat it, so every thread issues the same loads per stage and the wait
// counts are fixed.  Tokens past t and rows past n load clamped rows and are
// not stored.  K must be a multiple of 64.  kEpi 2 is the split-K form:
// workgroup z = blockIdx.z sums K slice [z kslice, (z + 1) kslice) and stores
// its fp32 tile to p.part.  kEpi 3 is the joint gate/up form: a workgroup
// takes 32 intermediate rows, its W tile holding them from W1 (tile rows
// 0..31) and W2 (32..63); wave w's B blocks are gate rows 16 (w % 2) .. +16
// and the same up rows, so one lane holds g and u of the same output and writes
// act = half(g * (u / (1 + exp(-u)))) on the fp16-rounded g and u.
constexpr int kMmTile = 64;                 // tokens and rows per workgroup
constexpr int kMmK = 64;                    // K per stage
constexpr int kMmOps = kMmTile * kMmK / 8 / 256;   // direct loads per thread per operand per stage (2)

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));

struct __align__(16) MmStage {
  uint16_t x[kMmTile * kMmK];
  uint16_t w[kMmTile * kMmK];
};
// ds_read_b128 is served eight lanes at a time over 32 four-byte banks (128
// bytes), and every 128-byte row starts on bank 0: r % 8 puts the eight rows of
// one such group (lanes l % 16 = 8g .. 8g + 7 of an operand read) on distinct
// 16-byte positions.  (The earlier (r / 2) % 8, right for 64 banks, left rows
// 2i and 2i + 1 on the same banks.)
__device__ __forceinline__ int mmswz(int r) { return r & 7; }

template <int kEpi>
__global__ __launch_bounds__(256) void gemm_nt_mfma_kernel(BatchedGemvParams p) {
  __shared__ MmStage s0, s1, s2, s3, s4, s5, s6, s7;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n0 = blockIdx.x * (kEpi == 3 ? kMmTile / 2 : kMmTile);
  const int t0 = blockIdx.y * kMmTile;
  int kbeg = 0, kend = p.k;
  if constexpr (kEpi == 2) {
    kbeg = blockIdx.z * p.kslice;
    kend = min(p.k, kbeg + p.kslice);
  }
  const int ktiles = kend > kbeg ? (kend - kbeg) / kMmK : 0;

  // Load i of wave w writes 1 KB at chunk 256 i + 64 w + lane of the stage's
  // operand: row 32 i + 8 w + lane / 8, position lane % 8.
  const uint16_t* xg[kMmOps];
  const uint16_t* wg[kMmOps];
#pragma unroll
  for (int i = 0; i < kMmOps; ++i) {
    const int row = 32 * i + 8 * wave + (lane >> 3);
    const int ch = (lane & 7) ^ mmswz(row);
    xg[i] = p.x + (long long)min(t0 + row, p.t - 1) * p.ldx + kbeg + 8 * ch;
    if constexpr (kEpi == 3)
      wg[i] = (row < 32 ? p.w : p.w2) + (long long)min(n0 + (row & 31), p.n - 1) * p.k + kbeg + 8 * ch;
    else
      wg[i] = p.w + (long long)min(n0 + row, p.n - 1) * p.k + kbeg + 8 * ch;
  }
  auto issue = [&](int kt, MmStage& st) {
    const long long ko = (long long)min(kt, ktiles - 1) * kMmK;
#pragma unroll
    for (int i = 0; i < kMmOps; ++i) {
      __builtin_amdgcn_global_load_lds(xg[i] + ko, (__attribute__((address_space(3))) void*)&st.x[(256 * i + 64 * wave) * 8],
                                       16, 0, 0);
      __builtin_amdgcn_global_load_lds(wg[i] + ko, (__attribute__((address_space(3))) void*)&st.w[(256 * i + 64 * wave) * 8],
                                       16, 0, 0);
    }
  };

  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
  const int fr = lane & 15, fg = lane >> 4;
  f32x4_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  // Byte offsets within a stage of the lane's A (X) and B (W) fragments for K
  // step ks of the tile: A[fr][8 fg .. +8] of token block i, B of row block j.
  unsigned aoff[2][2], boff[2][2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int ar = wm + 16 * i + fr;
      aoff[ks][i] = (unsigned)((ar * kMmK + 8 * ((4 * ks + fg) ^ mmswz(ar))) * 2);
      const int br = (kEpi == 3 ? 32 * i + 16 * (wave & 1) : wn + 16 * i) + fr;
      boff[ks][i] = (unsigned)((kMmTile * kMmK + br * kMmK + 8 * ((4 * ks + fg) ^ mmswz(br))) * 2);
    }
  auto compute = [&](const MmStage& st) {
    const unsigned base = (unsigned)(size_t)(const __attribute__((address_space(3))) void*)&st;
    f16x8 a[2][2], b[2][2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        asm volatile("ds_read_b128 %0, %1" : "=v"(a[ks][i]) : "v"(base + aoff[ks][i]) : "memory");
        asm volatile("ds_read_b128 %0, %1" : "=v"(b[ks][i]) : "v"(base + boff[ks][i]) : "memory");
      }
    asm volatile("s_waitcnt lgkmcnt(4)" : "+v"(a[0][0]), "+v"(a[0][1]), "+v"(b[0][0]), "+v"(b[0][1]));
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[0][i], b[0][j], acc[i][j], 0, 0, 0);
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a[1][0]), "+v"(a[1][1]), "+v"(b[1][0]), "+v"(b[1][1]));
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[1][i], b[1][j], acc[i][j], 0, 0, 0);
  };
  // Tile kt sits in stage kt % 8.  Each thread waits for its own loads of it
  // (6 newer stages of 4 loads each stay in flight) and for its reads of the
  // previous stage; after the barrier every thread's part of tile kt is in LDS
  // and the previous stage, read by all, takes tile kt + 7.  The barrier is
  // s_barrier alone: __syncthreads' fence would wait for every load in flight.
  auto body = [&](int kt, const MmStage& cur, MmStage& prev) {
    asm volatile("s_waitcnt vmcnt(24) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    issue(kt + 7, prev);
    compute(cur);
  };
  if (ktiles > 0) {
    issue(0, s0); issue(1, s1); issue(2, s2); issue(3, s3); issue(4, s4); issue(5, s5); issue(6, s6);
    for (int kt = 0; kt < ktiles; kt += 8) {
      body(kt, s0, s7);
      if (kt + 1 < ktiles) body(kt + 1, s1, s0);
      if (kt + 2 < ktiles) body(kt + 2, s2, s1);
      if (kt + 3 < ktiles) body(kt + 3, s3, s2);
      if (kt + 4 < ktiles) body(kt + 4, s4, s3);
      if (kt + 5 < ktiles) body(kt + 5, s5, s4);
      if (kt + 6 < ktiles) body(kt + 6, s6, s5);
      if (kt + 7 < ktiles) body(kt + 7, s7, s6);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the repeated tail loads land before the workgroup ends
  }
  if constexpr (kEpi == 3) {
    // blocks (i, 0) and (i, 1): gate and up of row n0 + 16 (w % 2) + l % 16 for
    // token t0 + wm + 16 i + 4 (l / 16) + r
    const int n = n0 + 16 * (wave & 1) + fr;
    if (n >= p.n) return;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = t0 + wm + 16 * i + (lane >> 4) * 4 + r;
        if (t >= p.t) continue;
        const float gh = (float)to_f16(acc[i][0][r]);
        const float uh = (float)to_f16(acc[i][1][r]);
        const float e = exp2_rep(-uh * kLog2e);
        reinterpret_cast<_Float16*>(p.y)[(long long)t * p.ldy + n] = to_f16(gh * (uh / (1.0f + e)));
      }
    return;
  }
  // D[4 (l / 16) + r][l % 16] of block (i, j): token t0 + wm + 16 i + 4 (l / 16) + r,
  // row n0 + wn + 16 j + l % 16
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + wn + 16 * j + fr;
      if (n >= p.n) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = t0 + wm + 16 * i + (lane >> 4) * 4 + r;
        if (t >= p.t) continue;
        if constexpr (kEpi == 2) {
          p.part[((long long)blockIdx.z * p.t + t) * p.n + n] = acc[i][j][r];
          continue;
        }
        const _Float16 y = to_f16(acc[i][j][r]);
        _Float16* dst = reinterpret_cast<_Float16*>(p.y) + (long long)t * p.ldy + n;
        if constexpr (kEpi == 0) {
          *dst = y;
        } else {
          const float rr = (float)reinterpret_cast<const _Float16*>(p.res)[(long long)t * p.ldy + n];
          *dst = (_Float16)(rr + (float)y);
        }
      }
    }
}

// Folds the split-K partials of gemm_nt_mfma_kernel<2>: the slices' fp32 sums
// added in slice order, then the epilogue of kEpi (0: half(sum); 1: half(R +
// half(sum))).  One thread per output.
template <int kEpi>
__global__ __launch_bounds__(256) void splitk_fold_kernel(BatchedGemvParams p, int splits) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long tn = (long long)p.t * p.n;
  if (i >= tn) return;
  float s = p.part[i];
  for (int z = 1; z < splits; ++z) s += p.part[z * tn + i];
  const long long t = i / p.n, n = i - t * p.n;
  _Float16 y = to_f16(s);
  if constexpr (kEpi == 1) y = (_Float16)((float)reinterpret_cast<const _Float16*>(p.res)[t * p.ldy + n] + (float)y);
  reinterpret_cast<_Float16*>(p.y)[t * p.ldy + n] = y;
}

// Buffer resource over `bytes` bytes from `base` (raw: no stride, no
// swizzle; word 3 the data format gfx9 parts take for untyped loads), and the
// buffer load of 16 bytes per lane into LDS (lane l at lds + 16 l; M0 holds
// the wave-uniform LDS base) at base + voffset + soffset.  Bytes at or past
// `bytes` read as zeros.
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4 buffer_rsrc(const void* base, unsigned bytes) {
  const unsigned long long a = reinterpret_cast<unsigned long long>(base);
  i32x4 r;
  r[0] = (int)(unsigned)a;
  r[1] = (int)(unsigned)(a >> 32);
  r[2] = (int)bytes;
  r[3] = 0x00020000;
  return r;
}
__device__ void raw_buffer_load_lds(i32x4 rsrc, __attribute__((address_space(3))) unsigned* lds, int size,
                                    int voffset, int soffset, int offset, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.lds");
__device__ __forceinline__ void buffer_load_lds16(i32x4 rsrc, __attribute__((address_space(3))) unsigned* lds,
                                                  unsigned voffset, int soffset) {
  raw_buffer_load_lds(rsrc, lds, 16, (int)voffset, soffset, 0, 0);
}
__device__ i32x4 raw_buffer_load_b128(i32x4 rsrc, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.v4i32");

constexpr int kGemmXcds = 8;                 // MI355X: workgroups are dealt to 8 XCDs in turn
constexpr int kRingMinRows = 128;            // the ring tiles from this many tokens
constexpr int kGemmMaxSplits = 8;            // K slices of a split product

// Large-M product on a ring of direct-to-LDS stages (M >= 128: the matrix-core
// prefill's passes): a 128 x 128 workgroup tile computed as Y^T = W X^T, so
// the MFMA's A operand is W's rows and B the tokens' rows and accumulator lane
// (g = l / 16, c = l % 16) holds rows 4 g .. 4 g + 3 of W for token c: four
// adjacent outputs of one token, stored as 8 bytes.  Four waves of 64 x 64
// (4 x 4 MFMA blocks).  K goes in tiles of 64 through a ring of 5 LDS stages of 32 KB
// (W tile then X tile, 128-byte rows with their 16-byte chunks swizzled by
// r % 8 as in gemm_nt_mfma_kernel) filled by direct loads
// (global_load_lds_dwordx4, 8 per thread per stage), 4 tiles in flight
// beyond the one being read: a register-staged version of this tile, with one
// tile (~0.2 us of matrix-core work) in flight against an L2/MALL round trip
// and two barriers per tile, ran the 2048-token QKV product in 72 us.  One
// barrier per tile here, and the next tile's operand fragments are read from
// LDS while the matrix cores consume the current tile's (with the reads and
// the products of a tile in sequence, the kernel ran at ~25% of the matrix
// cores' rate).  Operand reads are inline assembly with their own waits (see
// gemm_nt_mfma_kernel).  The grid is
// one-dimensional and XCD-major: XCD x computes a contiguous eighth of the
// (W row tile, token tile) pairs, W row tile major, so its L2 holds an eighth
// of W.  kEpi 0: half(sum); 1: half(R + half(sum)); 2: split K, slice z =
// blockIdx.y stores its fp32 sums to p.part ([z][t][n], n a multiple of 4)
// for splitk_fold_kernel; 3: the joint gate/up form
// (64 intermediate rows per workgroup, W tile rows 0..63 from W1 and 64..127
// the same rows of W2; wave (wy = w / 2) takes gate rows 32 wy .. +32 as its A
// blocks 0-1 and the same up rows as blocks 2-3; act = half(g * (u / (1 +
// exp(-u)))) on the fp16-rounded g and u).  Requires k a multiple of 64, y and
// res 8-byte aligned and ldy a multiple of 4.
constexpr int kRgT = 128;                        // tokens per workgroup
constexpr int kRgN = 128;                        // W rows per workgroup (64 outputs when kEpi == 3)
constexpr int kRgK = 64;                         // K per stage
constexpr int kRgOps = kRgN * kRgK / 8 / 256;    // direct loads per thread per operand per stage (4)
constexpr int kRgGroupN = 4;                     // W row tiles per group of the tile order

struct __align__(16) RingStage {
  uint16_t w[kRgN * kRgK];
  uint16_t x[kRgT * kRgK];
};

template <int kEpi>
__global__ __launch_bounds__(256, 1) void gemm_nt_ring128_kernel(BatchedGemvParams p) {
  __shared__ RingStage s0, s1, s2, s3, s4;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: scalar LDS bases
  constexpr int kRows = kEpi == 3 ? kRgN / 2 : kRgN;   // output rows per workgroup
  const int ttiles = (p.t + kRgT - 1) / kRgT;
  const int ntiles = (p.n + kRows - 1) / kRows;
  const int nwg = ttiles * ntiles;
  int pi = blockIdx.x;
  if (nwg % kGemmXcds == 0) pi = (pi % kGemmXcds) * (nwg / kGemmXcds) + pi / kGemmXcds;
  // Tile pi in groups of kRgGroupN W row tiles (fewer in the last group) x all
  // token tiles, W tile fastest: 32 consecutive pi (one XCD's CUs) cover 4 W
  // tiles x 8 token tiles, so each K slab an XCD fetches into its L2 serves 8
  // or 4 workgroups (16 and 2 with W tile major order: 26% of L2 requests
  // missed).
  const int grp = pi / (kRgGroupN * ttiles);
  const int gn = min(kRgGroupN, ntiles - grp * kRgGroupN);
  const int rem = pi - grp * kRgGroupN * ttiles;
  const int n0 = (grp * kRgGroupN + rem % gn) * kRows;
  const int t0 = (rem / gn) * kRgT;
  // kEpi 2 (split K): slice z = blockIdx.y sums K [z kslice, (z + 1) kslice)
  const int kbeg = kEpi == 2 ? (int)blockIdx.y * p.kslice : 0;
  const int ktiles = (kEpi == 2 ? min(p.k - kbeg, p.kslice) : p.k) / kRgK;

  // Load i of wave w writes 1 KB at chunk 256 i + 64 w + lane of the stage's
  // operand: row 32 i + 8 w + lane / 8, position lane % 8, which holds the
  // row's global chunk (lane % 8) ^ mmswz(row).  Buffer loads over each
  // operand (W or W1 and W2, X): a fixed 32-bit byte offset per lane and load,
  // the tile's K offset in a scalar register; rows past an operand's end lie
  // past its buffer's size and read as zeros (they feed only outputs that are
  // not stored).
  const int ch = (lane & 7) ^ ((lane >> 3) & 7);   // row % 8 == (lane / 8) % 8
  const i32x4 rw = buffer_rsrc(p.w, (unsigned)((long long)p.n * p.k * 2));
  const i32x4 rw2 = kEpi == 3 ? buffer_rsrc(p.w2, (unsigned)((long long)p.n * p.k * 2)) : rw;
  const i32x4 rx = buffer_rsrc(p.x, (unsigned)(((long long)(p.t - 1) * p.ldx + p.k) * 2));
  unsigned vw[kRgOps], vx[kRgOps];
#pragma unroll
  for (int i = 0; i < kRgOps; ++i) {
    const int row = 32 * i + 8 * wave + (lane >> 3);
    vw[i] = kEpi == 3 ? (unsigned)(n0 + (row & 63)) * (unsigned)p.k * 2u + 16u * ch
                      : (unsigned)(n0 + row) * (unsigned)p.k * 2u + (unsigned)kbeg * 2u + 16u * ch;
    vx[i] = (unsigned)(t0 + row) * (unsigned)p.ldx * 2u + (unsigned)kbeg * 2u + 16u * ch;
  }
  auto issue = [&](int kt, RingStage& st) {
    const int so = min(kt, ktiles - 1) * kRgK * 2;   // tiles past the last repeat it
#pragma unroll
    for (int i = 0; i < kRgOps; ++i) {
      // rows 64.. of the gate/up form's W tile are W2's (i >= 2)
      buffer_load_lds16((kEpi == 3 && i >= kRgOps / 2) ? rw2 : rw,
                        (__attribute__((address_space(3))) unsigned*)&st.w[(256 * i + 64 * wave) * 8], vw[i], so);
      buffer_load_lds16(rx, (__attribute__((address_space(3))) unsigned*)&st.x[(256 * i + 64 * wave) * 8], vx[i], so);
    }
  };

  const int wy = wave >> 1, wx = wave & 1;
  const int fr = lane & 15, fg = lane >> 4;
  f32x4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  // Byte offsets within a stage of the lane's fragments for K step ks: A (W)
  // rows of block i, B (X) tokens of block j; chunk 4 ks + fg of the row.
  unsigned aoff[2][4], boff[2][4];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ar = (kEpi == 3 ? (i >> 1) * 64 + wy * 32 + 16 * (i & 1) : wy * 64 + 16 * i) + fr;
      aoff[ks][i] = (unsigned)((ar * kRgK + 8 * ((4 * ks + fg) ^ mmswz(ar))) * 2);
      const int br = wx * 64 + 16 * i + fr;
      boff[ks][i] = (unsigned)((kRgN * kRgK + br * kRgK + 8 * ((4 * ks + fg) ^ mmswz(br))) * 2);
    }
  // Fragments of one K tile: f[ks][i] (A, W rows of block i) and f[ks][4 + j]
  // (B, tokens of block j) for the two K steps of 32.
  typedef f16x8 Frags[2][8];
  auto read_frags = [&](const RingStage& st, Frags& f) {
    const unsigned base = (unsigned)(size_t)(const __attribute__((address_space(3))) void*)&st;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        asm volatile("ds_read_b128 %0, %1" : "=v"(f[ks][i]) : "v"(base + aoff[ks][i]) : "memory");
        asm volatile("ds_read_b128 %0, %1" : "=v"(f[ks][4 + i]) : "v"(base + boff[ks][i]) : "memory");
      }
  };
  auto mfma_tile = [&](const Frags& f) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(f[ks][i], f[ks][4 + j], acc[i][j], 0, 0, 0);
  };
  // The fragments' registers are bound to the wait, so no use of them can be
  // scheduled before it.
  auto wait_frags = [&](Frags& f, int) {
    asm volatile("s_waitcnt vmcnt(24) lgkmcnt(0)\n\ts_barrier"
                 : "+v"(f[0][0]), "+v"(f[0][1]), "+v"(f[0][2]), "+v"(f[0][3]), "+v"(f[0][4]),
                   "+v"(f[0][5]), "+v"(f[0][6]), "+v"(f[0][7]), "+v"(f[1][0]), "+v"(f[1][1]),
                   "+v"(f[1][2]), "+v"(f[1][3]), "+v"(f[1][4]), "+v"(f[1][5]), "+v"(f[1][6]),
                   "+v"(f[1][7])
                 :
                 : "memory");
  };
  // Tile kt sits in stage kt % 5.  Iteration kt holds tile kt's fragments in
  // registers (read during iteration kt - 1) and tiles kt + 1 .. kt + 4 in
  // flight.  Each thread waits for its own loads of tile kt + 1 (three newer
  // tiles of 8 loads stay in flight) and for its reads of tile kt; after the
  // barrier tile kt + 1 is whole in LDS and tile kt's stage, which every wave
  // has read, takes tile kt + 5.  Then tile kt + 1's fragments are read while
  // the matrix cores consume tile kt's: the LDS reads and the products
  // overlap.  The barrier is s_barrier alone: __syncthreads' fence would wait
  // for every load in flight.
  Frags fa, fb;
  auto body = [&](int kt, Frags& cur, Frags& nxt, RingStage& own, const RingStage& next) {
    wait_frags(cur, kt);
    issue(kt + 5, own);
    read_frags(next, nxt);
    mfma_tile(cur);
  };
  issue(0, s0);
  issue(1, s1);
  issue(2, s2);
  issue(3, s3);
  issue(4, s4);
  asm volatile("s_waitcnt vmcnt(32)\n\ts_barrier" ::: "memory");
  read_frags(s0, fa);
  for (int kt = 0; kt < ktiles; kt += 10) {
    body(kt, fa, fb, s0, s1);
    if (kt + 1 < ktiles) body(kt + 1, fb, fa, s1, s2);
    if (kt + 2 < ktiles) body(kt + 2, fa, fb, s2, s3);
    if (kt + 3 < ktiles) body(kt + 3, fb, fa, s3, s4);
    if (kt + 4 < ktiles) body(kt + 4, fa, fb, s4, s0);
    if (kt + 5 < ktiles) body(kt + 5, fb, fa, s0, s1);
    if (kt + 6 < ktiles) body(kt + 6, fa, fb, s1, s2);
    if (kt + 7 < ktiles) body(kt + 7, fb, fa, s2, s3);
    if (kt + 8 < ktiles) body(kt + 8, fa, fb, s3, s4);
    if (kt + 9 < ktiles) body(kt + 9, fb, fa, s4, s0);
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the repeated tail loads land before the workgroup ends

  if constexpr (kEpi == 3) {
    // blocks (i, j) and (i + 2, j), i < 2: gate and up of intermediate rows
    // n0 + 32 wy + 16 i + 4 (l / 16) + r, token t0 + 64 wx + 16 j + l % 16
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = t0 + wx * 64 + 16 * j + fr;
      if (t >= p.t) continue;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int n = n0 + wy * 32 + 16 * i + fg * 4;
        if (n >= p.n) continue;
        f16x4_t v;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float gh = (float)to_f16(acc[i][j][r]);
          const float uh = (float)to_f16(acc[i + 2][j][r]);
          const float e = exp2_rep(-uh * kLog2e);
          v[r] = to_f16(gh * (uh / (1.0f + e)));
        }
        _Float16* dst = reinterpret_cast<_Float16*>(p.y) + (long long)t * p.ldy + n;
        if (n + 4 <= p.n) {
          *reinterpret_cast<f16x4_t*>(dst) = v;
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n + r < p.n) dst[r] = v[r];
        }
      }
    }
    return;
  }
  // block (i, j): rows n0 + 64 wy + 16 i + 4 (l / 16) + r of W, token t0 + 64 wx + 16 j + l % 16
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int t = t0 + wx * 64 + 16 * j + fr;
    if (t >= p.t) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int n = n0 + wy * 64 + 16 * i + fg * 4;
      if (n >= p.n) continue;
      if constexpr (kEpi == 2) {   // the slice's fp32 sums, [z][t][n] (n a multiple of 4)
        *reinterpret_cast<f32x4_t*>(p.part + ((long long)blockIdx.y * p.t + t) * p.n + n) = acc[i][j];
        continue;
      }
      _Float16* dst = reinterpret_cast<_Float16*>(p.y) + (long long)t * p.ldy + n;
      const _Float16* res = reinterpret_cast<const _Float16*>(p.res) + (long long)t * p.ldy + n;
      if (n + 4 <= p.n) {
        f16x4_t v;
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = to_f16(acc[i][j][r]);
        if constexpr (kEpi == 1) {
          const f16x4_t rv = *reinterpret_cast<const f16x4_t*>(res);
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] = (_Float16)((float)rv[r] + (float)v[r]);
        }
        *reinterpret_cast<f16x4_t*>(dst) = v;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (n + r >= p.n) break;
          _Float16 y = to_f16(acc[i][j][r]);
          if constexpr (kEpi == 1) y = (_Float16)((float)res[r] + (float)y);
          dst[r] = y;
        }
      }
    }
  }
}

// The same product with a 192-row x 256-token workgroup tile (products whose
// grid of such tiles still covers the device: QKV and gate/up at 2048 tokens,
// one and two tiles per CU).  Per K, a 128 x 128 tile moves 64 bytes from L2
// into LDS and reads 128 from LDS per 2048 flops of its four 64 x 64 waves;
// at the matrix cores' rate that is the whole measured direct-load rate of a
// CU (~64 B per clock) and more than its LDS, and the 128 x 128 kernel ran at
// ~35% of the matrix-core time (rocprofv3: SQ_VALU_MFMA_BUSY_CYCLES against
// SQ_BUSY_CYCLES).  Here each of the four waves computes 96 W rows x 128
// tokens (6 x 8 MFMA blocks, 192 accumulator registers): 37 B per clock from
// L2 and ~110 from LDS at the matrix cores' rate.  K goes in tiles of 64
// through two stages each for W (192 x 128 B) and X (256 x 128 B); chunk q of
// row r at q ^ (r % 8), so the eight rows that one eight-lane group of a
// fragment read covers fall on distinct banks.  Every load is 16 bytes per
// lane, eight lanes to one row's whole 128-byte line: X's 8 per thread and
// tile go straight into LDS, W's 6 go through registers and are stored one
// tile later.  (With both operands on one path the kernel was slower: direct
// loads alone 6% on gate/up, registers alone 15-20%; the two paths together
// move more.)  Fragments go in K steps of 32, two per tile: the next step's
// fragments are read from LDS while the matrix cores consume the current
// one's, and a stage takes tile kt + 2 as soon as every wave has read tile
// kt's second step.  (32-wide tiles through a ring of 5 stages of 28 KB, 4
// tiles in flight, sent twice the L2 requests for the same bytes, each half a
// line, and waited twice as long on instructions as hipBLASLt's
// MT192x256x64.)  kEpi 0: half(sum); 1: half(R + half(sum)); 3: joint
// gate/up, 96 outputs per workgroup (W tile rows 0..95 from W1, 96..191 the
// same rows of W2; wave (wy = w / 2) takes gate rows 48 wy + 16 i as its A
// blocks i < 3 and the same up rows as blocks i + 3).
constexpr int kR2N = 192;                        // W rows per workgroup (96 outputs when kEpi == 3)
constexpr int kR2T = 256;                        // tokens per workgroup
constexpr int kR2K = 64;                         // K per stage
constexpr int kR2A = kR2N * kR2K / 8 / 64;       // 1 KB direct loads per stage: W (24)
constexpr int kR2B = kR2T * kR2K / 8 / 64;       // X (32)
constexpr int kR2Loads = (kR2A + kR2B) / 4;      // per thread per stage (14)

template <int S>
struct StageIdx {
  static constexpr int value = S;
};

template <int kEpi>
__global__ __launch_bounds__(256, 1) void gemm_nt_ring192_kernel(BatchedGemvParams p) {
  // W and X tiles in two stages each; 128-aligned, so the step-1 XOR below
  // commutes with every stage base
  __shared__ __align__(128) uint16_t lw[2][kR2N * kR2K];
  __shared__ __align__(128) uint16_t lx[2][kR2T * kR2K];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: scalar LDS bases
  constexpr int kRows = kEpi == 3 ? kR2N / 2 : kR2N;   // output rows per workgroup
  const int ttiles = (p.t + kR2T - 1) / kR2T;
  const int ntiles = (p.n + kRows - 1) / kRows;
  const int nwg = ttiles * ntiles;
  int pi = blockIdx.x;
  if (nwg % kGemmXcds == 0) pi = (pi % kGemmXcds) * (nwg / kGemmXcds) + pi / kGemmXcds;
  const int n0 = (pi / ttiles) * kRows;
  const int t0 = (pi % ttiles) * kR2T;
  const int ktiles = p.k / kR2K;

  // Load j of this wave is 1 KB load L = wave + 4 j of a tile: W rows 8 L ..
  // +8 for L < 24, else X rows 8 (L - 24) .. +8; lane l fills row 8 L' + l / 8
  // of its stage, position l % 8, with the row's global chunk (l % 8) ^ (row %
  // 8): eight lanes read one row's whole 128-byte line.  The loads are buffer
  // loads over each operand (W or W1, W2, X) with a fixed byte offset per lane
  // and load and the tile's K offset in a scalar register; rows past the
  // operand's end lie past its buffer's size and read as zeros (they feed only
  // outputs that are not stored).
  const int ch = (lane & 7) ^ ((lane >> 3) & 7);   // row % 8 == (lane / 8) % 8
  const i32x4 rw = buffer_rsrc(p.w, (unsigned)((long long)p.n * p.k * 2));
  const i32x4 rw2 = kEpi == 3 ? buffer_rsrc(p.w2, (unsigned)((long long)p.n * p.k * 2)) : rw;
  const i32x4 rx = buffer_rsrc(p.x, (unsigned)(((long long)(p.t - 1) * p.ldx + p.k) * 2));
  // Load j reads W (W1, then W2 from j = kR2A / 8 in the gate/up form) for
  // j < kR2A / 4 and X after, whatever the wave: the operand, and so the
  // descriptor, is known at compile time (a descriptor chosen at run time is
  // a vector value, and every load then loops over its distinct values).
  static_assert(kR2A % 8 == 0 && kR2B % 4 == 0, "loads of one operand per j");
  unsigned voff[kR2Loads];
#pragma unroll
  for (int j = 0; j < kR2Loads; ++j) {
    const int L = wave + 4 * j;
    if (j < kR2A / 4) {
      const int row = 8 * L + (lane >> 3);
      voff[j] = (unsigned)(n0 + row % kRows) * (unsigned)p.k * 2u + 16u * ch;
    } else {
      const int row = 8 * (L - kR2A) + (lane >> 3);
      voff[j] = (unsigned)(t0 + row) * (unsigned)p.ldx * 2u + 16u * ch;
    }
  }
  // W goes through registers (a tile's loads land in wr while the tile before
  // is multiplied, then are stored to LDS in the same layout); X goes
  // straight into LDS.
  i32x4 wr[kR2A / 4];
  auto load_w = [&](int kt) {
#pragma unroll
    for (int j = 0; j < kR2A / 4; ++j)
      wr[j] = raw_buffer_load_b128((kEpi == 3 && j >= kR2A / 8) ? rw2 : rw, (int)voff[j], kt * kR2K * 2, 0);
  };
  auto store_w = [&](int stage) {
    char* base = reinterpret_cast<char*>(lw[stage]);
#pragma unroll
    for (int j = 0; j < kR2A / 4; ++j)
      *reinterpret_cast<__attribute__((address_space(3))) i32x4*>(
          (__attribute__((address_space(3))) char*)(base + (wave + 4 * j) * 1024 + 16 * lane)) = wr[j];
  };
  auto issue_x = [&](int kt, int stage) {
    char* base = reinterpret_cast<char*>(lx[stage]);
#pragma unroll
    for (int j = kR2A / 4; j < kR2Loads; ++j)
      buffer_load_lds16(rx, (__attribute__((address_space(3))) unsigned*)(base + (wave + 4 * j - kR2A) * 1024),
                        voff[j], kt * kR2K * 2);
  };

  const int wy = wave >> 1, wx = wave & 1;
  const int fr = lane & 15, fg = lane >> 4;
  f32x4_t acc[6][8];
#pragma unroll
  for (int i = 0; i < 6; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  // LDS addresses in stage 0 of the lane's fragments for K step 0 of a tile:
  // A (W) rows of block i, B (X) tokens of block j; chunk fg of the row, at
  // position fg ^ (row % 8).  Step 1's chunk 4 + fg sits at address ^ 64, and
  // stage 1 is the read instruction's immediate offset.
  const unsigned lw0 = (unsigned)(size_t)(__attribute__((address_space(3))) void*)&lw[0][0];
  const unsigned lx0 = (unsigned)(size_t)(__attribute__((address_space(3))) void*)&lx[0][0];
  constexpr int kWStage = kR2N * kR2K * 2, kXStage = kR2T * kR2K * 2;   // bytes
  unsigned aoff[6], boff[8];
#pragma unroll
  for (int i = 0; i < 6; ++i) {
    const int ar = (kEpi == 3 ? (i / 3) * kRows + wy * 48 + 16 * (i % 3) : wy * 96 + 16 * i) + fr;
    aoff[i] = lw0 + (unsigned)(ar * kR2K * 2 + 16 * (fg ^ (ar & 7)));
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int br = wx * 128 + 16 * j + fr;
    boff[j] = lx0 + (unsigned)(br * kR2K * 2 + 16 * (fg ^ (br & 7)));
  }
  typedef f16x8 Frags[14];   // A blocks 0..5, then B blocks 0..7
  // Step 1's addresses are made opaque where they are formed, so they are
  // computed at each read rather than kept live across the loop.
  auto read1 = [&](f16x8& v, unsigned a, auto off) {
    constexpr int o = decltype(off)::value;
    if constexpr (o == 0)
      asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(a) : "memory");
    else
      asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(a), "i"(o) : "memory");
  };
  auto read_frags = [&](auto stage, int ks, Frags& f) {
    constexpr StageIdx<decltype(stage)::value * kWStage> wo{};
    constexpr StageIdx<decltype(stage)::value * kXStage> xo{};
#pragma unroll
    for (int i = 0; i < 14; ++i) {
      unsigned a = i < 6 ? aoff[i] : boff[i - 6];
      if (ks) {
        a ^= 64u;
        asm volatile("" : "+v"(a));
      }
      if (i < 6)
        read1(f[i], a, wo);
      else
        read1(f[i], a, xo);
    }
  };
  auto mfma_tile = [&](const Frags& f) {
#pragma unroll
    for (int i = 0; i < 6; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(f[i], f[6 + j], acc[i][j], 0, 0, 0);
  };
  // The fragments' registers are bound to each wait, so no use of them can be
  // scheduled before it.  Tile kt sits in stage kt % 2.  Step 0 of tile kt:
  // wait for the reads of its fragments, read step 1's from the same stage,
  // multiply.  Step 1: wait for those reads and for this thread's loads of
  // tile kt + 1 (the only loads in flight), and after the barrier every wave
  // has read tile kt's stage and every load of tile kt + 1 has landed: the
  // stage takes tile kt + 2, and tile kt + 1's step-0 fragments are read while
  // step 1 of tile kt is multiplied.
  auto wait_reads = [&](Frags& f) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]),
                   "+v"(f[6]), "+v"(f[7]), "+v"(f[8]), "+v"(f[9]), "+v"(f[10]), "+v"(f[11]),
                   "+v"(f[12]), "+v"(f[13])
                 :
                 : "memory");
  };
  auto wait_all = [&](Frags& f) {
    asm volatile("s_waitcnt vmcnt(6) lgkmcnt(0)\n\ts_barrier"
                 : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]),
                   "+v"(f[6]), "+v"(f[7]), "+v"(f[8]), "+v"(f[9]), "+v"(f[10]), "+v"(f[11]),
                   "+v"(f[12]), "+v"(f[13])
                 :
                 : "memory");
  };
  Frags fa, fb;
  // No branch splits a tile's products (the register allocator then moved
  // every accumulator at each tile): the last two tiles load the last tile
  // again into their free stage, and after the last tile the step-0 read of
  // the other stage only reads LDS that is never used.
  // Step 0 of tile kt also stores W(kt + 1) from wr into the other W stage
  // (every wave has read tile kt - 1's, which sat there, before the last
  // barrier) and loads W(kt + 2) into wr; step 1 waits for X(kt + 1), the
  // newest loads in flight being W(kt + 2)'s 6.
  auto tile = [&](int kt, auto own, auto next) {
    wait_reads(fa);
    store_w(decltype(next)::value);
    load_w(min(kt + 2, ktiles - 1));
    read_frags(own, 1, fb);
    mfma_tile(fa);
    wait_all(fb);
    issue_x(min(kt + 2, ktiles - 1), decltype(own)::value);
    read_frags(next, 0, fa);
    mfma_tile(fb);
  };
  constexpr StageIdx<0> k0{};
  constexpr StageIdx<1> k1{};
  load_w(0);
  issue_x(0, 0);
  store_w(0);
  load_w(min(1, ktiles - 1));
  issue_x(min(1, ktiles - 1), 1);
  asm volatile("s_waitcnt vmcnt(14) lgkmcnt(0)\n\ts_barrier" ::: "memory");   // W(0) stored, X(0) landed
  read_frags(k0, 0, fa);
  // Four tiles per trip with guards (two per trip, or a separate odd tile
  // after the loop, made the allocator move accumulators at every trip).
  for (int kt = 0; kt < ktiles; kt += 4) {
    tile(kt, k0, k1);
    if (kt + 1 < ktiles) tile(kt + 1, k1, k0);
    if (kt + 2 < ktiles) tile(kt + 2, k0, k1);
    if (kt + 3 < ktiles) tile(kt + 3, k1, k0);
  }
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");

  if constexpr (kEpi == 3) {
    // blocks (i, j) and (i + 3, j), i < 3: gate and up of outputs
    // n0 + 48 wy + 16 i + 4 (l / 16) + r, token t0 + 128 wx + 16 j + l % 16
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int t = t0 + wx * 128 + 16 * j + fr;
      if (t >= p.t) continue;
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        const int n = n0 + wy * 48 + 16 * i + fg * 4;
        if (n >= p.n) continue;
        f16x4_t v;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float gh = (float)to_f16(acc[i][j][r]);
          const float uh = (float)to_f16(acc[i + 3][j][r]);
          const float e = exp2_rep(-uh * kLog2e);
          v[r] = to_f16(gh * (uh / (1.0f + e)));
        }
        _Float16* dstp = reinterpret_cast<_Float16*>(p.y) + (long long)t * p.ldy + n;
        if (n + 4 <= p.n) {
          *reinterpret_cast<f16x4_t*>(dstp) = v;
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n + r < p.n) dstp[r] = v[r];
        }
      }
    }
    return;
  }
  // block (i, j): rows n0 + 96 wy + 16 i + 4 (l / 16) + r of W, token t0 + 128 wx + 16 j + l % 16
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int t = t0 + wx * 128 + 16 * j + fr;
    if (t >= p.t) continue;
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      const int n = n0 + wy * 96 + 16 * i + fg * 4;
      if (n >= p.n) continue;
      _Float16* dstp = reinterpret_cast<_Float16*>(p.y) + (long long)t * p.ldy + n;
      const _Float16* res = reinterpret_cast<const _Float16*>(p.res) + (long long)t * p.ldy + n;
      if (n + 4 <= p.n) {
        f16x4_t v;
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = to_f16(acc[i][j][r]);
        if constexpr (kEpi == 1) {
          const f16x4_t rv = *reinterpret_cast<const f16x4_t*>(res);
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] = (_Float16)((float)rv[r] + (float)v[r]);
        }
        *reinterpret_cast<f16x4_t*>(dstp) = v;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (n + r >= p.n) break;
          _Float16 y = to_f16(acc[i][j][r]);
          if constexpr (kEpi == 1) y = (_Float16)((float)res[r] + (float)y);
          dstp[r] = y;
        }
      }
    }
  }
}

}  // namespace

hipError_t launch_rmsnorm_batched(const uint16_t* x, const uint16_t* w, float eps, uint16_t* xn,
                                  int hidden, int T, hipStream_t stream) {
  const dim3 grid((T + 3) / 4), block(256);
  switch (hidden / 512) {
#define QD_CASE(n) \
    case n: hipLaunchKernelGGL(rmsnorm_batched_kernel<n>, grid, block, 0, stream, x, w, eps, xn, T); break;
    QD_CASE(1) QD_CASE(2) QD_CASE(3) QD_CASE(4) QD_CASE(5) QD_CASE(6) QD_CASE(7) QD_CASE(8)
#undef QD_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Compute units of the current device, read once per device.
static int device_cus() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = cached[dev].load(std::memory_order_relaxed);
  if (v <= 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    cached[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

hipError_t launch_gemv_batched(const BatchedGemvParams& p, int epi, hipStream_t stream) {
  const int nj = (p.k + 511) / 512;
  if (nj < 1 || nj > 16) return hipErrorInvalidValue;
  // Four rows per wave where it measured faster: K in (1536, 2048] with n >= 4096
  // (QKV and the gate/up rows of hidden 2048: 4.5-5% per launch inside the
  // engine's prefill, cold weights).  At n = 2048 (o_proj) it was no faster at
  // 127 tokens and 4% slower in 256-token chunks; narrower products have too few
  // workgroups for its 16-row workgroups of four waves.
  if (nj == 4 && p.n >= 4096) {
    const dim3 grid((p.n + 4 * kR4Waves - 1) / (4 * kR4Waves), (p.t + kTokPerWg - 1) / kTokPerWg);
    const size_t lds = (size_t)kR4Tile * nj * 512 * sizeof(float);
    switch (nj * 2 + epi) {
#define QD_CASE(n)                                                                                  \
    case 2 * n:                                                                                      \
      hipLaunchKernelGGL((gemv_batched_r4_kernel<n, 0>), grid, dim3(kR4Waves * 64), lds, stream, p); \
      break;                                                                                         \
    case 2 * n + 1:                                                                                  \
      hipLaunchKernelGGL((gemv_batched_r4_kernel<n, 1>), grid, dim3(kR4Waves * 64), lds, stream, p); \
      break;
      QD_CASE(1) QD_CASE(2) QD_CASE(3) QD_CASE(4)
#undef QD_CASE
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  const int waves = gemv_waves(nj);
  // From K > 4096 (one workgroup per CU) a workgroup takes 64 tokens instead of 32
  // when the grid still covers every CU and the last 64-token block is more than
  // half full: each weight row is then loaded half as often (c_proj at K = 5504:
  // 78.9 -> 70.4 us at 127 tokens, 152.9 -> 139.9 us at 256).  Narrower grids and
  // ragged last blocks ran slower that way.  Each output's sum is the same either way.
  BatchedGemvParams q = p;
  q.tok_per_wg = kTokPerWg;
  if (nj >= 9) {
    const long long wgs = (long long)((p.n + 2 * waves - 1) / (2 * waves)) * ((p.t + 63) / 64);
    const int rem = p.t % 64;
    if (wgs >= device_cus() && (rem == 0 || rem > 32)) q.tok_per_wg = 64;
  }
  const dim3 grid((p.n + 2 * waves - 1) / (2 * waves), (p.t + q.tok_per_wg - 1) / q.tok_per_wg);
  const size_t lds = (size_t)tok_tile(nj) * nj * 512 * sizeof(uint16_t);
  switch (nj * 2 + epi) {
#define QD_CASE(n)                                                                                  \
    case 2 * n:                                                                                      \
      hipLaunchKernelGGL((gemv_batched_kernel<n, 0>), grid, dim3(waves * 64), lds, stream, q);       \
      break;                                                                                         \
    case 2 * n + 1:                                                                                  \
      hipLaunchKernelGGL((gemv_batched_kernel<n, 1>), grid, dim3(waves * 64), lds, stream, q);       \
      break;
    QD_CASE(1) QD_CASE(2) QD_CASE(3) QD_CASE(4) QD_CASE(5) QD_CASE(6) QD_CASE(7) QD_CASE(8)
    QD_CASE(9) QD_CASE(10) QD_CASE(11) QD_CASE(12) QD_CASE(13) QD_CASE(14) QD_CASE(15) QD_CASE(16)
#undef QD_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_rope_batched(uint16_t* qkv, const uint16_t* bias, uint16_t* k_layer,
                               uint16_t* v_layer, const float2* rope_cs, long long row_stride,
                               long long head_stride, int pos0, int num_heads, int T,
                               hipStream_t stream) {
  // 8-byte vectors of Q, K, V and the cache rows; 16-byte reads of the table
  if (((reinterpret_cast<uintptr_t>(qkv) | reinterpret_cast<uintptr_t>(k_layer) |
        reinterpret_cast<uintptr_t>(v_layer)) & 7u) || (reinterpret_cast<uintptr_t>(rope_cs) & 15u) ||
      row_stride % 4 || head_stride % 4)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(rope_batched_kernel, dim3((num_heads + kRopeHeads - 1) / kRopeHeads, T),
                     dim3(kRopeHeads * 16), 0, stream, qkv, bias, k_layer,
                     v_layer, rope_cs, row_stride, head_stride, pos0, num_heads);
  return hipGetLastError();
}

hipError_t launch_swiglu_batched(const uint16_t* g, const uint16_t* u, uint16_t* act, int rows,
                                 int cols, long long ld, hipStream_t stream) {
  const long long n = (long long)rows * cols;
  if (rows < 1 || cols < 1 || ld < cols) return hipErrorInvalidValue;
  const bool vec8 = cols % 8 == 0 && ld % 8 == 0 &&
                    ((reinterpret_cast<uintptr_t>(g) | reinterpret_cast<uintptr_t>(u) |
                      reinterpret_cast<uintptr_t>(act)) & 15u) == 0;
  if (vec8)
    hipLaunchKernelGGL(swiglu_batched_kernel<8>, dim3((unsigned)((n / 8 + 255) / 256)), dim3(256), 0,
                       stream, g, u, act, rows, cols, ld);
  else
    hipLaunchKernelGGL(swiglu_batched_kernel<1>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       stream, g, u, act, rows, cols, ld);
  return hipGetLastError();
}

// Tile choice of a plain product from kRingMinRows tokens: 192 x 256 where
// that grid covers every CU (2048-token QKV: 256 tiles), else 128 x 128 where
// that grid covers at least half of them (a 128 x 128 grid of 192 tiles ran
// the 512-token QKV product as fast as hipBLASLt), else the 64 x 64 tile.
enum class GemmTile { k64, k128, k192 };

// The 128 x 128 tile's buffer loads take 32-bit byte offsets up to a tile past each operand's end.
static bool ring128_offsets32(const BatchedGemvParams& p) {
  return (long long)(p.n + kRgN) * p.k * 2 < (1LL << 32) && (long long)(p.t + kRgT) * p.ldx * 2 < (1LL << 32);
}

static GemmTile pick_tile(const BatchedGemvParams& p, int rows_per_out) {
  const bool vec8 = ((reinterpret_cast<uintptr_t>(p.y) | reinterpret_cast<uintptr_t>(p.res)) & 7u) == 0 &&
                    p.ldy % 4 == 0;
  if (p.t < kRingMinRows || !vec8) return GemmTile::k64;
  const int cus = device_cus();
  const long long big = (long long)((p.n * rows_per_out + kR2N - 1) / kR2N) * ((p.t + kR2T - 1) / kR2T);
  // the 192 x 256 tile's buffer loads take 32-bit byte offsets up to a tile past each operand's end
  const bool offsets32 = (long long)(p.n + kR2N) * p.k * 2 < (1LL << 32) &&
                         (long long)(p.t + kR2T) * p.ldx * 2 < (1LL << 32);
  if (big >= cus && offsets32) return GemmTile::k192;
  const long long mid = (long long)((p.n * rows_per_out + kRgN - 1) / kRgN) * ((p.t + kRgT - 1) / kRgT);
  return 2 * mid >= cus && ring128_offsets32(p) ? GemmTile::k128 : GemmTile::k64;
}

hipError_t launch_gemm_mfma(const BatchedGemvParams& p, int epi, hipStream_t stream) {
  if (p.k < 64 || p.k % 64 != 0 || p.t < 1 || p.n < 1) return hipErrorInvalidValue;
  switch (pick_tile(p, 1)) {
    case GemmTile::k192: {
      const dim3 grid((unsigned)(((p.n + kR2N - 1) / kR2N) * ((p.t + kR2T - 1) / kR2T)));
      if (epi == 0)
        hipLaunchKernelGGL(gemm_nt_ring192_kernel<0>, grid, dim3(256), 0, stream, p);
      else
        hipLaunchKernelGGL(gemm_nt_ring192_kernel<1>, grid, dim3(256), 0, stream, p);
      return hipGetLastError();
    }
    case GemmTile::k128: {
      const dim3 grid((unsigned)(((p.n + kRgN - 1) / kRgN) * ((p.t + kRgT - 1) / kRgT)));
      if (epi == 0)
        hipLaunchKernelGGL(gemm_nt_ring128_kernel<0>, grid, dim3(256), 0, stream, p);
      else
        hipLaunchKernelGGL(gemm_nt_ring128_kernel<1>, grid, dim3(256), 0, stream, p);
      return hipGetLastError();
    }
    default:
      break;
  }
  const dim3 grid((p.n + kMmTile - 1) / kMmTile, (p.t + kMmTile - 1) / kMmTile);
  if (epi == 0)
    hipLaunchKernelGGL(gemm_nt_mfma_kernel<0>, grid, dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(gemm_nt_mfma_kernel<1>, grid, dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_gemm_mfma_swiglu(const BatchedGemvParams& p, hipStream_t stream) {
  if (p.k < 64 || p.k % 64 != 0 || p.n < 1 || p.t < 1 || !p.w2) return hipErrorNotSupported;
  switch (pick_tile(p, 2)) {   // two W rows (gate and up) per output
    case GemmTile::k192:
      hipLaunchKernelGGL(gemm_nt_ring192_kernel<3>,
                         dim3((unsigned)(((p.n + kR2N / 2 - 1) / (kR2N / 2)) * ((p.t + kR2T - 1) / kR2T))),
                         dim3(256), 0, stream, p);
      break;
    case GemmTile::k128:
      hipLaunchKernelGGL(gemm_nt_ring128_kernel<3>,
                         dim3((unsigned)(((p.n + kRgN / 2 - 1) / (kRgN / 2)) * ((p.t + kRgT - 1) / kRgT))),
                         dim3(256), 0, stream, p);
      break;
    default: {
      const dim3 grid((p.n + kMmTile / 2 - 1) / (kMmTile / 2), (p.t + kMmTile - 1) / kMmTile);
      hipLaunchKernelGGL(gemm_nt_mfma_kernel<3>, grid, dim3(256), 0, stream, p);
      break;
    }
  }
  return hipGetLastError();
}

// Splits K over up to kGemmMaxSplits slices of whole 64-wide tiles when the
// product's grid leaves CUs idle and the workspace holds the slices' fp32
// partials; one launch then adds the slices in order with the epilogue
// (splitk_fold_kernel).  From kRingMinRows tokens with n a multiple of 4 the
// slices run on the 128 x 128 ring tile (the 256-token c_proj product: 32
// tiles of K = 5504), below it on the 64 x 64 tile.
hipError_t launch_gemm_mfma_split(const BatchedGemvParams& p, int epi, float* workspace,
                                  size_t workspace_bytes, hipStream_t stream) {
  if (p.k < 64 || p.k % 64 != 0 || p.t < 1 || p.n < 1) return hipErrorInvalidValue;
  const GemmTile tile = pick_tile(p, 1);
  const bool ring = p.t >= kRingMinRows && p.n % 4 == 0 && tile != GemmTile::k192 && ring128_offsets32(p) &&
                    ((reinterpret_cast<uintptr_t>(p.y) | reinterpret_cast<uintptr_t>(p.res)) & 7u) == 0 &&
                    p.ldy % 4 == 0;
  const int tn = ring ? kRgN : kMmTile, tt = ring ? kRgT : kMmTile;
  const long long tiles = (long long)((p.n + tn - 1) / tn) * ((p.t + tt - 1) / tt);
  const int cus = device_cus();
  int splits = 1;
  if (workspace && tile != GemmTile::k192 && tiles < cus)
    splits = (int)std::min<long long>(kGemmMaxSplits, (cus + tiles - 1) / tiles);
  if (splits > 1) {
    // slices of whole K tiles, none empty, as many as the workspace holds
    while (splits > 1 && (size_t)splits * p.t * p.n * sizeof(float) > workspace_bytes) --splits;
    const int kslice = ((p.k + splits - 1) / splits + kMmK - 1) / kMmK * kMmK;
    splits = (p.k + kslice - 1) / kslice;
    if (splits > 1) {
      BatchedGemvParams q = p;
      q.part = workspace;
      q.kslice = kslice;
      if (ring)
        hipLaunchKernelGGL(gemm_nt_ring128_kernel<2>, dim3((unsigned)tiles, splits), dim3(256), 0, stream, q);
      else
        hipLaunchKernelGGL(gemm_nt_mfma_kernel<2>,
                           dim3((p.n + kMmTile - 1) / kMmTile, (p.t + kMmTile - 1) / kMmTile, splits),
                           dim3(256), 0, stream, q);
      hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
      const dim3 fgrid((unsigned)(((long long)p.t * p.n + 255) / 256));
      if (epi == 0)
        hipLaunchKernelGGL(splitk_fold_kernel<0>, fgrid, dim3(256), 0, stream, q, splits);
      else
        hipLaunchKernelGGL(splitk_fold_kernel<1>, fgrid, dim3(256), 0, stream, q, splits);
      return hipGetLastError();
    }
  }
  return launch_gemm_mfma(p, epi, stream);
}

hipError_t launch_embed(const uint16_t* wte, const int* tokens, uint16_t* x, int hidden, int T,
                        hipStream_t stream) {
  hipLaunchKernelGGL(embed_kernel, dim3(T), dim3(256), 0, stream, wte, tokens, x, hidden);
  return hipGetLastError();
}

}  // namespace qd
