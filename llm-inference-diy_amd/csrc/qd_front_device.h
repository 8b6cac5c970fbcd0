// Device code of the decode step's attention front end, shared by
// qkv_front_kernel (qd_decode_ops.hip) and the fused front end + attention
// kernel (qd_attention.hip): the GEMV lane layout, the RMSNorm, and one wave's
// work for one (head, rotation pair), bias, RoPE and KV append included.
#pragma once

#include "qd_device.h"
#include "qd_internal.h"

namespace qd {
namespace {

constexpr float kLog2e = 1.44269504088896340736f;

// This lane's x elements k = 512*j + 8*l + e, and the RMSNorm weights when
// norm_w is non-null.  Issued before a kernel's weight loads: x and norm_w are
// small and L2-resident, so the normalisation below waits only for them while
// the weight rows are still in flight (loads complete in issue order).
template <int NJ>
__device__ __forceinline__ void issue_input(const uint16_t* __restrict__ x,
                                            const uint16_t* __restrict__ norm_w, int lane,
                                            f16x8 (&xv)[NJ], f16x8 (&nv)[NJ]) {
#pragma unroll
  for (int j = 0; j < NJ; ++j) xv[j] = *reinterpret_cast<const f16x8*>(x + 512 * j + 8 * lane);
  if (norm_w == nullptr) return;
#pragma unroll
  for (int j = 0; j < NJ; ++j) nv[j] = *reinterpret_cast<const f16x8*>(norm_w + 512 * j + 8 * lane);
}

// RMSNorm in place (rmsnorm.cuh:6-57): x * (1 / sqrt(sum(x^2) / n + eps)) * w
// with the sum of squares in the wave64 order, correctly rounded sqrt and
// divide, each product rounded to fp32 and the result to fp16.  (HIP's
// __fsqrt_rn is the native v_sqrt_f32, not correctly rounded; sqrtf and '/'
// are, by hipcc's default -fhip-fp32-correctly-rounded-divide-sqrt.)
template <int NJ>
__device__ __forceinline__ void normalise(f16x8 (&xv)[NJ], const f16x8 (&nv)[NJ], float eps) {
  constexpr int hidden = NJ * 512;
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = (float)xv[j][e];
      acc = __builtin_fmaf(v, v, acc);   // exact square: rounds only the sum
    }
  const float var = wave64_sum(acc) / (float)hidden;
  const float r = 1.0f / __builtin_sqrtf(var + eps);
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) xv[j][e] = to_f16(((float)xv[j][e] * r) * (float)nv[j][e]);
}

// Non-temporal loads of this lane's chunks of a weight row (read once).
template <int NJ>
__device__ __forceinline__ void issue_row(const uint16_t* __restrict__ w_row, int lane,
                                          f16x8 (&wv)[NJ]) {
#pragma unroll
  for (int j = 0; j < NJ; ++j)
    wv[j] = __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(w_row + 512 * j + 8 * lane));
}

// This lane's sequential sum over (j, e) of exact fp16 products.
template <int NJ>
__device__ __forceinline__ float lane_sum(const f16x8 (&wv)[NJ], const f16x8 (&xv)[NJ]) {
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e)   // exact product: the fmaf rounds only the sum
      acc = __builtin_fmaf((float)wv[j][e], (float)xv[j][e], acc);
  return acc;
}

// The final values of one pair (h, i): rotated Q (q1 at dim i, q2 at i + 64),
// biased K (kb, qkv's K section), rotated K (kr, the cache row) and biased V
// (v, qkv's V section and the cache row).
struct FrontPair {
  _Float16 q1, q2, kb1, kb2, kr1, kr2, v1, v2;
};

// Bias and rotate-half RoPE of pair (h, i), evaluated as written (each
// product and sum rounded; no contraction), on the six GEMV outputs
// y = {q1, q2, k1, k2, v1, v2}.
__device__ __forceinline__ FrontPair front_finish(bool bias, const _Float16* y,
                                                  const _Float16 (&bias6)[6], float2 cs) {
  _Float16 v6[6];
#pragma unroll
  for (int r = 0; r < 6; ++r) v6[r] = bias ? (_Float16)((float)y[r] + (float)bias6[r]) : y[r];
  const float q1 = (float)v6[0], q2 = (float)v6[1], k1 = (float)v6[2], k2 = (float)v6[3];
  const float q1c = q1 * cs.x, q2s = q2 * cs.y, q2c = q2 * cs.x, q1s = q1 * cs.y;
  const float k1c = k1 * cs.x, k2s = k2 * cs.y, k2c = k2 * cs.x, k1s = k1 * cs.y;
  FrontPair o;
  o.q1 = to_f16(q1c - q2s);
  o.q2 = to_f16(q2c + q1s);
  o.kb1 = v6[2];
  o.kb2 = v6[3];
  o.kr1 = to_f16(k1c - k2s);
  o.kr2 = to_f16(k2c + k1s);
  o.v1 = v6[4];
  o.v2 = v6[5];
  return o;
}

// Stores of pair (h, i): qkv (Q rotated, K and V biased) and the cache row at
// p.pos (K rotated, V).
__device__ __forceinline__ void front_store(const QkvFrontParams& p, int h, int i, int hidden,
                                            const FrontPair& o) {
  _Float16* qkv = reinterpret_cast<_Float16*>(p.qkv);
  const int idx1 = h * 128 + i;
  qkv[idx1] = o.q1;
  qkv[idx1 + 64] = o.q2;
  qkv[hidden + idx1] = o.kb1;
  qkv[hidden + idx1 + 64] = o.kb2;
  qkv[2 * hidden + idx1] = o.v1;
  qkv[2 * hidden + idx1 + 64] = o.v2;
  const long long base = (long long)p.pos * p.row_stride + (long long)h * p.head_stride;
  _Float16* kc = reinterpret_cast<_Float16*>(p.k_layer) + base;
  _Float16* vc = reinterpret_cast<_Float16*>(p.v_layer) + base;
  kc[i] = o.kr1;
  kc[64 + i] = o.kr2;
  vc[i] = o.v1;
  vc[64 + i] = o.v2;
}

// Rows of one pair in flight per phase: at most 24 16-byte chunks per lane
// (all six rows up to hidden 2048, then two phases of three rows).
constexpr int qkv_rows_per_phase(int nj) { return nj <= 4 ? 6 : 3; }
constexpr int kQkvPairsPerBlock = 4;

struct NoLoads {
  __device__ void operator()() const {}
};

// One wave's share of the front end (qkv_front_kernel's work for pair (h, i)):
// rows q(i), q(i+64), k(i), k(i+64), v(i), v(i+64) as six GEMVs in flight,
// then the bias and rotation (front_finish) and, with kStore, lane 0's stores
// to qkv and the cache (front_store).  Returns the pair's final values in
// every lane.  kBiasWords: the bias pointer is 4-byte aligned, so each bias
// value is read with a scalar load of its 32-bit word.  after_rows() runs
// once the weight rows' loads (and the epilogue's operands) are issued: loads
// it issues go out behind them and stay in flight through the sums (loads
// complete in issue order).
template <int NJ, bool kBiasWords, bool kStore = true, class After = NoLoads>
__device__ __forceinline__ FrontPair qkv_front_pair(const QkvFrontParams& p, int h, int i, int lane,
                                                    After&& after_rows = After{}) {
  constexpr int RG = qkv_rows_per_phase(NJ);
  const int hidden = NJ * 512;
  // row r: (r >> 1) selects Q, K, V; (r & 1) the rotation half
  auto row_ptr = [&](int r) {
    return p.w + (long long)((r >> 1) * hidden + h * 128 + i + (r & 1) * 64) * hidden;
  };
  f16x8 xv[NJ], nv[NJ], wv[RG][NJ];
  issue_input<NJ>(p.x, p.norm_w, lane, xv, nv);
#pragma unroll
  for (int r = 0; r < RG; ++r) issue_row<NJ>(row_ptr(r), lane, wv[r]);
  __builtin_amdgcn_sched_barrier(0);
  // The epilogue's operands (wave-uniform), fetched while the weight rows are
  // in flight: a 4-byte-aligned bias with scalar loads of the 32-bit word
  // holding each value, any other 2-byte-aligned one 16 bits at a time into
  // registers that stay untouched until the epilogue.  Either way nothing here
  // waits for the weight stream.
  // Read through the constant address space: the values are read-only here
  // and wave-uniform, so they are scalar loads whatever code surrounds them.
  typedef const __attribute__((address_space(4))) uint64_t ConstU64;
  typedef const __attribute__((address_space(4))) uint32_t ConstU32;
  uint32_t bias_bits[6] = {};
  const uint64_t cs_bits = *(ConstU64*)(uintptr_t)(p.rope_cs + p.pos * 64 + i);
  float2 cs;
  cs.x = __uint_as_float((uint32_t)cs_bits);
  cs.y = __uint_as_float((uint32_t)(cs_bits >> 32));
  if (p.bias) {
#pragma unroll
    for (int r = 0; r < 6; ++r) {
      const int idx = (r >> 1) * hidden + h * 128 + i + (r & 1) * 64;
      if constexpr (kBiasWords)
        bias_bits[r] = (((ConstU32*)(uintptr_t)p.bias)[idx >> 1] >> (16 * (idx & 1))) & 0xFFFFu;
      else
        bias_bits[r] = p.bias[idx];
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  after_rows();
  __builtin_amdgcn_sched_barrier(0);
  if (p.norm_w) normalise<NJ>(xv, nv, p.eps);
  _Float16 y[6];                               // hgemv's half outputs
#pragma unroll
  for (int r = 0; r < RG; ++r) y[r] = to_f16(wave64_sum(lane_sum<NJ>(wv[r], xv)));
  if constexpr (RG < 6) {
#pragma unroll
    for (int r = 0; r < 6 - RG; ++r) issue_row<NJ>(row_ptr(RG + r), lane, wv[r]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < 6 - RG; ++r) y[RG + r] = to_f16(wave64_sum(lane_sum<NJ>(wv[r], xv)));
  }
  _Float16 bias6[6];
#pragma unroll
  for (int r = 0; r < 6; ++r) bias6[r] = __builtin_bit_cast(_Float16, (uint16_t)bias_bits[r]);
  const FrontPair o = front_finish(p.bias != nullptr, y, bias6, cs);
  if (kStore && lane == 0) front_store(p, h, i, hidden, o);
  return o;
}

}  // namespace
}  // namespace qd
