// Device helpers shared by the gfx950 kernels: fp16 vector types and the
// wave64 reductions built on DPP row operations.
#pragma once

#include <hip/hip_runtime.h>

namespace qd {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// fp32 -> fp16, round to nearest even, of a value already rounded to fp32.
// The empty asm pins x as an fp32 register value, so the compiler cannot fold
// the multiply or add that produced it into the conversion (v_fma_mixlo_f16
// and v_mad_mixlo_f16 round once, straight to fp16, which differs from
// rounding to fp32 first wherever the fp32 value sits on an fp16 tie).
__device__ __forceinline__ _Float16 to_f16(float x) {
  asm volatile("" : "+v"(x));
  return (_Float16)x;
}

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

// Sum over the 16 lanes of a DPP row: ((a0+a1)+(a2+a3)) + ((a4+a5)+(a6+a7)),
// then the two half-rows.  All 16 lanes receive the same value (each step adds
// a partner whose value is the mirror image of its own).
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_mov<kDppQuadSwap1>(x);
  x += dpp_mov<kDppQuadSwap2>(x);
  x += dpp_mov<kDppHalfMirror>(x);
  x += dpp_mov<kDppMirror>(x);
  return x;
}

// Maximum over the 16 lanes of a DPP row (fmaxf: exact in any order, NaN only
// if every lane is NaN).  All 16 lanes receive it.
__device__ __forceinline__ float row16_max(float x) {
  x = fmaxf(x, dpp_mov<kDppQuadSwap1>(x));
  x = fmaxf(x, dpp_mov<kDppQuadSwap2>(x));
  x = fmaxf(x, dpp_mov<kDppHalfMirror>(x));
  x = fmaxf(x, dpp_mov<kDppMirror>(x));
  return x;
}

// Maximum over all 64 lanes; every lane receives it.
__device__ __forceinline__ float wave64_max(float x) {
  x = row16_max(x);
  x = fmaxf(x, __shfl_xor(x, 16));
  x = fmaxf(x, __shfl_xor(x, 32));
  return x;
}

// Sum over all 64 lanes: row sums, then (row0 + row1) + (row2 + row3).  Every
// lane receives the same value.
__device__ __forceinline__ float wave64_sum(float x) {
  x = row16_sum(x);
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}

// 2^x, reproducible bit for bit by a host implementation of the same steps
// (all library code is built with -ffp-contract=off, so each operation below
// rounds exactly once):
//   n = rint(x) (ties to even), f = x - n (exact, |f| <= 1/2),
//   2^f ~= 1 + f*q(f), q(f) = c1 + c2 f + ... + c6 f^5 evaluated in Estrin
//   form: (c1 + c2 f) + f^2 ((c3 + c4 f) + f^2 (c5 + c6 f)), each bracket an
//   fmaf, then one fmaf for 1 + f*q;
//   result = ldexp(2^f, n).
// Dependency depth is 4 fmaf after f (Horner would be 6); the kernels that
// call it run one wave per SIMD, so latency is what matters.  The
// coefficients were fitted to 2^f on [-1/2, 1/2] by iteratively reweighted
// least squares on 4000 Chebyshev nodes and rounded to fp32; this evaluation
// is within 1.25 ulp of 2^f there (1.17 the largest error seen in 2e7
// samples).  exp2_rep(0) == 1 exactly.  Inputs <= -125
// and NaN give 0 (so no result is subnormal); inputs >= 128 give +inf.
//
// Branch-free: the polynomial runs on x clamped to [-126, 128] (v_med3_f32;
// a NaN clamps to -126) and the out-of-range results are selected at the end,
// so a wave never splits on it.  In range the clamp leaves x unchanged.
__device__ __forceinline__ float exp2_rep(float x) {
  const float xc = __builtin_amdgcn_fmed3f(x, -126.0f, 128.0f);
  const float n = __builtin_rintf(xc);
  const float f = xc - n;
  const float f2 = f * f;
  const float a = __builtin_fmaf(0x1.ebfbdcp-3f, f, 0x1.62e430p-1f);
  const float b = __builtin_fmaf(0x1.3b2d4ep-7f, f, 0x1.c6aee8p-5f);
  const float c = __builtin_fmaf(0x1.41fbb0p-13f, f, 0x1.5f3e54p-10f);
  const float q = __builtin_fmaf(__builtin_fmaf(c, f2, b), f2, a);
  const float r = __builtin_ldexpf(__builtin_fmaf(q, f, 1.0f), (int)n);
  return x >= 128.0f ? __builtin_inff() : (x > -125.0f ? r : 0.0f);
}

// exp2_rep for arguments known to be <= 0 (or -inf / NaN), as every softmax
// exponent is: the same operations on the same clamped value, so the result is
// bit-identical to exp2_rep(x), without the overflow select.
__device__ __forceinline__ float exp2_rep_nonpos(float x) {
  const float xc = fmaxf(x, -126.0f);
  const float n = __builtin_rintf(xc);
  const float f = xc - n;
  const float f2 = f * f;
  const float a = __builtin_fmaf(0x1.ebfbdcp-3f, f, 0x1.62e430p-1f);
  const float b = __builtin_fmaf(0x1.3b2d4ep-7f, f, 0x1.c6aee8p-5f);
  const float c = __builtin_fmaf(0x1.41fbb0p-13f, f, 0x1.5f3e54p-10f);
  const float q = __builtin_fmaf(__builtin_fmaf(c, f2, b), f2, a);
  const float r = __builtin_ldexpf(__builtin_fmaf(q, f, 1.0f), (int)n);
  return x > -125.0f ? r : 0.0f;
}

}  // namespace qd
