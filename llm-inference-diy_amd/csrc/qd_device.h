// Device helpers shared by the gfx950 kernels: fp16 vector types and the
// wave64 reductions built on DPP row operations.
#pragma once

#include <hip/hip_runtime.h>

namespace qd {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

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

// Sum over all 64 lanes: row sums, then (row0 + row1) + (row2 + row3).  Every
// lane receives the same value.
__device__ __forceinline__ float wave64_sum(float x) {
  x = row16_sum(x);
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}

}  // namespace qd
