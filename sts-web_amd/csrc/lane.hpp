// lane.hpp -- cross-lane exchanges inside a 64-wide CDNA wavefront.
//
// DPP row operations act within 16-lane rows; ds_swizzle bitmask mode acts
// within 32-lane halves; a 32-lane exchange goes through ds_bpermute, or, for
// reductions, through the gfx950 permlane swaps at the end of this file.
// All exchanges here are involutions, so both partners see each other.
#pragma once

#include <hip/hip_runtime.h>

namespace sts {

// GFX9 DPP control encodings.
constexpr int kDppQuadXor1 = 0xB1;      // quad_perm [1,0,3,2]       : lane ^ 1
constexpr int kDppQuadXor2 = 0x4E;      // quad_perm [2,3,0,1]       : lane ^ 2
constexpr int kDppRowHalfMirror = 0x141;  // row_half_mirror (8 lanes) : lane ^ 7
constexpr int kDppRowMirror = 0x140;    // row_mirror (16 lanes)     : lane ^ 15

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// ds_swizzle bitmask mode: and=0x1F, or=0, xor=0x10 -> lane ^ 16 within 32 lanes.
__device__ __forceinline__ float swizzle_xor16(float x) {
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x401F));
}

__device__ __forceinline__ float xor32(float x) { return __shfl_xor(x, 32, 64); }

// Exchange with the partner lane whose index differs in bit LEVEL of the lane
// index (LEVEL 0..4).  Levels 2, 3 use the mirror forms (lane ^ 7, lane ^ 15),
// which flip the wanted bit and lower bits only; for butterflies the xor masks
// {1, 2, 7, 15, 16} span all five bits, so reductions over them are complete.
template <int LEVEL>
__device__ __forceinline__ float xchg(float x) {
  if constexpr (LEVEL == 0) return dpp_f32<kDppQuadXor1>(x);
  else if constexpr (LEVEL == 1) return dpp_f32<kDppQuadXor2>(x);
  else if constexpr (LEVEL == 2) return dpp_f32<kDppRowHalfMirror>(x);
  else if constexpr (LEVEL == 3) return dpp_f32<kDppRowMirror>(x);
  else return swizzle_xor16(x);
}

// gfx950 v_permlane16_swap / v_permlane32_swap called with x in both
// operands return a pair that holds, on every lane, x itself and the value of
// the partner lane (lane ^ 16, resp. lane ^ 32), in an order that depends on
// the lane.  A commutative op of the pair is therefore x op partner(x) on
// every lane, computed on the VALU without a trip through the LDS unit.
__device__ __forceinline__ float max_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

}  // namespace sts
