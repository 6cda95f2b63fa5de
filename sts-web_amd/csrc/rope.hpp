// rope.hpp -- interleaved rotary embedding of two adjacent pairs, as
// RoPE::apply_rope_to_tensor computes it (crates/sts-wasm/src/model.rs:99-100):
// (x0, x1) -> (x0*c - x1*s, x0*s + x1*c), every product and sum rounded
// separately, so rows rotated here equal the oracle's bit for bit.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sts {

// Pairs (x.x, x.y) and (x.z, x.w) rotated by (cs.x, sn.x) and (cs.y, sn.y).
__device__ __forceinline__ float4 rope4(float4 x, float2 cs, float2 sn) {
#pragma clang fp contract(off)
  float4 y;
  y.x = x.x * cs.x - x.y * sn.x;
  y.y = x.x * sn.x + x.y * cs.x;
  y.z = x.z * cs.y - x.w * sn.y;
  y.w = x.z * sn.y + x.w * cs.y;
  return y;
}

// Table entries for the pairs of dims d0, d0+1, d0+2, d0+3 (d0 % 4 == 0) at
// position pos of [max_pos][D/2] cos/sin tables.
template <int D>
__device__ __forceinline__ void rope_coeffs(const float* cos_t, const float* sin_t, uint32_t pos,
                                            int d0, float2& cs, float2& sn) {
  const size_t ro = (size_t)pos * (D / 2) + d0 / 2;
  cs = *reinterpret_cast<const float2*>(cos_t + ro);
  sn = *reinterpret_cast<const float2*>(sin_t + ro);
}

}  // namespace sts
