// q4k.hpp -- Q4_K weight dequantisation and matrix-vector product (gfx950).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sts {

// A Q4_K matrix [N][K]: N rows of K/256 super-blocks of 144 bytes each
// (crates/sts-wasm/src/wgsl/shader_q4k_matvec.wgsl:13-19).
constexpr uint32_t kQ4kBlockBytes = 144;
constexpr uint32_t kQ4kBlockWeights = 256;

// Exact binary16 -> binary32 (v_cvt_f32_f16), as WGSL unpack2x16float.
__device__ __forceinline__ float half_bits_to_float(uint32_t bits) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)(bits & 0xFFFFu));
}

// 6-bit scale and min of sub-block j from the packed scale bytes held in
// s0 (bytes 0-3), s1 (4-7), s2 (8-11); shader_q4k_matvec.wgsl:85-113.
__device__ __forceinline__ void scale_min(uint32_t s0, uint32_t s1, uint32_t s2, uint32_t j,
                                          uint32_t& sc, uint32_t& mn) {
  const uint32_t sh = 8u * (j & 3u);
  const uint32_t b0 = (s0 >> sh) & 0xFFu, b1 = (s1 >> sh) & 0xFFu, b2 = (s2 >> sh) & 0xFFu;
  if (j < 4) {
    sc = b0 & 63u;
    mn = b1 & 63u;
  } else {
    sc = (b2 & 0xFu) | ((b0 >> 6) << 4);
    mn = (b2 >> 4) | ((b1 >> 6) << 4);
  }
}

struct Q4kParams {
  const uint8_t* w = nullptr;    // N * K/256 blocks
  const float* x = nullptr;      // [B][K]
  const float* res = nullptr;    // [B][N] or null
  float* y = nullptr;            // [B][N]
  uint32_t B = 0, K = 0, N = 0;
};

// y[b][n] = sum_k W[n][k] x[b][k] (+ res[b][n]).
int launch_q4k_matvec(const Q4kParams& p, hipStream_t stream);

// out[n][k] = W[n][k] as f32, in the reference shader's rounding order.
int launch_q4k_dequant(const uint8_t* w, float* out, uint32_t N, uint32_t K, hipStream_t stream);

}  // namespace sts
