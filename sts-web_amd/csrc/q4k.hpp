// q4k.hpp -- Q4_K weight dequantisation and matrix-vector product (gfx950).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sts {

// A Q4_K matrix [N][K]: N rows of K/256 super-blocks of 144 bytes each
// (crates/sts-wasm/src/wgsl/shader_q4k_matvec.wgsl:13-19).
constexpr uint32_t kQ4kBlockBytes = 144;
constexpr uint32_t kQ4kBlockWeights = 256;

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
