// depformer.hpp -- the depformer step chain (crates/sts-wasm/src/depth_engine.rs:884-1491)
// batched over streams: Q4_K GEMM on f32 MFMA, RMSNorm, embedding + add, top-k sampling.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sts {

constexpr int kGemmMaxZ = 16;        // weight matrices per batched GEMM launch
constexpr uint32_t kMaxPenalty = 30; // penalty tokens per (stream, step), depth_engine.rs:909
constexpr uint32_t kMaxTopK = 256;   // shader_sample_topk.wgsl:18
constexpr uint32_t kMaxVocab = 4096; // logits row held in LDS by the sampler

// Y_z[m][n] = sum_k W_z[n][k] X_z[m][k] (+ R[m][n]) for m < M, n < N, one Q4_K
// matrix W_z per grid z.  With swiglu_f > 0 the matrix has 2F rows and the
// output is Y[m][j] = silu(G[m][j]) * G[m][j + F] for j < F
// (shader_swiglu.wgsl:30-34 applied to the product).
struct Q4kGemmParams {
  const uint8_t* w[kGemmMaxZ] = {};
  const float* x = nullptr;
  const float* res = nullptr;
  float* y = nullptr;
  uint32_t M = 0, N = 0, K = 0, Z = 1;
  uint64_t ldx = 0, ldy = 0, ldr = 0;  // row strides (floats)
  uint64_t x_zstride = 0, y_zstride = 0;
  uint32_t swiglu_f = 0;
  // With norm_alpha set, each x row is RMS-normalised: x * (1 / sqrt(sum x^2 /
  // K + norm_eps)) * norm_alpha (shader_rmsnorm.wgsl's formula), with the sum
  // of squares taken in this kernel's order, alpha applied to x on load and
  // the row's 1/rms to its outputs.
  const float* norm_alpha = nullptr;
  float norm_eps = 0.f;
  // Super-blocks per weight row when the launch covers only part of K (a
  // split-K slice of a wider matrix); 0: K / 256.
  uint32_t w_row_blocks = 0;
};
// K above 4096 (no RMSNorm or SwiGLU, Z = 1) runs as ceil(K / 4096) slices
// into a stream workspace, summed in slice order by a second kernel that also
// adds the residual: deterministic, and refused while the stream is being
// captured if the workspace has to grow.
int launch_q4k_gemm(const Q4kGemmParams& p, hipStream_t stream);

// out[b][i] = x[b][i] * (1 / sqrt(sum x^2 / D + eps)) * alpha[i] in the
// order of shader_rmsnorm.wgsl:27-92, one workgroup per row.
int launch_rmsnorm(const float* x, const float* alpha, float* out, uint32_t rows, uint32_t D,
                   float eps, hipStream_t stream);

// h[b][e] = proj[b][e] + embed(table, token of stream b)[e] for a Q4_0 table
// [vocab][D] (shader_embed_q4.wgsl:58-107, shader_vec_add.wgsl:20-28).  The
// token of stream b is tokens[b * tok_stride].
int launch_embed_add(const uint8_t* table, uint32_t vocab, const uint32_t* tokens,
                     uint64_t tok_stride, const float* proj, float* h, uint32_t B, uint32_t D,
                     hipStream_t stream);

// shader_sample_topk.wgsl on logits[b] [V] for each stream b (the logits are
// not modified).  Per stream: rand[b * rs_stride], penalty tokens
// ptoks[b * pt_stride .. + num_penalty[b * rs_stride]]; the token goes to
// out[b * out_stride].
struct SampleParams {
  const float* logits = nullptr;
  uint64_t ld_logits = 0;
  uint32_t B = 0, V = 0, top_k = 0;
  float temperature = 1.f, penalty = 1.f;
  const float* rand = nullptr;
  const uint32_t* ptoks = nullptr;
  const uint32_t* num_penalty = nullptr;
  uint64_t rs_stride = 1, pt_stride = 0;
  uint32_t* out = nullptr;
  uint64_t out_stride = 1;
};
int launch_sample_topk(const SampleParams& p, hipStream_t stream);

}  // namespace sts
