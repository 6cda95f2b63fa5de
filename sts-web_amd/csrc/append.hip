// append.hip -- ring-buffer KV append and RoPE for gfx950.
//
// cache_write replaces shader_cache_write.wgsl (crates/sts-wasm/src/wgsl/
// shader_cache_write.wgsl:19-49): the same slot formula, moved as 128-bit
// vectors when head_dim allows (bit-identical, it is a copy).  rope_apply
// replaces RoPE::apply_rope_to_tensor (crates/sts-wasm/src/model.rs:79-105).
#include <algorithm>

#include "append.hpp"
#include "common.hpp"
#include "rope.hpp"

namespace sts {

namespace {

// One thread per 4 consecutive elements of input [B][S][H][D] (D % 4 == 0).
__global__ __launch_bounds__(256) void cache_write_vec4(const float4* __restrict__ in,
                                                        float* __restrict__ cache,
                                                        uint32_t pos_offset, uint32_t S,
                                                        uint32_t H, uint32_t D4,
                                                        uint32_t max_len, uint64_t total4) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total4) return;
  const uint32_t d4 = (uint32_t)(i % D4);
  const uint64_t rem = i / D4;
  const uint32_t h = (uint32_t)(rem % H);
  const uint64_t rem2 = rem / H;
  const uint32_t s = (uint32_t)(rem2 % S);
  const uint64_t b = rem2 / S;
  const uint32_t slot = (uint32_t)(((uint64_t)pos_offset + s) % max_len);
  const uint64_t dst = ((b * H + h) * max_len + slot) * D4 + d4;
  reinterpret_cast<float4*>(cache)[dst] = in[i];
}

// Scalar form for head_dim not a multiple of 4 (the shader's own shape).
__global__ __launch_bounds__(256) void cache_write_scalar(const float* __restrict__ in,
                                                          float* __restrict__ cache,
                                                          uint32_t pos_offset, uint32_t S,
                                                          uint32_t H, uint32_t D,
                                                          uint32_t max_len, uint64_t total) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const uint32_t d = (uint32_t)(i % D);
  const uint64_t rem = i / D;
  const uint32_t h = (uint32_t)(rem % H);
  const uint64_t rem2 = rem / H;
  const uint32_t s = (uint32_t)(rem2 % S);
  const uint64_t b = rem2 / S;
  const uint32_t slot = (uint32_t)(((uint64_t)pos_offset + s) % max_len);
  cache[((b * H + h) * max_len + slot) * D + d] = in[i];
}

// Four floats rounded to bf16 (nearest even, as the bf16 prefill kernels round
// their operands), packed as 8 bytes.
__device__ __forceinline__ uint2 bf16x4_bits(float4 x) {
  typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
  bf16x4 y;
  y[0] = (__bf16)x.x;
  y[1] = (__bf16)x.y;
  y[2] = (__bf16)x.z;
  y[3] = (__bf16)x.w;
  return __builtin_bit_cast(uint2, y);
}

// K and V appended in one launch: one thread per 4 consecutive elements of
// k_in / v_in [B][S][H][D] (D % 4 == 0) writes them to slot
// (pos_offset + s) % max_len of their caches, the K row rotated first at
// table row rope_pos0 + s when cos_t is set (RoPE then cache write, as
// model.rs:760-764 runs them).
__global__ __launch_bounds__(256) void kv_append_vec4(const float4* __restrict__ k_in,
                                                      const float4* __restrict__ v_in,
                                                      float4* __restrict__ k_cache,
                                                      float4* __restrict__ v_cache,
                                                      const float2* __restrict__ cos_t,
                                                      const float2* __restrict__ sin_t,
                                                      uint2* __restrict__ k16, uint2* __restrict__ v16,
                                                      uint32_t rope_pos0, uint32_t pos_offset,
                                                      uint32_t S, uint32_t H, uint32_t D4,
                                                      uint32_t max_len, uint64_t total4) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total4) return;
  const uint32_t d4 = (uint32_t)(i % D4);
  const uint64_t rem = i / D4;
  const uint32_t h = (uint32_t)(rem % H);
  const uint64_t rem2 = rem / H;
  const uint32_t s = (uint32_t)(rem2 % S);
  const uint64_t b = rem2 / S;
  const uint32_t slot = (uint32_t)(((uint64_t)pos_offset + s) % max_len);
  const uint64_t dst = ((b * H + h) * max_len + slot) * D4 + d4;
  float4 k = k_in[i];
  const float4 v = v_in[i];
  if (cos_t) {
    const uint64_t row = (uint64_t)(rope_pos0 + s) * D4 + d4;
    k = rope4(k, cos_t[row], sin_t[row]);
  }
  k_cache[dst] = k;
  v_cache[dst] = v;
  if (k16) {
    k16[dst] = bf16x4_bits(k);
    v16[dst] = bf16x4_bits(v);
  }
}

// The bf16 copy of caches [n4 float4s]: every value rounded to nearest even.
__global__ __launch_bounds__(256) void to_bf16_kernel(const float4* __restrict__ x,
                                                      uint2* __restrict__ y, uint64_t n4) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4;
       i += (uint64_t)gridDim.x * blockDim.x)
    y[i] = bf16x4_bits(x[i]);
}

// One thread per two adjacent rotation pairs (4 floats) of x [B][S][H][D].
__global__ __launch_bounds__(256) void rope_kernel(float4* __restrict__ x,
                                                   const float2* __restrict__ cos_t,
                                                   const float2* __restrict__ sin_t,
                                                   uint32_t S, uint32_t H, uint32_t D4,
                                                   uint32_t offset, uint64_t total4) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total4) return;
  const uint32_t d4 = (uint32_t)(i % D4);
  const uint32_t s = (uint32_t)((i / D4 / H) % S);
  // A table row holds D/2 floats; float2 entry d4 covers pairs 2*d4, 2*d4+1.
  const uint64_t row = (uint64_t)(offset + s) * D4 + d4;
  x[i] = rope4(x[i], cos_t[row], sin_t[row]);
}

}  // namespace

int launch_cache_write(const float* input, float* cache, uint32_t pos_offset, uint32_t batch,
                       uint32_t seq, uint32_t heads, uint32_t head_dim, uint32_t max_len,
                       hipStream_t stream) {
  const uint64_t total = (uint64_t)batch * seq * heads * head_dim;
  if (total == 0) return STS_OK;
  const bool vec = (head_dim % 4 == 0) && ((uintptr_t)input % 16 == 0) &&
                   ((uintptr_t)cache % 16 == 0);
  if (vec) {
    const uint64_t total4 = total / 4;
    const uint64_t blocks = (total4 + 255) / 256;
    hipLaunchKernelGGL(cache_write_vec4, dim3((uint32_t)blocks), dim3(256), 0, stream,
                       reinterpret_cast<const float4*>(input), cache, pos_offset, seq, heads,
                       head_dim / 4, max_len, total4);
  } else {
    const uint64_t blocks = (total + 255) / 256;
    hipLaunchKernelGGL(cache_write_scalar, dim3((uint32_t)blocks), dim3(256), 0, stream, input,
                       cache, pos_offset, seq, heads, head_dim, max_len, total);
  }
  STS_HIP(hipGetLastError());
  return STS_OK;
}

int launch_kv_append(const float* k_in, const float* v_in, float* k_cache, float* v_cache,
                     uint32_t pos_offset, uint32_t batch, uint32_t seq, uint32_t heads,
                     uint32_t head_dim, uint32_t max_len, const float* cos_t, const float* sin_t,
                     uint32_t rope_pos0, uint16_t* k16, uint16_t* v16, hipStream_t stream) {
  const uint64_t total4 = (uint64_t)batch * seq * heads * head_dim / 4;
  if (total4 == 0) return STS_OK;
  if (head_dim % 4 != 0 || ((uintptr_t)k_in | (uintptr_t)v_in | (uintptr_t)k_cache |
                            (uintptr_t)v_cache) % 16 != 0)
    return fail(STS_ERR_INVALID, "fused K/V append needs head_dim %% 4 == 0 and 16-byte aligned rows");
  const uint64_t blocks = (total4 + 255) / 256;
  hipLaunchKernelGGL(kv_append_vec4, dim3((uint32_t)blocks), dim3(256), 0, stream,
                     reinterpret_cast<const float4*>(k_in), reinterpret_cast<const float4*>(v_in),
                     reinterpret_cast<float4*>(k_cache), reinterpret_cast<float4*>(v_cache),
                     reinterpret_cast<const float2*>(cos_t), reinterpret_cast<const float2*>(sin_t),
                     reinterpret_cast<uint2*>(k16), reinterpret_cast<uint2*>(v16), rope_pos0,
                     pos_offset, seq, heads, head_dim / 4, max_len, total4);
  STS_HIP(hipGetLastError());
  return STS_OK;
}

int launch_to_bf16(const float* x, uint16_t* y, uint64_t n, hipStream_t stream) {
  if (n == 0) return STS_OK;
  if (n % 4 != 0 || ((uintptr_t)x % 16) || ((uintptr_t)y % 8))
    return fail(STS_ERR_INVALID, "bf16 copy needs a multiple of 4 values, aligned");
  const uint64_t n4 = n / 4;
  const uint64_t blocks = std::min<uint64_t>((n4 + 255) / 256, 65536);
  hipLaunchKernelGGL(to_bf16_kernel, dim3((uint32_t)blocks), dim3(256), 0, stream,
                     reinterpret_cast<const float4*>(x), reinterpret_cast<uint2*>(y), n4);
  STS_HIP(hipGetLastError());
  return STS_OK;
}

int launch_rope(float* x, const float* cos_t, const float* sin_t, uint32_t batch, uint32_t seq,
                uint32_t heads, uint32_t head_dim, uint32_t offset, hipStream_t stream) {
  const uint64_t total4 = (uint64_t)batch * seq * heads * head_dim / 4;
  if (total4 == 0) return STS_OK;
  const uint64_t blocks = (total4 + 255) / 256;
  hipLaunchKernelGGL(rope_kernel, dim3((uint32_t)blocks), dim3(256), 0, stream,
                     reinterpret_cast<float4*>(x), reinterpret_cast<const float2*>(cos_t),
                     reinterpret_cast<const float2*>(sin_t), seq, heads, head_dim / 4, offset,
                     total4);
  STS_HIP(hipGetLastError());
  return STS_OK;
}

}  // namespace sts
