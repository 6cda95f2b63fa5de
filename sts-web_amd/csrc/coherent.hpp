// coherent.hpp -- device-coherent loads and stores for data that one
// workgroup publishes and another (possibly on another XCD, with its own L2)
// reads within the same launch.
//
// Buffer loads and stores carrying the sc1 cache policy are coherent at
// device scope by themselves, so publishing needs only a wait for the
// stores' acknowledgement (s_waitcnt) before the arrival atomic, not an L2
// write-back or invalidate of everything the workgroup touched.  16-byte
// accesses per lane fill whole 64-byte segments, so the write-through costs
// no more HBM traffic than the data itself.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sts {

typedef float coh_f4 __attribute__((ext_vector_type(4)));
typedef uint32_t coh_u4 __attribute__((ext_vector_type(4)));

constexpr int kSc1 = 16;                  // cache-policy bit of sc1
constexpr int kBufferWord3 = 0x00020000;  // raw 32-bit buffer, no swizzle

// A raw buffer resource over `bytes` bytes at p; accesses past the end load
// zeros and drop stores.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t coherent_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)bytes, kBufferWord3);
}

__device__ __forceinline__ void st_coherent4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, coh_f4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(coh_u4, v), r, byte_off, 0, kSc1);
}
__device__ __forceinline__ void st_coherent(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, byte_off, 0, kSc1);
}
__device__ __forceinline__ coh_f4 ld_coherent4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(coh_f4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kSc1));
}
__device__ __forceinline__ float ld_coherent(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, kSc1));
}

}  // namespace sts
