// append.hpp -- KV append and RoPE launchers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sts {

// cache[((b*H + h)*max_len + (pos_offset + s) % max_len)*D + d] = input[((b*S + s)*H + h)*D + d]
int launch_cache_write(const float* input, float* cache, uint32_t pos_offset, uint32_t batch,
                       uint32_t seq, uint32_t heads, uint32_t head_dim, uint32_t max_len,
                       hipStream_t stream);

// In-place interleaved RoPE of x [B][S][H][D] with table rows offset..offset+S-1.
int launch_rope(float* x, const float* cos_t, const float* sin_t, uint32_t batch, uint32_t seq,
                uint32_t heads, uint32_t head_dim, uint32_t offset, hipStream_t stream);

}  // namespace sts
