// append.hpp -- KV append and RoPE launchers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sts {

// cache[((b*H + h)*max_len + (pos_offset + s) % max_len)*D + d] = input[((b*S + s)*H + h)*D + d]
int launch_cache_write(const float* input, float* cache, uint32_t pos_offset, uint32_t batch,
                       uint32_t seq, uint32_t heads, uint32_t head_dim, uint32_t max_len,
                       hipStream_t stream);

// K and V rows of [B][S][H][D] appended to their caches in one launch (same
// slot formula); with cos_t set, the K row is rotated at table row
// rope_pos0 + s first.  With k16/v16 set, the rows also go, rounded to bf16
// (nearest even), to the same slots of those bf16 copies.  head_dim % 4 == 0,
// all pointers 16-byte aligned.
int launch_kv_append(const float* k_in, const float* v_in, float* k_cache, float* v_cache,
                     uint32_t pos_offset, uint32_t batch, uint32_t seq, uint32_t heads,
                     uint32_t head_dim, uint32_t max_len, const float* cos_t, const float* sin_t,
                     uint32_t rope_pos0, uint16_t* k16, uint16_t* v16, hipStream_t stream);

// y[i] = bf16(x[i]) (nearest even) for n values (n % 4 == 0, x 16-byte aligned).
int launch_to_bf16(const float* x, uint16_t* y, uint64_t n, hipStream_t stream);

// In-place interleaved RoPE of x [B][S][H][D] with table rows offset..offset+S-1.
int launch_rope(float* x, const float* cos_t, const float* sin_t, uint32_t batch, uint32_t seq,
                uint32_t heads, uint32_t head_dim, uint32_t offset, hipStream_t stream);

}  // namespace sts
