// decode.hpp -- split-KV decode attention over a ring-buffer KV cache.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sts {

// One launch of the decode kernel.  Row i (0 <= i < len) of stream b, query
// head h lives in slot (start + i) % M of
//   k + b*kv_bstride + (h / group)*kv_hstride
// (rows of head_dim floats; group > 1 is grouped-query attention, each K/V
// head serving `group` consecutive query heads).  With k_new set, row len-1
// is taken from k_new/v_new and written to its slot of k_wr/v_wr (a fused
// append; with group > 1 by the first query head of each group only).
struct DecodeParams {
  const float* q = nullptr;      // stream b, head h at q + b*q_bstride + h*D
  const float* k = nullptr;
  const float* v = nullptr;
  float* out = nullptr;          // stream b, head h at out + b*out_bstride + h*D
  const float* k_new = nullptr;  // stream b, K/V head j at k_new + b*kn_bstride + j*D, or null
  const float* v_new = nullptr;
  float* k_wr = nullptr;
  float* v_wr = nullptr;
  uint16_t* k16_wr = nullptr;  // bf16 copies of k_wr/v_wr (same layout) that the
  uint16_t* v16_wr = nullptr;  // appended row also goes to, rounded, or null
  const float* rope_cos = nullptr;  // [max_pos][D/2]; with rope, q and k_new are
  const float* rope_sin = nullptr;  // rotated in registers at position rope_pos
  const int32_t* lens = nullptr;    // per-stream device arrays, or null for the
  const int32_t* starts = nullptr;  // uniform len/start below
  uint32_t len = 0, start = 0;
  uint32_t rope_pos = 0;
  uint32_t H = 0, M = 0;
  uint64_t q_bstride = 0, out_bstride = 0;
  uint64_t kv_bstride = 0, kv_hstride = 0;
  uint64_t kn_bstride = 0;  // k_new/v_new stream stride; 0: q_bstride
  uint32_t group = 1;       // query heads per K/V head
  float scale_log2 = 0.f;  // softmax scale * log2(e)
  uint32_t chunk = 0;      // rows per split
  uint32_t nsplit_max = 1; // grid x
  float* part = nullptr;   // [B][H][nsplit_max][D+4] partials (nsplit > 1 only)
  uint32_t* counters = nullptr;  // [B][H] arrival counters, zero between calls
  // Last, so that the fields the kernel's prologue needs keep their shared
  // 16-byte kernel-argument loads.  The head dim in memory, set by the
  // launcher (64 and 128 run their own layouts; other multiples of 4 up to
  // 128 a padded one).
  uint32_t head_dim = 0;
  // Padded head dims only, with lens == null: stream b's window has
  // len + b * len_step rows and its RoPE position is rope_pos + b * len_step
  // (the queries of a causal chunk as streams over one cache: kv_bstride 0).
  uint32_t len_step = 0;
};

// scale * log2(e), the factor the decode and prefill kernels fold into q.
float softmax_scale_log2(float scale);

// Chooses chunk / nsplit_max / waves for `units` (stream, head) pairs whose
// longest window is max_rows, then launches.  Allocates the split workspace
// from the per-stream pool when more than one split is needed.
int launch_decode(DecodeParams p, uint32_t batch, uint32_t head_dim, uint32_t max_rows,
                  hipStream_t stream);

// Makes sure the split workspace that launch_decode needs for these sizes on
// `stream` exists (allocating it now if not), so that a caller can fail before
// it changes any state; launch_decode then finds it and cannot fail on it.
int reserve_decode(uint32_t batch, uint32_t heads, uint32_t head_dim, uint32_t max_rows,
                   hipStream_t stream);

// launch_decode without allocating: the split records and arrival counters
// live in a static device array of the library (8 MiB of records, 16384
// counters per GPU); launches that need more fail with STS_ERR_INVALID.  All
// calls on one GPU share that array: calls that overlap in time race.
int launch_decode_noalloc(DecodeParams p, uint32_t batch, uint32_t head_dim, uint32_t max_rows,
                          hipStream_t stream);

}  // namespace sts
