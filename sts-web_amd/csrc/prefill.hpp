// prefill.hpp -- chunked causal prefill attention over a ring-buffer KV cache.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sts {

// Query i (0 <= i < S) is window row len - S + i and attends window rows
// 0..len-S+i; window row r of query head h is slot (start + r) % M of
// k + (h / group)*M*D (group > 1: grouped-query attention, each K/V head
// serving `group` consecutive query heads).  q, out are [S][H][D].
struct PrefillParams {
  const float* q = nullptr;
  const float* k = nullptr;
  const float* v = nullptr;
  float* out = nullptr;
  uint32_t S = 0, H = 0, M = 0;
  uint32_t start = 0, len = 0;
  float scale_log2 = 0.f;
  // Key-range split: up to nsplit workgroups share a (head, query tile); each
  // publishes a partial (O, max, sum) to part and the last to arrive (counted
  // in counters, one per (head, tile), left at zero) merges them.
  uint32_t nsplit = 1;
  float* part = nullptr;
  uint32_t* counters = nullptr;
  // With rope_cos set, query i is rotated in registers at table row
  // rope_pos0 + i before it is scaled (tables [max_pos][D/2]).
  const float* rope_cos = nullptr;
  const float* rope_sin = nullptr;
  uint32_t rope_pos0 = 0;
  // Polls after which a bounded wait of the bf16 kernels gives up and records
  // STS_DEVERR_WAIT_TIMEOUT in the device error word.
  uint32_t wait_limit = 1u << 24;
  uint32_t* err = nullptr;  // the device error word
  // bf16 copies of the caches ([H][M][D], bf16 bits); when set, the bf16-MFMA
  // kernel reads them instead of k / v.
  const void* k16 = nullptr;
  const void* v16 = nullptr;
  // Query heads per K/V head (last, so the other fields keep their
  // kernel-argument load groups).  The kernels take the K/V head of query
  // head h as umulhi(h, group_magic) = h / group (exact for h, group < 2^16),
  // group_magic = ceil(2^32 / group), set by launch_prefill; 0 for group 1.
  uint32_t group = 1;
  uint32_t group_magic = 0;
  // Start stagger of the bf16-mirror kernel, set by its launch when the grid
  // fits in one round on the device: a query tile with fewer key blocks than
  // the launch's longest sleeps start_stagger x ~128 clocks per block of
  // difference before its first loads.  0: no stagger.
  uint32_t start_stagger = 0;
};

// Checks everything launch_prefill would reject for these sizes, without
// launching (callers that mutate state first validate with it).
int check_prefill(uint32_t seq, uint32_t heads, uint32_t head_dim, uint32_t max_len,
                  int precision);

int launch_prefill(const PrefillParams& p, uint32_t head_dim, int precision, hipStream_t stream);

// Acquires, ahead of time, everything launch_prefill would acquire for these
// sizes on `stream` (split workspace, device error word), so that a caller
// that changes state before launching can fail first; afterwards
// launch_prefill with the same sizes finds them and cannot fail on them.
// bf16_rows: the launch will read bf16 copies of the caches.
int reserve_prefill(uint32_t S, uint32_t H, uint32_t len, uint32_t head_dim, int precision,
                    bool bf16_rows, hipStream_t stream);


}  // namespace sts
