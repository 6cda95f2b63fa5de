// common.hpp -- error reporting and per-stream workspace for the sts_attn library.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <string>

#include "sts_attn.h"

namespace sts {

// Records `msg` as the calling thread's last error and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the calling thread's last error.
void clear_error();
const char* last_error_cstr();

#define STS_HIP(call)                                                              \
  do {                                                                             \
    hipError_t e_ = (call);                                                        \
    if (e_ != hipSuccess)                                                          \
      return ::sts::fail(STS_ERR_HIP, "%s failed: %s (%d) at %s:%d", #call,        \
                         hipGetErrorString(e_), (int)e_, __FILE__, __LINE__);      \
  } while (0)

#define STS_CHECK(cond, ...)                                                       \
  do {                                                                             \
    if (!(cond)) return ::sts::fail(STS_ERR_INVALID, __VA_ARGS__);                 \
  } while (0)

// Split-KV partial results and arrival counters for one (device, stream).
struct Workspace {
  float* part = nullptr;       // partial (acc[D], m, l) records
  size_t part_floats = 0;
  uint32_t* counters = nullptr;  // one arrival counter per (stream, head); zero between calls
  size_t n_counters = 0;
};

// Returns a workspace for `stream` on the current device holding at least the
// requested sizes.  Growing allocates new buffers (new counters zero-filled on
// the stream) and retires the old ones without freeing them, so work queued
// earlier and graphs captured earlier stay valid.  Fails with STS_ERR_STATE
// when it would have to allocate while the stream is being captured.
int get_workspace(hipStream_t stream, size_t part_floats, size_t n_counters, Workspace** out);

// Number of compute units of the current device (cached per device).
int device_cu_count();

// Poll bound of the kernels' bounded waits (0 restores the default, 2^24).
void set_wait_limit(uint32_t polls);
uint32_t wait_limit();

}  // namespace sts
