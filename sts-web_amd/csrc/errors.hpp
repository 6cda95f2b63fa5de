// errors.hpp -- the per-GPU device error word (STS_DEVERR_* bits).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sts {

// Address of the current device's error word, for kernel arguments.
int device_error_word(uint32_t** word);

// Synchronises `stream`, then reads and clears the current device's error word.
int take_device_errors(hipStream_t stream, uint32_t* flags);

}  // namespace sts
