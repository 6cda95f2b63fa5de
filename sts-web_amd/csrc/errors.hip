// errors.hip -- the device error word: STS_DEVERR_* bits that kernels raise
// instead of hanging or faulting (a bounded wait that gave up), read back and
// cleared by sts_device_errors.  One word per GPU, in device memory the code
// object owns; kernels receive its address as an argument.
#include <map>
#include <mutex>

#include "common.hpp"
#include "errors.hpp"

namespace sts {

namespace {

__device__ uint32_t g_error_word;
__device__ uint32_t g_error_taken;

__global__ void take_errors_kernel(uint32_t* word, uint32_t* taken) {
  if (threadIdx.x == 0) *taken = atomicExch(word, 0u);
}

struct ErrorWords {
  uint32_t* word = nullptr;
  uint32_t* taken = nullptr;
};

std::mutex g_mutex;
std::map<int, ErrorWords> g_words;  // device -> addresses on it

int words_for_device(ErrorWords* out) {
  int dev = 0;
  STS_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(g_mutex);
  auto it = g_words.find(dev);
  if (it == g_words.end()) {
    ErrorWords w;
    STS_HIP(hipGetSymbolAddress(reinterpret_cast<void**>(&w.word), HIP_SYMBOL(g_error_word)));
    STS_HIP(hipGetSymbolAddress(reinterpret_cast<void**>(&w.taken), HIP_SYMBOL(g_error_taken)));
    it = g_words.emplace(dev, w).first;
  }
  *out = it->second;
  return STS_OK;
}

}  // namespace

int device_error_word(uint32_t** word) {
  ErrorWords w;
  if (int rc = words_for_device(&w)) return rc;
  *word = w.word;
  return STS_OK;
}

int take_device_errors(hipStream_t stream, uint32_t* flags) {
  // The swap must run now, not be recorded into a graph, and the stream must
  // be waited for: neither is possible while it is being captured.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  STS_HIP(hipStreamIsCapturing(stream, &cap));
  if (cap != hipStreamCaptureStatusNone)
    return fail(STS_ERR_STATE,
                "the device error word cannot be read while the stream is being captured; "
                "read it after the capture or the graph's replay");
  ErrorWords w;
  if (int rc = words_for_device(&w)) return rc;
  // Swapped to zero on the device after the work queued on `stream`, so no
  // bit raised between the read and the clear is lost.
  hipLaunchKernelGGL(take_errors_kernel, dim3(1), dim3(64), 0, stream, w.word, w.taken);
  STS_HIP(hipGetLastError());
  STS_HIP(hipStreamSynchronize(stream));
  uint32_t v = 0;
  STS_HIP(hipMemcpy(&v, w.taken, sizeof v, hipMemcpyDeviceToHost));
  *flags = v;
  return STS_OK;
}

}  // namespace sts
