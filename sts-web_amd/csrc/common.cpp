// common.cpp -- error reporting and per-(device, stream) workspace.
#include "common.hpp"

#include <algorithm>
#include <atomic>
#include <map>
#include <mutex>
#include <utility>
#include <vector>

namespace sts {

namespace {
thread_local std::string g_last_error;

std::mutex g_ws_mutex;
std::map<std::pair<int, hipStream_t>, Workspace> g_ws;
// Workspace buffers replaced by larger ones; kept until the process ends.
std::vector<void*> g_retired;

std::mutex g_cu_mutex;
std::map<int, int> g_cu;
}  // namespace

int fail(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

void clear_error() { g_last_error.clear(); }

const char* last_error_cstr() { return g_last_error.c_str(); }

int get_workspace(hipStream_t stream, size_t part_floats, size_t n_counters, Workspace** out) {
  int dev = 0;
  STS_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(g_ws_mutex);
  Workspace& ws = g_ws[{dev, stream}];
  if (ws.part_floats < part_floats || ws.n_counters < n_counters) {
    // A stream being captured into a HIP graph must not allocate: the graph
    // would record the counters' initialisation and keep pointers that the
    // eager path could later replace.
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    STS_HIP(hipStreamIsCapturing(stream, &cap));
    if (cap != hipStreamCaptureStatusNone)
      return fail(STS_ERR_STATE,
                  "split workspace of %zu floats / %zu counters needed while the stream is "
                  "being captured; run the call once on this stream before capturing it",
                  part_floats, n_counters);
    // The old buffers are retired, not freed: kernels queued on the stream
    // and graphs captured earlier keep using them.  Growth at least doubles,
    // so the retired buffers never exceed the live ones.
    auto grow = [](size_t want, size_t have, size_t round) {
      const size_t n = std::max<size_t>(std::max(want, have < want ? 2 * have : have), 1);
      return (n + round - 1) / round * round;
    };
    const size_t pf = grow(part_floats, ws.part_floats, 65536);
    const size_t nc = grow(n_counters, ws.n_counters, 1024);
    float* part = nullptr;
    uint32_t* counters = nullptr;
    if (hipMalloc(&part, pf * sizeof(float)) != hipSuccess)
      return fail(STS_ERR_NOMEM, "workspace allocation of %zu bytes failed", pf * sizeof(float));
    if (hipMalloc(&counters, nc * sizeof(uint32_t)) != hipSuccess) {
      (void)hipFree(part);
      return fail(STS_ERR_NOMEM, "workspace counter allocation failed");
    }
    // The counters start at zero; every launch leaves them at zero.
    if (hipMemsetAsync(counters, 0, nc * sizeof(uint32_t), stream) != hipSuccess) {
      (void)hipFree(part);
      (void)hipFree(counters);
      return fail(STS_ERR_HIP, "workspace counter initialisation failed");
    }
    if (ws.part) g_retired.push_back(ws.part);
    if (ws.counters) g_retired.push_back(ws.counters);
    ws.part = part;
    ws.counters = counters;
    ws.part_floats = pf;
    ws.n_counters = nc;
  }
  *out = &ws;
  return STS_OK;
}

namespace {
std::atomic<uint32_t> g_wait_limit{1u << 24};
}  // namespace

void set_wait_limit(uint32_t polls) { g_wait_limit = polls ? polls : (1u << 24); }
uint32_t wait_limit() { return g_wait_limit; }

int device_cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> lock(g_cu_mutex);
  auto it = g_cu.find(dev);
  if (it != g_cu.end()) return it->second;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = 256;
  g_cu[dev] = cus;
  return cus;
}

}  // namespace sts

extern "C" const char* sts_last_error(void) { return sts::last_error_cstr(); }

extern "C" int sts_abi_version(void) { return STS_ATTN_ABI_VERSION; }
