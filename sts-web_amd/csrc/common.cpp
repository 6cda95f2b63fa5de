// common.cpp -- error reporting and per-(device, stream) workspace.
#include "common.hpp"

#include <map>
#include <mutex>
#include <utility>

namespace sts {

namespace {
thread_local std::string g_last_error;

std::mutex g_ws_mutex;
std::map<std::pair<int, hipStream_t>, Workspace> g_ws;

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
    // Work already queued on this stream may still use the old buffers.
    if (ws.part || ws.counters) STS_HIP(hipStreamSynchronize(stream));
    if (ws.part) STS_HIP(hipFree(ws.part));
    if (ws.counters) STS_HIP(hipFree(ws.counters));
    ws = Workspace{};
    size_t pf = part_floats > 0 ? part_floats : 1;
    size_t nc = n_counters > 0 ? n_counters : 1;
    // Round up so that slowly growing workloads do not reallocate every call.
    pf = (pf + 65535) & ~size_t(65535);
    nc = (nc + 1023) & ~size_t(1023);
    if (hipMalloc(&ws.part, pf * sizeof(float)) != hipSuccess) {
      ws.part = nullptr;
      return fail(STS_ERR_NOMEM, "workspace allocation of %zu bytes failed", pf * sizeof(float));
    }
    if (hipMalloc(&ws.counters, nc * sizeof(uint32_t)) != hipSuccess) {
      (void)hipFree(ws.part);
      ws.part = nullptr;
      ws.counters = nullptr;
      return fail(STS_ERR_NOMEM, "workspace counter allocation failed");
    }
    STS_HIP(hipMemsetAsync(ws.counters, 0, nc * sizeof(uint32_t), stream));
    ws.part_floats = pf;
    ws.n_counters = nc;
  }
  *out = &ws;
  return STS_OK;
}

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
