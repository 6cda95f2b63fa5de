// probe.hip -- the plain-read roofline probe (measurement only; no counterpart
// in the reference).
//
// sts_probe_stream_read reads two buffers once with 16-byte nontemporal
// buffer loads, the access the HBM-bound kernels of this library make, and
// nothing else: no arithmetic beyond one running sum per lane, one float
// stored per workgroup.  Timed on the same bytes and the same grid as a
// kernel, it gives the rate that a read of those bytes reaches on this chip,
// which is the practical ceiling that kernel is compared with.
//
// Each workgroup streams a contiguous share of each buffer (the shares of
// `a` first, then of `b`); every thread keeps 8 loads in flight.
#include "coherent.hpp"
#include "common.hpp"

namespace sts {

namespace {

constexpr int kProbeThreads = 256;
constexpr int kProbeInFlight = 8;
constexpr int kProbeNt = 2;  // buffer-load cache policy bit: nontemporal

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Sum of this thread's 16-byte pieces of [lo, hi) (16-byte units) of buf.
__device__ __forceinline__ float read_share(const void* buf, uint64_t lo, uint64_t hi) {
  if (hi <= lo) return 0.f;
  const uint32_t bytes = (uint32_t)((hi - lo) * 16);
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char*>(static_cast<const char*>(buf)) + lo * 16, 0, (int)bytes, kBufferWord3);
  float acc = 0.f;
  constexpr uint32_t step = kProbeThreads * kProbeInFlight * 16;
  for (uint32_t off = threadIdx.x * 16; off < bytes; off += step) {
    u32x4 x[kProbeInFlight];
    // Pieces past the share read zeros (buffer bounds), so all 8 loads issue.
#pragma unroll
    for (int j = 0; j < kProbeInFlight; ++j)
      x[j] = __builtin_amdgcn_raw_buffer_load_b128(r, off + j * kProbeThreads * 16, 0, kProbeNt);
#pragma unroll
    for (int j = 0; j < kProbeInFlight; ++j)
      acc += __builtin_bit_cast(float, x[j].x ^ x[j].y ^ x[j].z ^ x[j].w);
  }
  return acc;
}

__global__ __launch_bounds__(kProbeThreads) void stream_read_kernel(const void* a, uint64_t na,
                                                                    const void* b, uint64_t nb,
                                                                    float* sink) {
  const uint64_t wg = blockIdx.x, nwg = gridDim.x;
  const uint64_t ca = (na + nwg - 1) / nwg, cb = (nb + nwg - 1) / nwg;
  float acc = read_share(a, min(na, wg * ca), min(na, (wg + 1) * ca));
  acc += read_share(b, min(nb, wg * cb), min(nb, (wg + 1) * cb));
  // One value per workgroup keeps every load live.
  acc += __shfl_xor(acc, 32, 64);
  if (threadIdx.x == 0) sink[blockIdx.x] = acc;
}

}  // namespace

}  // namespace sts

extern "C" int sts_probe_stream_read(const void* a, uint64_t a_bytes, const void* b,
                                     uint64_t b_bytes, uint32_t workgroups, float* sink,
                                     void* stream) {
  sts::clear_error();
  STS_CHECK(a && sink && (b || b_bytes == 0), "null pointer argument");
  STS_CHECK(a_bytes % 16 == 0 && b_bytes % 16 == 0, "sizes must be multiples of 16 bytes");
  STS_CHECK(((uintptr_t)a & 15u) == 0 && ((uintptr_t)b & 15u) == 0,
            "buffers must be 16-byte aligned");
  STS_CHECK(workgroups >= 1 && workgroups <= 65535, "workgroups %u out of 1..65535", workgroups);
  // One workgroup's share of a buffer is addressed through one buffer resource.
  STS_CHECK((a_bytes + workgroups - 1) / workgroups < 0x7FFFFFF0ull &&
                (b_bytes + workgroups - 1) / workgroups < 0x7FFFFFF0ull,
            "a workgroup's share must be below 2 GiB");
  hipLaunchKernelGGL(sts::stream_read_kernel, dim3(workgroups), dim3(sts::kProbeThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), a, a_bytes / 16, b, b_bytes / 16,
                     sink);
  STS_HIP(hipGetLastError());
  return STS_OK;
}
