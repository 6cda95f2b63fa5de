// q4k.hip -- Q4_K dequantisation and matrix-vector product for gfx950.
//
// Reference: crates/sts-wasm/src/gguf.rs:808-905 (q4k_matmul with M = 1, the
// single-token path, and q4k_matmul_with_residual), whose kernel is
// wgsl/shader_q4k_matvec.wgsl: one output per thread, dequantising
// w = (d*scale)*q - (dmin*min) weight by weight in f32.
//
// Work split.  A row of K weights is S = K/64 slots of 64 consecutive
// weights: slot s is iteration it = s%4 of super-block s/4, i.e. 32 quant
// bytes whose low nibbles are sub-block 2it and high nibbles sub-block 2it+1
// (weights 64s .. 64s+63), plus the block's 16-byte header (d, dmin, packed
// scales).  Lane l of a wave owns slot 64*kp + l, where kp numbers the KP
// waves that share a row when K > 4096; it keeps the 64 x values of its slot
// in registers for the whole launch and walks rows, adding per row
//     d1 * sum(q_lo * x_lo) - m1 * sum(x_lo) + d2 * sum(q_hi * x_hi) - m2 * sum(x_hi)
// with the two sums of x computed once.  Per row a lane loads 48 bytes; the
// lanes of a wave together read the row as one contiguous stream (2304
// bytes at K = 4096).  The regrouping changes the rounding of the sum
// (tolerance-checked against the shader-order oracle), not the weights: the
// dequantisation kernel below reproduces the shader's f32 weights bit for
// bit.
//
// Rows are dealt to groups of KP waves (KP = 1 up to K = 4096): group g owns
// the contiguous rows g*R .. g*R + R-1 (R <= 12), one row ahead: row j + 1
// is requested just before row j is reduced, and row 0 before x is staged.
// The KP waves of a group keep their partial sums and combine through LDS
// once, at the end.  K <= 4096: eight waves per CU in workgroups of four;
// K > 4096: one workgroup of 12 waves per CU, so that x is staged once per
// CU.  Measured per projection shape against the alternatives: rows requested
// two to twelve ahead (or two ahead, after the reduction), four, six,
// twelve or sixteen waves per CU at K <= 4096, rows dealt round-robin over
// the waves, and nontemporal weight loads were all slower (the last by up to
// 15% on the FFN's linear_in: the three loads of a row share cache lines,
// which plain loads let the CU's cache serve).
//
// HBM-bound: 0.5625 bytes and 2 flops per weight (x and y are negligible).
#include <algorithm>
#include <cstdint>

#include "common.hpp"
#include "lane.hpp"
#include "q4k.hpp"

namespace sts {

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x4 ld16(const uint8_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

// d1*sum(q_lo*x_lo) - m1*sum(x_lo) + d2*sum(q_hi*x_hi) - m2*sum(x_hi) for one slot.
// xv[32..63] hold x_hi / 16 (the high nibbles are taken in place, as 16 q_hi);
// sxl and sxh are the sums of the unscaled x_lo and x_hi.
__device__ __forceinline__ float slot_dot(u32x4 hd, u32x4 qa, u32x4 qb, uint32_t jl,
                                          const float (&xv)[64], float sxl, float sxh) {
  const float d = half_bits_to_float(hd.x), dmin = half_bits_to_float(hd.x >> 16);
  uint32_t scl, mnl, sch, mnh;
  scale_min(hd.y, hd.z, hd.w, jl, scl, mnl);
  scale_min(hd.y, hd.z, hd.w, jl + 1, sch, mnh);
  const uint32_t words[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
  // Four independent chains per half, so consecutive FMAs do not wait on
  // each other.
  float ql[4] = {0.f, 0.f, 0.f, 0.f}, qh[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    uint32_t lo = words[w] & 0x0F0F0F0Fu;
    uint32_t hi = words[w] & 0xF0F0F0F0u;  // 16 q: its x values are scaled by 1/16
    // Opaque to the optimiser, so that each byte below becomes one
    // v_cvt_f32_ubyte{0..3} instead of a bit-field extract plus a convert.
    asm("" : "+v"(lo), "+v"(hi));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ql[i] = fmaf((float)((lo >> (8 * i)) & 0xFFu), xv[4 * w + i], ql[i]);
      qh[i] = fmaf((float)((hi >> (8 * i)) & 0xFFu), xv[32 + 4 * w + i], qh[i]);
    }
  }
  const float qls = (ql[0] + ql[1]) + (ql[2] + ql[3]);
  const float qhs = (qh[0] + qh[1]) + (qh[2] + qh[3]);
  const float d1 = d * (float)scl, m1 = dmin * (float)mnl;
  const float d2 = d * (float)sch, m2 = dmin * (float)mnh;
  return (d1 * qls - m1 * sxl) + (d2 * qhs - m2 * sxh);
}

__device__ __forceinline__ float wave_sum(float x) {
  x += xchg<0>(x);
  x += xchg<1>(x);
  x += xchg<2>(x);
  x += xchg<3>(x);
  return sum_xor32(sum_xor16(x));
}

// Group g of the grid owns the contiguous rows g*R .. g*R + R-1; its KP
// waves cover slots 64*kp + lane of each of them (KP = 1 up to K = 4096),
// one row ahead, and keep their partial sums until the end, where the KP
// waves of a group combine through LDS once.  G groups per workgroup.

template <int R, int KP, int G>
__global__ __launch_bounds__(64 * KP * G) void q4k_matvec_rows_kernel(const Q4kParams p) {
  constexpr int NT = 64 * KP * G;     // threads
  constexpr int XL = (1024 * KP + NT - 1) / NT;  // float4 of x per thread, K <= 4096 KP
  static_assert(XL >= 1 && XL * NT >= 1024 * KP, "x staging shape");
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int kp = wv % KP;
  const int grp = wv / KP;
  const uint32_t row0 = (blockIdx.x * G + grp) * R;  // this group's first row
  const uint32_t nb = p.K / kQ4kBlockWeights;
  const uint32_t s = 64u * kp + lane;  // this lane's slot
  const bool has = s < 4u * nb;
  // A lane without a slot reads slot 0 (valid memory) and contributes zero:
  // its x values and their sums are zero.
  const uint32_t blk = has ? s >> 2 : 0u, it = has ? s & 3u : 0u;
  const uint32_t b = blockIdx.y;
  const size_t row_bytes = (size_t)nb * kQ4kBlockBytes;
  const uint8_t* wslot = p.w + (size_t)blk * kQ4kBlockBytes + 16 + 32 * it;
  const uint8_t* whead = p.w + (size_t)blk * kQ4kBlockBytes;

  // x is requested first, then the first row, so that waiting for x does
  // not wait for the weights.  The workgroup stages x in LDS, slot c at row c
  // of pitch 68 floats (the 16 lanes of a read phase then hit distinct
  // banks), and each lane copies its slot into registers.
  extern __shared__ __align__(16) float xs[];  // [K/64][68]
  const float4* xb = reinterpret_cast<const float4*>(p.x + (size_t)b * p.K);
  const uint32_t n4 = p.K / 4;
  // A vector value, not an array: an array would be kept in scratch memory
  // across the scheduling barrier below.
  typedef float xvec __attribute__((ext_vector_type(4 * XL)));
  xvec xr;
#pragma unroll
  for (int k = 0; k < XL; ++k) {
    const uint32_t i = threadIdx.x + k * NT;
    const float4 t = xb[i < n4 ? i : 0u];
    xr[4 * k] = t.x;
    xr[4 * k + 1] = t.y;
    xr[4 * k + 2] = t.z;
    xr[4 * k + 3] = t.w;
  }
  // Keeps the x loads ahead of the weight loads in the issue order.
  __builtin_amdgcn_sched_barrier(0);

  u32x4 hd[R], qa[R], qb[R];
  auto load = [&](int j) {
    // Rows past the end re-read row N-1 and are not stored.
    const size_t off = (size_t)min(row0 + j, p.N - 1) * row_bytes;
    hd[j] = ld16(whead + off);
    qa[j] = ld16(wslot + off);
    qb[j] = ld16(wslot + off + 16);
  };
  load(0);
  __builtin_amdgcn_sched_barrier(0);

#pragma unroll
  for (int k = 0; k < XL; ++k) {
    const uint32_t i = threadIdx.x + k * NT;
    if (i < n4)
      *reinterpret_cast<float4*>(&xs[(i >> 4) * 68 + 4 * (i & 15)]) =
          make_float4(xr[4 * k], xr[4 * k + 1], xr[4 * k + 2], xr[4 * k + 3]);
  }
  __syncthreads();
  float xv[64];
  const uint32_t xs0 = has ? s * 68 : 0u;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const float4 t = *reinterpret_cast<const float4*>(&xs[xs0 + 4 * j]);
    xv[4 * j] = has ? t.x : 0.f;
    xv[4 * j + 1] = has ? t.y : 0.f;
    xv[4 * j + 2] = has ? t.z : 0.f;
    xv[4 * j + 3] = has ? t.w : 0.f;
  }
  float sxl = 0.f, sxh = 0.f;
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    sxl += xv[j];
    sxh += xv[32 + j];
  }
  // The high-nibble products take the nibble in place (16 q, one mask, no
  // shift) times x / 16: both scalings are exact, so the products are q x.
#pragma unroll
  for (int j = 0; j < 32; ++j) xv[32 + j] *= 0.0625f;

  float acc[R];
#pragma unroll
  for (int j = 0; j < R; ++j) {
    // Row j + 1 is requested before row j is reduced.
    if (j + 1 < R) load(j + 1);
    acc[j] = wave_sum(slot_dot(hd[j], qa[j], qb[j], 2 * it, xv, sxl, sxh));
  }
  auto store = [&](int j, float v) {
    const uint32_t row = row0 + j;
    if (row < p.N) {
      if (p.res) v += p.res[(size_t)b * p.N + row];
      p.y[(size_t)b * p.N + row] = v;
    }
  };
  if constexpr (KP == 1) {
    if (lane == 0) {
#pragma unroll
      for (int j = 0; j < R; ++j) store(j, acc[j]);
    }
  } else {
    // x is in registers by now: its LDS rows hold the partial sums, in the
    // order of the slots (wave 0 first), so the sum runs as the KP = 1
    // kernel would add the waves' shares.
    __syncthreads();
    float* red = xs;  // [G][R][KP]
    if (lane == 0) {
#pragma unroll
      for (int j = 0; j < R; ++j) red[(grp * R + j) * KP + kp] = acc[j];
    }
    __syncthreads();
    if (kp == 0 && lane < R) {
      float v = red[(grp * R + lane) * KP];
#pragma unroll
      for (int k = 1; k < KP; ++k) v += red[(grp * R + lane) * KP + k];
      store(lane, v);
    }
  }
}

// One thread per slot: the 64 weights of slot s of row n, rounded as the
// shader rounds them (products and difference separately).
__global__ __launch_bounds__(256) void q4k_dequant_kernel(const uint8_t* __restrict__ w,
                                                          float* __restrict__ out, uint32_t N,
                                                          uint32_t K) {
#pragma clang fp contract(off)
  const uint32_t S = K / 64;
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (uint64_t)N * S) return;
  const uint32_t n = (uint32_t)(t / S), s = (uint32_t)(t % S);
  const uint32_t blk = s >> 2, it = s & 3u;
  const uint8_t* bp = w + ((size_t)n * (K / kQ4kBlockWeights) + blk) * kQ4kBlockBytes;
  const u32x4 hd = ld16(bp), qa = ld16(bp + 16 + 32 * it), qb = ld16(bp + 32 + 32 * it);
  const float d = half_bits_to_float(hd.x), dmin = half_bits_to_float(hd.x >> 16);
  uint32_t scl, mnl, sch, mnh;
  scale_min(hd.y, hd.z, hd.w, 2 * it, scl, mnl);
  scale_min(hd.y, hd.z, hd.w, 2 * it + 1, sch, mnh);
  const float d1 = d * (float)scl, m1 = dmin * (float)mnl;
  const float d2 = d * (float)sch, m2 = dmin * (float)mnh;
  const uint32_t words[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
  float* o = out + (size_t)n * K + (size_t)s * 64;
#pragma unroll
  for (int wd = 0; wd < 8; ++wd) {
    float4 lo, hi;
    const uint32_t q = words[wd];
    lo.x = (float)(q & 0xFu) * d1 - m1;
    lo.y = (float)((q >> 8) & 0xFu) * d1 - m1;
    lo.z = (float)((q >> 16) & 0xFu) * d1 - m1;
    lo.w = (float)((q >> 24) & 0xFu) * d1 - m1;
    hi.x = (float)((q >> 4) & 0xFu) * d2 - m2;
    hi.y = (float)((q >> 12) & 0xFu) * d2 - m2;
    hi.z = (float)((q >> 20) & 0xFu) * d2 - m2;
    hi.w = (float)((q >> 28) & 0xFu) * d2 - m2;
    *reinterpret_cast<float4*>(o + 4 * wd) = lo;
    *reinterpret_cast<float4*>(o + 32 + 4 * wd) = hi;
  }
}

template <int R, int KP, int G>
int launch_rows(const Q4kParams& p, uint32_t wgs, hipStream_t stream) {
  const size_t lds = std::max((size_t)(p.K / 64) * 68, (size_t)G * R * KP) * sizeof(float);
  hipLaunchKernelGGL((q4k_matvec_rows_kernel<R, KP, G>), dim3(wgs, p.B), dim3(64 * KP * G), lds,
                     stream, p);
  STS_HIP(hipGetLastError());
  return STS_OK;
}

// K <= 4096: eight waves per CU in workgroups of four.  K > 4096: one
// workgroup of G groups (12 waves) per CU, so that x, up to 64 KB, is staged
// once per CU (for the FFN's linear_out [4096, 11264]: 7.3 us, against 8.3
// with two groups per workgroup and 9.4-11.0 with one).  In both cases as
// many more groups as keep each at 12 rows or fewer, and no more groups than
// rows; R = rows per group.
template <int KP, int G>
int launch_rows_kp(const Q4kParams& p, hipStream_t stream) {
  const uint32_t cus = (uint32_t)device_cu_count();
  const uint32_t min_groups = KP == 1 ? 8u * cus : G * cus;
  const uint32_t groups = std::min(std::max(min_groups, (p.N + 11) / 12), p.N);
  const uint32_t wgs = (groups + G - 1) / G;
  const uint32_t r = (p.N + G * wgs - 1) / (G * wgs);
  switch (r) {
    case 1: return launch_rows<1, KP, G>(p, wgs, stream);
    case 2: return launch_rows<2, KP, G>(p, wgs, stream);
    case 3: return launch_rows<3, KP, G>(p, wgs, stream);
    case 4: return launch_rows<4, KP, G>(p, wgs, stream);
    case 5: return launch_rows<5, KP, G>(p, wgs, stream);
    case 6: return launch_rows<6, KP, G>(p, wgs, stream);
    case 7: return launch_rows<7, KP, G>(p, wgs, stream);
    case 8: return launch_rows<8, KP, G>(p, wgs, stream);
    case 9: return launch_rows<9, KP, G>(p, wgs, stream);
    case 10: return launch_rows<10, KP, G>(p, wgs, stream);
    case 11: return launch_rows<11, KP, G>(p, wgs, stream);
    default: return launch_rows<12, KP, G>(p, wgs, stream);
  }
}

}  // namespace

int launch_q4k_matvec(const Q4kParams& p, hipStream_t stream) {
  const uint32_t kp = (p.K / 64 + 63) / 64;
  if (kp == 1) return launch_rows_kp<1, 4>(p, stream);
  if (kp == 2) return launch_rows_kp<2, 6>(p, stream);
  if (kp == 3) return launch_rows_kp<3, 4>(p, stream);
  if (kp == 4) return launch_rows_kp<4, 3>(p, stream);
  return fail(STS_ERR_INVALID, "K = %u too large (at most 16384)", p.K);
}

int launch_q4k_dequant(const uint8_t* w, float* out, uint32_t N, uint32_t K, hipStream_t stream) {
  const uint64_t threads = (uint64_t)N * (K / 64);
  const uint64_t wgs = (threads + 255) / 256;
  if (wgs > 0x7FFFFFFFull) return fail(STS_ERR_INVALID, "matrix too large for one launch");
  hipLaunchKernelGGL(q4k_dequant_kernel, dim3((uint32_t)wgs), dim3(256), 0, stream, w, out, N, K);
  STS_HIP(hipGetLastError());
  return STS_OK;
}

}  // namespace sts
