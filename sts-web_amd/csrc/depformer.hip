// depformer.hip -- kernels of the depformer step chain for gfx950, batched over streams.
//
// The reference (crates/sts-wasm/src/depth_engine.rs:884-1491) runs one stream
// per frame: per step an embedding lookup and add, six layers of RMSNorm,
// Q4_K matvecs, cache writes, attention, SwiGLU and residual adds, then an
// output matvec and top-k sampling, each a separate WGSL dispatch.  Here the
// streams of a batch share every weight read: the Q4_K products become
// GEMMs with the streams as the M dimension.
//
// q4k_gemm_kernel.  Workgroup = one 16-stream tile x all K: wave kb owns
// super-block column kb (256 weights of every row) and keeps the 64 x values
// of its lane in registers; the workgroup walks 16-row tiles.  Per tile a
// wave dequantises the shader's f32 weights w = (d*scale)*q - dmin*min
// (shader_q4k_matvec.wgsl:117-136, products and difference rounded
// separately, so the weights are bit-identical) and feeds them to
// v_mfma_f32_16x16x4f32: lane (r, g) supplies W[n0 + r][k] and X[m0 + r][k]
// for k = 256 kb + 64 g + i at instruction i, g = lane / 16 being slot g of
// the super-block (its 32 quant bytes, low nibbles sub-block 2g, high 2g+1).
// The waves' partial tiles are summed through LDS in wave order
// (deterministic), with the residual or the SwiGLU of a gate/value row pair
// applied on the way out.
#include <algorithm>
#include <cfloat>
#include <cstdint>
#include <type_traits>

#include "common.hpp"
#include "depformer.hpp"
#include "q4k.hpp"

namespace sts {

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kGemmBufferWord3 = 0x00020000;  // raw 32-bit buffer, no swizzle

__device__ __forceinline__ u32x4 ld16(const uint8_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

// The 48 weight bytes lane (r, g) needs of one super-block row: header and
// the 32 quant bytes of slot g.
struct WTile {
  u32x4 hd, qa, qb;
};

// MAXT: the largest workgroup (64 * K/256 threads) the instance runs with;
// 256 (K <= 1024) leaves the register file to the prefetch buffers.  Three
// waves per SIMD (three 4-wave workgroups per CU at K <= 1024): one register
// past 168 would leave room for two.
template <bool SWIGLU, int MAXT>
__global__ __launch_bounds__(MAXT) __attribute__((amdgpu_waves_per_eu(3)))
void q4k_gemm_kernel(const Q4kGemmParams p) {
#pragma clang fp contract(off)
  constexpr int NH = SWIGLU ? 2 : 1;
  __shared__ float part[16][NH][256];
  __shared__ float ssq[16][16];
  __shared__ float s_inv[16];  // 1/rms of the tile's rows (RMSNorm)
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int kb = tid >> 6;
  const int r = lane & 15, g = lane >> 4;
  const uint32_t KB = p.K / kQ4kBlockWeights;  // waves in the workgroup
  const uint32_t z = blockIdx.z, mt = blockIdx.y;
  const uint8_t* W = p.w[z];
  const float* X = p.x + z * p.x_zstride;
  float* Y = p.y + z * p.y_zstride;
  const uint32_t nout = SWIGLU ? p.swiglu_f : p.N;
  const uint32_t ntiles = (nout + 15) / 16;
  const size_t row_bytes = (size_t)(p.w_row_blocks ? p.w_row_blocks : KB) * kQ4kBlockBytes;

  // Rows past the end (and tiles past the last) re-read valid rows; their
  // outputs are not stored.
  auto load_w = [&](WTile (&wt)[NH], uint32_t t) {
    t = min(t, ntiles - 1);
#pragma unroll
    for (int hv = 0; hv < NH; ++hv) {
      const uint32_t n = min(t * 16 + r + (hv ? p.swiglu_f : 0u), p.N - 1);
      const uint8_t* blk = W + n * row_bytes + (size_t)kb * kQ4kBlockBytes;
      wt[hv].hd = ld16(blk);
      wt[hv].qa = ld16(blk + 16 + 32 * g);
      wt[hv].qb = ld16(blk + 32 + 32 * g);
    }
  };
  // The first tile's weights are requested before x, so both latencies overlap.
  WTile cur[NH], nxt[NH];
  load_w(cur, blockIdx.x);

  // x values of this lane: X[m][256 kb + 64 g + j], j < 64 (zero past M).
  // The tile's rows come in through a buffer resource that ends with its last
  // row inside M, so rows past M read zeros: no per-row branch or select.
  const uint32_t rows_here = min(16u, p.M - mt * 16);
  const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(X) + (size_t)mt * 16 * p.ldx, 0,
      (int)(((uint64_t)(rows_here - 1) * p.ldx + p.K) * sizeof(float)), kGemmBufferWord3);
  auto ldx4 = [&](uint32_t row, uint32_t col) {
    return __builtin_bit_cast(
        float4, __builtin_amdgcn_raw_buffer_load_b128(
                    xrs, (uint32_t)((row * p.ldx + col) * sizeof(float)), 0, 0));
  };
  float xv[64];
  {
    // Through a per-wave LDS chunk (16 rows x 64 floats, pitch 68) so the
    // global loads are coalesced: instruction i of chunk c reads rows
    // 4i..4i+3, 256 contiguous bytes each; the lanes of slot g then copy
    // chunk g (the 16 lanes of a read phase hit distinct banks).  (Each lane
    // reading its own 256 bytes would touch 64 cache lines per instruction.)
    // Chunks in flight at once: all four where a wave may hold 168 registers,
    // two in the 16-wave instance (128).
    constexpr int CIF = MAXT <= 256 ? 4 : 2;
    __shared__ __align__(16) float xs[MAXT / 64][16][68];
#pragma unroll
    for (int c0 = 0; c0 < 4; c0 += CIF) {
      float4 ld[CIF][4];
#pragma unroll
      for (int c = 0; c < CIF; ++c)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          ld[c][i] = ldx4(4 * i + (lane >> 4), 256 * kb + 64 * (c0 + c) + 4 * (lane & 15));
#pragma unroll
      for (int c = 0; c < CIF; ++c) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          *reinterpret_cast<float4*>(&xs[kb][4 * i + (lane >> 4)][4 * (lane & 15)]) = ld[c][i];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (g == c0 + c) {
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const float4 t = *reinterpret_cast<const float4*>(&xs[kb][r][4 * j]);
            xv[4 * j] = t.x;
            xv[4 * j + 1] = t.y;
            xv[4 * j + 2] = t.z;
            xv[4 * j + 3] = t.w;
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
    }
  }
  if (p.norm_alpha) {
    // RMSNorm of the 16 rows (shader_rmsnorm.wgsl:80-90), x * (1/rms) * alpha,
    // with the sum of squares taken over this workgroup's registers.  alpha
    // scales x here and 1/rms (one factor per row) scales the row's outputs
    // in the epilogue: sum_k w (x alpha) / rms, one multiply per x value
    // instead of two.
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < 64; ++j) q = __builtin_fmaf(xv[j], xv[j], q);
    q += __shfl_xor(q, 16, 64);
    q += __shfl_xor(q, 32, 64);
    if (g == 0) ssq[kb][r] = q;
    __syncthreads();
    if (tid < 16) {
      float tot = ssq[0][tid];
      for (uint32_t w = 1; w < KB; ++w) tot += ssq[w][tid];
      s_inv[tid] = 1.0f / sqrtf(tot / (float)p.K + p.norm_eps);
    }
    const float4* al = reinterpret_cast<const float4*>(p.norm_alpha + 256 * kb + 64 * g);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float4 a = al[j];
      xv[4 * j] = xv[4 * j] * a.x;
      xv[4 * j + 1] = xv[4 * j + 1] * a.y;
      xv[4 * j + 2] = xv[4 * j + 2] * a.z;
      xv[4 * j + 3] = xv[4 * j + 3] * a.w;
    }
  }

  for (uint32_t t = blockIdx.x; t < ntiles; t += gridDim.x) {
    // The next tile's weights are in flight during this one (the condition
    // is uniform over the workgroup).
    if (t + gridDim.x < ntiles) load_w(nxt, t + gridDim.x);
#pragma unroll
    for (int hv = 0; hv < NH; ++hv) {
      const u32x4 hd = cur[hv].hd, qa = cur[hv].qa, qb = cur[hv].qb;
      const float d = half_bits_to_float(hd.x), dmin = half_bits_to_float(hd.x >> 16);
      uint32_t scl, mnl, sch, mnh;
      scale_min(hd.y, hd.z, hd.w, 2 * g, scl, mnl);
      scale_min(hd.y, hd.z, hd.w, 2 * g + 1, sch, mnh);
      // d1 = d*scale and m1 = dmin*min are exact in f32 (11-bit f16
      // significands times 6-bit integers), and so is q*d1 (4-bit q), so
      // fma(q, d1, -m1) rounds once, where the shader's (d*scale)*q - dmin*min
      // rounds: the same weight, bit for bit.
      const float d1 = d * (float)scl, m1 = dmin * (float)mnl;
      const float d2 = d * (float)sch, m2 = dmin * (float)mnh;
      const uint32_t words[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
      floatx4 acc[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        uint32_t lo = words[w] & 0x0F0F0F0Fu;
        uint32_t hi = (words[w] >> 4) & 0x0F0F0F0Fu;
        // Opaque to the optimiser, so each byte below is one v_cvt_f32_ubyte.
        asm("" : "+v"(lo), "+v"(hi));
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const float wl = __builtin_fmaf((float)((lo >> (8 * b)) & 0xFFu), d1, -m1);
          acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(wl, xv[4 * w + b], acc[b], 0, 0, 0);
        }
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const float wh = __builtin_fmaf((float)((hi >> (8 * b)) & 0xFFu), d2, -m2);
          acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(wh, xv[32 + 4 * w + b], acc[b], 0, 0, 0);
        }
      }
      const floatx4 s = (acc[0] + acc[1]) + (acc[2] + acc[3]);
      // Accumulator element e of lane (r, g) is row 4g + e, stream r of the tile.
#pragma unroll
      for (int e = 0; e < 4; ++e) part[kb][hv][(4 * g + e) * 16 + r] = s[e];
    }
    __syncthreads();
    for (int o = tid; o < 256; o += blockDim.x) {
      const uint32_t mo = mt * 16 + (o & 15), no = t * 16 + (o >> 4);
      float v = part[0][0][o];
      for (uint32_t w = 1; w < KB; ++w) v += part[w][0][o];
      const float inv = p.norm_alpha ? s_inv[o & 15] : 1.0f;
      v *= inv;
      if constexpr (SWIGLU) {
        float u = part[0][NH - 1][o];
        for (uint32_t w = 1; w < KB; ++w) u += part[w][NH - 1][o];
        u *= inv;
        v = v / (1.0f + expf(-v)) * u;
      }
      if (mo < p.M && no < nout) {
        if (p.res) v += p.res[(size_t)mo * p.ldr + no];
        Y[(size_t)mo * p.ldy + no] = v;
      }
    }
    __syncthreads();
#pragma unroll
    for (int hv = 0; hv < NH; ++hv) cur[hv] = nxt[hv];
  }
}

// One workgroup of 256 per row, shader_rmsnorm.wgsl:27-92 step for step.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ x,
                                                      const float* __restrict__ alpha,
                                                      float* __restrict__ out, uint32_t D,
                                                      float eps) {
#pragma clang fp contract(off)
  __shared__ float sums[256];
  const uint32_t t = threadIdx.x;
  const float* xr = x + (size_t)blockIdx.x * D;
  float* yr = out + (size_t)blockIdx.x * D;
  float acc = 0.f;
  for (uint32_t i = t; i < D; i += 256) acc += xr[i] * xr[i];
  sums[t] = acc;
  __syncthreads();
  for (uint32_t half = 128; half >= 2; half >>= 1) {
    if (t < half) sums[t] += sums[t + half];
    __syncthreads();
  }
  const float total = sums[0] + sums[1];
  const float rms = sqrtf(total / (float)D + eps);
  const float inv = 1.0f / rms;
  for (uint32_t i = t; i < D; i += 256) yr[i] = xr[i] * inv * alpha[i];
}

// shader_embed_q4.wgsl:58-107 fused with shader_vec_add.wgsl:20-28.
__global__ __launch_bounds__(256) void embed_add_kernel(const uint8_t* __restrict__ table,
                                                        uint32_t vocab,
                                                        const uint32_t* __restrict__ tokens,
                                                        uint64_t tok_stride,
                                                        const float* __restrict__ proj,
                                                        float* __restrict__ h, uint32_t D) {
  const uint32_t e = blockIdx.x * 256 + threadIdx.x;
  const uint32_t b = blockIdx.y;
  if (e >= D) return;
  // Two memory round trips: the projection with the token, then the three
  // bytes of the token's Q4_0 block this element needs, all at once (an
  // out-of-range token reads row 0 and adds nothing).
  const float pv = proj[(size_t)b * D + e];
  const uint32_t tok = tokens[(size_t)b * tok_stride];
  const bool ok = tok < vocab;
  const uint8_t* blk = table + ((size_t)(ok ? tok : 0u) * (D / 32) + e / 32) * 18;
  const uint32_t pos = e % 32;
  // The f16 scale as one 16-bit load (18-byte blocks keep it 2-byte aligned).
  const uint32_t bits = *reinterpret_cast<const uint16_t*>(blk);
  const uint32_t qb = blk[2 + (pos & 15u)];
  // An Inf/NaN scale reads as 0 (shader_embed_q4.wgsl:48-51).
  const float scale = ((bits >> 10) & 0x1Fu) == 0x1Fu ? 0.f : half_bits_to_float(bits);
  const uint32_t nib = pos < 16 ? (qb & 0xFu) : (qb >> 4);
  const float emb = ok ? ((float)nib - 8.0f) * scale : 0.f;
  h[(size_t)b * D + e] = pv + emb;
}

// Monotone map of a float to a uint32 (larger float -> larger key), and back.
__device__ __forceinline__ uint32_t order_key(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_value(uint32_t k) {
  return __builtin_bit_cast(float, (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// Inclusive prefix sum over the 64 lanes: Hillis-Steele inside each 16-lane
// row (DPP row_shr 1, 2, 4, 8), then the row totals carried across rows by
// the GFX9 row broadcasts (lane 15 into rows 1 and 3, lane 31 into rows 2
// and 3).
__device__ __forceinline__ uint32_t wave_scan_incl(uint32_t v) {
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, false);  // row_shr:8
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false);  // row_bcast:15
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return v;
}

// The value of lane ^ MASK (MASK < 16): quad permutations on DPP, the
// ds_swizzle bitmask mode (xor) above that.
template <int MASK>
__device__ __forceinline__ uint32_t lane_xor(uint32_t x) {
  if constexpr (MASK == 1)
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
  else if constexpr (MASK == 2)
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
  else
    return (uint32_t)__builtin_amdgcn_ds_swizzle((int)x, 0x1F | (MASK << 10));
}

// Bitonic sort of 64 64-bit keys, one per lane, into descending order (lane l
// ends with the wave's key of rank l).  Partners at lane distance 16 and 32
// come from the gfx950 permlane swaps, which return the lane's own key and
// its partner's in a lane-dependent order: the compare-exchange takes the
// larger or smaller of the two, which does not depend on that order.
template <int SIZE, int STRIDE>
__device__ __forceinline__ void wave_bitonic_steps(uint64_t& x, uint32_t lane) {
  // The lower partner of a pair keeps the larger key in blocks that sort
  // descending (lane & SIZE clear), the smaller one in blocks that sort
  // ascending.
  const bool keep_max = ((lane & STRIDE) == 0) == ((lane & SIZE) == 0);
  if constexpr (STRIDE >= 16) {
    const uint32_t lo = (uint32_t)x, hi = (uint32_t)(x >> 32);
    const auto l2 = STRIDE == 16 ? __builtin_amdgcn_permlane16_swap(lo, lo, false, false)
                                 : __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
    const auto h2 = STRIDE == 16 ? __builtin_amdgcn_permlane16_swap(hi, hi, false, false)
                                 : __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
    const uint64_t a = ((uint64_t)h2[0] << 32) | l2[0], c = ((uint64_t)h2[1] << 32) | l2[1];
    const uint64_t mx = a > c ? a : c, mn = a > c ? c : a;
    x = keep_max ? mx : mn;
  } else {
    const uint32_t lo = lane_xor<STRIDE>((uint32_t)x), hi = lane_xor<STRIDE>((uint32_t)(x >> 32));
    const uint64_t y = ((uint64_t)hi << 32) | lo;
    x = (keep_max ? y > x : y < x) ? y : x;
  }
  if constexpr (STRIDE > 1) wave_bitonic_steps<SIZE, STRIDE / 2>(x, lane);
}
template <int SIZE>
__device__ __forceinline__ void wave_bitonic_sort(uint64_t& x, uint32_t lane) {
  wave_bitonic_steps<SIZE, SIZE / 2>(x, lane);
  if constexpr (SIZE < 64) wave_bitonic_sort<SIZE * 2>(x, lane);
}

// Number of keys of the descending list L[0..64) above x (STRICT) or at or
// above x: a branch-free binary search, 6 halving steps and a last check.
template <bool STRICT>
__device__ __forceinline__ uint32_t count_above(const uint64_t* L, uint64_t x) {
  uint32_t pos = 0;
#pragma unroll
  for (uint32_t step = 32; step >= 1; step >>= 1) {
    const uint64_t y = L[pos + step - 1];
    pos += (STRICT ? y > x : y >= x) ? step : 0u;
  }
  const uint64_t y = L[pos];  // pos <= 63 here
  return pos + ((STRICT ? y > x : y >= x) ? 1u : 0u);
}

// shader_sample_topk.wgsl for one stream per workgroup, token for token.
// Penalty, temperature and (top_k <= 1) the argmax follow the shader's lanes
// and tree exactly.  The top K are found by a radix select of the K-th
// largest value and ranked by (value descending, index ascending) keys,
// per-wave bitonic sorts merged by binary-search ranks, which is the shader's
// selection and insertion sort unless logits the order depends on are equal;
// then wave 0 replays the shader's selection (first minimum replaced) and the
// slots are ranked as its stable sort ranks them.  exp(v - max) is taken
// correctly rounded; the draw comes from a wave scan, checked against the
// shader's running total and redone on one lane where they could differ.
// Thread t holds logits t, t + 256, ... in registers: NJ of them,
// NJ * 256 >= V.

// Bound on how far the sampler's wave-scan running total can be from the
// shader's single-lane one: each is within about 2K ulps of 1 of the exact
// total (positive terms, K <= 256: 2 * 256 * 2^-24 = 3.1e-5), so they differ
// by less than 6.2e-5 < 2^-13.
constexpr float kDrawSlack = 1.0f / 8192.0f;

template <int NJ>
__global__ __launch_bounds__(256) void sample_topk_kernel(const SampleParams p) {
  __shared__ float vals[NJ * 256];
  __shared__ float tv[256];
  __shared__ uint32_t ti[256];
  __shared__ __align__(16) uint32_t hist[3][256];
  __shared__ uint32_t s_cnt[2][64];
  __shared__ __align__(16) float ev[kMaxTopK];
  __shared__ uint32_t ri[kMaxTopK];
  __shared__ float s_maxv;
  __shared__ uint32_t s_pbits[4096 / 32];  // the listed penalty tokens, one bit each
  __shared__ uint64_t sbuf[2 * kMaxTopK];
  __shared__ uint32_t slot_idx[kMaxTopK];  // replayed selection: slot -> logit index
  __shared__ uint32_t s_tie[2];            // keys >= the K-th, any equal neighbours
  __shared__ __align__(16) float cumv[kMaxTopK];  // the scan's running totals, then the weights
  static_assert(kMaxTopK == 256, "one key per thread in the ranking sort");
  const uint32_t tid = threadIdx.x, b = blockIdx.x, V = p.V;
  const uint32_t lane = tid & 63u, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const float* lg = p.logits + (size_t)b * p.ld_logits;

  // The logits first; the penalty tokens once their count is in (only that
  // many are guaranteed readable).
  const uint32_t np = min(p.num_penalty[(size_t)b * p.rs_stride], kMaxPenalty);
  const float rnd = p.rand[(size_t)b * p.rs_stride];  // the draw's, requested now
  float x[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const uint32_t i = tid + 256u * j;
    x[j] = i < V ? lg[i] : 0.f;
  }
  const uint32_t tok = tid < np ? p.ptoks[(size_t)b * p.pt_stride + tid] : 0u;
  hist[0][tid] = 0;
  hist[1][tid] = 0;

  // Repetition penalty (:56-69); a token listed twice is penalised once (the
  // shader's lanes all read before they write).  The listed tokens set their
  // bits in an LDS bitmap, and each thread penalises the logits it holds.
  static_assert(NJ * 256 <= 4096, "penalty bitmap");
  if (np > 0) {
    if (tid < 4096 / 32) s_pbits[tid] = 0;
    __syncthreads();
    if (tid < np && tok < V) atomicOr(&s_pbits[tok >> 5], 1u << (tok & 31u));
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const uint32_t i = tid + 256u * j;
      if (i < V && ((s_pbits[i >> 5] >> (i & 31u)) & 1u))
        x[j] = x[j] > 0.f ? x[j] / p.penalty : x[j] * p.penalty;
    }
  }
  // Temperature (:72-88).
#pragma unroll
  for (int j = 0; j < NJ; ++j) x[j] = x[j] / p.temperature;

  uint32_t* outp = p.out + (size_t)b * p.out_stride;
  const uint32_t K = p.top_k;
  if (K <= 1) {
    // Per-lane maxima and the tree argmax (:95-106), first index on ties
    // within a lane.
    float lmax = -3.402823466e+38f;
    uint32_t lidx = 0;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const uint32_t i = tid + 256u * j;
      if (i < V && x[j] > lmax) {
        lmax = x[j];
        lidx = i;
      }
    }
    tv[tid] = lmax;
    ti[tid] = lidx;
    __syncthreads();
    for (uint32_t half = 128; half > 0; half >>= 1) {
      if (tid < half && tv[tid + half] > tv[tid]) {
        tv[tid] = tv[tid + half];
        ti[tid] = ti[tid + half];
      }
      __syncthreads();
    }
    if (tid == 0) *outp = ti[0];
    return;
  }

  // -0 takes the key of +0: the two compare equal as floats, so they tie
  // (and go by index) as in a float comparison.
  uint32_t k[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) k[j] = order_key(x[j] == 0.f ? 0.f : x[j]);
  __syncthreads();  // histograms cleared

  // Radix select of the Ks-th largest key, 8 bits at a time from the top,
  // stopping early once the bin holding it is taken whole.  Every wave picks
  // the digit itself from the histogram (one barrier per pass); the three
  // histograms rotate, pass p clearing the one pass p + 2 counts into, whose
  // last reads (pass p - 1) all precede this pass's barrier.
  const uint32_t Ks = min(K, V);
  uint32_t prefix = 0, mask = 0, rem = Ks;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    uint32_t* H = hist[pass % 3];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      if (tid + 256u * j < V && (k[j] & mask) == prefix) atomicAdd(&H[(k[j] >> shift) & 0xFFu], 1u);
    }
    __syncthreads();
    // Lane l holds bins 4g .. 4g+3 with g = 63 - l, so the lane prefix sum
    // counts the keys in bins >= 4g; the lane whose bins straddle the
    // rem-th largest key has above < rem <= incl.
    const uint32_t g = 63u - lane;
    const uint4 hb = *reinterpret_cast<const uint4*>(&H[4 * g]);
    const uint32_t own = hb.x + hb.y + hb.z + hb.w;
    const uint32_t incl = wave_scan_incl(own);
    const uint32_t above = incl - own;
    const uint32_t h[4] = {hb.x, hb.y, hb.z, hb.w};
    uint32_t cum = above, dig = 0, nrem = 0, exact = 0;
    bool found = false;
#pragma unroll
    for (int d = 3; d >= 0; --d) {
      const bool here = !found && cum + h[d] >= rem;
      dig = here ? 4 * g + d : dig;
      nrem = here ? rem - cum : nrem;
      exact = here ? (uint32_t)(h[d] == rem - cum) : exact;
      found |= here;
      cum += h[d];
    }
    // Read with every lane active (the source lane must hold its values).
    const uint64_t hit = __ballot(above < rem && incl >= rem);
    const int src = hit ? (int)__builtin_ctzll(hit) : 0;  // one lane hits
    const uint32_t digit = __builtin_amdgcn_readlane(dig, src);
    rem = __builtin_amdgcn_readlane(nrem, src);
    const uint32_t ex = __builtin_amdgcn_readlane(exact, src);
    hist[(pass + 2) % 3][tid] = 0;
    prefix |= digit << shift;
    mask |= 0xFFu << shift;
    if (ex) break;
  }

  // Collection in index order: keys above the threshold prefix all, of those
  // on it the first `rem` (all of them when the bin was taken whole).  Slots
  // come from per-(j, wave) ballot counts, so the order is deterministic.
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const bool valid = tid + 256u * j < V;
    const uint64_t bg = __ballot(valid && (k[j] & mask) > prefix);
    const uint64_t be = __ballot(valid && (k[j] & mask) == prefix);
    if (lane == 0) {
      s_cnt[0][4 * j + wave] = (uint32_t)__builtin_popcountll(bg);
      s_cnt[1][4 * j + wave] = (uint32_t)__builtin_popcountll(be);
    }
  }
  __syncthreads();
  // Entries past 4 * NJ are never written: they count nothing.
  const uint32_t cg = lane < 4u * NJ ? s_cnt[0][lane] : 0u;
  const uint32_t ce = lane < 4u * NJ ? s_cnt[1][lane] : 0u;
  const uint32_t ig = wave_scan_incl(cg), ie = wave_scan_incl(ce);
  const uint32_t xg = ig - cg, xe = ie - ce;  // exclusive prefix over (j, wave)
  const uint32_t total_g = __builtin_amdgcn_readlane(ig, 63);
  uint64_t* ck = sbuf;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const uint32_t i = tid + 256u * j;
    const bool valid = i < V;
    const bool gt = valid && (k[j] & mask) > prefix, eq = valid && (k[j] & mask) == prefix;
    const uint64_t bg = __ballot(gt), be = __ballot(eq);
    // The bases are read with every lane active: inside the divergent branch
    // below, the source lane 4j + wave may be inactive, and the compiler is
    // free to compute xg / xe there for the active lanes only.
    const uint32_t gbase = __builtin_amdgcn_readlane(xg, 4 * j + wave);
    const uint32_t ebase = __builtin_amdgcn_readlane(xe, 4 * j + wave);
    const uint64_t key = ((uint64_t)k[j] << 32) | (0xFFFFFFFFu - i);
    if (gt) {
      const uint32_t slot = gbase + __builtin_amdgcn_mbcnt_hi(
                                        (uint32_t)(bg >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bg, 0u));
      if (slot < kMaxTopK) ck[slot] = key;
    } else if (eq) {
      const uint32_t e = ebase + __builtin_amdgcn_mbcnt_hi(
                                     (uint32_t)(be >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)be, 0u));
      if (e < rem && total_g + e < kMaxTopK) ck[total_g + e] = key;
    }
  }
  // Slots past the Ks taken hold 0, below every real key (the index part of
  // a real key is at least 2^32 - kMaxVocab).
  if (tid >= Ks) ck[tid] = 0;
  __syncthreads();

  // Rank the keys of ck, descending.  Each wave sorts its 64 keys; a key's
  // rank is its place in its wave's list plus the keys above it in the other
  // three lists (equal keys, the padding zeros, count as above when they are
  // in a lower wave, so the ranks are distinct).  Leaves the key of rank tid
  // in sbuf[256 + tid] and returns it.
  auto rank_keys = [&]() -> uint64_t {
    uint64_t key = ck[tid];
    wave_bitonic_sort<2>(key, lane);
    uint64_t* lists = sbuf;  // each thread overwrites only the slot it read
    lists[tid] = key;
    __syncthreads();
    uint32_t rank = lane;
#pragma unroll
    for (uint32_t i = 1; i < 4; ++i) {
      const uint32_t w2 = (wave + i) & 3u;
      rank += w2 > wave ? count_above<true>(lists + 64 * w2, key)
                        : count_above<false>(lists + 64 * w2, key);
    }
    sbuf[256 + rank] = key;
    __syncthreads();
    return sbuf[256 + tid];
  };
  // Value descending, index ascending: the shader's selection and insertion
  // sort (:134-196) whenever no two of the logits the order depends on are
  // equal.
  uint64_t key = rank_keys();
  bool tied = false;
  if (V > K) {
    // Ties: two of the K taken with equal values (the stable insertion sort
    // orders them by the shader's slot, not by index), or a logit left out
    // with the value of the K-th (which of those the shader keeps depends on
    // its slots).  Either changes only which index stands at the ranks of
    // the equal values, never the values at any rank.
    const uint32_t tkey = (uint32_t)(sbuf[256 + K - 1] >> 32);
    bool tie = tid + 1 < K && (uint32_t)(sbuf[256 + tid + 1] >> 32) == (uint32_t)(key >> 32);
    uint32_t n_ge = 0;
#pragma unroll
    for (int j = 0; j < NJ; ++j) n_ge += (tid + 256u * j < V && k[j] >= tkey) ? 1u : 0u;
    n_ge = __builtin_amdgcn_readlane(wave_scan_incl(n_ge), 63);  // the wave's total
    if (tid == 0) s_tie[0] = s_tie[1] = 0;
    __syncthreads();
    if (lane == 0 && n_ge) atomicAdd(&s_tie[0], n_ge);
    if (tie) s_tie[1] = 1;
    __syncthreads();
    tied = s_tie[1] != 0 || s_tie[0] > K;
  }
  // K > V: the shader's unused slots hold (-3.402823466e+38, 0).
  const bool real = tid < Ks;
  const float v = real ? key_value((uint32_t)(key >> 32)) : -3.402823466e+38f;
  ri[tid] = real ? 0xFFFFFFFFu - (uint32_t)key : 0u;
  if (tid == 0) s_maxv = v;
  __syncthreads();
  // Softmax over the K (:198-210): exp(v - max) correctly rounded to f32
  // (through f64), the rounding the oracle takes for WGSL's exp.
  const float max_v = s_maxv;
  ev[tid] = tid < K ? (float)exp((double)(v - max_v)) : 0.f;  // +0 past K
  __syncthreads();
  if (tid < 64) {
    // The cumulative draw (:212-221).  Wave 0: lane l holds values 4l..4l+3;
    // the sum and the running total come from a wave scan, a different f32
    // order from the shader's single-lane loop, less than kDrawSlack away
    // from it.  The scan's pick is therefore the shader's whenever rand lies
    // further than kDrawSlack from the boundaries around it; otherwise lane 0
    // redoes the shader's loop.
    float e[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) e[c] = 4 * tid + c < K ? ev[4 * tid + c] : 0.f;
    float sum = (e[0] + e[1]) + (e[2] + e[3]);
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) sum += __shfl_xor(sum, off, 64);
    float q[4], run = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      run += e[c] / sum;
      q[c] = run;  // inclusive prefix within the lane
    }
    // Exclusive prefix of the lane totals.
    float pre = run;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float w = __shfl_up(pre, off, 64);
      if (tid >= off) pre += w;
    }
    pre -= run;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (4 * tid + c < K) cumv[4 * tid + c] = pre + q[c];
    int first = 4;
#pragma unroll
    for (int c = 3; c >= 0; --c)
      if (4 * tid + c < K && rnd < pre + q[c]) first = c;
    const uint64_t hits = __ballot(first < 4);
    uint32_t pick = K - 1;
    if (hits) {
      const int lane0 = __builtin_ctzll(hits);
      pick = 4 * lane0 + __shfl(first, lane0, 64);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // Certain when rand sits clear of the pick's upper boundary (or, with no
    // hit, of the last total) and of its lower one.
    const bool sure = hits ? (rnd < cumv[pick] - kDrawSlack &&
                              (pick == 0 || rnd >= cumv[pick - 1] + kDrawSlack))
                           : rnd >= cumv[K - 1] + kDrawSlack;
    if (!sure) {
      // The shader's order: the sum in slot order, each weight divided by
      // it, the running total in slot order.  Both chains run on lane 0 over
      // 16 values at a time from LDS (the loads ahead of the additions; the
      // slots past K hold +0, which leaves a sum unchanged), the divisions on
      // every lane in between.
      float sq = 0.f;
      if (tid == 0) {
        for (uint32_t j0 = 0; j0 < K; j0 += 16) {
          float4 t[4];
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) t[q4] = *reinterpret_cast<const float4*>(&ev[j0 + 4 * q4]);
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            sq = sq + t[q4].x;
            sq = sq + t[q4].y;
            sq = sq + t[q4].z;
            sq = sq + t[q4].w;
          }
        }
      }
      sq = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sq)));
#pragma unroll
      for (int c = 0; c < 4; ++c) cumv[4 * tid + c] = e[c] / sq;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      uint32_t pk = K - 1;
      if (tid == 0) {
        float cum = 0.f;
        bool found = false;
        for (uint32_t j0 = 0; j0 < K && !found; j0 += 16) {
          float4 t[4];
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) t[q4] = *reinterpret_cast<const float4*>(&cumv[j0 + 4 * q4]);
          const float w[16] = {t[0].x, t[0].y, t[0].z, t[0].w, t[1].x, t[1].y, t[1].z, t[1].w,
                               t[2].x, t[2].y, t[2].z, t[2].w, t[3].x, t[3].y, t[3].z, t[3].w};
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            cum = cum + w[i];
            if (!found && j0 + i < K && rnd < cum) {
              pk = j0 + i;
              found = true;
            }
          }
        }
      }
      pick = __builtin_amdgcn_readfirstlane(pk);
    }
    if (tid == 0) {
      // The draw picked a rank (the values by rank, and so the draw, are the
      // same whatever order equal values take).  Only a rank whose value
      // another rank among the K shares, or the K-th value when more logits
      // share it than were taken, can hold a different index in the shader.
      bool need = false;
      if (tied) {
        const uint32_t vp = (uint32_t)(sbuf[256 + pick] >> 32);
        need = (pick > 0 && (uint32_t)(sbuf[256 + pick - 1] >> 32) == vp) ||
               (pick + 1 < K && (uint32_t)(sbuf[256 + pick + 1] >> 32) == vp) ||
               (s_tie[0] > K && vp == (uint32_t)(sbuf[256 + K - 1] >> 32));
      }
      s_tie[1] = pick;
      s_tie[0] = need ? 1u : 0u;
      if (!need) *outp = ri[pick];
    }
  }
  __syncthreads();
  if (s_tie[0] == 0) return;
  const uint32_t pick = s_tie[1];
  // Then the shader's selection is replayed: wave 0 runs its loop over the
  // logits' keys in index order (vals is free once the keys exist), the
  // slots are ranked as its stable insertion sort ranks them, and the index
  // at the drawn rank is the token.
  uint32_t* lk = reinterpret_cast<uint32_t*>(vals);
#pragma unroll
  for (int j = 0; j < NJ; ++j)
    if (tid + 256u * j < V) lk[tid + 256u * j] = k[j];
  if (tid >= K) ck[tid] = 0;
  __syncthreads();
  if (wave == 0) {
    // Slot s = lane + 64c holds (key << 32 | s) and its logit's index.
    // Thread 0's loop (:148-178): slots 0..K-1 start with logits 0..K-1;
    // logit j >= K replaces the first slot holding the minimum when it is
    // strictly greater, and the minimum is found again.
    uint64_t sk[4];
    uint32_t sidx[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t sl = lane + 64u * c;
      sk[c] = sl < K ? ((uint64_t)lk[sl] << 32) | sl : ~0ull;
      sidx[c] = sl;
    }
    // The wave's minimum in every lane: partners within quads (DPP quad
    // permutations), mirrored within 8 and 16 lanes (DPP), then across 16
    // and 32 lanes (permlane swaps) -- register exchanges only.
    auto wave_min = [&]() {
      uint64_t m = sk[0];
#pragma unroll
      for (int c = 1; c < 4; ++c) m = sk[c] < m ? sk[c] : m;
      auto dpp_min = [&](auto ctrl) {
        constexpr int C = decltype(ctrl)::value;
        const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)m, C, 0xF, 0xF, false);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(m >> 32), C, 0xF, 0xF, false);
        const uint64_t o = ((uint64_t)hi << 32) | lo;
        m = o < m ? o : m;
      };
      dpp_min(std::integral_constant<int, 0xB1>{});   // quad_perm [1,0,3,2]
      dpp_min(std::integral_constant<int, 0x4E>{});   // quad_perm [2,3,0,1]
      dpp_min(std::integral_constant<int, 0x141>{});  // row_half_mirror
      dpp_min(std::integral_constant<int, 0x140>{});  // row_mirror
      {
        const auto l2 = __builtin_amdgcn_permlane16_swap((uint32_t)m, (uint32_t)m, false, false);
        const auto h2 = __builtin_amdgcn_permlane16_swap((uint32_t)(m >> 32), (uint32_t)(m >> 32), false, false);
        const uint64_t a = ((uint64_t)h2[0] << 32) | l2[0], c = ((uint64_t)h2[1] << 32) | l2[1];
        m = a < c ? a : c;
      }
      {
        const auto l2 = __builtin_amdgcn_permlane32_swap((uint32_t)m, (uint32_t)m, false, false);
        const auto h2 = __builtin_amdgcn_permlane32_swap((uint32_t)(m >> 32), (uint32_t)(m >> 32), false, false);
        const uint64_t a = ((uint64_t)h2[0] << 32) | l2[0], c = ((uint64_t)h2[1] << 32) | l2[1];
        m = a < c ? a : c;
      }
      return m;
    };
    uint64_t mn = wave_min();
    for (uint32_t j0 = K; j0 < V; j0 += 64) {
      const uint32_t j = j0 + lane;
      const bool in = j < V;
      const uint32_t kj = in ? lk[j] : 0u;
      uint64_t bits = __ballot(in && kj > (uint32_t)(mn >> 32));
      while (bits) {
        const int bl = __builtin_ctzll(bits);
        const uint32_t kb = __builtin_amdgcn_readlane(kj, bl);
        const uint32_t sl = (uint32_t)mn;
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (lane + 64u * c == sl) {
            sk[c] = ((uint64_t)kb << 32) | sl;
            sidx[c] = j0 + (uint32_t)bl;
          }
        mn = wave_min();
        bits &= ~((2ull << bl) - 1ull);
        bits &= __ballot(in && kj > (uint32_t)(mn >> 32));
      }
    }
    // Ranked as the insertion sort orders them: value descending, slot
    // ascending among equal values.
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t sl = lane + 64u * c;
      if (sl < K) {
        ck[sl] = (sk[c] & 0xFFFFFFFF00000000ull) | (0xFFFFFFFFu - sl);
        slot_idx[sl] = sidx[c];
      }
    }
  }
  __syncthreads();
  key = rank_keys();
  if (tid == pick) *outp = slot_idx[0xFFFFFFFFu - (uint32_t)key];
}

// y[m][n] = sum over the slices s of part[s][m][n] in slice order, plus
// res[m][n]: the split-K sum of launch_q4k_gemm.
__global__ __launch_bounds__(256) void splitk_sum_kernel(const float* __restrict__ part,
                                                         uint32_t nsl, uint32_t M, uint32_t N,
                                                         const float* __restrict__ res,
                                                         uint64_t ldr, float* __restrict__ y,
                                                         uint64_t ldy) {
#pragma clang fp contract(off)
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (uint64_t)M * N) return;
  const uint32_t m = (uint32_t)(i / N), n = (uint32_t)(i % N);
  float v = part[i];
  for (uint32_t s = 1; s < nsl; ++s) v += part[(uint64_t)s * M * N + i];
  if (res) v += res[(size_t)m * ldr + n];
  y[(size_t)m * ldy + n] = v;
}

}  // namespace

int launch_q4k_gemm(const Q4kGemmParams& p, hipStream_t stream) {
  // Every check runs before anything is allocated or launched.
  if (p.K % kQ4kBlockWeights != 0 || p.K == 0 || p.K > 64 * kQ4kBlockWeights)
    return fail(STS_ERR_INVALID, "GEMM K = %u must be a multiple of 256 in 256..16384", p.K);
  if (p.M == 0 || p.N == 0 || p.Z == 0 || p.Z > (uint32_t)kGemmMaxZ)
    return fail(STS_ERR_INVALID, "GEMM shape M=%u N=%u Z=%u", p.M, p.N, p.Z);
  if ((p.M + 15) / 16 > 65535u) return fail(STS_ERR_INVALID, "M = %u too large", p.M);
  if (p.swiglu_f && (p.swiglu_f * 2 != p.N))
    return fail(STS_ERR_INVALID, "SwiGLU GEMM needs N = 2F (N=%u F=%u)", p.N, p.swiglu_f);
  if (p.ldx % 4 != 0 || p.x_zstride % 4 != 0 || (reinterpret_cast<uintptr_t>(p.x) & 15))
    return fail(STS_ERR_INVALID, "GEMM x rows must be 16-byte aligned");
  // A 16-row tile of x is addressed through one buffer resource (31-bit range).
  if ((uint64_t)p.ldx * 15 * sizeof(float) + (uint64_t)p.K * sizeof(float) > 0x7FFFFFF0ull)
    return fail(STS_ERR_INVALID, "GEMM x row stride %llu too large",
                (unsigned long long)p.ldx);
  for (uint32_t z = 0; z < p.Z; ++z)
    if (!p.w[z] || (reinterpret_cast<uintptr_t>(p.w[z]) & 15))
      return fail(STS_ERR_INVALID, "GEMM weights %u null or not 16-byte aligned", z);
  if (p.K > 16 * kQ4kBlockWeights) {
    // Split K: slices of up to 16 super-blocks into a workspace, then the sum.
    if (p.Z != 1 || p.swiglu_f || p.norm_alpha)
      return fail(STS_ERR_INVALID, "GEMM with K = %u > 4096 takes no SwiGLU, RMSNorm or Z > 1",
                  p.K);
    const uint32_t KB = p.K / kQ4kBlockWeights;
    const uint32_t nsl = (KB + 15) / 16;
    const size_t mn = (size_t)p.M * p.N;
    const uint64_t blocks = (mn + 255) / 256;
    if (blocks > 0x7FFFFFFFull) return fail(STS_ERR_INVALID, "GEMM M x N = %zu too large", mn);
    Workspace* ws = nullptr;
    if (int rc = get_workspace(stream, nsl * mn, 0, &ws)) return rc;
    for (uint32_t sl = 0; sl < nsl; ++sl) {
      const uint32_t kb0 = sl * 16, kbs = std::min(16u, KB - kb0);
      Q4kGemmParams q = p;
      q.w[0] = p.w[0] + (size_t)kb0 * kQ4kBlockBytes;
      q.x = p.x + (size_t)kb0 * kQ4kBlockWeights;
      q.K = kbs * kQ4kBlockWeights;
      q.w_row_blocks = KB;
      q.res = nullptr;
      q.y = ws->part + sl * mn;
      q.ldy = p.N;
      if (int rc = launch_q4k_gemm(q, stream)) return rc;
    }
    hipLaunchKernelGGL(splitk_sum_kernel, dim3((uint32_t)blocks), dim3(256), 0, stream,
                       ws->part, nsl, p.M, p.N, p.res, p.ldr, p.y, p.ldy);
    STS_HIP(hipGetLastError());
    return STS_OK;
  }
  const uint32_t KB = p.K / kQ4kBlockWeights;
  const uint32_t mtiles = (p.M + 15) / 16;
  const uint32_t nout = p.swiglu_f ? p.swiglu_f : p.N;
  const uint32_t ntiles = (nout + 15) / 16;
  // Up to 4 workgroups per CU in total; each walks ntiles / gx row tiles and
  // reads its 16 x rows once.
  const uint32_t cus = (uint32_t)device_cu_count();
  const uint32_t gx = std::max(1u, std::min(ntiles, 4 * cus / std::max(1u, mtiles * p.Z)));
  const dim3 grid(gx, mtiles, p.Z), block(64 * KB);
  if (KB <= 4) {
    if (p.swiglu_f)
      hipLaunchKernelGGL((q4k_gemm_kernel<true, 256>), grid, block, 0, stream, p);
    else
      hipLaunchKernelGGL((q4k_gemm_kernel<false, 256>), grid, block, 0, stream, p);
  } else {
    if (p.swiglu_f)
      hipLaunchKernelGGL((q4k_gemm_kernel<true, 1024>), grid, block, 0, stream, p);
    else
      hipLaunchKernelGGL((q4k_gemm_kernel<false, 1024>), grid, block, 0, stream, p);
  }
  STS_HIP(hipGetLastError());
  return STS_OK;
}

int launch_rmsnorm(const float* x, const float* alpha, float* out, uint32_t rows, uint32_t D,
                   float eps, hipStream_t stream) {
  if (rows == 0 || D == 0) return fail(STS_ERR_INVALID, "empty RMSNorm");
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, stream, x, alpha, out, D, eps);
  STS_HIP(hipGetLastError());
  return STS_OK;
}

int launch_embed_add(const uint8_t* table, uint32_t vocab, const uint32_t* tokens,
                     uint64_t tok_stride, const float* proj, float* h, uint32_t B, uint32_t D,
                     hipStream_t stream) {
  if (D % 32 != 0 || B == 0 || B > 65535u)
    return fail(STS_ERR_INVALID, "embedding: dim %u must be a multiple of 32, batch %u", D, B);
  if (reinterpret_cast<uintptr_t>(table) & 1)
    return fail(STS_ERR_INVALID, "embedding table must be 2-byte aligned (its f16 scales)");
  hipLaunchKernelGGL(embed_add_kernel, dim3((D + 255) / 256, B), dim3(256), 0, stream, table,
                     vocab, tokens, tok_stride, proj, h, D);
  STS_HIP(hipGetLastError());
  return STS_OK;
}

int launch_sample_topk(const SampleParams& p, hipStream_t stream) {
  if (p.V == 0 || p.V > kMaxVocab)
    return fail(STS_ERR_INVALID, "sampling vocab %u must be in 1..%u", p.V, kMaxVocab);
  if (p.top_k > kMaxTopK)
    return fail(STS_ERR_INVALID, "top_k %u exceeds %u", p.top_k, kMaxTopK);
  if (p.B == 0) return STS_OK;
  if (p.V <= 2048)
    hipLaunchKernelGGL(sample_topk_kernel<8>, dim3(p.B), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(sample_topk_kernel<16>, dim3(p.B), dim3(256), 0, stream, p);
  STS_HIP(hipGetLastError());
  return STS_OK;
}

}  // namespace sts
