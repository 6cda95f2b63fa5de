// prefill.hip -- chunked causal prefill attention on MFMA for gfx950.
//
// Semantics of the reference's prefill branch (crates/sts-wasm/src/model.rs:760-797):
// softmax((Q K^T) * scale + mask) V with key j masked when j > offset + i
// (apply_causal_mask, model.rs:539-563), here over a ring window that may wrap.
//
// One workgroup = one head x 64 queries (16 per wave); keys stream through LDS
// in blocks of 64.  Each wave computes S^T = K Q^T for its 16 queries, so that
// the accumulator layout of S^T (lane l: keys 4*(l/16)+j of each 16-key tile,
// query l%16) is, after the online softmax, directly the B operand P^T of
// O^T = V^T P^T.  The contraction order over keys is permuted identically in
// V^T and P^T, so P never goes through LDS.  Each query's max and sum are
// reduced over the 4 lanes {l%16 + 16g} that hold its keys.
//
//   BF16 = true : f32 K/V/Q rounded to bf16 while staging, v_mfma_f32_16x16x32_bf16,
//                 f32 softmax and accumulation.
//   BF16 = false: f32 throughout, v_mfma_f32_16x16x4f32.
//
// Blocks are indexed (head, q-tile) with head fastest, so all q-tiles of a
// head land on the same XCD (workgroup id % 8) and share its L2 copy of the
// head's K/V; the heaviest (last) q-tiles are dispatched first.
#include <cfloat>
#include <type_traits>

#include "common.hpp"
#include "lane.hpp"
#include "prefill.hpp"

namespace sts {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kBQ = 64;  // queries per workgroup
constexpr int kBK = 64;  // keys per LDS block

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }

template <int D, bool BF16>
struct PrefillSmem {
  using T = typename std::conditional<BF16, __bf16, float>::type;
  static constexpr int KP = BF16 ? D + 8 : D + 4;  // K row pitch: 16 rows hit distinct banks
  static constexpr int VP = 80;                    // V^T row pitch (keys), see vt_col
  alignas(16) T ks[kBK * KP];
  alignas(16) T vt[D * VP];
};

// V^T is stored d-major with the 4-key quads of each row permuted by
// ((d >> 2) ^ (d >> 4)) & 15: with a 80-element pitch the staging writes
// (32 lanes on 32 different rows) and the MFMA operand reads (16 rows x 4
// quads) both hit 64 distinct banks.
__device__ __forceinline__ int vt_col(int d, int quad) {
  return 4 * (quad ^ (((d >> 2) ^ (d >> 4)) & 15));
}

template <int D, bool BF16>
__global__ __launch_bounds__(256) void prefill_kernel(const PrefillParams p) {
  using Smem = PrefillSmem<D, BF16>;
  constexpr int KP = Smem::KP;
  constexpr int VP = Smem::VP;
  constexpr int DT = D / 16;         // O^T tiles of 16 dims
  constexpr int C4 = D / 4;          // float4 columns of a row
  constexpr int KPER = kBK * C4 / 256;        // K float4 per thread per block
  constexpr int VQ = (kBK / 4) * C4 / 256;    // V 4-key x 4-dim squares per thread
  __shared__ Smem sm;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 4;
  const int l16 = lane & 15;
  const uint32_t h = blockIdx.x;
  const uint32_t nqt = (p.S + kBQ - 1) / kBQ;
  const uint32_t qt = nqt - 1 - blockIdx.y;
  const uint32_t base_w = p.len - p.S;
  const uint32_t qi = qt * kBQ + wave * 16 + l16;
  const bool q_ok = qi < p.S;
  const uint32_t w_q = base_w + qi;  // window row of this lane's query
  // Last window row any query of this wave can see (blocks beyond it are skipped).
  const uint32_t w_wave = base_w + min(p.S - 1, qt * kBQ + wave * 16 + 15);

  // B operand of S^T = K Q^T: this lane's query row, permuted per MFMA.
  constexpr int QN = BF16 ? D / 32 : D / 16;
  typename std::conditional<BF16, bf16x8, float4>::type qop[QN];
  const float* qrow = p.q + ((size_t)(q_ok ? qi : 0) * p.H + h) * D;
#pragma unroll
  for (int a = 0; a < QN; ++a) {
    if constexpr (BF16) {
      // dims 32a + 8g .. +7
      float4 x0 = make_float4(0.f, 0.f, 0.f, 0.f), x1 = x0;
      if (q_ok) {
        x0 = ld4(qrow + a * 32 + g * 8);
        x1 = ld4(qrow + a * 32 + g * 8 + 4);
      }
      bf16x8 b;
      b[0] = (__bf16)x0.x; b[1] = (__bf16)x0.y; b[2] = (__bf16)x0.z; b[3] = (__bf16)x0.w;
      b[4] = (__bf16)x1.x; b[5] = (__bf16)x1.y; b[6] = (__bf16)x1.z; b[7] = (__bf16)x1.w;
      qop[a] = b;
    } else {
      // dims 16a + 4g .. +3 (instruction (a, j) contracts dim 16a + 4g + j)
      qop[a] = q_ok ? ld4(qrow + a * 16 + g * 4) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }

  float m = -FLT_MAX;
  float lsum = 0.f;
  floatx4 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) o[t] = floatx4{0.f, 0.f, 0.f, 0.f};

  const uint32_t q_last = min(p.S, (qt + 1) * kBQ) - 1;
  const uint32_t kend = min(p.len, base_w + q_last + 1);  // keys this workgroup needs
  const float* kh = p.k + (size_t)h * p.M * D;
  const float* vh = p.v + (size_t)h * p.M * D;
  const int d4 = tid % C4;

  // Next block's K and V rows, in flight while the current block computes.
  // Rows past kend re-read row kend-1 (finite, and masked out of the softmax).
  float4 kreg[KPER];
  float4 vreg[VQ][4];
  auto row_ptr = [&](const float* base, uint32_t r) {
    r = r < kend ? r : kend - 1;
    uint32_t slot = p.start + r;
    slot = slot >= p.M ? slot - p.M : slot;
    return base + (size_t)slot * D + d4 * 4;
  };
  auto prefetch = [&](uint32_t kb) {
#pragma unroll
    for (int i = 0; i < KPER; ++i) kreg[i] = ld4(row_ptr(kh, kb + tid / C4 + i * (256 / C4)));
#pragma unroll
    for (int i = 0; i < VQ; ++i) {
      const int kq = tid / C4 + i * (256 / C4);
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) vreg[i][r4] = ld4(row_ptr(vh, kb + kq * 4 + r4));
    }
  };
  auto stage = [&]() {
#pragma unroll
    for (int i = 0; i < KPER; ++i) {
      const int key = tid / C4 + i * (256 / C4);
      const float4 x = kreg[i];
      if constexpr (BF16) {
        bf16x4 y;
        y[0] = (__bf16)x.x; y[1] = (__bf16)x.y; y[2] = (__bf16)x.z; y[3] = (__bf16)x.w;
        *reinterpret_cast<bf16x4*>(&sm.ks[key * KP + d4 * 4]) = y;
      } else {
        *reinterpret_cast<float4*>(&sm.ks[key * KP + d4 * 4]) = x;
      }
    }
#pragma unroll
    for (int i = 0; i < VQ; ++i) {
      const int kq = tid / C4 + i * (256 / C4);
      const float4* x = vreg[i];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d = d4 * 4 + c;
        const float e0 = c == 0 ? x[0].x : c == 1 ? x[0].y : c == 2 ? x[0].z : x[0].w;
        const float e1 = c == 0 ? x[1].x : c == 1 ? x[1].y : c == 2 ? x[1].z : x[1].w;
        const float e2 = c == 0 ? x[2].x : c == 1 ? x[2].y : c == 2 ? x[2].z : x[2].w;
        const float e3 = c == 0 ? x[3].x : c == 1 ? x[3].y : c == 2 ? x[3].z : x[3].w;
        if constexpr (BF16) {
          bf16x4 y;
          y[0] = (__bf16)e0; y[1] = (__bf16)e1; y[2] = (__bf16)e2; y[3] = (__bf16)e3;
          *reinterpret_cast<bf16x4*>(&sm.vt[d * VP + vt_col(d, kq)]) = y;
        } else {
          *reinterpret_cast<float4*>(&sm.vt[d * VP + vt_col(d, kq)]) = make_float4(e0, e1, e2, e3);
        }
      }
    }
  };

  prefetch(0);
  for (uint32_t kb = 0; kb < kend; kb += kBK) {
    __syncthreads();  // the previous block's LDS reads are done
    stage();
    __syncthreads();
    if (kb + kBK < kend) prefetch(kb + kBK);
    if (kb > w_wave) continue;  // every key of this block is masked for this wave

    // S^T tiles t: keys kb + 16t + 4g + j, query qi.
    floatx4 s[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      s[t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int a = 0; a < QN; ++a) {
        if constexpr (BF16) {
          const bf16x8 kop =
              *reinterpret_cast<const bf16x8*>(&sm.ks[(16 * t + l16) * KP + a * 32 + g * 8]);
          s[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop, qop[a], s[t], 0, 0, 0);
        } else {
          const float4 kf =
              *reinterpret_cast<const float4*>(&sm.ks[(16 * t + l16) * KP + a * 16 + g * 4]);
          s[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf.x, qop[a].x, s[t], 0, 0, 0);
          s[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf.y, qop[a].y, s[t], 0, 0, 0);
          s[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf.z, qop[a].z, s[t], 0, 0, 0);
          s[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf.w, qop[a].w, s[t], 0, 0, 0);
        }
      }
    }

    // Causal mask and online softmax for query qi over this block.
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t key = kb + 16 * t + 4 * g + j;
        float x = s[t][j] * p.scale_log2;
        x = (key <= w_q && key < kend) ? x : -INFINITY;
        s[t][j] = x;
        mx = fmaxf(mx, x);
      }
    mx = fmaxf(mx, swizzle_xor16(mx));
    mx = fmaxf(mx, xor32(mx));
    const float mn = fmaxf(m, mx);
    const float alpha = fast_exp2(m - mn);
    m = mn;
    float ps = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float e = fast_exp2(s[t][j] - mn);
        s[t][j] = e;
        ps += e;
      }
    ps += swizzle_xor16(ps);
    ps += xor32(ps);
    lsum = lsum * alpha + ps;
#pragma unroll
    for (int t = 0; t < DT; ++t) o[t] *= alpha;

    // O^T += V^T P^T
    if constexpr (BF16) {
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        bf16x8 pb;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          pb[j] = (__bf16)s[2 * kk][j];
          pb[4 + j] = (__bf16)s[2 * kk + 1][j];
        }
#pragma unroll
        for (int t = 0; t < DT; ++t) {
          const int d = 16 * t + l16;
          const bf16x4 lo = *reinterpret_cast<const bf16x4*>(&sm.vt[d * VP + vt_col(d, 8 * kk + g)]);
          const bf16x4 hi =
              *reinterpret_cast<const bf16x4*>(&sm.vt[d * VP + vt_col(d, 8 * kk + 4 + g)]);
          bf16x8 vop;
          vop[0] = lo[0]; vop[1] = lo[1]; vop[2] = lo[2]; vop[3] = lo[3];
          vop[4] = hi[0]; vop[5] = hi[1]; vop[6] = hi[2]; vop[7] = hi[3];
          o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, pb, o[t], 0, 0, 0);
        }
      }
    } else {
#pragma unroll
      for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int tk = 0; tk < 4; ++tk) {
          const int d = 16 * t + l16;
          const float4 vf = *reinterpret_cast<const float4*>(&sm.vt[d * VP + vt_col(d, 4 * tk + g)]);
          o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf.x, s[tk][0], o[t], 0, 0, 0);
          o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf.y, s[tk][1], o[t], 0, 0, 0);
          o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf.z, s[tk][2], o[t], 0, 0, 0);
          o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf.w, s[tk][3], o[t], 0, 0, 0);
        }
    }
  }

  if (q_ok) {
    float* orow = p.out + ((size_t)qi * p.H + h) * D;
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      float4 r;
      r.x = o[t][0] / lsum;
      r.y = o[t][1] / lsum;
      r.z = o[t][2] / lsum;
      r.w = o[t][3] / lsum;
      *reinterpret_cast<float4*>(orow + 16 * t + 4 * g) = r;
    }
  }
}

template <int D, bool BF16>
int launch_t(const PrefillParams& p, hipStream_t stream) {
  const uint32_t nqt = (p.S + kBQ - 1) / kBQ;
  if (nqt > 65535u) return fail(STS_ERR_INVALID, "seq %u too long for one launch", p.S);
  hipLaunchKernelGGL((prefill_kernel<D, BF16>), dim3(p.H, nqt), dim3(256), 0, stream, p);
  STS_HIP(hipGetLastError());
  return STS_OK;
}

}  // namespace

int launch_prefill(const PrefillParams& p, uint32_t head_dim, int precision, hipStream_t stream) {
  const bool bf16 = precision == STS_PREC_BF16_MFMA;
  if (head_dim == 128) return bf16 ? launch_t<128, true>(p, stream) : launch_t<128, false>(p, stream);
  if (head_dim == 64) return bf16 ? launch_t<64, true>(p, stream) : launch_t<64, false>(p, stream);
  return fail(STS_ERR_INVALID, "head_dim %u not supported (64 or 128)", head_dim);
}

}  // namespace sts
