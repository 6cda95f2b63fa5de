// prefill.hip -- chunked causal prefill attention on MFMA for gfx950.
//
// Semantics of the reference's prefill branch (crates/sts-wasm/src/model.rs:760-797):
// softmax((Q K^T) * scale + mask) V with key j masked when j > offset + i
// (apply_causal_mask, model.rs:539-563), here over a ring window that may wrap.
//
// One workgroup = one head x 64 queries; keys stream through LDS in blocks of
// 64.  Eight waves: wave w owns queries 16*(w%4)..+15 and key slice w/4 (32
// keys) of every block, with its own online softmax; the two slices of a
// query group merge through LDS at the end.  Each wave computes S^T = K Q^T,
// so that the accumulator layout of S^T (lane l: keys 4*(l/16)+j of each
// 16-key tile, query l%16) is, after the online softmax, directly the B
// operand P^T of O^T = V^T P^T.  The contraction order over keys is permuted
// identically in V^T and P^T, so P never goes through LDS.  Each query's max
// and sum are reduced over the 4 lanes {l%16 + 16g} that hold its keys.
//
//   BF16 = true : f32 K/V/Q rounded to bf16 while staging, v_mfma_f32_16x16x32_bf16,
//                 f32 softmax and accumulation.
//   BF16 = false: f32 throughout, v_mfma_f32_16x16x4f32.
//
// The f32 variant also splits each tile's key range over up to four
// workgroups (blockIdx.z); each publishes (O, max, sum) with device-coherent
// stores and the last to arrive folds them in split order.
//
// Blocks are indexed (head, q-tile, split) with head fastest, so all
// workgroups of a head land on the same XCD (workgroup id % 8) and share its
// L2 copy of the head's K/V; the heaviest (last) q-tiles are dispatched first.
#include <algorithm>
#include <cfloat>
#include <type_traits>

#include "coherent.hpp"
#include "common.hpp"
#include "lane.hpp"
#include "prefill.hpp"

namespace sts {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

constexpr int kBQ = 64;  // queries per workgroup
constexpr int kBK = 64;  // keys per LDS block

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ float4 scale4(float4 x, float c) {
  return make_float4(x.x * c, x.y * c, x.z * c, x.w * c);
}

template <int D, bool BF16>
struct PrefillSmem {
  using T = typename std::conditional<BF16, __bf16, float>::type;
  static constexpr int KP = BF16 ? D + 8 : D + 4;  // K row pitch: 16 rows hit distinct banks
  static constexpr int VP = 80;                    // V^T row pitch (keys), see vt_col
  alignas(16) T ks[kBK * KP];
  alignas(16) T vt[D * VP];
};

constexpr int kMaxPrefillSplits = 4;
constexpr int kKsplit = 2;  // waves per query group (key slices of a block)

// V^T is stored d-major with the 4-key quads of each row permuted by
// ((d >> 2) ^ (d >> 4)) & 15: with a 80-element pitch the staging writes
// (32 lanes on 32 different rows) and the MFMA operand reads (16 rows x 4
// quads) both hit 64 distinct banks.
__device__ __forceinline__ int vt_col(int d, int quad) {
  return 4 * (quad ^ (((d >> 2) ^ (d >> 4)) & 15));
}

// KSPLIT (= 2) waves share each group of 16 queries: wave w handles queries
// 16 * (w % 4) .. +15 of the tile and the key slice w / 4 (32 keys) of every
// 64-key block, with its own online softmax; the slices merge once at the
// end.  More waves per SIMD hide the latency of each wave's serial
// softmax/MFMA chain.
template <int D, bool BF16, int KSPLIT>
__global__ __launch_bounds__(256 * KSPLIT) void prefill_kernel(const PrefillParams p) {
  using Smem = PrefillSmem<D, BF16>;
  constexpr int NT = 256 * KSPLIT;
  constexpr int KP = Smem::KP;
  constexpr int VP = Smem::VP;
  constexpr int DT = D / 16;           // O^T tiles of 16 dims
  constexpr int C4 = D / 4;            // float4 columns of a row
  constexpr int KW = kBK / KSPLIT;     // keys per wave per block
  constexpr int TW = KW / 16;          // S^T tiles per wave per block
  constexpr int KPER = kBK * C4 / NT;  // K float4 per thread per block
  constexpr int VSQ = (kBK / 4) * C4;  // V 4-key x 4-dim squares per block
  constexpr int VPER = VSQ >= NT ? VSQ / NT : 1;
  static_assert(KPER >= 1 && TW == 2, "tile shape: 32-key slices");
  // bf16 tiles are double-buffered (block i+1 is staged while block i is
  // computed, one barrier per block); f32 tiles are twice as large and use one
  // buffer with a barrier on each side of the staging.
  constexpr int NBUF = BF16 ? 2 : 1;
  __shared__ Smem sm_buf[NBUF];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int qg = wave & 3;       // query group
  const int kslice = wave >> 2;  // key slice
  const int g = lane >> 4;
  const int l16 = lane & 15;
  const uint32_t h = blockIdx.x;
  const uint32_t nqt = (p.S + kBQ - 1) / kBQ;
  const uint32_t qt = nqt - 1 - blockIdx.y;
  const uint32_t split = blockIdx.z;
  const uint32_t base_w = p.len - p.S;
  const uint32_t qi = qt * kBQ + qg * 16 + l16;
  const bool q_ok = qi < p.S;
  const uint32_t w_q = base_w + qi;  // window row of this lane's query
  // Window rows of the first and last query of this wave: keys up to w_first
  // need no causal mask, keys past w_wave are skipped.
  const uint32_t w_first = base_w + qt * kBQ + qg * 16;
  const uint32_t w_wave = base_w + min(p.S - 1, qt * kBQ + qg * 16 + 15);

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
        x0 = scale4(ld4(qrow + a * 32 + g * 8), p.scale_log2);
        x1 = scale4(ld4(qrow + a * 32 + g * 8 + 4), p.scale_log2);
      }
      bf16x8 b;
      b[0] = (__bf16)x0.x; b[1] = (__bf16)x0.y; b[2] = (__bf16)x0.z; b[3] = (__bf16)x0.w;
      b[4] = (__bf16)x1.x; b[5] = (__bf16)x1.y; b[6] = (__bf16)x1.z; b[7] = (__bf16)x1.w;
      qop[a] = b;
    } else {
      // dims 16a + 4g .. +3 (instruction (a, j) contracts dim 16a + 4g + j)
      qop[a] = q_ok ? scale4(ld4(qrow + a * 16 + g * 4), p.scale_log2)
                    : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }

  float m = -FLT_MAX;
  float lsum = 0.f;
  floatx4 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) o[t] = floatx4{0.f, 0.f, 0.f, 0.f};

  const uint32_t q_last = min(p.S, (qt + 1) * kBQ) - 1;
  const uint32_t kend = min(p.len, base_w + q_last + 1);  // keys this query tile needs
  // This workgroup's share of the tile's key blocks (sizes differ by at most one).
  const uint32_t nb = (kend + kBK - 1) / kBK;
  const uint32_t ns = min(p.nsplit, nb);
  if (split >= ns) return;  // the tile has fewer blocks than splits
  const uint32_t kb_begin = split * nb / ns * kBK;
  const uint32_t kb_end = min(kend, (split + 1) * nb / ns * kBK);
  const int d4 = tid % C4;

  // K/V rows come in through buffer loads on per-head resources (byte offset
  // slot * D * 4 + column).  A block whose 64 rows are all inside the window
  // and do not wrap needs no per-row arithmetic: per-thread constant offsets
  // plus one scalar block offset.  Other blocks compute each row's slot; rows
  // past the tile's last key get an offset past the resource, which loads
  // zeros (finite, and masked out of the softmax).
  constexpr uint32_t ROWB = D * sizeof(float);
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(p.k) + (size_t)h * p.M * D, 0, (int)(p.M * ROWB), kBufferWord3);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(p.v) + (size_t)h * p.M * D, 0, (int)(p.M * ROWB), kBufferWord3);
  const bool v_thread = VSQ >= NT || tid < VSQ;
  auto k_row = [&](int i) { return (uint32_t)(tid / C4 + i * (NT / C4)); };
  auto v_row = [&](int i, int r4) { return (uint32_t)((tid / C4 + i * (NT / C4)) * 4 + r4); };

  struct Buf {
    floatx4 k[KPER];
    floatx4 v[VPER][4];
  };
  Buf buf;
  // Loads block kb into b; valid == false loads zeros (keeps the number of
  // loads in flight the same on every path).  Only the offsets depend on the
  // path; the loads themselves are issued unconditionally, so the compiler's
  // wait counts see one fixed order of loads.
  constexpr int NL = KPER + 4 * VPER;
  auto fetch = [&](Buf& b, uint32_t kb, bool valid) {
    uint32_t slot0 = p.start + kb;
    slot0 = slot0 >= p.M ? slot0 - p.M : slot0;
    uint32_t vo[NL];
    uint32_t so = 0;
    if (valid && kb + kBK <= kend && slot0 + kBK <= p.M) {
      so = slot0 * ROWB;
#pragma unroll
      for (int i = 0; i < KPER; ++i) vo[i] = k_row(i) * ROWB + d4 * 16;
#pragma unroll
      for (int i = 0; i < VPER; ++i)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) vo[KPER + 4 * i + r4] = v_row(i, r4) * ROWB + d4 * 16;
    } else {
      const uint32_t lim = valid ? kend : 0u;
      auto off = [&](uint32_t r) {
        const uint32_t row = kb + r;
        uint32_t slot = slot0 + r;
        slot = min(slot, slot - p.M);  // wrap (slot < 2M)
        return row < lim ? slot * ROWB + d4 * 16 : 0xFFFFFFF0u;
      };
#pragma unroll
      for (int i = 0; i < KPER; ++i) vo[i] = off(k_row(i));
#pragma unroll
      for (int i = 0; i < VPER; ++i)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) vo[KPER + 4 * i + r4] = off(v_row(i, r4));
    }
#pragma unroll
    for (int i = 0; i < KPER; ++i)
      b.k[i] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(krs, vo[i], so, 0));
    if (v_thread) {
#pragma unroll
      for (int i = 0; i < VPER; ++i)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
          b.v[i][r4] = __builtin_bit_cast(
              floatx4, __builtin_amdgcn_raw_buffer_load_b128(vrs, vo[KPER + 4 * i + r4], so, 0));
    }
  };
  auto stage = [&](const Buf& b, int nb_) {
    Smem& sm = sm_buf[nb_];
#pragma unroll
    for (int i = 0; i < KPER; ++i) {
      const int key = tid / C4 + i * (NT / C4);
      const floatx4 x = b.k[i];
      if constexpr (BF16) {
        bf16x4 y;
        y[0] = (__bf16)x.x; y[1] = (__bf16)x.y; y[2] = (__bf16)x.z; y[3] = (__bf16)x.w;
        *reinterpret_cast<bf16x4*>(&sm.ks[key * KP + d4 * 4]) = y;
      } else {
        *reinterpret_cast<floatx4*>(&sm.ks[key * KP + d4 * 4]) = x;
      }
    }
    if (v_thread) {
#pragma unroll
      for (int i = 0; i < VPER; ++i) {
        const int kq = tid / C4 + i * (NT / C4);
        const floatx4* x = b.v[i];
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
            *reinterpret_cast<float4*>(&sm.vt[d * VP + vt_col(d, kq)]) =
                make_float4(e0, e1, e2, e3);
          }
        }
      }
    }
  };

  const uint32_t nblk = (kb_end - kb_begin + kBK - 1) / kBK;
  // One block out of LDS: S^T, online softmax, O^T update.
  auto compute = [&](uint32_t kb, int nb_, bool active) {
    const Smem& sm = sm_buf[nb_];
    const uint32_t k0 = kb + kslice * KW;  // first key of this wave's slice
    if (!active || k0 > w_wave) return;    // every key of the slice is masked for this wave
    const bool unmasked = k0 + KW <= kend && k0 + KW - 1 <= w_first;

    // S^T tiles t: keys k0 + 16t + 4g + j, query qi.  The bf16 operands of
    // the whole block (K for S^T, V^T for O^T) are read from LDS first, so
    // the reads overlap each other, the MFMAs and the softmax.
    const int q0 = kslice * (KW / 4);  // first 4-key quad of the slice
    floatx4 s[TW];
    [[maybe_unused]] bf16x8 vop[DT];
    if constexpr (BF16) {
      bf16x8 kop[TW][QN];
#pragma unroll
      for (int t = 0; t < TW; ++t)
#pragma unroll
        for (int a = 0; a < QN; ++a)
          kop[t][a] = *reinterpret_cast<const bf16x8*>(
              &sm.ks[(kslice * KW + 16 * t + l16) * KP + a * 32 + g * 8]);
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const int d = 16 * t + l16;
        const bf16x4 lo = *reinterpret_cast<const bf16x4*>(&sm.vt[d * VP + vt_col(d, q0 + g)]);
        const bf16x4 hi = *reinterpret_cast<const bf16x4*>(&sm.vt[d * VP + vt_col(d, q0 + 4 + g)]);
        vop[t] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
#pragma unroll
      for (int t = 0; t < TW; ++t) {
        s[t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int a = 0; a < QN; ++a)
          s[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[t][a], qop[a], s[t], 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int t = 0; t < TW; ++t) {
        const int krow = kslice * KW + 16 * t + l16;
        float4 kf[QN];
#pragma unroll
        for (int a = 0; a < QN; ++a)
          kf[a] = *reinterpret_cast<const float4*>(&sm.ks[krow * KP + a * 16 + g * 4]);
        s[t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int a = 0; a < QN; ++a) {
          s[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[a].x, qop[a].x, s[t], 0, 0, 0);
          s[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[a].y, qop[a].y, s[t], 0, 0, 0);
          s[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[a].z, qop[a].z, s[t], 0, 0, 0);
          s[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[a].w, qop[a].w, s[t], 0, 0, 0);
        }
      }
    }

    // Causal mask and online softmax for query qi over this slice (q carries
    // the scale, so scores are already in log2 units).
    float mx = -INFINITY;
    if (unmasked) {
#pragma unroll
      for (int t = 0; t < TW; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) mx = fmaxf(mx, s[t][j]);
    } else {
#pragma unroll
      for (int t = 0; t < TW; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t key = k0 + 16 * t + 4 * g + j;
          const float x = (key <= w_q && key < kend) ? s[t][j] : -INFINITY;
          s[t][j] = x;
          mx = fmaxf(mx, x);
        }
    }
    mx = max_xor32(max_xor16(mx));
    const float mn = fmaxf(m, mx);
    const float alpha = fast_exp2(m - mn);
    m = mn;
    float ps = 0.f;
#pragma unroll
    for (int t = 0; t < TW; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float e = fast_exp2(s[t][j] - mn);
        s[t][j] = e;
        ps += e;
      }
    ps = sum_xor32(sum_xor16(ps));
    lsum = lsum * alpha + ps;
    // Rescale only when some lane's running max moved (alpha == 1 otherwise).
    if (__any(alpha != 1.f)) {
#pragma unroll
      for (int t = 0; t < DT; ++t) o[t] *= alpha;
    }

    // O^T += V^T P^T over this wave's 32 keys.
    if constexpr (BF16) {
      bf16x8 pb;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pb[j] = (__bf16)s[0][j];
        pb[4 + j] = (__bf16)s[1][j];
      }
#pragma unroll
      for (int t = 0; t < DT; ++t)
        o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop[t], pb, o[t], 0, 0, 0);
    } else {
#pragma unroll
      for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int tk = 0; tk < TW; ++tk) {
          const int d = 16 * t + l16;
          const float4 vf =
              *reinterpret_cast<const float4*>(&sm.vt[d * VP + vt_col(d, q0 + 4 * tk + g)]);
          o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf.x, s[tk][0], o[t], 0, 0, 0);
          o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf.y, s[tk][1], o[t], 0, 0, 0);
          o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf.z, s[tk][2], o[t], 0, 0, 0);
          o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf.w, s[tk][3], o[t], 0, 0, 0);
        }
    }
  };

  // One block in flight in registers while the previous one computes.
  auto blk = [&](uint32_t i) { return kb_begin + min(i, nblk - 1) * kBK; };
  if constexpr (NBUF == 2) {
    // While block i is computed from one LDS buffer, block i+1 (in registers
    // since the previous trip) is staged into the other and block i+2 is
    // fetched.  The other buffer was last read by block i-1, which every wave
    // finished before the previous barrier.
    fetch(buf, blk(0), true);
    stage(buf, 0);
    fetch(buf, blk(1), nblk > 1);
    __syncthreads();
    for (uint32_t i = 0; i < nblk; ++i) {
      compute(blk(i), i & 1, true);
      if (i + 1 < nblk) stage(buf, (i + 1) & 1);
      fetch(buf, blk(i + 2), i + 2 < nblk);
      __syncthreads();
    }
  } else {
    fetch(buf, kb_begin, true);
    for (uint32_t i = 0; i < nblk; ++i) {
      const uint32_t kb = kb_begin + i * kBK;
      __syncthreads();  // the previous block's LDS reads are done
      stage(buf, 0);
      __syncthreads();
      fetch(buf, blk(i + 1), i + 1 < nblk);
      compute(kb, 0, true);
    }
  }

  // Merge the key slices of each query group: slice r > 0 parks (m, l, O^T)
  // in LDS (reusing the K/V tiles), slice 0 folds it in; one round per slice.
  if constexpr (KSPLIT > 1) {
    float* red = reinterpret_cast<float*>(&sm_buf[0]);  // [4 groups][64 lanes][DT*4 + 2]
    constexpr int RS = DT * 4 + 2;
    static_assert(4 * 64 * RS * sizeof(float) <= sizeof(Smem), "merge scratch");
#pragma unroll
    for (int r = 1; r < KSPLIT; ++r) {
      __syncthreads();
      if (kslice == r) {
        float* dst = red + (qg * 64 + lane) * RS;
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
          for (int j = 0; j < 4; ++j) dst[4 * t + j] = o[t][j];
        dst[DT * 4] = m;
        dst[DT * 4 + 1] = lsum;
      }
      __syncthreads();
      if (kslice == 0) {
        const float* src = red + (qg * 64 + lane) * RS;
        const float m2 = src[DT * 4], l2 = src[DT * 4 + 1];
        const float mm = fmaxf(m, m2);
        const float f1 = fast_exp2(m - mm), f2 = fast_exp2(m2 - mm);
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
          for (int j = 0; j < 4; ++j) o[t][j] = o[t][j] * f1 + src[4 * t + j] * f2;
        lsum = lsum * f1 + l2 * f2;
        m = mm;
      }
    }
  }
  // From here on, the waves of key slice 0 hold each query group's result.
  const bool owner = kslice == 0;
  float* orow = p.out + ((size_t)qi * p.H + h) * D;

  if (ns == 1) {
    if (owner && q_ok) {
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
    return;
  }

  // Publish this split's partial with device-coherent stores (the splits of a
  // tile may run on different XCDs), wait for their acknowledgement, then take
  // an arrival ticket.  Record layout: O as [t][group][lane] float4, then the
  // running max and sum as [group][lane].
  constexpr int REC = 256 * (DT * 4 + 2);
  const size_t tile = (size_t)h * nqt + qt;
  float* rec_tile = p.part + tile * p.nsplit * REC;
  const int slot = qg * 64 + lane;
  const __amdgpu_buffer_rsrc_t rsrc = coherent_rsrc(rec_tile, ns * REC * sizeof(float));
  if (owner) {
    const uint32_t rec = split * REC * sizeof(float);
#pragma unroll
    for (int t = 0; t < DT; ++t) st_coherent4(rsrc, rec + (t * 256 + slot) * 16, o[t]);
    st_coherent(rsrc, rec + (DT * 4 * 256 + slot) * 4, m);
    st_coherent(rsrc, rec + (DT * 4 * 256 + 256 + slot) * 4, lsum);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __shared__ uint32_t s_ticket;
  uint32_t* ctr = p.counters + tile;
  __syncthreads();
  if (tid == 0) s_ticket = atomicAdd(ctr, 1u);
  __syncthreads();
  if (s_ticket != ns - 1) return;
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");

  // Last to arrive: fold the splits in split order (whichever arrived last),
  // so the result does not depend on arrival order.
  if (owner) {
    float ms[kMaxPrefillSplits], ls[kMaxPrefillSplits];
#pragma unroll
    for (int s2 = 0; s2 < kMaxPrefillSplits; ++s2) {
      ms[s2] = -FLT_MAX;
      ls[s2] = 0.f;
      if (s2 == (int)split) {
        ms[s2] = m;
        ls[s2] = lsum;
      } else if (s2 < (int)ns) {
        const uint32_t rec = s2 * REC * sizeof(float);
        ms[s2] = ld_coherent(rsrc, rec + (DT * 4 * 256 + slot) * 4);
        ls[s2] = ld_coherent(rsrc, rec + (DT * 4 * 256 + 256 + slot) * 4);
      }
    }
    float mm = ms[0];
#pragma unroll
    for (int s2 = 1; s2 < kMaxPrefillSplits; ++s2) mm = fmaxf(mm, ms[s2]);
    float l = 0.f;
    floatx4 acc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s2 = 0; s2 < kMaxPrefillSplits; ++s2) {
      if (s2 < (int)ns) {
        const float f = fast_exp2(ms[s2] - mm);
        l += f * ls[s2];
        floatx4 os[DT];
        if (s2 == (int)split) {
#pragma unroll
          for (int t = 0; t < DT; ++t) os[t] = o[t];
        } else {
          const uint32_t rec = s2 * REC * sizeof(float);
#pragma unroll
          for (int t = 0; t < DT; ++t)
            os[t] = ld_coherent4(rsrc, rec + (t * 256 + slot) * 16);
        }
#pragma unroll
        for (int t = 0; t < DT; ++t) acc[t] += f * os[t];
      }
    }
    if (q_ok) {
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        float4 r;
        r.x = acc[t][0] / l;
        r.y = acc[t][1] / l;
        r.z = acc[t][2] / l;
        r.w = acc[t][3] / l;
        *reinterpret_cast<float4*>(orow + 16 * t + 4 * g) = r;
      }
    }
  }
  if (tid == 0) atomicExch(ctr, 0u);
}

template <int D, bool BF16>
int launch_t(const PrefillParams& p, hipStream_t stream) {
  const uint32_t nqt = (p.S + kBQ - 1) / kBQ;
  if (nqt > 65535u) return fail(STS_ERR_INVALID, "seq %u too long for one launch", p.S);
  if ((uint64_t)p.M * D * sizeof(float) > 0x7FFFFFF0ull)
    return fail(STS_ERR_INVALID, "max_len %u too large for one head's buffer resource", p.M);
  // f32 tiles carry four times the MFMA work of bf16 ones: split their key
  // ranges until there are about two workgroups per CU.  bf16 tiles are
  // bound by the CU's load rate and gain nothing from splitting.
  const uint32_t tiles = p.H * nqt;
  const uint32_t cus = (uint32_t)device_cu_count();
  uint32_t nsplit = BF16 ? 1u : (2 * cus + tiles - 1) / tiles;
  nsplit = std::max(1u, std::min<uint32_t>(nsplit, kMaxPrefillSplits));
  PrefillParams q = p;
  q.nsplit = nsplit;
  if (nsplit > 1) {
    Workspace* ws = nullptr;
    const int rc = get_workspace(stream, (size_t)tiles * nsplit * 256 * (D + 2), tiles, &ws);
    if (rc != STS_OK) return rc;
    q.part = ws->part;
    q.counters = ws->counters;
  }
  hipLaunchKernelGGL((prefill_kernel<D, BF16, kKsplit>), dim3(p.H, nqt, nsplit),
                     dim3(256 * kKsplit), 0, stream, q);
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
