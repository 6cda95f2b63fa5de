// prefill.hip -- chunked causal prefill attention on MFMA for gfx950.
//
// Semantics of the reference's prefill branch (crates/sts-wasm/src/model.rs:760-797):
// softmax((Q K^T) * scale + mask) V with key j masked when j > offset + i
// (apply_causal_mask, model.rs:539-563), here over a ring window that may wrap.
//
// Two kernels, one workgroup = one head x 64 queries, keys in blocks of 64:
//
//   prefill_kernel (f32, v_mfma_f32_16x16x4f32): eight waves; wave w owns
//   queries 16*(w%4)..+15 and key slice w/4 (32 keys) of every block, with
//   its own online softmax; the two slices of a query group merge through
//   LDS at the end.  Each wave computes S^T = K Q^T, so that the accumulator
//   layout of S^T (lane l: keys 4*(l/16)+j of each 16-key tile, query l%16)
//   is, after the online softmax, directly the B operand P^T of
//   O^T = V^T P^T; the contraction order over keys is permuted identically
//   in V^T and P^T, so P never goes through LDS.  Each tile's key range is
//   also split over up to four workgroups (blockIdx.z); each publishes
//   (O, max, sum) with device-coherent stores and the last to arrive folds
//   them in split order.
//
//   prefill_ws_kernel (bf16 MFMA, f32 softmax and accumulation): specialised
//   producer and consumer waves, described above the kernel.  Its SPLIT
//   instance is the split variant: operands split into bf16 hi and lo parts,
//   three bf16 products per f32 product (f32-grade for moderate score ranges).
//
// Blocks are indexed (head, q-tile[, split]) with head fastest, so all
// workgroups of a head land on the same XCD (workgroup id % 8) and share its
// L2 copy of the head's K/V; the heaviest (last) q-tiles are dispatched first.
// In prefill_ws_kernel (not its SPLIT instance) the tiles within two blocks
// of the longest visit their key blocks last to first, ending on the blocks
// every tile of the head shares (by then in L2); on the bf16-mirror path the
// shorter tiles also start staggered when all tiles are resident at once.
// Both kernels write the output rows with nontemporal stores, which keep the
// finished tiles' output from pushing those shared blocks out of L2.
#include <algorithm>
#include <cfloat>

#include "coherent.hpp"
#include "common.hpp"
#include "decode.hpp"
#include "errors.hpp"
#include "lane.hpp"
#include "prefill.hpp"
#include "rope.hpp"

namespace sts {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kBQ = 64;  // queries per workgroup
constexpr int kBK = 64;  // keys per LDS block

// Query row of q (scaled by zero when the lane has no query) with optional
// RoPE at table row rope_pos0 + i: four dims d0..d0+3.
template <int D>
__device__ __forceinline__ float4 load_query4(const PrefillParams& p, const float* qrow,
                                              uint32_t i, int d0, float qscale) {
  float4 x = *reinterpret_cast<const float4*>(qrow + d0);
  if (p.rope_cos) {
    float2 cs, sn;
    rope_coeffs<D>(p.rope_cos, p.rope_sin, p.rope_pos0 + i, d0, cs, sn);
    x = rope4(x, cs, sn);
  }
  return make_float4(x.x * qscale, x.y * qscale, x.z * qscale, x.w * qscale);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
// Output rows are written once and not read in the launch: nontemporal
// stores keep them from pushing out of L2 the K/V blocks that the longer
// tiles of a head read after the shorter tiles have finished (512 queries
// after 256 cached, f32 K/V: 19.4 -> 18.4 us per layer in the bf16 kernel,
// 56.6 -> 55.9 us in the f32 one).
__device__ __forceinline__ void st4_stream(float* p, float4 v) {
  __builtin_nontemporal_store(coh_f4{v.x, v.y, v.z, v.w}, reinterpret_cast<coh_f4*>(p));
}
__device__ __forceinline__ float4 scale4(float4 x, float c) {
  return make_float4(x.x * c, x.y * c, x.z * c, x.w * c);
}

template <int D>
struct PrefillSmem {
  static constexpr int KP = D + 4;  // K row pitch: 16 rows hit distinct banks
  static constexpr int VP = 80;     // V^T row pitch (keys), see vt_col
  alignas(16) float ks[kBK * KP];
  alignas(16) float vt[D * VP];
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
// softmax/MFMA chain.  f32 throughout.
template <int D, int KSPLIT>
__global__ __launch_bounds__(256 * KSPLIT) void prefill_kernel(const PrefillParams p) {
  using Smem = PrefillSmem<D>;
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
  // One LDS buffer, with a barrier on each side of the staging.
  __shared__ Smem sm_buf[1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int qg = wave & 3;       // query group
  const int kslice = wave >> 2;  // key slice
  const int g = lane >> 4;
  const int l16 = lane & 15;
  const uint32_t h = blockIdx.x;
  const uint32_t kvh = p.group_magic ? __umulhi(h, p.group_magic) : h;  // its K/V head
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
  constexpr int QN = D / 16;
  float4 qop[QN];
  // Every lane loads (a row past the tile's end reads row 0) and scales by
  // zero when it has no query: no branch, so all loads issue at once.
  const uint32_t qrow_i = q_ok ? qi : 0;
  const float* qrow = p.q + ((size_t)qrow_i * p.H + h) * D;
  const float qs = q_ok ? p.scale_log2 : 0.f;
#pragma unroll
  for (int a = 0; a < QN; ++a) {
    // dims 16a + 4g .. +3 (instruction (a, j) contracts dim 16a + 4g + j)
    qop[a] = load_query4<D>(p, qrow, qrow_i, a * 16 + g * 4, qs);
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
      const_cast<float*>(p.k) + (size_t)kvh * p.M * D, 0, (int)(p.M * ROWB),
      kBufferWord3);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(p.v) + (size_t)kvh * p.M * D, 0, (int)(p.M * ROWB),
      kBufferWord3);
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
      *reinterpret_cast<floatx4*>(&sm.ks[key * KP + d4 * 4]) = x;
    
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
          *reinterpret_cast<float4*>(&sm.vt[d * VP + vt_col(d, kq)]) =
              make_float4(e0, e1, e2, e3);
        
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

    // S^T tiles t: keys k0 + 16t + 4g + j, query qi.  The operands of
    // the whole block (K for S^T, V^T for O^T) are read from LDS first, so
    // the reads overlap each other, the MFMAs and the softmax.
    const int q0 = kslice * (KW / 4);  // first 4-key quad of the slice
    floatx4 s[TW];
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
  
  };

  // One block in flight in registers while the previous one computes.
  auto blk = [&](uint32_t i) { return kb_begin + min(i, nblk - 1) * kBK; };
  fetch(buf, kb_begin, true);
  for (uint32_t i = 0; i < nblk; ++i) {
    const uint32_t kb = kb_begin + i * kBK;
    __syncthreads();  // the previous block's LDS reads are done
    stage(buf, 0);
    __syncthreads();
    fetch(buf, blk(i + 1), i + 1 < nblk);
    compute(kb, 0, true);
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
        st4_stream(orow + 16 * t + 4 * g, r);
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
  // Every other split has taken its ticket: reset the counter now, its round
  // trip overlapping the loads of the fold.
  if (tid == 0) atomicExch(ctr, 0u);

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
        st4_stream(orow + 16 * t + 4 * g, r);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// bf16 prefill with specialised waves.
//
// One workgroup = one head x 64 queries, eight waves.  Waves 4..7 (producers)
// load the f32 K/V rows of 64-key blocks, three blocks in flight in registers,
// round them to bf16 and write them into a ring of kWsStages LDS stages (K
// row-major, V transposed).  Waves 0..3 (consumers) each own 32 queries
// (w & 1) and one 32-key slice (w >> 1) of every block; per block a consumer
// computes S^T = K_slice Q^T as one 32x32 tile (v_mfma_f32_32x32x16_bf16,
// Q^T in registers), the online softmax, and O^T += V^T P^T with the S^T
// accumulator itself as the B operand (lane l: query l%32, register v: key
// 8*(v/4) + 4*(l/32) + v%4 of the slice; V^T holds the keys of every 16-key
// group in the order bit 3 <-> bit 2 so the A operand reads them in the same
// order).  Producers and consumers of a stage hand over through two LDS
// counters per stage (filled: +1 per producer wave, released: +1 per
// consumer wave), so loading and converting overlap the matrix and softmax
// work instead of alternating with it at workgroup barriers.
constexpr int kWsStages = 4;
constexpr int kWsKB = 64;
// Lazy rescaling threshold of the bf16 kernels' online softmax (log2 units).
constexpr float kLazyLog2 = 8.f;

// SPLIT stages hold two bf16 planes of every value, x_hi = bf16(x) and
// x_lo = bf16(x - x_hi) (16 significant bits between them).
template <int D, bool SPLIT>
struct WsStage {
  static constexpr int KP = D + 8;      // K row pitch (bf16)
  static constexpr int VP = kWsKB + 8;  // V^T row pitch (bf16)
  static constexpr int NPL = SPLIT ? 2 : 1;
  alignas(16) __bf16 ks[NPL][kWsKB * KP];
  alignas(16) __bf16 vt[NPL][D * VP];
};

// x = hi + lo to 16 significant bits: hi = bf16(x), lo = bf16(x - hi) (the
// difference is exact in f32).
__device__ __forceinline__ __bf16 bf16_lo(float x, __bf16 hi) { return (__bf16)(x - (float)hi); }

// bf16 offset of block key k (0..63) inside V^T row d: key bits 2 and 3
// swapped, then 8-key units XOR-permuted by (d/4)%8 (bank spread for the
// transposing writes and the operand reads).
__device__ __forceinline__ int ws_vt_pos(int d, int k) {
  const int kp = (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1);
  return (((kp >> 3) ^ ((d >> 2) & 7)) << 3) | (kp & 7);
}

typedef float f32x16 __attribute__((ext_vector_type(16)));

// s_waitcnt lgkmcnt(0) alone (vmcnt and expcnt at their maxima).
constexpr int kWaitLgkm0 = 0xC07F;

// Spins until the LDS counter reaches target, for at most `limit` polls.  The
// handover completes within microseconds; the bound guarantees that every
// wave leaves the loop.  A wait that gives up records STS_DEVERR_WAIT_TIMEOUT
// in the device error word (the stage it goes on with may not hold its block,
// so the output is wrong, and the host learns it from that word).
__device__ __forceinline__ void ws_wait_ge(const uint32_t* ctr, uint32_t target, uint32_t limit,
                                           int lane, uint32_t* err) {
  bool done = false;
  for (uint32_t spin = 0; spin < limit && !done; ++spin) {
    done = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= target;
    if (!done) __builtin_amdgcn_s_sleep(1);
  }
  if (!done && lane == 0 && err) atomicOr(err, (uint32_t)STS_DEVERR_WAIT_TIMEOUT);
  asm volatile("" ::: "memory");
}
// Publishes this wave's LDS writes (or the end of its LDS reads) and counts it.
__device__ __forceinline__ void ws_signal(uint32_t* ctr, int lane) {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  if (lane == 0) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// SPLIT: the split variant (f32-grade while the scores' ~2^-16 relative error
// stays small next to the tolerance).  Every operand is split into bf16 hi and
// lo planes and each product runs as three bf16 MFMAs (hi*hi + hi*lo +
// lo*hi, f32 accumulate; the dropped lo*lo term is 2^-16 relative), which
// on this chip's 16:1 bf16:f32 matrix rate is ~5x the f32 MFMA rate.  Two
// stages (the planes double a stage) and no LDS query tile: the consumers
// split their own queries.
// KV16: the K/V rows come from bf16 copies of the caches (p.k16, p.v16,
// [H][M][D] bf16, rounded to nearest even as the f32 path rounds them in its
// producers), so the producers move half the bytes and convert nothing; the
// stages, and therefore the result, are those of the f32-input kernel.
template <int D, bool SPLIT, bool KV16 = false>
__global__ __launch_bounds__(512) void prefill_ws_kernel(const PrefillParams p) {
  static_assert(!(SPLIT && KV16), "the split variant needs the f32 rows");
  using Stage = WsStage<D, SPLIT>;
  constexpr int KB = kWsKB;
  constexpr int NS = SPLIT ? 2 : kWsStages;
  constexpr int QT = 64;
  constexpr int KP = Stage::KP;
  constexpr int VP = Stage::VP;
  constexpr int C4 = D / 4;               // float4 columns of a row
  constexpr int KA = D / 16;              // k-chunks of S^T
  constexpr int OT = D / 32;              // O^T row tiles
  constexpr int NP = 256;                 // producer threads
  constexpr int KPER = KB * C4 / NP;      // K float4 per producer thread per block
  constexpr int VSQ = (KB / 4) * C4;      // V 4-key x 4-dim squares per block
  constexpr int VPER = VSQ >= NP ? VSQ / NP : 1;
  static_assert(KPER >= 1 && (VSQ % NP == 0 || NP % VSQ == 0), "tile shape");
  __shared__ Stage st[NS];
  __shared__ uint32_t filled[NS], vfilled[NS], released[NS], q_ready;
  // The tile's queries, scaled and rounded to bf16 once by the producers
  // (each query row is the B operand of two consumer waves).
  constexpr int QP = D + 8;  // row pitch (bf16)
  __shared__ __align__(16) __bf16 qs[SPLIT ? 8 : QT * QP];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t h = blockIdx.x;
  const uint32_t kvh = p.group_magic ? __umulhi(h, p.group_magic) : h;  // its K/V head
  const uint32_t nqt = (p.S + QT - 1) / QT;
  const uint32_t qt = nqt - 1 - blockIdx.y;  // heaviest tiles first
  const uint32_t base_w = p.len - p.S;
  const uint32_t q_last = min(p.S, (qt + 1) * QT) - 1;
  const uint32_t kend = min(p.len, base_w + q_last + 1);
  const uint32_t nblk = (kend + KB - 1) / KB;
  // Visit order of the key blocks: the tiles within two blocks of the
  // launch's longest take theirs last to first.  They then start on blocks
  // few other tiles read and end on the ones every tile of the head has
  // already brought into L2 (512 queries after 256 cached, f32 K/V: 20.0 ->
  // 19.0 us per layer; the same order on the mirror path keeps its result
  // bit-identical to this one's; the split kernel, 0.25 us slower with it,
  // keeps the forward order).  Step i of producers and consumers handles
  // block blk(i); steps past the last block stay past it (zero loads).
  const uint32_t maxblk = (p.len + KB - 1) / KB;
  const bool reverse = !SPLIT && nblk + 2 >= maxblk;
  auto blk = [&](uint32_t i) { return reverse && i < nblk ? nblk - 1 - i : i; };
  if (tid < NS) {
    filled[tid] = 0;
    vfilled[tid] = 0;
    released[tid] = 0;
    if (tid == 0) q_ready = 0;
  }
  __syncthreads();
  // Start stagger (bf16 mirror, all tiles resident at once): the shorter a
  // tile's key range, the later it requests its queries and first blocks, so
  // the longest tiles, which set the kernel's end, start under less HBM
  // traffic; the shorter ones still finish first (measured at 512 queries
  // after 256 cached: 17.6 -> 16.5 us per layer).
  if (KV16 && p.start_stagger) {
    // At most 16 blocks' worth: a bounded head start for the long tiles,
    // however many blocks a launch has.
    const uint32_t n = min(maxblk - nblk, 16u) * p.start_stagger;
    for (uint32_t i = 0; i < n; ++i) __builtin_amdgcn_s_sleep(2);
  }

  // Consumer state (also the merge's inputs).
  const int qg = wave & 1;
  const int ks = (wave >> 1) & 1;
  const int l32 = lane & 31;
  const int hh = lane >> 5;
  const uint32_t qi = qt * QT + qg * 32 + l32;
  const bool q_ok = qi < p.S;
  float m = -FLT_MAX;
  float lsum = 0.f;
  f32x16 o[OT];
#pragma unroll
  for (int t = 0; t < OT; ++t)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[t][v] = 0.f;

  if (wave >= 4 && KV16) {
    // ---- producers, bf16 rows ----
    const int pt = tid - 256;
    constexpr int C8 = D / 8;               // 16-byte chunks (8 dims) of a bf16 row
    constexpr int KP16 = KB * C8 / NP;      // K chunks per producer thread and block
    constexpr int VQ16 = (KB / 4) * C8;     // V pieces (4 keys x 8 dims) per block
    constexpr int VP16 = VQ16 >= NP ? VQ16 / NP : 1;
    static_assert(KP16 >= 1 && (VQ16 % NP == 0 || NP % VQ16 == 0), "bf16 tile shape");
    constexpr uint32_t ROWB = D * 2;
    const int c8 = pt % C8;
    const __amdgpu_buffer_rsrc_t k16rs = __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<uint16_t*>(const_cast<void*>(p.k16)) + (size_t)kvh * p.M * D,
        0, (int)(p.M * ROWB), kBufferWord3);
    const __amdgpu_buffer_rsrc_t v16rs = __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<uint16_t*>(const_cast<void*>(p.v16)) + (size_t)kvh * p.M * D,
        0, (int)(p.M * ROWB), kBufferWord3);
    const bool v_thread = VQ16 >= NP || pt < VQ16;
    auto k_row = [&](int i) { return (uint32_t)(pt / C8 + i * (NP / C8)); };
    auto v_row = [&](int i, int r4) { return (uint32_t)((pt / C8 + i * (NP / C8)) * 4 + r4); };
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    struct Buf {
      u32x4 k[KP16];
      u32x4 v[VP16][4];
    };
    constexpr int NL = KP16 + 4 * VP16;
    auto fetch = [&](Buf& bf, uint32_t b) {
      const uint32_t kb = blk(b) * KB;
      const uint32_t lim = b < nblk ? kend : 0u;
      uint32_t slot0 = p.start + kb;
      slot0 = slot0 >= p.M ? slot0 - p.M : slot0;
      uint32_t vo[NL];
      uint32_t so = 0;
      if (kb + KB <= lim && slot0 + KB <= p.M) {
        so = slot0 * ROWB;
#pragma unroll
        for (int i = 0; i < KP16; ++i) vo[i] = k_row(i) * ROWB + c8 * 16;
#pragma unroll
        for (int i = 0; i < VP16; ++i)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) vo[KP16 + 4 * i + r4] = v_row(i, r4) * ROWB + c8 * 16;
      } else {
        auto off = [&](uint32_t r) {
          const uint32_t row = kb + r;
          uint32_t slot = slot0 + r;
          slot = min(slot, slot - p.M);  // wrap (slot < 2M)
          return row < lim ? slot * ROWB + c8 * 16 : 0xFFFFFFF0u;
        };
#pragma unroll
        for (int i = 0; i < KP16; ++i) vo[i] = off(k_row(i));
#pragma unroll
        for (int i = 0; i < VP16; ++i)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) vo[KP16 + 4 * i + r4] = off(v_row(i, r4));
      }
#pragma unroll
      for (int i = 0; i < KP16; ++i)
        bf.k[i] = __builtin_amdgcn_raw_buffer_load_b128(k16rs, vo[i], so, 0);
      if (v_thread) {
#pragma unroll
        for (int i = 0; i < VP16; ++i)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4)
            bf.v[i][r4] = __builtin_amdgcn_raw_buffer_load_b128(v16rs, vo[KP16 + 4 * i + r4], so, 0);
      }
    };
    // K chunks go to their rows as they are; each V piece (4 keys x 8 dims) is
    // transposed into 8 runs of 4 keys (dims c8*8 .. +7).
    auto put_k = [&](const Buf& bf, Stage& sg) {
#pragma unroll
      for (int i = 0; i < KP16; ++i)
        *reinterpret_cast<u32x4*>(&sg.ks[0][k_row(i) * KP + c8 * 8]) = bf.k[i];
    };
    auto put_v = [&](const Buf& bf, Stage& sg) {
      if (!v_thread) return;
#pragma unroll
      for (int i = 0; i < VP16; ++i) {
        const int key0 = (pt / C8 + i * (NP / C8)) * 4;
        const u32x4* x = bf.v[i];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int d = c8 * 8 + e;
          const int w = e >> 1, sh = (e & 1) * 16;
          const uint32_t r0 = (x[0][w] >> sh) & 0xFFFFu, r1 = (x[1][w] >> sh) & 0xFFFFu;
          const uint32_t r2 = (x[2][w] >> sh) & 0xFFFFu, r3 = (x[3][w] >> sh) & 0xFFFFu;
          typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
          *reinterpret_cast<u32x2*>(&sg.vt[0][d * VP + ws_vt_pos(d, key0)]) =
              u32x2{r0 | (r1 << 16), r2 | (r3 << 16)};
        }
      }
    };
    auto produce = [&](const Buf& bf, uint32_t i) {
      const uint32_t s = i % NS, use = i / NS;
      ws_wait_ge(&released[s], 4 * use, p.wait_limit, lane, p.err);
      // The split kernel's consumers (its three products per block make them
      // the slower side) may start the scores once K is in (vfilled then
      // counts V); elsewhere one signal covers the block (two measured
      // slower there).
      put_k(bf, st[s]);
      if constexpr (SPLIT) ws_signal(&filled[s], lane);
      put_v(bf, st[s]);
      ws_signal(SPLIT ? &vfilled[s] : &filled[s], lane);
    };
    // Queries: as the f32 producers stage them.
    constexpr int QPER = QT * C4 / NP;
    const int d4 = pt % C4;
    auto q_row = [&](int i) { return (uint32_t)(pt / C4 + i * (NP / C4)); };
    float4 qv[QPER];
#pragma unroll
    for (int i = 0; i < QPER; ++i) {
      const uint32_t qq = qt * QT + q_row(i);
      qv[i] = ld4(p.q + ((size_t)(qq < p.S ? qq : 0) * p.H + h) * D + d4 * 4);
    }
    float2 qcs[QPER], qsn[QPER];
    if (p.rope_cos) {
#pragma unroll
      for (int i = 0; i < QPER; ++i) {
        const uint32_t qq = qt * QT + q_row(i);
        rope_coeffs<D>(p.rope_cos, p.rope_sin, p.rope_pos0 + (qq < p.S ? qq : 0), d4 * 4, qcs[i],
                       qsn[i]);
      }
    }
    // The second block is requested once the queries are in: at the start
    // every tile asks for its queries and first block together, and a
    // second block each would lengthen that burst for all of them.
    Buf b0, b1, b2;
    fetch(b0, 0);
#pragma unroll
    for (int i = 0; i < QPER; ++i) {
      const uint32_t qq = qt * QT + q_row(i);
      if (p.rope_cos) qv[i] = rope4(qv[i], qcs[i], qsn[i]);
      const float4 x = scale4(qv[i], qq < p.S ? p.scale_log2 : 0.f);
      bf16x4 y;
      y[0] = (__bf16)x.x; y[1] = (__bf16)x.y; y[2] = (__bf16)x.z; y[3] = (__bf16)x.w;
      *reinterpret_cast<bf16x4*>(&qs[q_row(i) * QP + d4 * 4]) = y;
    }
    ws_signal(&q_ready, lane);
    fetch(b1, 1);
    produce(b0, 0);
    for (uint32_t i = 1; i < nblk; i += 3) {
      fetch(b2, i + 1);
      produce(b1, i);
      if (i + 1 >= nblk) break;
      fetch(b0, i + 2);
      produce(b2, i + 1);
      if (i + 2 >= nblk) break;
      fetch(b1, i + 3);
      produce(b0, i + 2);
    }
  } else if (wave >= 4) {
    // ---- producers ----
    const int pt = tid - 256;
    const int d4 = pt % C4;
    constexpr uint32_t ROWB = D * sizeof(float);
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.k) + (size_t)kvh * p.M * D, 0, (int)(p.M * ROWB),
        kBufferWord3);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.v) + (size_t)kvh * p.M * D, 0, (int)(p.M * ROWB),
        kBufferWord3);
    const bool v_thread = VSQ >= NP || pt < VSQ;
    auto k_row = [&](int i) { return (uint32_t)(pt / C4 + i * (NP / C4)); };
    auto v_row = [&](int i, int r4) { return (uint32_t)((pt / C4 + i * (NP / C4)) * 4 + r4); };
    struct Buf {
      floatx4 k[KPER];
      floatx4 v[VPER][4];
    };
    constexpr int NL = KPER + 4 * VPER;
    // Loads block b (rows past the tile's last key, and every row of a block
    // past the last, read zeros: the loads are issued unconditionally so the
    // compiler's wait counts see one fixed order).
    auto fetch = [&](Buf& bf, uint32_t b) {
      const uint32_t kb = blk(b) * KB;
      const uint32_t lim = b < nblk ? kend : 0u;
      uint32_t slot0 = p.start + kb;
      slot0 = slot0 >= p.M ? slot0 - p.M : slot0;
      uint32_t vo[NL];
      uint32_t so = 0;
      if (kb + KB <= lim && slot0 + KB <= p.M) {
        so = slot0 * ROWB;
#pragma unroll
        for (int i = 0; i < KPER; ++i) vo[i] = k_row(i) * ROWB + d4 * 16;
#pragma unroll
        for (int i = 0; i < VPER; ++i)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) vo[KPER + 4 * i + r4] = v_row(i, r4) * ROWB + d4 * 16;
      } else {
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
        bf.k[i] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(krs, vo[i], so, 0));
      if (v_thread) {
#pragma unroll
        for (int i = 0; i < VPER; ++i)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4)
            bf.v[i][r4] = __builtin_bit_cast(
                floatx4, __builtin_amdgcn_raw_buffer_load_b128(vrs, vo[KPER + 4 * i + r4], so, 0));
      }
    };
    // Four values rounded to bf16 at one offset of the hi plane (and, for
    // SPLIT, their remainders in the lo plane).
    auto store4 = [&](__bf16* hi_plane, __bf16* lo_plane, int off, float a, float b, float c, float d) {
      bf16x4 yh;
      yh[0] = (__bf16)a; yh[1] = (__bf16)b; yh[2] = (__bf16)c; yh[3] = (__bf16)d;
      *reinterpret_cast<bf16x4*>(&hi_plane[off]) = yh;
      if constexpr (SPLIT) {
        bf16x4 yl;
        yl[0] = bf16_lo(a, yh[0]); yl[1] = bf16_lo(b, yh[1]);
        yl[2] = bf16_lo(c, yh[2]); yl[3] = bf16_lo(d, yh[3]);
        *reinterpret_cast<bf16x4*>(&lo_plane[off]) = yl;
      } else {
        (void)lo_plane;
      }
    };
    auto put_k = [&](const Buf& bf, Stage& sg) {
#pragma unroll
      for (int i = 0; i < KPER; ++i) {
        const floatx4 x = bf.k[i];
        store4(sg.ks[0], sg.ks[Stage::NPL - 1], k_row(i) * KP + d4 * 4, x.x, x.y, x.z, x.w);
      }
    };
    auto put_v = [&](const Buf& bf, Stage& sg) {
      if (!v_thread) return;
#pragma unroll
      for (int i = 0; i < VPER; ++i) {
        const int key0 = (pt / C4 + i * (NP / C4)) * 4;
        const floatx4* x = bf.v[i];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int d = d4 * 4 + c;
          store4(sg.vt[0], sg.vt[Stage::NPL - 1], d * VP + ws_vt_pos(d, key0), x[0][c], x[1][c], x[2][c], x[3][c]);
        }
      }
    };
    // Block i goes to stage i % NS once the consumers have released that
    // stage's previous block (4 releases per use).
    auto produce = [&](const Buf& bf, uint32_t i) {
      const uint32_t s = i % NS, use = i / NS;
      ws_wait_ge(&released[s], 4 * use, p.wait_limit, lane, p.err);
      put_k(bf, st[s]);
      if constexpr (SPLIT) ws_signal(&filled[s], lane);
      put_v(bf, st[s]);
      ws_signal(SPLIT ? &vfilled[s] : &filled[s], lane);
    };
    // Three blocks in flight in registers: block i is converted and stored
    // while blocks i+1 and i+2 load (the per-CU load rate, not the issue,
    // bounds this loop).
    // Queries first: row pt/C4 + i*(NP/C4), columns 4*d4..+3 (a row past the
    // tile's end reads row 0 and is scaled by zero, so every load is issued).
    constexpr int QPER = SPLIT ? 1 : QT * C4 / NP;
    float4 qv[QPER];
    if constexpr (!SPLIT) {
#pragma unroll
      for (int i = 0; i < QPER; ++i) {
        const uint32_t qq = qt * QT + k_row(i);
        qv[i] = ld4(p.q + ((size_t)(qq < p.S ? qq : 0) * p.H + h) * D + d4 * 4);
      }
    }
    // RoPE coefficients of those query rows (issued with the loads).
    float2 qcs[QPER], qsn[QPER];
    if (!SPLIT && p.rope_cos) {
#pragma unroll
      for (int i = 0; i < QPER; ++i) {
        const uint32_t qq = qt * QT + k_row(i);
        rope_coeffs<D>(p.rope_cos, p.rope_sin, p.rope_pos0 + (qq < p.S ? qq : 0), d4 * 4, qcs[i],
                       qsn[i]);
      }
    }
    // The second block is requested once the queries are in (as above;
    // 512 queries after 256 cached: 18.2 -> 17.7 us per layer; the split
    // kernel, which loads no queries here, requests both at once).
    Buf b0, b1, b2;
    fetch(b0, 0);
    if constexpr (SPLIT) fetch(b1, 1);
    if constexpr (!SPLIT) {
#pragma unroll
      for (int i = 0; i < QPER; ++i) {
        const uint32_t qq = qt * QT + k_row(i);
        if (p.rope_cos) qv[i] = rope4(qv[i], qcs[i], qsn[i]);
        const float4 x = scale4(qv[i], qq < p.S ? p.scale_log2 : 0.f);
        bf16x4 y;
        y[0] = (__bf16)x.x; y[1] = (__bf16)x.y; y[2] = (__bf16)x.z; y[3] = (__bf16)x.w;
        *reinterpret_cast<bf16x4*>(&qs[k_row(i) * QP + d4 * 4]) = y;
      }
      ws_signal(&q_ready, lane);
      fetch(b1, 1);
    }
    produce(b0, 0);
    for (uint32_t i = 1; i < nblk; i += 3) {
      fetch(b2, i + 1);
      produce(b1, i);
      if (i + 1 >= nblk) break;
      fetch(b0, i + 2);
      produce(b2, i + 1);
      if (i + 2 >= nblk) break;
      fetch(b1, i + 3);
      produce(b0, i + 2);
    }
  } else {
    // ---- consumers ----
    const uint32_t w_q = base_w + qi;
    const uint32_t w_first = base_w + qt * QT + qg * 32;
    // B operands of S^T: this lane's query, dims 16a + 8hh .. +7 (planes hi
    // and, for SPLIT, lo).
    constexpr int QPL = SPLIT ? 2 : 1;
    bf16x8 qop[QPL][KA];
    if constexpr (SPLIT) {
      // Every lane loads (a row past the tile's end reads row 0) and scales
      // by zero when it has no query: no branch, so all loads issue at once.
      const uint32_t qrow_i = q_ok ? qi : 0;
      const float* qrow = p.q + ((size_t)qrow_i * p.H + h) * D;
      const float qsc = q_ok ? p.scale_log2 : 0.f;
#pragma unroll
      for (int a = 0; a < KA; ++a) {
        const float4 x0 = load_query4<D>(p, qrow, qrow_i, a * 16 + hh * 8, qsc);
        const float4 x1 = load_query4<D>(p, qrow, qrow_i, a * 16 + hh * 8 + 4, qsc);
        const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const __bf16 hi = (__bf16)xs[e];
          qop[0][a][e] = hi;
          qop[QPL - 1][a][e] = bf16_lo(xs[e], hi);
        }
      }
    } else {
      ws_wait_ge(&q_ready, 4, p.wait_limit, lane, p.err);
#pragma unroll
      for (int a = 0; a < KA; ++a)
        qop[0][a] = *reinterpret_cast<const bf16x8*>(&qs[(qg * 32 + l32) * QP + a * 16 + hh * 8]);
    }
    // Scores S^T of block i: waits for its stage, K operands from LDS, MFMAs.
    // The scores accumulate onto -mb, mb the running maximum when they are
    // issued (0 before the first block), so they come out of the MFMAs
    // relative to it: the softmax subtracts nothing unless the base has
    // moved since (the first block, a lazy rescale).
    // The base's negation is kept in a tile of its own, the first MFMA's
    // accumulator input, and rewritten only when the base moves.
    float mbase = 0.f;
    f32x16 nbase;
#pragma unroll
    for (int v = 0; v < 16; ++v) nbase[v] = -0.f;
    auto s_block = [&](uint32_t i) {
      const uint32_t s = i % NS, use = i / NS;
      ws_wait_ge(&filled[s], 4 * (use + 1), p.wait_limit, lane, p.err);
      const Stage& sg = st[s];
      f32x16 sc = nbase;
#pragma unroll
      for (int pl = 0; pl < QPL; ++pl) {
        // K plane pl against Q hi, and (SPLIT, K hi only) against Q lo.
        bf16x8 kop[KA];
#pragma unroll
        for (int a = 0; a < KA; ++a)
          kop[a] = *reinterpret_cast<const bf16x8*>(&sg.ks[pl][(ks * 32 + l32) * KP + a * 16 + hh * 8]);
#pragma unroll
        for (int a = 0; a < KA; ++a)
          sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kop[a], qop[0][a], sc, 0, 0, 0);
        if (SPLIT && pl == 0) {
#pragma unroll
          for (int a = 0; a < KA; ++a)
            sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kop[a], qop[QPL - 1][a], sc, 0, 0, 0);
        }
      }
      return sc;
    };
    // Mask, online softmax and O^T += V^T P^T of block i; releases its stage.
    auto finish_block = [&](uint32_t i, f32x16 sc, float mb) {
      const uint32_t s = i % NS;
      const Stage& sg = st[s];
      const uint32_t k0 = blk(i) * KB + ks * 32;
      const bool unmasked = k0 + 31 < kend && k0 + 31 <= w_first;
      if (!unmasked) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const uint32_t key = k0 + 8 * (v >> 2) + 4 * hh + (v & 3);
          sc[v] = (key <= w_q && key < kend) ? sc[v] : -INFINITY;
        }
      }
      // sc holds the scores less mb; the block maximum is mx + mb.
      float mx = sc[0];
#pragma unroll
      for (int v = 1; v < 16; ++v) mx = fmaxf(mx, sc[v]);
      mx = max_xor32(mx) + mb;
      // Lazy rescaling: the weights stay relative to the base m until some
      // query's block maximum exceeds it by more than kLazyLog2 (weights then
      // stay <= 2^kLazyLog2); only then does the base move and O get
      // rescaled.  The same softmax; the rescale no longer runs every block.
      if (__any(mx > m + kLazyLog2)) {
        const float mn = fmaxf(m, mx);
        const float alpha = fast_exp2(m - mn);
        m = mn;
        lsum *= alpha;
#pragma unroll
        for (int t = 0; t < OT; ++t) o[t] *= alpha;
        mbase = m == -FLT_MAX ? 0.f : m;
#pragma unroll
        for (int v = 0; v < 16; ++v) nbase[v] = -mbase;
      }
      // The weights exp2(s - m): sc already less mb, so only a moved base
      // needs a subtraction.
      const float dm = m - mb;
      if (__any(dm != 0.f)) {
#pragma unroll
        for (int v = 0; v < 16; ++v) sc[v] -= dm;
      }
      float ps = 0.f;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float e = fast_exp2(sc[v]);
        sc[v] = e;
        if constexpr (SPLIT) ps += e;
      }
      bf16x8 pb[QPL][2];
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const __bf16 hi = (__bf16)sc[8 * c + j];
          pb[0][c][j] = hi;
          if constexpr (SPLIT) pb[QPL - 1][c][j] = bf16_lo(sc[8 * c + j], hi);
        }
      if constexpr (!SPLIT) {
        // The row sum of the weights as the products will use them, rounded
        // to bf16: two bf16 weights per v_dot2 with (1, 1), f32 accumulate.
        const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};
        float ps1 = 0.f;
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
          ps = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{pb[0][0][j], pb[0][0][j + 1]}, ones, ps, false);
          ps1 = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{pb[0][1][j], pb[0][1][j + 1]}, ones, ps1, false);
        }
        ps += ps1;
      }
      lsum += sum_xor32(ps);
      // V^T operands are read per output tile after the softmax (the stage
      // stays claimed until they are in registers), then the stage is released.
      if constexpr (SPLIT) ws_wait_ge(&vfilled[s], 4 * (i / NS + 1), p.wait_limit, lane, p.err);
#pragma unroll
      for (int t = 0; t < OT; ++t) {
#pragma unroll
        for (int pl = 0; pl < QPL; ++pl) {
          // V plane pl against P hi, and (SPLIT, V hi only) against P lo.
          bf16x8 vop[2];
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            const int d = 32 * t + l32;
            const int oct = (ks * 4 + 2 * c + hh) ^ ((d >> 2) & 7);
            vop[c] = *reinterpret_cast<const bf16x8*>(&sg.vt[pl][d * VP + oct * 8]);
          }
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vop[c], pb[0][c], o[t], 0, 0, 0);
            if (SPLIT && pl == 0)
              o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vop[c], pb[QPL - 1][c], o[t], 0, 0, 0);
          }
        }
      }
      ws_signal(&released[s], lane);
    };
    // (Consumers one block ahead, the next block's score MFMAs issued before
    // this block's softmax, measured slower once the softmax lost the
    // subtraction and the row-sum additions: mirror 16.9 against 16.1 us.)
    for (uint32_t i = 0; i < nblk; ++i) {
      const float mb = mbase;
      finish_block(i, s_block(i), mb);
    }
  }

  // Merge the two key slices of each query group through LDS (stage 0, free
  // once every wave has passed the barrier) and write the rows.
  __syncthreads();
  constexpr int RS = OT * 16 + 2;
  float* red = reinterpret_cast<float*>(&st[0]);  // [2 groups][64 lanes][RS]
  static_assert(2 * 64 * RS * sizeof(float) <= sizeof(Stage), "merge scratch");
  if (wave < 4 && ks == 1) {
    float* dst = red + (qg * 64 + lane) * RS;
#pragma unroll
    for (int t = 0; t < OT; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) dst[16 * t + v] = o[t][v];
    dst[OT * 16] = m;
    dst[OT * 16 + 1] = lsum;
  }
  __syncthreads();
  if (wave >= 4 || ks != 0 || !q_ok) return;
  const float* src = red + (qg * 64 + lane) * RS;
  const float m2 = src[OT * 16], l2 = src[OT * 16 + 1];
  const float mm = fmaxf(m, m2);
  const float f1 = fast_exp2(m - mm), f2 = fast_exp2(m2 - mm);
  const float inv = 1.f / (lsum * f1 + l2 * f2);
  float* orow = p.out + ((size_t)qi * p.H + h) * D;
#pragma unroll
  for (int t = 0; t < OT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float4 y;
      y.x = (o[t][4 * r + 0] * f1 + src[16 * t + 4 * r + 0] * f2) * inv;
      y.y = (o[t][4 * r + 1] * f1 + src[16 * t + 4 * r + 1] * f2) * inv;
      y.z = (o[t][4 * r + 2] * f1 + src[16 * t + 4 * r + 2] * f2) * inv;
      y.w = (o[t][4 * r + 3] * f1 + src[16 * t + 4 * r + 3] * f2) * inv;
      st4_stream(orow + 32 * t + 8 * r + 4 * hh, y);
    }
}

template <int D, bool SPLIT, bool KV16 = false>
int launch_ws(const PrefillParams& p, hipStream_t stream) {
  const uint32_t nqt = (p.S + 63) / 64;
  if (nqt > 65535u) return fail(STS_ERR_INVALID, "seq %u too long for one launch", p.S);
  if ((uint64_t)p.M * D * sizeof(float) > 0x7FFFFFF0ull)
    return fail(STS_ERR_INVALID, "max_len %u too large for one head's buffer resource", p.M);
  PrefillParams q = p;
  // A sleeping workgroup costs nothing only while no other waits for its CU.
  q.start_stagger = KV16 && !SPLIT && (uint64_t)p.H * nqt <= (uint64_t)device_cu_count() ? 10u : 0u;
  hipLaunchKernelGGL((prefill_ws_kernel<D, SPLIT, KV16>), dim3(p.H, nqt, 1), dim3(512), 0, stream,
                     q);
  STS_HIP(hipGetLastError());
  return STS_OK;
}

// Key-range splits of the f32 kernel: f32 tiles carry four times the MFMA
// work of bf16 ones, so their key ranges are split until there are about two
// workgroups per CU.
uint32_t f32_splits(uint32_t S, uint32_t H) {
  const uint32_t tiles = H * ((S + kBQ - 1) / kBQ);
  const uint32_t cus = (uint32_t)device_cu_count();
  const uint32_t nsplit = (2 * cus + tiles - 1) / tiles;
  return std::max(1u, std::min<uint32_t>(nsplit, kMaxPrefillSplits));
}

// The split workspace of the f32 kernel (null with one split).
template <int D>
int f32_workspace(uint32_t S, uint32_t H, hipStream_t stream, uint32_t* nsplit, Workspace** out) {
  *out = nullptr;
  *nsplit = f32_splits(S, H);
  if (*nsplit <= 1) return STS_OK;
  const uint32_t tiles = H * ((S + kBQ - 1) / kBQ);
  return get_workspace(stream, (size_t)tiles * *nsplit * 256 * (D / 4 + 2), tiles, out);
}

template <int D>
int launch_f32(const PrefillParams& p, hipStream_t stream) {
  const uint32_t nqt = (p.S + kBQ - 1) / kBQ;
  if (nqt > 65535u) return fail(STS_ERR_INVALID, "seq %u too long for one launch", p.S);
  if ((uint64_t)p.M * D * sizeof(float) > 0x7FFFFFF0ull)
    return fail(STS_ERR_INVALID, "max_len %u too large for one head's buffer resource", p.M);
  PrefillParams q = p;
  Workspace* ws = nullptr;
  if (int rc = f32_workspace<D>(p.S, p.H, stream, &q.nsplit, &ws)) return rc;
  if (ws) {
    q.part = ws->part;
    q.counters = ws->counters;
  }
  const uint32_t nsplit = q.nsplit;
  hipLaunchKernelGGL((prefill_kernel<D, kKsplit>), dim3(p.H, nqt, nsplit),
                     dim3(256 * kKsplit), 0, stream, q);
  STS_HIP(hipGetLastError());
  return STS_OK;
}

}  // namespace


int check_prefill(uint32_t seq, uint32_t heads, uint32_t head_dim, uint32_t max_len,
                  int precision) {
  if (head_dim == 0 || head_dim > 128 || head_dim % 4 != 0)
    return fail(STS_ERR_INVALID, "head_dim %u not supported (a multiple of 4 up to 128)",
                head_dim);
  if (precision != STS_PREC_F32 && precision != STS_PREC_BF16_MFMA &&
      precision != STS_PREC_F32_SPLIT_BF16)
    return fail(STS_ERR_INVALID, "precision %d unknown", precision);
  if (heads < 1 || heads > 65535u) return fail(STS_ERR_INVALID, "heads %u out of 1..65535", heads);
  if ((seq + 63u) / 64u > 65535u) return fail(STS_ERR_INVALID, "seq %u too long for one launch", seq);
  // Other head dims run the queries as streams of one decode launch.
  if (head_dim != 64 && head_dim != 128 && seq > 65535u)
    return fail(STS_ERR_INVALID, "seq %u too long for one launch at head_dim %u", seq, head_dim);
  if ((uint64_t)max_len * head_dim * sizeof(float) > 0x7FFFFFF0ull)
    return fail(STS_ERR_INVALID, "max_len %u too large for one head's buffer resource", max_len);
  return STS_OK;
}

// Head dims other than 64 and 128 (multiples of 4 up to 128, which the
// reference's shader also takes, shader_attention.wgsl:36): query i of the
// chunk is a decode over window rows 0..len-S+i, exactly the S sequential
// decodes the reference's prefill stands for, run as one launch of the
// padded decode kernel with the queries as streams over the shared cache.
// Always f32, whatever precision was asked for.
static int launch_prefill_by_decode(const PrefillParams& p, uint32_t head_dim,
                                    hipStream_t stream) {
  if (!p.k || !p.v) return fail(STS_ERR_INVALID, "head_dim %u needs the f32 caches", head_dim);
  DecodeParams d;
  d.q = p.q;
  d.k = p.k;
  d.v = p.v;
  d.out = p.out;
  d.H = p.H;
  d.M = p.M;
  d.group = p.group;
  d.q_bstride = (uint64_t)p.H * head_dim;
  d.out_bstride = (uint64_t)p.H * head_dim;
  d.kv_bstride = 0;
  d.kv_hstride = (uint64_t)p.M * head_dim;
  d.len = p.len - p.S + 1;
  d.len_step = 1;
  d.start = p.start;
  d.scale_log2 = p.scale_log2;
  if (p.rope_cos) {
    d.rope_cos = p.rope_cos;
    d.rope_sin = p.rope_sin;
    d.rope_pos = p.rope_pos0;
  }
  return launch_decode(d, p.S, head_dim, p.len, stream);
}

int reserve_prefill(uint32_t S, uint32_t H, uint32_t len, uint32_t head_dim, int precision,
                    bool bf16_rows, hipStream_t stream) {
  uint32_t* err = nullptr;
  if (int rc = device_error_word(&err)) return rc;
  if (head_dim != 64 && head_dim != 128)
    return reserve_decode(S, H, head_dim, len, stream);  // launch_prefill_by_decode's plan
  if (bf16_rows || precision != STS_PREC_F32) return STS_OK;  // no workspace
  uint32_t nsplit = 1;
  Workspace* ws = nullptr;
  return head_dim == 128 ? f32_workspace<128>(S, H, stream, &nsplit, &ws)
                         : f32_workspace<64>(S, H, stream, &nsplit, &ws);
}

int launch_prefill(const PrefillParams& p0, uint32_t head_dim, int precision, hipStream_t stream) {
  if (int rc = check_prefill(p0.S, p0.H, head_dim, p0.M, precision)) return rc;
  if (p0.group == 0 || p0.H % p0.group != 0)
    return fail(STS_ERR_INVALID, "query heads %u not a multiple of the K/V group %u", p0.H,
                p0.group);
  if (head_dim != 64 && head_dim != 128) return launch_prefill_by_decode(p0, head_dim, stream);
  PrefillParams p = p0;
  p.group_magic = p.group > 1 ? (uint32_t)(((1ull << 32) + p.group - 1) / p.group) : 0u;
  p.wait_limit = wait_limit();
  if (int rc = device_error_word(&p.err)) return rc;
  const bool d128 = head_dim == 128;
  if (!(p.k16 && p.v16) && !(p.k && p.v))
    return fail(STS_ERR_INVALID, "prefill needs the K/V caches (f32 or their bf16 copies)");
  if (p.k16) {
    if (precision != STS_PREC_BF16_MFMA)
      return fail(STS_ERR_INVALID, "bf16 K/V rows serve the bf16-MFMA precision only");
    return d128 ? launch_ws<128, false, true>(p, stream) : launch_ws<64, false, true>(p, stream);
  }
  switch (precision) {
    case STS_PREC_BF16_MFMA:
      return d128 ? launch_ws<128, false>(p, stream) : launch_ws<64, false>(p, stream);
    case STS_PREC_F32_SPLIT_BF16:
      return d128 ? launch_ws<128, true>(p, stream) : launch_ws<64, true>(p, stream);
    default:
      return d128 ? launch_f32<128>(p, stream) : launch_f32<64>(p, stream);
  }
}

}  // namespace sts
