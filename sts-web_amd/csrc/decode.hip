// decode.hip -- split-KV decode attention for gfx950.
//
// Replaces shader_attention.wgsl (crates/sts-wasm/src/wgsl/shader_attention.wgsl:43-156),
// which runs one 256-lane workgroup per head, each lane streaming whole
// 512-byte rows.  Here the window of every (stream, head) is dealt to splits
// in 16-row units, round-robin; each workgroup streams one split with 128-bit
// loads that are contiguous across lanes, keeps an online softmax per row
// group, merges its waves through LDS, and the last workgroup of a
// (stream, head) to finish merges the splits (log-sum-exp) and writes out.
//
// Layout per wave (D = head_dim, G = D/4 lanes per row, NG = 64/G row groups):
//   lane = g*G + c holds dims [4c, 4c+4) of the rows of group g; one loop
//   iteration covers RPI = NG * (G/4) = 16 rows, row r0 + j*NG + g for j < G/4.
// Dot products are reduced over the G lanes of a group with a transposing
// butterfly (DPP + ds_swizzle), which leaves lane c holding the score of row
// j = (c >> 2) & (G/4 - 1), replicated over a quad.
//
// Softmax uses exp(x) = 2^(x log2 e): q is pre-multiplied by scale*log2(e) and
// the hardware base-2 exponential is applied to (s - m) <= 0.
#include <cfloat>
#include <map>
#include <mutex>

#include "common.hpp"
#include "coherent.hpp"
#include "decode.hpp"
#include "lane.hpp"
#include "rope.hpp"

namespace sts {

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kMaxSplits = 64;  // splits per (stream, head), bounded by the merge's LDS

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ void st4(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }

// K/V rows are read once per launch: nontemporal (streaming) loads keep them
// from displacing useful lines and measure ~9% faster on this access pattern.
constexpr int kNt = 2;  // buffer-load cache policy bit: nontemporal

// One transposing butterfly level: N values in, N/2 out.  The lane whose bit
// LEVEL is set keeps the upper half, its partner the lower half.
template <int LEVEL, int N>
__device__ __forceinline__ void transpose_level(float* s, int c) {
  const bool hi = (c >> LEVEL) & 1;
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    const float lo_v = s[i], hi_v = s[i + N / 2];
    const float send = hi ? lo_v : hi_v;
    const float keep = hi ? hi_v : lo_v;
    s[i] = keep + xchg<LEVEL>(send);
  }
}

// Sums RPG = G/4 per-lane partial dots over the G lanes of a row group; lane c
// ends with row (c >> 2) & (RPG-1).
template <int G>
__device__ __forceinline__ float reduce_rows(float* s, int c) {
  if constexpr (G == 32) {
    transpose_level<4, 8>(s, c);
    transpose_level<3, 4>(s, c);
    transpose_level<2, 2>(s, c);
  } else {
    static_assert(G == 16, "head_dim 64 or 128");
    transpose_level<3, 4>(s, c);
    transpose_level<2, 2>(s, c);
  }
  float x = s[0];
  x += xchg<1>(x);
  x += xchg<0>(x);
  return x;
}

// Max over the RPG distinct rows of a group (quads hold replicas).
template <int G>
__device__ __forceinline__ float group_max(float x) {
  x = fmaxf(x, xchg<2>(x));
  x = fmaxf(x, xchg<3>(x));
  if constexpr (G == 32) x = fmaxf(x, xchg<4>(x));
  return x;
}

// Sum over all 64 lanes.
__device__ __forceinline__ float wave_sum(float x) {
  x += xchg<0>(x);
  x += xchg<1>(x);
  x += xchg<2>(x);
  x += xchg<3>(x);
  x += xchg<4>(x);
  x += xor32(x);
  return x;
}

// PAD: a head dim below D (a multiple of 4, p.head_dim) on the D-wide lane
// layout: the lanes past it load zeros, so they add nothing to the scores or
// the weighted sums, and store nothing.
template <int D, int WAVES, bool PAD = false>
__global__ __launch_bounds__(WAVES * 64) void decode_kernel(const DecodeParams p) {
  constexpr int G = D / 4;
  constexpr int NG = 64 / G;
  constexpr int RPG = G / 4;
  constexpr int RPI = NG * RPG;
  static_assert(RPI == 16, "16 rows per wave iteration");

  __shared__ __align__(16) float s_p[WAVES][RPI];
  __shared__ __align__(16) float s_acc[WAVES * NG][D];
  __shared__ float s_ml[WAVES * NG][2];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane / G;
  const int c = lane % G;
  const uint32_t split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;

  uint32_t len, start;
  if (p.lens) {
    const int32_t L = p.lens[b];
    len = L <= 0 ? 0u : min((uint32_t)L, p.M);
    const int32_t st = p.starts[b] % (int32_t)p.M;
    start = (uint32_t)(st < 0 ? st + (int32_t)p.M : st);
  } else {
    len = p.len + (PAD ? b * p.len_step : 0u);
    start = p.start;
  }

  const uint32_t dh = PAD ? p.head_dim : (uint32_t)D;  // the head dim in memory
  const bool lane_ok = !PAD || (uint32_t)c * 4 < dh;   // this lane's 4 dims exist
  float* outp = p.out + b * p.out_bstride + (size_t)h * dh;
  if (len == 0) {
    if (split == 0)
      for (int t = tid; t < (int)dh; t += WAVES * 64) outp[t] = 0.f;
    return;
  }
  // This (stream, head) gets ceil(len / chunk) splits (at most nsplit_max);
  // split s takes the 16-row units s, s + nsplit, ... so that every
  // workgroup streams from the whole window and XCDs share the load evenly.
  uint32_t nsplit = (len + p.chunk - 1) / p.chunk;
  nsplit = nsplit < p.nsplit_max ? nsplit : p.nsplit_max;
  if (split >= nsplit) return;
  const uint32_t nunits = (len + RPI - 1) / RPI;

  const size_t qoff = b * p.q_bstride + (size_t)h * dh + c * 4;
  // The 4-wave kernel rotates and scales q before its first K/V loads are
  // issued: issuing them first and waiting for q afterwards measured ~1 us
  // slower per config-2 launch (20.3 vs 19.25 us), the chip-wide burst of K/V
  // requests delaying every wave's q.  The one-wave kernel (a few rows per
  // wave) issues its K/V loads first, so the two round trips overlap.
  float4 q4 = make_float4(0.f, 0.f, 0.f, 0.f);
  if (lane_ok) q4 = ld4(p.q + qoff);
  float2 rc = make_float2(0.f, 0.f), rs = make_float2(0.f, 0.f);
  const bool rope = p.rope_cos != nullptr && lane_ok;
  if (rope) {
    const uint32_t pos = p.rope_pos + (PAD ? b * p.len_step : 0u);
    const size_t ro = (size_t)pos * (dh / 2) + c * 2;
    rc = *reinterpret_cast<const float2*>(p.rope_cos + ro);
    rs = *reinterpret_cast<const float2*>(p.rope_sin + ro);
  }
  auto prep_q = [&]() {
    if (rope) q4 = rope4(q4, rc, rs);
    q4.x *= p.scale_log2;
    q4.y *= p.scale_log2;
    q4.z *= p.scale_log2;
    q4.w *= p.scale_log2;
  };
  if constexpr (WAVES > 1) prep_q();

  // The K/V head of this query head (no division on the common group-1 path).
  const uint32_t kvh = p.group == 1 ? h : h / p.group;
  const size_t kvoff = b * p.kv_bstride + kvh * p.kv_hstride;
  // K/V rows come in through buffer loads on per-(stream, head) resources:
  // a row outside the window gets an offset past the resource and loads
  // zeros, so every load is issued unconditionally and the compiler's wait
  // counts see one fixed order of loads (no drain before each batch).
  const uint32_t head_bytes = p.M * dh * (uint32_t)sizeof(float);
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(p.k) + kvoff, 0, (int)head_bytes, kBufferWord3);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(p.v) + kvoff, 0, (int)head_bytes, kBufferWord3);
  const bool append = p.k_new != nullptr;
  const uint32_t new_row = len - 1;
  const uint32_t new_unit = new_row / RPI;
  const int new_g = (int)((new_row % RPI) % NG), new_j = (int)((new_row % RPI) / NG);

  // The fused-append row: written to its slot once, RoPE'd, by the lanes of
  // the wave whose unit holds it, which also use it from registers.
  float4 kn = make_float4(0.f, 0.f, 0.f, 0.f), vn = kn;
  if (append) {
    const size_t knoff = b * (p.kn_bstride ? p.kn_bstride : p.q_bstride) + (size_t)kvh * dh + c * 4;
    if (lane_ok) {
      kn = ld4(p.k_new + knoff);
      vn = ld4(p.v_new + knoff);
    }
  }

  float m = -FLT_MAX;
  float lsum = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  const int jj = (c >> 2) & (RPG - 1);

  // Byte offset of window row r in this lane's K/V resource (rows outside the
  // window get an offset past it and load zeros).
  auto row_off = [&](uint32_t r) {
    uint32_t slot = start + r;
    slot = slot >= p.M ? slot - p.M : slot;
    return r < len && lane_ok ? slot * (dh * (uint32_t)sizeof(float)) + c * 16 : 0x80000000u;
  };
  // Rows r0 + j*NG + g (j < RPG) of this lane's group: K into kk, V into vv,
  // or both, K and V of each row together.
  auto load_k = [&](uint32_t r0, float4* kk) {
#pragma unroll
    for (int j = 0; j < RPG; ++j)
      kk[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                             krs, row_off(r0 + j * NG + g), 0, kNt));
  };
  auto load_v = [&](uint32_t r0, float4* vv) {
#pragma unroll
    for (int j = 0; j < RPG; ++j)
      vv[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                             vrs, row_off(r0 + j * NG + g), 0, kNt));
  };
  auto load_rows = [&](uint32_t r0, float4* kk, float4* vv) {
#pragma unroll
    for (int j = 0; j < RPG; ++j) {
      const uint32_t off = row_off(r0 + j * NG + g);
      kk[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(krs, off, 0, kNt));
      vv[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(vrs, off, 0, kNt));
    }
  };
  // The online-softmax update with the 16 rows starting at r0, in two halves.
  // score_rows: the rows' scores from K, the running maximum and sum; leaves
  // the weights of this lane's group's rows in pp and returns the factor the
  // running sum of V rows is rescaled by.  accumulate_rows: that rescale and
  // the weighted sum of the rows' V.
  auto score_rows = [&](uint32_t r0, float4* kk, float* pp) {
    if (append && r0 == new_unit * RPI && g == new_g) {
#pragma unroll
      for (int j = 0; j < RPG; ++j)
        if (j == new_j) kk[j] = kn;
    }
    float s[RPG];
#pragma unroll
    for (int j = 0; j < RPG; ++j)
      s[j] = q4.x * kk[j].x + q4.y * kk[j].y + q4.z * kk[j].z + q4.w * kk[j].w;
    float sc = reduce_rows<G>(s, c);
    const uint32_t my_row = r0 + jj * NG + g;
    sc = my_row < len ? sc : -INFINITY;
    const float mn = fmaxf(m, group_max<G>(sc));
    const float alpha = fast_exp2(m - mn);
    const float pj = fast_exp2(sc - mn);
    m = mn;
    lsum = lsum * alpha + pj;
    if ((c & 3) == 0) s_p[wave][g * RPG + jj] = pj;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int j = 0; j < RPG; j += 4) {
      const float4 t = *reinterpret_cast<const float4*>(&s_p[wave][g * RPG + j]);
      pp[j] = t.x;
      pp[j + 1] = t.y;
      pp[j + 2] = t.z;
      pp[j + 3] = t.w;
    }
    return alpha;
  };
  auto accumulate_rows = [&](uint32_t r0, float4* vv, const float* pp, float alpha) {
    if (append && r0 == new_unit * RPI && g == new_g) {
#pragma unroll
      for (int j = 0; j < RPG; ++j)
        if (j == new_j) vv[j] = vn;
    }
    acc.x *= alpha;
    acc.y *= alpha;
    acc.z *= alpha;
    acc.w *= alpha;
#pragma unroll
    for (int j = 0; j < RPG; ++j) {
      acc.x += pp[j] * vv[j].x;
      acc.y += pp[j] * vv[j].y;
      acc.z += pp[j] * vv[j].z;
      acc.w += pp[j] * vv[j].w;
    }
  };

  // Writes the fused-append row to its slot (RoPE'd first).  The one-wave
  // kernel (short windows) issues its first loads before this store; the
  // 4-wave kernel stores first (measured: 19.1 vs 20.3 us per config-2 launch
  // the other way round; 3.93 vs 4.03 us per depformer step).
  auto store_new_row = [&]() {
    if (!append) return;
    const uint32_t owner_split = new_unit % nsplit;
    const uint32_t owner_wave = (new_unit / nsplit) % WAVES;
    if (split == owner_split && (uint32_t)wave == owner_wave && g == new_g) {
      // Only these lanes wait for k_new and the table: the others go on to
      // their first loads.
      if (rope) kn = rope4(kn, rc, rs);
      // Every query head of a K/V group uses the row from registers; the
      // group's first head stores it.
      if (h == kvh * p.group && lane_ok) {
        uint32_t slot = start + new_row;
        slot = slot >= p.M ? slot - p.M : slot;
        st4(p.k_wr + kvoff + (size_t)slot * dh + c * 4, kn);
        st4(p.v_wr + kvoff + (size_t)slot * dh + c * 4, vn);
        if (p.k16_wr) {
          typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
          const bf16x4 kb = {(__bf16)kn.x, (__bf16)kn.y, (__bf16)kn.z, (__bf16)kn.w};
          const bf16x4 vb = {(__bf16)vn.x, (__bf16)vn.y, (__bf16)vn.z, (__bf16)vn.w};
          *reinterpret_cast<bf16x4*>(p.k16_wr + kvoff + (size_t)slot * dh + c * 4) = kb;
          *reinterpret_cast<bf16x4*>(p.v16_wr + kvoff + (size_t)slot * dh + c * 4) = vb;
        }
      }
    }
  };
  // At most one unit of 16 rows in flight per wave (16 KB, 64 KB per CU):
  // deeper register pipelines (2-4 units) lowered the HBM rate through the
  // extra outstanding requests (32 heads x 128, 3000 rows: 19.4 us per launch
  // with one unit, 20.4-21.1 us with 2-4).
  const uint32_t ustep = nsplit * WAVES;
  uint32_t u = split + nsplit * wave;
  float4 kk[RPG], vv[RPG];
  float pp[RPG];
  if constexpr (WAVES > 1) {
    // Within that: the next unit's K rows are requested as soon as this
    // unit's scores are formed and its V rows once the weighted sum has used
    // this unit's, so the wave is never without loads in flight while it
    // computes (19.51 vs 19.69 us per config-2 fused launch).  Rows past the
    // window read zeros, so these loads need no condition.
    store_new_row();
    load_k(u * RPI, kk);
    // Every K load ahead of every V load: a wait for K never waits for V.
    __builtin_amdgcn_sched_barrier(0);
    load_v(u * RPI, vv);
    while (u < nunits) {
      const uint32_t r0 = u * RPI;
      const uint32_t un = u + ustep;
      const float alpha = score_rows(r0, kk, pp);
      load_k(un * RPI, kk);
      accumulate_rows(r0, vv, pp, alpha);
      load_v(un * RPI, vv);
      u = un;
    }
  } else {
    // u = 0 < nunits here (the window is not empty); no condition, so the
    // wait for q below does not wait for these loads.
    load_rows(u * RPI, kk, vv);
    prep_q();
    store_new_row();
    while (u < nunits) {
      const float alpha = score_rows(u * RPI, kk, pp);
      accumulate_rows(u * RPI, vv, pp, alpha);
      u += ustep;
      if (u < nunits) load_rows(u * RPI, kk, vv);
    }
  }

  // Each row's weight sits in the 4 lanes of a quad: the group's sum of
  // weights is the sum over its quads.
  float lg = lsum;
  lg += xchg<2>(lg);
  lg += xchg<3>(lg);
  if constexpr (G == 32) lg += xchg<4>(lg);

  // The WAVES x NG row groups' states (acc, m, l) go to LDS as they are, and
  // wave 0 merges them all at once (no exchanges between lanes before the
  // barrier, no more workgroup barriers after it): lane (grp, col) of wave 0
  // handles the float4 column col = lane % C4 of the head.
  constexpr int C4 = D / 4;
  constexpr int NG2 = 64 / C4;  // lane groups per wave: 2 for D = 128, 4 for D = 64
  constexpr int NST = WAVES * NG;
  st4(&s_acc[wave * NG + g][c * 4], acc);
  if (c == 0) {
    s_ml[wave * NG + g][0] = m;
    s_ml[wave * NG + g][1] = lg;
  }
  __syncthreads();
  if (wave != 0) return;
  float m_t = s_ml[0][0];
#pragma unroll
  for (int w = 1; w < NST; ++w) m_t = fmaxf(m_t, s_ml[w][0]);
  float fw[NST];
  float l_t = 0.f;
#pragma unroll
  for (int w = 0; w < NST; ++w) {
    fw[w] = fast_exp2(s_ml[w][0] - m_t);
    l_t += fw[w] * s_ml[w][1];
  }
  const int col = lane % C4, grp = lane / C4;
  float4 a4 = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int w = 0; w < NST; ++w) {
    const float4 x = *reinterpret_cast<const float4*>(&s_acc[w][col * 4]);
    a4.x += fw[w] * x.x;
    a4.y += fw[w] * x.y;
    a4.z += fw[w] * x.z;
    a4.w += fw[w] * x.w;
  }

  if (nsplit == 1) {
    if (lane < C4 && (!PAD || (uint32_t)col * 4 < dh))
      st4(outp + col * 4, make_float4(a4.x / l_t, a4.y / l_t, a4.z / l_t, a4.w / l_t));
    return;
  }

  // One-wave launches (windows of at most 64 rows) always run a single split.
  if constexpr (WAVES == 1) return;

  // Publish this split's partial (acc[D], m, l, 2 pad floats) with device-
  // coherent stores, wait for their acknowledgement, then take an arrival
  // ticket; the last split of (b, h) to arrive merges.  The wavefront fences
  // keep the compiler from reordering the atomics; s_waitcnt orders them in
  // hardware.
  constexpr int REC = D + 4;
  const size_t rec_base = ((size_t)b * p.H + h) * p.nsplit_max * REC;
  const __amdgpu_buffer_rsrc_t part_rs = coherent_rsrc(p.part + rec_base, p.nsplit_max * REC * 4);
  const uint32_t rec = split * REC * 4;  // byte offset of this split's record
  if (lane < C4) st_coherent4(part_rs, rec + col * 16, coh_f4{a4.x, a4.y, a4.z, a4.w});
  // (m, l) and the record's two pad words as one 16-byte store: whole
  // segments written through, like the rows above.
  if (lane == 0) st_coherent4(part_rs, rec + D * 4, coh_f4{m_t, l_t, 0.f, 0.f});
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  uint32_t* ctr = p.counters + (size_t)b * p.H + h;
  uint32_t ticket = 0;
  if (lane == 0) ticket = atomicAdd(ctr, 1u);
  ticket = __builtin_amdgcn_readfirstlane(ticket);
  if (ticket != nsplit - 1) return;
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  // Every other split of (b, h) has taken its ticket: the counter is reset
  // now, its round trip overlapping the merge's loads.
  if (lane == 0) atomicExch(ctr, 0u);

  // Merge: lane s < nsplit fetches split s's (m, l); lane (grp, col) fetches
  // column col of the splits grp, grp + NG2, ... in passes of kPass records,
  // all issued before the first use.
  constexpr int kPass = 4;
  float ms = -FLT_MAX, ls = 0.f;
  if (lane < (int)nsplit) {
    const coh_f4 ml = ld_coherent4(part_rs, (lane * REC + D) * 4);
    ms = ml.x;
    ls = ml.y;
  }
  float4 raw[kPass];
  auto fetch = [&](uint32_t s0) {
#pragma unroll
    for (int i = 0; i < kPass; ++i) {
      const uint32_t s = s0 + grp + NG2 * i;
      raw[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (s < nsplit) {
        const coh_f4 x = ld_coherent4(part_rs, (s * REC + col * 4) * 4);
        raw[i] = make_float4(x.x, x.y, x.z, x.w);
      }
    }
  };
  fetch(0);
  if (nsplit <= (uint32_t)(NG2 * kPass)) {
    // One pass: the splits' (m, l) broadcast from their lanes as uniform
    // values, so the weights need no exchange between lanes.
    constexpr int NSX = NG2 * kPass;
    float mu[NSX], lu[NSX];
#pragma unroll
    for (int t = 0; t < NSX; ++t) {
      mu[t] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ms), t));
      lu[t] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ls), t));
    }
    float mg = mu[0];
#pragma unroll
    for (int t = 1; t < NSX; ++t) mg = fmaxf(mg, mu[t]);
    float fl[NSX];
    float l = 0.f;
#pragma unroll
    for (int t = 0; t < NSX; ++t) {
      fl[t] = fast_exp2(mu[t] - mg);  // 0 for the lanes past nsplit (m = -FLT_MAX)
      l += fl[t] * lu[t];
    }
    float4 o4 = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < kPass; ++i) {
      float f = fl[NG2 * i];
#pragma unroll
      for (int g = 1; g < NG2; ++g) f = grp == g ? fl[g + NG2 * i] : f;
      o4.x += f * raw[i].x;
      o4.y += f * raw[i].y;
      o4.z += f * raw[i].z;
      o4.w += f * raw[i].w;
    }
    if constexpr (NG2 == 4) {
      o4.x += xchg<4>(o4.x);
      o4.y += xchg<4>(o4.y);
      o4.z += xchg<4>(o4.z);
      o4.w += xchg<4>(o4.w);
    }
    o4.x += xor32(o4.x);
    o4.y += xor32(o4.y);
    o4.z += xor32(o4.z);
    o4.w += xor32(o4.w);
    if (lane < C4 && (!PAD || (uint32_t)col * 4 < dh))
      st4(outp + col * 4, make_float4(o4.x / l, o4.y / l, o4.z / l, o4.w / l));
    return;
  }
  float mg = ms;
  mg = fmaxf(mg, xchg<0>(mg));
  mg = fmaxf(mg, xchg<1>(mg));
  mg = fmaxf(mg, xchg<2>(mg));
  mg = fmaxf(mg, xchg<3>(mg));
  mg = fmaxf(mg, xchg<4>(mg));
  mg = fmaxf(mg, xor32(mg));
  const float fl = fast_exp2(ms - mg);
  const float l = wave_sum(lane < (int)nsplit ? fl * ls : 0.f);
  float4 o4 = make_float4(0.f, 0.f, 0.f, 0.f);
  for (uint32_t s0 = 0; s0 < nsplit; s0 += NG2 * kPass) {
    if (s0 > 0) fetch(s0);
#pragma unroll
    for (int i = 0; i < kPass; ++i) {
      const uint32_t s = s0 + grp + NG2 * i;
      const float f = __shfl(fl, (int)(s < nsplit ? s : 0), 64);
      if (s < nsplit) {
        o4.x += f * raw[i].x;
        o4.y += f * raw[i].y;
        o4.z += f * raw[i].z;
        o4.w += f * raw[i].w;
      }
    }
  }
  // Sum the NG2 lane groups that hold the same column.
  if constexpr (NG2 == 4) {
    o4.x += xchg<4>(o4.x);
    o4.y += xchg<4>(o4.y);
    o4.z += xchg<4>(o4.z);
    o4.w += xchg<4>(o4.w);
  }
  o4.x += xor32(o4.x);
  o4.y += xor32(o4.y);
  o4.z += xor32(o4.z);
  o4.w += xor32(o4.w);
  if (lane < C4 && (!PAD || (uint32_t)col * 4 < dh))
    st4(outp + col * 4, make_float4(o4.x / l, o4.y / l, o4.z / l, o4.w / l));
}

}  // namespace

namespace {

struct DecodePlan {
  uint32_t chunk = 0;   // rows per split
  uint32_t nsplit = 1;  // grid x
  int waves = 1;        // waves per workgroup
};

// Chooses chunk / nsplit / waves for `units` (stream, head) pairs whose
// longest window is max_rows.
DecodePlan plan_decode(uint64_t units, uint32_t max_rows) {
  constexpr uint32_t kRpi = 16;
  DecodePlan pl;
  // Small windows (depformer) run one wave per (stream, head); long windows
  // use 4-wave workgroups and as many splits as it takes to give the chip
  // about `target` workgroups, with chunks of 64..512 rows.
  const bool small = max_rows <= 64;
  pl.waves = small ? 1 : 4;
  const uint32_t unit_rows = pl.waves * kRpi;
  if (small) {
    pl.chunk = (max_rows + kRpi - 1) / kRpi * kRpi;
    if (pl.chunk == 0) pl.chunk = kRpi;
    pl.nsplit = 1;
    return pl;
  }
  // One workgroup per CU (2-4 per CU measured slower: more partials to
  // merge, no more bytes in flight per CU).
  constexpr int chunk_max = 512, chunk_min = 64;
  const uint64_t target = (uint64_t)device_cu_count();
  uint64_t want = (target + units - 1) / units;
  if (want < 1) want = 1;
  uint64_t c = (max_rows + want - 1) / want;
  c = (c + unit_rows - 1) / unit_rows * unit_rows;
  if (c > (uint64_t)chunk_max) c = (uint64_t)chunk_max / unit_rows * unit_rows;
  if (c < (uint64_t)chunk_min) c = (uint64_t)chunk_min;
  if (c < unit_rows) c = unit_rows;
  pl.chunk = (uint32_t)c;
  pl.nsplit = (max_rows + pl.chunk - 1) / pl.chunk;
  if (pl.nsplit > (uint32_t)kMaxSplits) {
    pl.chunk = (max_rows + kMaxSplits - 1) / kMaxSplits;
    pl.chunk = (pl.chunk + unit_rows - 1) / unit_rows * unit_rows;
    pl.nsplit = (max_rows + pl.chunk - 1) / pl.chunk;
  }
  return pl;
}

// The lane layout a head dim runs on: 64 or 128 (padded for the others).
uint32_t padded_head_dim(uint32_t head_dim) { return head_dim <= 64 ? 64u : 128u; }

int check_decode(const DecodeParams& p, uint32_t batch, uint32_t head_dim) {
  if (head_dim == 0 || head_dim > 128 || head_dim % 4 != 0)
    return fail(STS_ERR_INVALID, "head_dim %u not supported (a multiple of 4 up to 128)",
                head_dim);
  if (p.len_step && (p.lens || (head_dim == 64 || head_dim == 128)))
    return fail(STS_ERR_INVALID, "per-stream window steps serve padded head dims only");
  if ((uint64_t)p.M * head_dim * sizeof(float) > 0x7FFFFFF0ull)
    return fail(STS_ERR_INVALID, "max_len %u too large for one head's buffer resource", p.M);
  if (batch > 65535u || p.H > 65535u)
    return fail(STS_ERR_INVALID, "batch (%u) and heads (%u) must be <= 65535", batch, p.H);
  if (p.group == 0 || p.H % p.group != 0)
    return fail(STS_ERR_INVALID, "query heads %u not a multiple of the K/V group %u", p.H, p.group);
  return STS_OK;
}

int launch_planned(DecodeParams p, const DecodePlan& pl, uint32_t batch, uint32_t head_dim,
                   hipStream_t stream) {
  p.chunk = pl.chunk;
  p.nsplit_max = pl.nsplit;
  p.head_dim = head_dim;
  const dim3 grid(pl.nsplit, p.H, batch);
  const bool one = pl.waves == 1;
  const dim3 block(one ? 64 : 256);
  if (head_dim == 128) {
    if (one)
      hipLaunchKernelGGL((decode_kernel<128, 1>), grid, block, 0, stream, p);
    else
      hipLaunchKernelGGL((decode_kernel<128, 4>), grid, block, 0, stream, p);
  } else if (head_dim == 64) {
    if (one)
      hipLaunchKernelGGL((decode_kernel<64, 1>), grid, block, 0, stream, p);
    else
      hipLaunchKernelGGL((decode_kernel<64, 4>), grid, block, 0, stream, p);
  } else if (head_dim < 64) {
    if (one)
      hipLaunchKernelGGL((decode_kernel<64, 1, true>), grid, block, 0, stream, p);
    else
      hipLaunchKernelGGL((decode_kernel<64, 4, true>), grid, block, 0, stream, p);
  } else {
    if (one)
      hipLaunchKernelGGL((decode_kernel<128, 1, true>), grid, block, 0, stream, p);
    else
      hipLaunchKernelGGL((decode_kernel<128, 4, true>), grid, block, 0, stream, p);
  }
  STS_HIP(hipGetLastError());
  return STS_OK;
}

// ---- allocation-free variant ------------------------------------------------
//
// Split workspace of launch_decode_noalloc, in device memory the code object
// owns (one copy per GPU, held until the process ends): words
// [0, kScratchCounters) are the arrival counters (zero between launches, as
// each launch's last arriver leaves them), the rest the partial records.
constexpr uint32_t kScratchCounters = 16384;         // 64 KiB
constexpr uint32_t kScratchPartFloats = 2u << 20;    // 8 MiB
static __device__ __align__(256) uint32_t scratch[kScratchCounters + kScratchPartFloats];

__global__ void zero_words(uint32_t* p, uint32_t n) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    p[i] = 0u;
}

std::mutex g_scratch_mutex;
std::map<int, uint32_t*> g_scratch;  // device -> address of `scratch` on it

// Device address of `scratch` on the current device.  The first call on a
// device looks it up (the array's name in host code is not a device address)
// and clears the counters with a fill kernel on `stream`.
int scratch_address(hipStream_t stream, uint32_t** out) {
  int dev = 0;
  STS_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  auto it = g_scratch.find(dev);
  if (it != g_scratch.end()) {
    *out = it->second;
    return STS_OK;
  }
  uint32_t* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(reinterpret_cast<void**>(&ptr), HIP_SYMBOL(scratch));
  if (e != hipSuccess || ptr == nullptr)
    return fail(STS_ERR_HIP, "hipGetSymbolAddress(scratch) failed: %s (%d)", hipGetErrorString(e),
                (int)e);
  hipLaunchKernelGGL(zero_words, dim3(16), dim3(256), 0, stream, ptr, kScratchCounters);
  STS_HIP(hipGetLastError());
  g_scratch[dev] = ptr;
  *out = ptr;
  return STS_OK;
}

// The split workspace of a launch planned for `units` (stream, head) pairs, or
// null when the plan has one split.
int decode_workspace(uint64_t units, uint32_t head_dim, const DecodePlan& pl, hipStream_t stream,
                     Workspace** out) {
  *out = nullptr;
  if (pl.nsplit <= 1) return STS_OK;
  // Partials and arrival counters.
  return get_workspace(stream, (size_t)units * pl.nsplit * (padded_head_dim(head_dim) + 4), units,
                       out);
}

}  // namespace

int reserve_decode(uint32_t batch, uint32_t heads, uint32_t head_dim, uint32_t max_rows,
                   hipStream_t stream) {
  const uint64_t units = (uint64_t)batch * heads;
  if (units == 0) return STS_OK;
  Workspace* ws = nullptr;
  return decode_workspace(units, head_dim, plan_decode(units, max_rows), stream, &ws);
}

int launch_decode(DecodeParams p, uint32_t batch, uint32_t head_dim, uint32_t max_rows,
                  hipStream_t stream) {
  const uint64_t units = (uint64_t)batch * p.H;
  if (units == 0) return STS_OK;
  if (int rc = check_decode(p, batch, head_dim)) return rc;
  const DecodePlan pl = plan_decode(units, max_rows);
  Workspace* ws = nullptr;
  if (int rc = decode_workspace(units, head_dim, pl, stream, &ws)) return rc;
  if (ws) {
    p.part = ws->part;
    p.counters = ws->counters;
  }
  return launch_planned(p, pl, batch, head_dim, stream);
}

int launch_decode_noalloc(DecodeParams p, uint32_t batch, uint32_t head_dim, uint32_t max_rows,
                          hipStream_t stream) {
  const uint64_t units = (uint64_t)batch * p.H;
  if (units == 0) return STS_OK;
  if (int rc = check_decode(p, batch, head_dim)) return rc;
  const DecodePlan pl = plan_decode(units, max_rows);
  if (pl.nsplit > 1) {
    const uint64_t need = units * pl.nsplit * (padded_head_dim(head_dim) + 4);
    if (need > kScratchPartFloats || units > kScratchCounters)
      return fail(STS_ERR_INVALID,
                  "this launch needs %llu floats of split records and %llu counters; the "
                  "static scratch holds %u and %u (use sts_decode_ring)",
                  (unsigned long long)need, (unsigned long long)units, kScratchPartFloats,
                  kScratchCounters);
    uint32_t* ptr = nullptr;
    if (int rc = scratch_address(stream, &ptr)) return rc;
    p.counters = ptr;
    p.part = reinterpret_cast<float*>(ptr + kScratchCounters);
  }
  return launch_planned(p, pl, batch, head_dim, stream);
}

float softmax_scale_log2(float scale) { return scale * kLog2e; }

}  // namespace sts
