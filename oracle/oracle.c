/*
 * oracle.c -- CPU restatement of sts-web's attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py as the checker (and as the timed CPU baseline),
 * never by the product library.  Built with -ffp-contract=off so every f32
 * multiply and add rounds separately, in the order the reference writes them.
 *
 * Reference paths are relative to crates/sts-wasm/src/ of
 * idle-intelligence/sts-web.
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <float.h>
#include <pthread.h>
#include <sched.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>

/* Hot loops are compiled for several x86-64 levels and dispatched at load time
 * by the CPU's features (the library is built here and runs on another host's
 * CPU).  The floating-point order does not depend on the level: every f32
 * product and sum is rounded separately (-ffp-contract=off, no fast-math). */
#if defined(__x86_64__)
#define ORC_MULTIARCH __attribute__((target_clones("avx512f", "avx2", "default")))
#else
#define ORC_MULTIARCH
#endif
#endif

/* ------------------------------------------------------------------------ */
/* RNG                                                                        */
/* ------------------------------------------------------------------------ */

uint64_t orc_splitmix64(uint64_t seed, uint64_t i) {
  uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ULL;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

static inline float normal_sample(uint64_t seed, uint64_t j) {
  const uint64_t k = j >> 1;
  const uint64_t c0 = orc_splitmix64(seed, 2 * k);
  const uint64_t c1 = orc_splitmix64(seed, 2 * k + 1);
  const double u1 = (double)((c0 >> 40) + 1) * (1.0 / 16777216.0);
  const double u2 = (double)(c1 >> 40) * (1.0 / 16777216.0);
  const double r = sqrt(-2.0 * log(u1));
  const double th = 6.283185307179586476925286766559 * u2;
  return (float)((j & 1) ? r * sin(th) : r * cos(th));
}

void orc_fill_normal(uint64_t seed, uint64_t first, uint64_t n, float* out) {
  int64_t nn = (int64_t)n;
#pragma omp parallel for schedule(static)
  for (int64_t j = 0; j < nn; ++j) out[j] = normal_sample(seed, first + (uint64_t)j);
}

/* ------------------------------------------------------------------------ */
/* RoPE                                                                       */
/* ------------------------------------------------------------------------ */

/* model.rs:46-66.  inv_freq and the angle are f32 operations as in the
 * reference (f32 powf, f32 divide, f32 multiply); the tables hold cos and sin
 * of that f32 angle rounded to nearest f32. */
void orc_rope_tables(uint32_t head_dim, uint32_t max_seq_len, float theta,
                     float* cos_t, float* sin_t) {
  const uint32_t half = head_dim / 2;
  float* inv_freq = (float*)malloc(sizeof(float) * (half ? half : 1));
  for (uint32_t i = 0; i < half; ++i) {
    const float e = (float)(2 * i) / (float)head_dim;           /* model.rs:50 */
    inv_freq[i] = 1.0f / powf(theta, e);
  }
  for (uint32_t p = 0; p < max_seq_len; ++p) {
    const float pos = (float)p;                                   /* model.rs:53 */
    for (uint32_t j = 0; j < half; ++j) {
      const float ang = pos * inv_freq[j];                        /* model.rs:58 */
      cos_t[(size_t)p * half + j] = (float)cos((double)ang);      /* model.rs:65 */
      sin_t[(size_t)p * half + j] = (float)sin((double)ang);      /* model.rs:66 */
    }
  }
  free(inv_freq);
}

/* model.rs:79-105: interleaved pairs (x[2j], x[2j+1]) of every [b,s,h] row,
 * rotated by the table row offset+s. */
void orc_rope_apply(float* x, uint32_t B, uint32_t S, uint32_t H, uint32_t D,
                    uint32_t offset, const float* cos_t, const float* sin_t) {
  const uint32_t half = D / 2;
  for (uint32_t b = 0; b < B; ++b)
    for (uint32_t s = 0; s < S; ++s) {
      const float* c = cos_t + (size_t)(offset + s) * half;
      const float* sn = sin_t + (size_t)(offset + s) * half;
      for (uint32_t h = 0; h < H; ++h) {
        float* row = x + (((size_t)b * S + s) * H + h) * D;
        for (uint32_t j = 0; j < half; ++j) {
          const float xr = row[2 * j], xi = row[2 * j + 1];
          const float a = xr * c[j];
          const float bb = xi * sn[j];
          const float e = xr * sn[j];
          const float f = xi * c[j];
          row[2 * j] = a - bb;        /* model.rs:100 */
          row[2 * j + 1] = e + f;     /* model.rs:101 */
        }
      }
    }
}

/* ------------------------------------------------------------------------ */
/* KV append and counters                                                     */
/* ------------------------------------------------------------------------ */

/* shader_cache_write.wgsl:26-49, one loop iteration per invocation id. */
void orc_cache_write(const float* input, float* cache, uint32_t pos_offset,
                     uint32_t B, uint32_t S, uint32_t H, uint32_t D, uint32_t max_len) {
  const uint32_t total = B * S * H * D;                           /* :28 */
  for (uint32_t idx = 0; idx < total; ++idx) {
    const uint32_t d = idx % D;                                   /* :35 */
    const uint32_t rem = idx / D;
    const uint32_t h = rem % H;
    const uint32_t rem2 = rem / H;
    const uint32_t s = rem2 % S;
    const uint32_t b = rem2 / S;
    const float val = input[idx];                                 /* :44 */
    const uint32_t cache_pos = (pos_offset + s) % max_len;        /* :47 */
    const uint32_t base_out = ((b * H + h) * max_len + cache_pos) * D + d;
    cache[base_out] = val;                                        /* :49 */
  }
}

/* The grouped-query expansion of the prefill branch (model.rs:766-783):
 * k [B][nkv][S][hd] -> unsqueeze_dim(2) -> repeat_dim(2, rep) -> reshape
 * [B][nkv * rep][S][hd], so expanded head h = j * rep + r holds K/V head j.
 * `rows` is S * hd floats per head. */
void orc_gqa_expand(const float* kv, float* out, uint32_t B, uint32_t nkv, uint32_t rep,
                    uint64_t rows) {
  for (uint32_t b = 0; b < B; ++b)
    for (uint32_t j = 0; j < nkv; ++j)
      for (uint32_t r = 0; r < rep; ++r) {                         /* :772-775 */
        const float* src = kv + ((uint64_t)b * nkv + j) * rows;
        float* dst = out + (((uint64_t)b * nkv + j) * rep + r) * rows;  /* :776 reshape */
        for (uint64_t i = 0; i < rows; ++i) dst[i] = src[i];
      }
}

void orc_kv_init(orc_kv* c, uint64_t max_len) {  /* model.rs:207-219 */
  c->offset = 0;
  c->len = 0;
  c->write_pos = 0;
  c->max_len = max_len;
}

void orc_kv_advance(orc_kv* c, uint64_t n) {     /* model.rs:293-298 */
  for (uint64_t i = 0; i < n; ++i) {
    c->write_pos = (c->write_pos + 1) % c->max_len;
    c->offset += 1;
    c->len = (c->len + 1 < c->max_len) ? c->len + 1 : c->max_len;
  }
}

void orc_kv_update(orc_kv* c) {                  /* model.rs:245-251 */
  orc_kv_advance(c, 1);
}

void orc_kv_reset(orc_kv* c) {                   /* model.rs:325-331 */
  c->offset = 0;
  c->len = 0;
  c->write_pos = 0;
}

void orc_kv_rollback(orc_kv* c, uint64_t n) {    /* model.rs:352-362 */
  if (n > c->len) n = c->len;
  c->offset -= n;
  c->len -= n;
  if (c->write_pos >= n)
    c->write_pos -= n;
  else
    c->write_pos = c->max_len - (n - c->write_pos);
}

/* ------------------------------------------------------------------------ */
/* Decode attention, shader order                                             */
/* ------------------------------------------------------------------------ */

#define WG 256u /* shader_attention.wgsl:35 */

/* Interleave width of phase 1: ILANES lanes' rows are processed together so
 * that their dot products (each a sequential sum over d, as the shader's) run
 * as independent dependency chains.  Every lane's arithmetic is performed in
 * exactly the shader's order; only lanes are interleaved. */
#define ILANES 8u

/* Row `pos` of a head's window: rows are contiguous (ring == 0) or live in
 * slot (start + pos) % M of a ring of M rows. */
static inline const float* win_row(const float* h, uint32_t D, uint32_t ring, uint32_t start,
                                   uint32_t pos) {
  const uint32_t slot = ring ? (uint32_t)(((uint64_t)start + pos) % ring) : pos;
  return h + (size_t)slot * D;
}

ORC_MULTIARCH
static void attention_wgsl_head(const float* q_reg, const float* kh, const float* vh,
                                float* out, uint32_t D, uint32_t S, float scale,
                                uint32_t ring, uint32_t start,
                                float* p_v /* [WG][D] */, float* p_max, float* p_sum,
                                float* sh_max, float* sh_sum, float* sh_v) {
  /* Phase 1 (:64-101): per-lane online softmax over rows tid, tid+WG, ... */
  for (uint32_t t0 = 0; t0 < WG; t0 += ILANES) {
    float m[ILANES], l[ILANES];
    for (uint32_t j = 0; j < ILANES; ++j) {
      m[j] = -3.402823e+38f;                                      /* :71 */
      l[j] = 0.0f;                                                /* :72 */
      float* pv = p_v + (size_t)(t0 + j) * D;
      for (uint32_t d = 0; d < D; ++d) pv[d] = 0.0f;              /* :74-76 */
    }
    for (uint32_t base = t0; base < S; base += WG) {              /* :78-100 */
      const uint32_t n = S - base < ILANES ? S - base : ILANES;   /* lanes with a row */
      const float* kr[ILANES];
      float dot[ILANES];
      for (uint32_t j = 0; j < ILANES; ++j) {
        kr[j] = win_row(kh, D, ring, start, j < n ? base + j : base);
        dot[j] = 0.0f;
      }
      for (uint32_t d = 0; d < D; ++d)
        for (uint32_t j = 0; j < ILANES; ++j) {
          const float prod = q_reg[d] * kr[j][d];
          dot[j] = dot[j] + prod;                                 /* :82-84 */
        }
      for (uint32_t j = 0; j < n; ++j) {
        const float sc = dot[j] * scale;                          /* :85 */
        const float old_max = m[j];
        m[j] = fmaxf(m[j], sc);                                   /* :88 */
        const float alpha = expf(old_max - m[j]);                 /* :89 */
        const float w = expf(sc - m[j]);                          /* :90 */
        l[j] = l[j] * alpha + w;                                  /* :92 */
        const float* vr = win_row(vh, D, ring, start, base + j);
        float* pv = p_v + (size_t)(t0 + j) * D;
        for (uint32_t d = 0; d < D; ++d) {
          const float a = pv[d] * alpha;
          const float b = w * vr[d];
          pv[d] = a + b;                                          /* :95-97 */
        }
      }
    }
    for (uint32_t j = 0; j < ILANES; ++j) {
      p_max[t0 + j] = m[j];
      p_sum[t0 + j] = l[j];
    }
  }
  /* Phase 2 (:106-124): tree merge of (max, sum). */
  for (uint32_t t = 0; t < WG; ++t) {
    sh_max[t] = p_max[t];
    sh_sum[t] = p_sum[t];
  }
  for (uint32_t stride = WG / 2; stride > 0; stride >>= 1) {
    for (uint32_t tid = 0; tid < stride; ++tid) {
      const uint32_t other = tid + stride;
      const float m1 = sh_max[tid], m2 = sh_max[other];
      const float s1 = sh_sum[tid], s2 = sh_sum[other];
      const float nm = fmaxf(m1, m2);
      const float a1 = expf(m1 - nm);
      const float a2 = expf(m2 - nm);
      sh_max[tid] = nm;
      const float x = s1 * a1;
      const float y = s2 * a2;
      sh_sum[tid] = x + y;
    }
  }
  const float gmax = sh_max[0];                                   /* :126 */
  const float gsum = sh_sum[0];                                   /* :127 */
  /* Phase 3 (:133-155): rescale each lane, tree-sum each dimension. */
  for (uint32_t tid = 0; tid < WG; ++tid) {
    const float corr = expf(p_max[tid] - gmax);                   /* :133 */
    float* pv = p_v + (size_t)tid * D;
    for (uint32_t d = 0; d < D; ++d) pv[d] = pv[d] * corr;        /* :134-136 */
  }
  for (uint32_t d = 0; d < D; ++d) {
    for (uint32_t t = 0; t < WG; ++t) sh_v[t] = p_v[(size_t)t * D + d];
    for (uint32_t stride = WG / 2; stride > 0; stride >>= 1)
      for (uint32_t tid = 0; tid < stride; ++tid) sh_v[tid] = sh_v[tid] + sh_v[tid + stride];
    out[d] = sh_v[0] / gsum;                                      /* :151-153 */
  }
}

void orc_attention_wgsl(const float* q, const float* k, const float* v, float* out,
                        uint32_t H, uint32_t D, uint32_t S, float scale,
                        uint64_t kv_head_stride) {
#pragma omp parallel
  {
    float* p_v = (float*)malloc(sizeof(float) * WG * D);
    float* scratch = (float*)malloc(sizeof(float) * WG * 5);
#pragma omp for schedule(dynamic, 1)
    for (int64_t hh = 0; hh < (int64_t)H; ++hh) {
      const uint32_t h = (uint32_t)hh;
      attention_wgsl_head(q + (size_t)h * D, k + (size_t)h * kv_head_stride,
                          v + (size_t)h * kv_head_stride, out + (size_t)h * D, D, S, scale, 0,
                          0, p_v, scratch, scratch + WG, scratch + 2 * WG, scratch + 3 * WG,
                          scratch + 4 * WG);
    }
    free(p_v);
    free(scratch);
  }
}

/* Gathers window rows 0..len-1 of every head into [H][len][D] order. */
static float* gather_window(const float* c, uint32_t H, uint32_t D, uint32_t M,
                            uint32_t start, uint32_t len) {
  float* g = (float*)malloc(sizeof(float) * (size_t)H * (len ? len : 1) * D);
#pragma omp parallel for schedule(static)
  for (int64_t hh = 0; hh < (int64_t)H; ++hh)
    for (uint32_t i = 0; i < len; ++i) {
      const uint32_t slot = (uint32_t)(((uint64_t)start + i) % M);
      memcpy(g + ((size_t)hh * len + i) * D, c + ((size_t)hh * M + slot) * D,
             sizeof(float) * D);
    }
  return g;
}

void orc_attention_ring_wgsl(const float* q, const float* kc, const float* vc, float* out,
                             uint32_t H, uint32_t D, uint32_t M, uint32_t start,
                             uint32_t len, float scale) {
  float* kg = gather_window(kc, H, D, M, start, len);
  float* vg = gather_window(vc, H, D, M, start, len);
  orc_attention_wgsl(q, kg, vg, out, H, D, len, scale, (uint64_t)len * D);
  free(kg);
  free(vg);
}

/* A temporal decode frame on the CPU: decode attention of every (layer, head)
 * over its ring window, in the shader's order, parallel over (layer, head) --
 * the CPU path a host without WebGPU would run for shader_attention.wgsl.
 * q[l], out[l]: [H][D]; kc[l], vc[l]: [H][M][D]; window of layer l: rows
 * 0..lens[l]-1 in slots (starts[l] + i) % M. */
void orc_decode_frame_wgsl(const float* const* q, const float* const* kc,
                           const float* const* vc, float* const* out, uint32_t L, uint32_t H,
                           uint32_t D, uint32_t M, const uint32_t* starts, const uint32_t* lens,
                           float scale) {
#pragma omp parallel
  {
    float* p_v = (float*)malloc(sizeof(float) * WG * D);
    float* scratch = (float*)malloc(sizeof(float) * WG * 5);
#pragma omp for schedule(dynamic, 1)
    for (int64_t t = 0; t < (int64_t)L * H; ++t) {
      const uint32_t l = (uint32_t)(t / H), h = (uint32_t)(t % H);
      attention_wgsl_head(q[l] + (size_t)h * D, kc[l] + (size_t)h * M * D,
                          vc[l] + (size_t)h * M * D, out[l] + (size_t)h * D, D, lens[l], scale, M,
                          starts[l] % M, p_v, scratch, scratch + WG, scratch + 2 * WG,
                          scratch + 3 * WG, scratch + 4 * WG);
    }
    free(p_v);
    free(scratch);
  }
}

/* ------------------------------------------------------------------------ */
/* Closed form in double                                                      */
/* ------------------------------------------------------------------------ */

static void softmax_head_f64(const float* qh, const float* kh, const float* vh, double* out,
                             uint32_t D, uint32_t M, uint32_t start, uint32_t n, double scale,
                             double* s /* [n] */) {
  double mx = -INFINITY;
  for (uint32_t i = 0; i < n; ++i) {
    const float* kr = kh + (size_t)((start + (uint64_t)i) % M) * D;
    double dot = 0.0;
    for (uint32_t d = 0; d < D; ++d) dot += (double)qh[d] * (double)kr[d];
    s[i] = dot * scale;
    if (s[i] > mx) mx = s[i];
  }
  double den = 0.0;
  for (uint32_t i = 0; i < n; ++i) {
    s[i] = exp(s[i] - mx);
    den += s[i];
  }
  for (uint32_t d = 0; d < D; ++d) out[d] = 0.0;
  for (uint32_t i = 0; i < n; ++i) {
    const float* vr = vh + (size_t)((start + (uint64_t)i) % M) * D;
    for (uint32_t d = 0; d < D; ++d) out[d] += s[i] * (double)vr[d];
  }
  for (uint32_t d = 0; d < D; ++d) out[d] /= den;
}

void orc_attention_ring_f64(const float* q, const float* kc, const float* vc, double* out,
                            uint32_t H, uint32_t D, uint32_t M, uint32_t start,
                            uint32_t len, double scale) {
#pragma omp parallel
  {
    double* s = (double*)malloc(sizeof(double) * (len ? len : 1));
#pragma omp for schedule(static)
    for (int64_t hh = 0; hh < (int64_t)H; ++hh) {
      const size_t h = (size_t)hh;
      if (len == 0) {
        for (uint32_t d = 0; d < D; ++d) out[h * D + d] = 0.0;
        continue;
      }
      softmax_head_f64(q + h * D, kc + h * M * D, vc + h * M * D, out + h * D, D, M, start,
                       len, scale, s);
    }
    free(s);
  }
}

void orc_prefill_f64(const float* q, const float* kc, const float* vc, double* out,
                     uint32_t S, uint32_t H, uint32_t D, uint32_t M, uint32_t start,
                     uint32_t len, double scale) {
  const int64_t total = (int64_t)S * H;
#pragma omp parallel
  {
    double* s = (double*)malloc(sizeof(double) * (len ? len : 1));
#pragma omp for schedule(dynamic, 4)
    for (int64_t t = 0; t < total; ++t) {
      const uint32_t i = (uint32_t)(t / H), h = (uint32_t)(t % H);
      const uint32_t n = len - S + i + 1; /* window rows 0..w_i */
      softmax_head_f64(q + ((size_t)i * H + h) * D, kc + (size_t)h * M * D,
                       vc + (size_t)h * M * D, out + ((size_t)i * H + h) * D, D, M, start,
                       n, scale, s);
    }
    free(s);
  }
}

void orc_prefill_seq_wgsl(const float* q, const float* kc, const float* vc, float* out,
                          uint32_t S, uint32_t H, uint32_t D, uint32_t M, uint32_t start,
                          uint32_t len, float scale) {
  float* kg = gather_window(kc, H, D, M, start, len);
  float* vg = gather_window(vc, H, D, M, start, len);
  for (uint32_t i = 0; i < S; ++i) {
    const uint32_t n = len - S + i + 1;
    orc_attention_wgsl(q + (size_t)i * H * D, kg, vg, out + (size_t)i * H * D, H, D, n, scale,
                       (uint64_t)len * D);
  }
  free(kg);
  free(vg);
}

/* ------------------------------------------------------------------------ */
/* Q4_K                                                                       */
/* ------------------------------------------------------------------------ */

enum { QK_K = 256, Q4K_BYTES = 144 };

/* WGSL unpack2x16float, which every Q4_K shader uses for d and dmin
 * (shader_q4k_matvec.wgsl:82): exact IEEE binary16 -> binary32.  Subnormals
 * are m * 2^-24 exactly; exponent 31 gives inf or NaN.  (The CPU helper
 * gguf.rs:65-88 f16_to_f32 returns half the value for subnormals; it is not
 * on the matvec path.) */
float orc_f16_to_f32(uint16_t bits) {
  const uint32_t sign = (uint32_t)(bits >> 15) << 31;
  const uint32_t exponent = (bits >> 10) & 0x1Fu;
  const uint32_t mantissa = bits & 0x3FFu;
  uint32_t out;
  if (exponent == 0) {
    float f = ldexpf((float)mantissa, -24);
    memcpy(&out, &f, 4);
    out |= sign;
  } else if (exponent == 31) {
    out = sign | (0xFFu << 23) | (mantissa << 13);
  } else {
    out = sign | ((exponent - 15u + 127u) << 23) | (mantissa << 13);
  }
  float f;
  memcpy(&f, &out, 4);
  return f;
}

void orc_f16_to_f32_n(const uint16_t* bits, float* out, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) out[i] = orc_f16_to_f32(bits[i]);
}

/* Round-to-nearest-even f32 -> f16 (what numpy's astype(np.float16) does). */
uint16_t orc_f32_to_f16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t absu = u & 0x7FFFFFFFu;
  if (absu >= 0x7F800000u) /* inf or NaN */
    return (uint16_t)(sign | 0x7C00u | (absu > 0x7F800000u ? 0x200u : 0u));
  if (absu >= 0x477FF000u) /* rounds to >= 65520: overflow to inf */
    return (uint16_t)(sign | 0x7C00u);
  if (absu < 0x38800000u) { /* below 2^-14: f16 subnormal or zero */
    if (absu < 0x33000000u) return (uint16_t)sign; /* below 2^-25: rounds to 0 */
    const uint32_t e = absu >> 23;                 /* biased f32 exponent 102..112 */
    const uint32_t mant = (absu & 0x7FFFFFu) | 0x800000u;
    const uint32_t shift = 126u - e;               /* 14..24 */
    uint32_t h = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
  }
  uint32_t h = ((absu >> 13) - (112u << 10)); /* rebias exponent, keep 10 mantissa bits */
  const uint32_t rem = absu & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
  return (uint16_t)(sign | h);
}

/* shader_q4k_matvec.wgsl:85-113. */
void orc_q4k_scale_min(const uint8_t* q, uint32_t j, uint32_t* sc, uint32_t* mn) {
  if (j < 4) {
    *sc = q[j] & 63u;
    *mn = q[j + 4] & 63u;
  } else {
    *sc = (q[j + 4] & 0xFu) | ((uint32_t)(q[j - 4] >> 6) << 4);
    *mn = (uint32_t)(q[j + 4] >> 4) | ((uint32_t)(q[j] >> 6) << 4);
  }
}

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* shader_q4k_matvec.wgsl:117-136: per iteration `it`, sub-blocks 2it (low
 * nibbles) and 2it+1 (high nibbles) of qs bytes it*32 .. it*32+31. */
void orc_q4k_dequant(const uint8_t* blocks, uint32_t N, uint32_t K, float* w) {
  const uint32_t nb = K / QK_K;
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < (int64_t)N; ++n) {
    for (uint32_t blk = 0; blk < nb; ++blk) {
      const uint8_t* b = blocks + ((size_t)n * nb + blk) * Q4K_BYTES;
      const float d = orc_f16_to_f32(rd16(b));
      const float dmin = orc_f16_to_f32(rd16(b + 2));
      float* out = w + (size_t)n * K + (size_t)blk * QK_K;
      for (uint32_t it = 0; it < 4; ++it) {
        uint32_t s0, m0, s1, m1;
        orc_q4k_scale_min(b + 4, 2 * it, &s0, &m0);
        orc_q4k_scale_min(b + 4, 2 * it + 1, &s1, &m1);
        const float d1 = d * (float)s0, mm1 = dmin * (float)m0;
        const float d2 = d * (float)s1, mm2 = dmin * (float)m1;
        for (uint32_t j = 0; j < 32; ++j) {
          const uint8_t byte = b[16 + it * 32 + j];
          out[it * 64 + j] = (float)(byte & 0xF) * d1 - mm1;
          out[it * 64 + 32 + j] = (float)(byte >> 4) * d2 - mm2;
        }
      }
    }
  }
}

/* scripts/quantize.py:162-253: per 32-weight sub-block, scale = (max-min)/15
 * and min value = -min; d = max scale / 63, dmin = max min value / 63 (1.0
 * when zero), both rounded to f16; 6-bit sub-block scales/mins and 4-bit
 * quants by round-half-even (np.round) and clipping, all in f32. */
void orc_q4k_quantize(const float* x, uint32_t N, uint32_t K, uint8_t* blocks) {
  const uint32_t nb = K / QK_K;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < (int64_t)N * nb; ++r) {
    const float* v = x + (size_t)r * QK_K;
    uint8_t* o = blocks + (size_t)r * Q4K_BYTES;
    float raw_scale[8], raw_min[8], max_scale = 0.f, max_min = 0.f;
    for (int j = 0; j < 8; ++j) {
      float mn = v[j * 32], mx = v[j * 32];
      for (int i = 1; i < 32; ++i) {
        mn = fminf(mn, v[j * 32 + i]);
        mx = fmaxf(mx, v[j * 32 + i]);
      }
      raw_scale[j] = mx > mn ? (mx - mn) / 15.0f : 0.f;
      raw_min[j] = -mn;
      if (j == 0 || raw_scale[j] > max_scale) max_scale = raw_scale[j];
      if (j == 0 || raw_min[j] > max_min) max_min = raw_min[j];
    }
    const uint16_t d16 = orc_f32_to_f16(max_scale > 0.f ? max_scale / 63.0f : 1.0f);
    const uint16_t dm16 = orc_f32_to_f16(max_min > 0.f ? max_min / 63.0f : 1.0f);
    const float d = orc_f16_to_f32(d16), dmin = orc_f16_to_f32(dm16);
    uint8_t sc[8], m[8];
    for (int j = 0; j < 8; ++j) {
      float a = d > 0.f ? nearbyintf(raw_scale[j] / d) : 0.f;
      float b = dmin > 0.f ? nearbyintf(raw_min[j] / dmin) : 0.f;
      a = a < 0.f ? 0.f : (a > 63.f ? 63.f : a);
      b = b < 0.f ? 0.f : (b > 63.f ? 63.f : b);
      sc[j] = (uint8_t)a;
      m[j] = (uint8_t)b;
    }
    o[0] = (uint8_t)(d16 & 0xFF);
    o[1] = (uint8_t)(d16 >> 8);
    o[2] = (uint8_t)(dm16 & 0xFF);
    o[3] = (uint8_t)(dm16 >> 8);
    uint8_t* sb = o + 4;
    for (int j = 0; j < 4; ++j) {
      sb[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
      sb[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
      sb[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4));
    }
    uint8_t q[8][32];
    for (int j = 0; j < 8; ++j) {
      const float es = d * (float)sc[j], em = dmin * (float)m[j];
      for (int i = 0; i < 32; ++i) {
        float t = es > 0.f ? nearbyintf((v[j * 32 + i] + em) / es) : 0.f;
        t = t < 0.f ? 0.f : (t > 15.f ? 15.f : t);
        q[j][i] = (uint8_t)t;
      }
    }
    for (int it = 0; it < 4; ++it)
      for (int i = 0; i < 32; ++i)
        o[16 + it * 32 + i] = (uint8_t)((q[2 * it][i] & 0xF) | ((q[2 * it + 1][i] & 0xF) << 4));
  }
}

static inline float dot4(float a0, float a1, float a2, float a3, const float* b) {
  return a0 * b[0] + a1 * b[1] + a2 * b[2] + a3 * b[3];
}

/* shader_q4k_matvec.wgsl:48-356 (the structure is the same for the chunked
 * shared-memory input: chunks only move where x is read from). */
void orc_q4k_matvec_wgsl(const uint8_t* blocks, const float* x, float* y, uint32_t B,
                         uint32_t K, uint32_t N) {
  const uint32_t nb = K / QK_K;
#pragma omp parallel for schedule(static)
  for (int64_t bn = 0; bn < (int64_t)B * N; ++bn) {
    const uint32_t b = (uint32_t)(bn / N), n = (uint32_t)(bn % N);
    const float* xb = x + (size_t)b * K;
    float acc = 0.f;
    for (uint32_t blk = 0; blk < nb; ++blk) {
      const uint8_t* p = blocks + ((size_t)n * nb + blk) * Q4K_BYTES;
      const float d = orc_f16_to_f32(rd16(p));
      const float dmin = orc_f16_to_f32(rd16(p + 2));
      for (uint32_t it = 0; it < 4; ++it) {
        uint32_t s0, m0, s1, m1;
        orc_q4k_scale_min(p + 4, 2 * it, &s0, &m0);
        orc_q4k_scale_min(p + 4, 2 * it + 1, &s1, &m1);
        const float d1 = d * (float)s0, mm1 = dmin * (float)m0;
        const float d2 = d * (float)s1, mm2 = dmin * (float)m1;
        const float* xlo = xb + blk * QK_K + it * 64;
        const float* xhi = xlo + 32;
        for (uint32_t w = 0; w < 8; ++w) {
          const uint8_t* q = p + 16 + it * 32 + w * 4;
          acc += dot4((float)(q[0] & 0xF) * d1 - mm1, (float)(q[1] & 0xF) * d1 - mm1,
                      (float)(q[2] & 0xF) * d1 - mm1, (float)(q[3] & 0xF) * d1 - mm1, xlo + w * 4);
          acc += dot4((float)(q[0] >> 4) * d2 - mm2, (float)(q[1] >> 4) * d2 - mm2,
                      (float)(q[2] >> 4) * d2 - mm2, (float)(q[3] >> 4) * d2 - mm2, xhi + w * 4);
        }
      }
    }
    y[(size_t)b * N + n] = acc;
  }
}

void orc_q4k_matvec_f64(const uint8_t* blocks, const float* x, double* y, uint32_t B,
                        uint32_t K, uint32_t N) {
  float* w = (float*)malloc(sizeof(float) * (size_t)N * K);
  orc_q4k_dequant(blocks, N, K, w);
#pragma omp parallel for schedule(static)
  for (int64_t bn = 0; bn < (int64_t)B * N; ++bn) {
    const uint32_t b = (uint32_t)(bn / N), n = (uint32_t)(bn % N);
    double acc = 0.0;
    for (uint32_t k = 0; k < K; ++k) acc += (double)w[(size_t)n * K + k] * (double)x[(size_t)b * K + k];
    y[bn] = acc;
  }
  free(w);
}

/* ---- depformer step chain -------------------------------------------------- */

void orc_rmsnorm_wgsl(const float* x, const float* alpha, float* out, uint32_t D, float eps) {
  float part[256];
  for (uint32_t t = 0; t < 256; ++t) { /* shader_rmsnorm.wgsl:47-57 */
    float acc = 0.f;
    for (uint32_t i = t; i < D; i += 256) acc += x[i] * x[i];
    part[t] = acc;
  }
  for (uint32_t half = 128; half >= 2; half >>= 1) /* :63-76 */
    for (uint32_t t = 0; t < half; ++t) part[t] += part[t + half];
  const float sum = part[0] + part[1];            /* :77 */
  const float rms = sqrtf(sum / (float)D + eps);  /* :81 */
  const float inv = 1.0f / rms;                   /* :82 */
  for (uint32_t i = 0; i < D; ++i) out[i] = x[i] * inv * alpha[i]; /* :90 */
}

void orc_swiglu(const float* in, float* out, uint32_t F) {
  for (uint32_t i = 0; i < F; ++i) {
    const float gate = in[i], value = in[F + i];
    out[i] = gate / (1.0f + expf(-gate)) * value; /* shader_swiglu.wgsl:30-34 */
  }
}

/* shader_embed_q4.wgsl:34-56: an Inf/NaN scale reads as 0, otherwise exact. */
static float q4_0_scale(uint16_t bits) {
  if (((bits >> 10) & 0x1F) == 0x1F) return 0.f;
  return orc_f16_to_f32(bits);
}

void orc_embed_q4_0(const uint8_t* table, uint32_t vocab, uint32_t dim, uint32_t token,
                    float* out) {
  if (token >= vocab) { /* :76-79 */
    memset(out, 0, sizeof(float) * dim);
    return;
  }
  const size_t row_bytes = (size_t)(dim / 32) * 18;
  const uint8_t* row = table + (size_t)token * row_bytes;
  for (uint32_t e = 0; e < dim; ++e) {
    const uint8_t* blk = row + (e / 32) * 18; /* :82-87 */
    const float scale = q4_0_scale(rd16(blk));
    const uint32_t pos = e % 32;
    const uint32_t nib = pos < 16 ? (blk[2 + pos] & 0xF) : (blk[2 + pos - 16] >> 4); /* :95-102 */
    out[e] = ((float)nib - 8.0f) * scale; /* :105 */
  }
}

uint32_t orc_sample_topk_wgsl(float* logits, uint32_t V, uint32_t top_k, float temperature,
                              float penalty, float rand, const uint32_t* penalty_tokens,
                              uint32_t num_penalty) {
  return orc_sample_topk_wgsl_ex(logits, V, top_k, temperature, penalty, rand, penalty_tokens,
                                 num_penalty, NULL, NULL);
}

/* As orc_sample_topk_wgsl; for top_k > 1 also stores the sorted slots' logit
 * indices and the running totals of the draw (top_k each) when given. */
uint32_t orc_sample_topk_wgsl_ex(float* logits, uint32_t V, uint32_t top_k, float temperature,
                                 float penalty, float rand, const uint32_t* penalty_tokens,
                                 uint32_t num_penalty, uint32_t* idx_out, float* cum_out) {
  /* Repetition penalty, shader_sample_topk.wgsl:56-69. */
  for (uint32_t p = 0; p < num_penalty; ++p) {
    const uint32_t tok = penalty_tokens[p];
    int seen = 0;
    for (uint32_t q = 0; q < p; ++q) seen |= penalty_tokens[q] == tok;
    if (seen || tok >= V) continue;
    const float val = logits[tok];
    logits[tok] = val > 0.f ? val / penalty : val * penalty;
  }
  /* Temperature and per-lane maxima, :72-88 (lane t takes t, t+256, ...). */
  float lmax[256];
  uint32_t lidx[256];
  for (uint32_t t = 0; t < 256; ++t) {
    lmax[t] = -3.402823466e+38f;
    lidx[t] = 0;
  }
  for (uint32_t i = 0; i < V; ++i) {
    logits[i] = logits[i] / temperature;
    const uint32_t t = i % 256;
    if (logits[i] > lmax[t]) {
      lmax[t] = logits[i];
      lidx[t] = i;
    }
  }
  for (uint32_t half = 128; half > 0; half >>= 1) /* :95-106 */
    for (uint32_t t = 0; t < half; ++t)
      if (lmax[t + half] > lmax[t]) {
        lmax[t] = lmax[t + half];
        lidx[t] = lidx[t + half];
      }
  if (top_k <= 1) return lidx[0]; /* :112-117 */

  /* Thread 0's selection of the top K, :134-178. */
  const uint32_t K = top_k;
  float* vals = (float*)malloc(sizeof(float) * K);
  uint32_t* idxs = (uint32_t*)malloc(sizeof(uint32_t) * K);
  for (uint32_t j = 0; j < K; ++j) {
    vals[j] = -3.402823466e+38f;
    idxs[j] = 0;
  }
  const uint32_t first_k = K < V ? K : V;
  for (uint32_t j = 0; j < first_k; ++j) {
    vals[j] = logits[j];
    idxs[j] = j;
  }
  float min_v = vals[0];
  uint32_t min_p = 0;
  for (uint32_t j = 1; j < first_k; ++j)
    if (vals[j] < min_v) {
      min_v = vals[j];
      min_p = j;
    }
  for (uint32_t j = K; j < V; ++j) {
    const float val = logits[j];
    if (val > min_v) {
      vals[min_p] = val;
      idxs[min_p] = j;
      min_v = vals[0];
      min_p = 0;
      for (uint32_t m = 1; m < K; ++m)
        if (vals[m] < min_v) {
          min_v = vals[m];
          min_p = m;
        }
    }
  }
  /* Insertion sort, descending, :184-196. */
  for (uint32_t si = 1; si < K; ++si) {
    const float kv = vals[si];
    const uint32_t ki = idxs[si];
    int sj = (int)si - 1;
    while (sj >= 0 && vals[sj] < kv) {
      vals[sj + 1] = vals[sj];
      idxs[sj + 1] = idxs[sj];
      --sj;
    }
    vals[sj + 1] = kv;
    idxs[sj + 1] = ki;
  }
  /* Softmax over the K and the cumulative draw, :198-221.  WGSL's exp has an
   * implementation-defined error bound (several ulp), so the reference fixes no
   * particular rounding of it; exp(v - max) is taken here correctly rounded to
   * f32 (exp in f64, then rounded), which the GPU sampler computes the same
   * way, so the draw is reproducible bit for bit. */
  float max_v = vals[0];
  for (uint32_t j = 1; j < K; ++j)
    if (vals[j] > max_v) max_v = vals[j];
  float sum = 0.f;
  for (uint32_t j = 0; j < K; ++j) {
    vals[j] = (float)exp((double)(vals[j] - max_v));
    sum = sum + vals[j];
  }
  float cum = 0.f;
  uint32_t tok = idxs[K - 1];
  int found = 0;
  for (uint32_t j = 0; j < K; ++j) {
    cum = cum + vals[j] / sum;
    if (cum_out) cum_out[j] = cum;
    if (idx_out) idx_out[j] = idxs[j];
    if (!found && rand < cum) {
      tok = idxs[j];
      found = 1;
      if (!cum_out && !idx_out) break;
    }
  }
  free(vals);
  free(idxs);
  return tok;
}

void orc_depformer_generate(const orc_depformer_cfg* c, const orc_depformer_weights* w,
                            const float* temporal_hidden, uint32_t text_token, uint32_t top_k,
                            float temperature, float penalty, const float* rand,
                            const uint32_t* penalty_tokens, const uint32_t* num_penalty,
                            uint32_t* tokens, float* logits_out, float* hidden_out) {
  const uint32_t D = c->dim, H = c->num_heads, hd = c->dim / c->num_heads, M = c->kv_max_len;
  const uint32_t F = c->ffn, S = c->num_steps;
  float* proj = (float*)malloc(sizeof(float) * (size_t)S * D);
  float* h = (float*)malloc(sizeof(float) * D);
  float* h2 = (float*)malloc(sizeof(float) * D);
  float* emb = (float*)malloc(sizeof(float) * D);
  float* nrm = (float*)malloc(sizeof(float) * D);
  float* qkv = (float*)malloc(sizeof(float) * 3 * D);
  float* att = (float*)malloc(sizeof(float) * D);
  float* gate = (float*)malloc(sizeof(float) * 2 * F);
  float* sw = (float*)malloc(sizeof(float) * F);
  float* logits = (float*)malloc(sizeof(float) * c->out_vocab);
  float* kc = (float*)calloc((size_t)c->num_layers * H * M * hd, sizeof(float));
  float* vc = (float*)calloc((size_t)c->num_layers * H * M * hd, sizeof(float));

  /* Phase 1: projected[step] = input_proj[step] . temporal_hidden (:953-983). */
  for (uint32_t st = 0; st < S; ++st)
    orc_q4k_matvec_wgsl(w->input_proj[st], temporal_hidden, proj + (size_t)st * D, 1,
                        c->temporal_dim, D);
  uint32_t prev = text_token;
  for (uint32_t st = 0; st < S; ++st) {
    /* Embedding lookup and add (:988-1057). */
    if (st == 0) {
      orc_embed_q4_0(w->text_emb, c->text_emb_vocab, D, prev, emb);
    } else {
      const uint32_t e = st - 1 < c->num_audio_emb - 1 ? st - 1 : c->num_audio_emb - 1;
      orc_embed_q4_0(w->audio_emb[e], c->audio_emb_vocab, D, prev, emb);
    }
    for (uint32_t i = 0; i < D; ++i) h[i] = proj[(size_t)st * D + i] + emb[i];
    for (uint32_t l = 0; l < c->num_layers; ++l) {
      const size_t wi = (size_t)l * S + st;
      float* kl = kc + (size_t)l * H * M * hd;
      float* vl = vc + (size_t)l * H * M * hd;
      orc_rmsnorm_wgsl(h, w->norm1_alpha[l], nrm, D, c->rms_eps);          /* :1069-1095 */
      orc_q4k_matvec_wgsl(w->attn_in_proj[wi], nrm, qkv, 1, D, 3 * D);     /* :1097-1119 */
      orc_cache_write(qkv + D, kl, st, 1, 1, H, hd, M);                    /* :1121-1150 */
      orc_cache_write(qkv + 2 * D, vl, st, 1, 1, H, hd, M);                /* :1152-1176 */
      orc_attention_wgsl(qkv, kl, vl, att, H, hd, st + 1, c->attn_scale,
                         (uint64_t)M * hd);                                /* :1178-1209 */
      orc_q4k_matvec_wgsl(w->attn_out_proj[wi], att, h2, 1, D, D);         /* :1211-1233 */
      for (uint32_t i = 0; i < D; ++i) h2[i] = h2[i] + h[i];               /* :1235-1257 */
      orc_rmsnorm_wgsl(h2, w->norm2_alpha[l], nrm, D, c->rms_eps);         /* :1262-1282 */
      orc_q4k_matvec_wgsl(w->ffn_linear_in[wi], nrm, gate, 1, D, 2 * F);   /* :1284-1306 */
      orc_swiglu(gate, sw, F);                                             /* :1308-1332 */
      orc_q4k_matvec_wgsl(w->ffn_linear_out[wi], sw, h, 1, F, D);          /* :1334-1356 */
      for (uint32_t i = 0; i < D; ++i) h[i] = h[i] + h2[i];                /* :1358-1382 */
    }
    if (hidden_out) memcpy(hidden_out + (size_t)st * D, h, sizeof(float) * D);
    orc_q4k_matvec_wgsl(w->output_linear[st], h, logits, 1, D, c->out_vocab); /* :1385-1409 */
    if (logits_out) memcpy(logits_out + (size_t)st * c->out_vocab, logits, sizeof(float) * c->out_vocab);
    prev = orc_sample_topk_wgsl(logits, c->out_vocab, top_k, temperature, penalty, rand[st],
                                penalty_tokens + (size_t)st * 30, num_penalty[st]); /* :1411-1439 */
    tokens[st] = prev;
  }
  free(proj); free(h); free(h2); free(emb); free(nrm); free(qkv); free(att);
  free(gate); free(sw); free(logits); free(kc); free(vc);
}

int orc_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void orc_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* Timing support for the CPU baseline: OpenMP thread t of the next n-thread
 * teams runs on CPU cpus[t] only (pin = 1), or on any of cpus[0..n) again
 * (pin = 0).  libgomp keeps its team threads between parallel regions, so the
 * binding holds for the regions that follow.  Returns the number of threads
 * whose binding failed. */
int orc_bind_threads(const int* cpus, int n, int pin) {
  int failed = 0;
#if defined(_OPENMP) && defined(__linux__)
  if (n <= 0) return 0;
  omp_set_num_threads(n);
#pragma omp parallel reduction(+ : failed)
  {
    cpu_set_t set;
    CPU_ZERO(&set);
    const int t = omp_get_thread_num();
    if (pin) {
      CPU_SET(cpus[t % n], &set);
    } else {
      for (int i = 0; i < n; ++i) CPU_SET(cpus[i], &set);
    }
    failed += pthread_setaffinity_np(pthread_self(), sizeof set, &set) != 0;
  }
#else
  (void)cpus;
  (void)n;
  (void)pin;
#endif
  return failed;
}
