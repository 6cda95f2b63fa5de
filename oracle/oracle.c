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
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
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

static void attention_wgsl_head(const float* q_reg, const float* kh, const float* vh,
                                float* out, uint32_t D, uint32_t S, float scale,
                                float* p_v /* [WG][D] */, float* p_max, float* p_sum,
                                float* sh_max, float* sh_sum, float* sh_v) {
  /* Phase 1 (:64-101): per-lane online softmax over rows tid, tid+WG, ... */
  for (uint32_t tid = 0; tid < WG; ++tid) {
    float m = -3.402823e+38f;                                     /* :71 */
    float l = 0.0f;                                               /* :72 */
    float* pv = p_v + (size_t)tid * D;
    for (uint32_t d = 0; d < D; ++d) pv[d] = 0.0f;                /* :74-76 */
    for (uint32_t pos = tid; pos < S; pos += WG) {                /* :78-100 */
      float dot = 0.0f;
      const float* kr = kh + (size_t)pos * D;
      for (uint32_t d = 0; d < D; ++d) {
        const float prod = q_reg[d] * kr[d];
        dot = dot + prod;                                         /* :82-84 */
      }
      dot = dot * scale;                                          /* :85 */
      const float old_max = m;
      m = fmaxf(m, dot);                                          /* :88 */
      const float alpha = expf(old_max - m);                      /* :89 */
      const float w = expf(dot - m);                              /* :90 */
      l = l * alpha + w;                                          /* :92 */
      const float* vr = vh + (size_t)pos * D;
      for (uint32_t d = 0; d < D; ++d) {
        const float a = pv[d] * alpha;
        const float b = w * vr[d];
        pv[d] = a + b;                                            /* :95-97 */
      }
    }
    p_max[tid] = m;
    p_sum[tid] = l;
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
                          v + (size_t)h * kv_head_stride, out + (size_t)h * D, D, S, scale,
                          p_v, scratch, scratch + WG, scratch + 2 * WG, scratch + 3 * WG,
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
