// api.cpp -- the extern "C" entry points of include/sts_attn.h.
//
// Host-side argument checks, the KV cache handle (KVCache / LayerCaches of
// crates/sts-wasm/src/model.rs:195-411) and the RoPE table handle
// (model.rs:38-122).  Kernels live in decode.hip, append.hip, prefill.hip.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <new>
#include <vector>

#include "append.hpp"
#include "common.hpp"
#include "decode.hpp"
#include "errors.hpp"
#include "prefill.hpp"
#include "q4k.hpp"

using sts::fail;

struct sts_rope {
  uint32_t head_dim = 0;
  uint32_t max_seq_len = 0;
  float* cos_t = nullptr;  // device [max_seq_len][head_dim/2]
  float* sin_t = nullptr;
};

struct sts_kv_cache {
  uint64_t max_len = 0, heads = 0, head_dim = 0;
  uint64_t q_heads = 0;  // query heads of q/out (a multiple of heads: GQA)
  uint64_t offset = 0, len = 0, write_pos = 0;
  uint64_t batch = 0;
  uint32_t flags = 0;
  float* k = nullptr;
  float* v = nullptr;
  uint16_t* k16 = nullptr;  // bf16 mirror (STS_KV_BF16_MIRROR)
  uint16_t* v16 = nullptr;
};

namespace {

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Any multiple of 4 up to 128 (shader_attention.wgsl:36 takes head_dim <= 128);
// 64 and 128 have their own kernels, the others run padded ones.
int check_head_dim(uint64_t d) {
  if (d == 0 || d > 128 || d % 4 != 0)
    return fail(STS_ERR_INVALID, "head_dim %llu not supported (a multiple of 4 up to 128)",
                (unsigned long long)d);
  return STS_OK;
}

// KVCache::advance (model.rs:293-298), n steps of the one-step update.
void kv_advance(sts_kv_cache* c, uint64_t n) {
  if (n >= c->max_len) {
    // Whole-ring advance: the same end state as n single steps.
    c->write_pos = (c->write_pos + n) % c->max_len;
    c->offset += n;
    c->len = c->max_len;
    return;
  }
  c->write_pos = (c->write_pos + n) % c->max_len;
  c->offset += n;
  c->len = (c->len + n < c->max_len) ? c->len + n : c->max_len;
}

// Oldest valid slot of the logical window.
uint64_t kv_start(const sts_kv_cache* c) {
  return (c->write_pos + c->max_len - c->len) % c->max_len;
}

int kv_ensure(sts_kv_cache* c, uint64_t batch, hipStream_t stream) {
  if (c->k) {
    if (batch != c->batch)
      return fail(STS_ERR_STATE, "cache allocated for batch %llu, called with batch %llu",
                  (unsigned long long)c->batch, (unsigned long long)batch);
    return STS_OK;
  }
  if (batch == 0) return fail(STS_ERR_INVALID, "batch must be >= 1");
  // The lazy allocation must not be recorded into a HIP graph (its zero fill
  // would be a memset node, and the graph would own nothing it addresses).
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  STS_HIP(hipStreamIsCapturing(stream, &cap));
  if (cap != hipStreamCaptureStatusNone)
    return fail(STS_ERR_STATE,
                "the cache's first use allocates its buffers, which cannot happen while the "
                "stream is being captured; allocate it first (sts_kv_ensure_allocated)");
  const uint64_t n = batch * c->heads * c->max_len * c->head_dim;
  if (hipMalloc(&c->k, n * sizeof(float)) != hipSuccess) {
    c->k = nullptr;
    return fail(STS_ERR_NOMEM, "K cache allocation of %llu bytes failed",
                (unsigned long long)(n * sizeof(float)));
  }
  if (hipMalloc(&c->v, n * sizeof(float)) != hipSuccess) {
    (void)hipFree(c->k);
    c->k = nullptr;
    c->v = nullptr;
    return fail(STS_ERR_NOMEM, "V cache allocation of %llu bytes failed",
                (unsigned long long)(n * sizeof(float)));
  }
  if (c->flags & STS_KV_BF16_MIRROR) {
    if (hipMalloc(&c->k16, n * sizeof(uint16_t)) != hipSuccess ||
        hipMalloc(&c->v16, n * sizeof(uint16_t)) != hipSuccess) {
      for (void* ptr : {(void*)c->k, (void*)c->v, (void*)c->k16, (void*)c->v16})
        if (ptr) (void)hipFree(ptr);
      c->k = c->v = nullptr;
      c->k16 = c->v16 = nullptr;
      return fail(STS_ERR_NOMEM, "bf16 mirror allocation of %llu bytes failed",
                  (unsigned long long)(2 * n * sizeof(uint16_t)));
    }
    STS_HIP(hipMemsetAsync(c->k16, 0, n * sizeof(uint16_t), stream));
    STS_HIP(hipMemsetAsync(c->v16, 0, n * sizeof(uint16_t), stream));
  }
  // Zero-filled like Tensor::zeros (model.rs:272-279).
  STS_HIP(hipMemsetAsync(c->k, 0, n * sizeof(float), stream));
  STS_HIP(hipMemsetAsync(c->v, 0, n * sizeof(float), stream));
  c->batch = batch;
  return STS_OK;
}

void kv_free(sts_kv_cache* c) {
  for (void* ptr : {(void*)c->k, (void*)c->v, (void*)c->k16, (void*)c->v16})
    if (ptr) (void)hipFree(ptr);
  c->k = c->v = nullptr;
  c->k16 = c->v16 = nullptr;
}

}  // namespace

extern "C" {

/* ---------------------------------------------------------------------- */
/* Stateless ops                                                            */
/* ---------------------------------------------------------------------- */

int sts_fused_attention(const float* q, const float* k, const float* v, float* out,
                        uint32_t num_heads, uint32_t head_dim, uint32_t seq_len, float scale,
                        uint64_t kv_head_stride, void* stream) {
  sts::clear_error();
  STS_CHECK(q && k && v && out, "null pointer argument");
  if (int rc = check_head_dim(head_dim)) return rc;
  STS_CHECK(num_heads >= 1, "num_heads must be >= 1");
  STS_CHECK(seq_len >= 1, "seq_len must be >= 1 (got 0)");
  STS_CHECK(kv_head_stride >= (uint64_t)seq_len * head_dim || num_heads == 1,
            "kv_head_stride %llu < seq_len*head_dim", (unsigned long long)kv_head_stride);
  STS_CHECK(kv_head_stride % 4 == 0, "kv_head_stride must be a multiple of 4");
  STS_CHECK(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out),
            "q, k, v, out must be 16-byte aligned");
  STS_CHECK(std::isfinite(scale), "scale must be finite");
  sts::DecodeParams p;
  p.q = q;
  p.k = k;
  p.v = v;
  p.out = out;
  p.len = seq_len;
  p.start = 0;
  p.M = seq_len;  // rows 0..seq_len-1, no wrap
  p.H = num_heads;
  p.kv_hstride = kv_head_stride;
  p.scale_log2 = sts::softmax_scale_log2(scale);
  return sts::launch_decode(p, 1, head_dim, seq_len, as_stream(stream));
}

int sts_cache_write(const float* input, float* cache, uint32_t pos_offset, uint32_t batch,
                    uint32_t seq, uint32_t heads, uint32_t head_dim, uint32_t max_len,
                    void* stream) {
  sts::clear_error();
  STS_CHECK(input && cache, "null pointer argument");
  STS_CHECK(max_len >= 1, "max_len must be >= 1");
  STS_CHECK(seq <= max_len, "seq %u > max_len %u: slots of one call would collide", seq, max_len);
  STS_CHECK(head_dim >= 1 && heads >= 1 && batch >= 1, "empty shape");
  return sts::launch_cache_write(input, cache, pos_offset, batch, seq, heads, head_dim, max_len,
                                 as_stream(stream));
}

}  // extern "C"

namespace {

// sts_decode_ring and its allocation-free variant: same checks, same launch
// plan; only where the split workspace lives differs.
int decode_ring(const float* q, const float* k_cache, const float* v_cache, float* out,
                const int32_t* lens, const int32_t* starts, uint32_t batch, uint32_t heads,
                uint32_t head_dim, uint32_t max_len, float scale, void* stream, bool noalloc) {
  sts::clear_error();
  STS_CHECK(q && k_cache && v_cache && out && lens && starts, "null pointer argument");
  if (int rc = check_head_dim(head_dim)) return rc;
  STS_CHECK(batch >= 1 && heads >= 1 && max_len >= 1, "empty shape");
  STS_CHECK(aligned16(q) && aligned16(k_cache) && aligned16(v_cache) && aligned16(out),
            "q, k_cache, v_cache, out must be 16-byte aligned");
  STS_CHECK(std::isfinite(scale), "scale must be finite");
  sts::DecodeParams p;
  p.q = q;
  p.k = k_cache;
  p.v = v_cache;
  p.out = out;
  p.lens = lens;
  p.starts = starts;
  p.M = max_len;
  p.H = heads;
  p.q_bstride = (uint64_t)heads * head_dim;
  p.out_bstride = (uint64_t)heads * head_dim;
  p.kv_hstride = (uint64_t)max_len * head_dim;
  p.kv_bstride = (uint64_t)heads * max_len * head_dim;
  p.scale_log2 = sts::softmax_scale_log2(scale);
  return noalloc ? sts::launch_decode_noalloc(p, batch, head_dim, max_len, as_stream(stream))
                 : sts::launch_decode(p, batch, head_dim, max_len, as_stream(stream));
}

}  // namespace

extern "C" {

int sts_decode_ring(const float* q, const float* k_cache, const float* v_cache, float* out,
                    const int32_t* lens, const int32_t* starts, uint32_t batch, uint32_t heads,
                    uint32_t head_dim, uint32_t max_len, float scale, void* stream) {
  return decode_ring(q, k_cache, v_cache, out, lens, starts, batch, heads, head_dim, max_len,
                     scale, stream, false);
}

int sts_decode_ring_noalloc(const float* q, const float* k_cache, const float* v_cache,
                            float* out, const int32_t* lens, const int32_t* starts,
                            uint32_t batch, uint32_t heads, uint32_t head_dim, uint32_t max_len,
                            float scale, void* stream) {
  return decode_ring(q, k_cache, v_cache, out, lens, starts, batch, heads, head_dim, max_len,
                     scale, stream, true);
}

int sts_depformer_step(const float* q, const float* k_new, const float* v_new,
                       uint64_t qkv_stride, float* k_cache, float* v_cache, float* out,
                       uint32_t batch, uint32_t heads, uint32_t head_dim, uint32_t max_len,
                       uint32_t step, float scale, void* stream) {
  sts::clear_error();
  STS_CHECK(q && k_new && v_new && k_cache && v_cache && out, "null pointer argument");
  if (int rc = check_head_dim(head_dim)) return rc;
  STS_CHECK(batch >= 1 && heads >= 1, "empty shape");
  STS_CHECK(step < max_len, "step %u must be < max_len %u", step, max_len);
  STS_CHECK(qkv_stride % 4 == 0 && (batch == 1 || qkv_stride >= (uint64_t)heads * head_dim),
            "qkv_stride must be a multiple of 4 and >= heads*head_dim");
  STS_CHECK(aligned16(q) && aligned16(k_new) && aligned16(v_new) && aligned16(k_cache) &&
                aligned16(v_cache) && aligned16(out),
            "pointers must be 16-byte aligned");
  STS_CHECK(std::isfinite(scale), "scale must be finite");
  sts::DecodeParams p;
  p.q = q;
  p.k = k_cache;
  p.v = v_cache;
  p.out = out;
  p.k_new = k_new;
  p.v_new = v_new;
  p.k_wr = k_cache;
  p.v_wr = v_cache;
  p.len = step + 1;
  p.start = 0;
  p.M = max_len;
  p.H = heads;
  p.q_bstride = qkv_stride;
  p.out_bstride = (uint64_t)heads * head_dim;
  p.kv_hstride = (uint64_t)max_len * head_dim;
  p.kv_bstride = (uint64_t)heads * max_len * head_dim;
  p.scale_log2 = sts::softmax_scale_log2(scale);
  return sts::launch_decode(p, batch, head_dim, step + 1, as_stream(stream));
}

int sts_prefill_attention(const float* q, const float* k_cache, const float* v_cache, float* out,
                          uint32_t seq, uint32_t heads, uint32_t head_dim, uint32_t max_len,
                          uint32_t win_start, uint32_t win_len, float scale, int precision,
                          void* stream) {
  sts::clear_error();
  STS_CHECK(q && k_cache && v_cache && out, "null pointer argument");
  STS_CHECK(heads >= 1 && max_len >= 1, "empty shape");
  STS_CHECK(seq >= 1 && seq <= win_len, "need 1 <= seq (%u) <= win_len (%u)", seq, win_len);
  STS_CHECK(win_len <= max_len, "win_len %u > max_len %u", win_len, max_len);
  STS_CHECK(win_start < max_len, "win_start %u >= max_len %u", win_start, max_len);
  if (int rc = sts::check_prefill(seq, heads, head_dim, max_len, precision)) return rc;
  STS_CHECK(aligned16(q) && aligned16(k_cache) && aligned16(v_cache) && aligned16(out),
            "pointers must be 16-byte aligned");
  STS_CHECK(std::isfinite(scale), "scale must be finite");
  sts::PrefillParams p;
  p.q = q;
  p.k = k_cache;
  p.v = v_cache;
  p.out = out;
  p.S = seq;
  p.H = heads;
  p.M = max_len;
  p.start = win_start;
  p.len = win_len;
  p.scale_log2 = sts::softmax_scale_log2(scale);
  return sts::launch_prefill(p, head_dim, precision, as_stream(stream));
}

int sts_prefill_attention_bf16kv(const float* q, const uint16_t* k16, const uint16_t* v16,
                                 float* out, uint32_t seq, uint32_t heads, uint32_t head_dim,
                                 uint32_t max_len, uint32_t win_start, uint32_t win_len,
                                 float scale, void* stream) {
  sts::clear_error();
  STS_CHECK(q && k16 && v16 && out, "null pointer argument");
  STS_CHECK(heads >= 1 && max_len >= 1, "empty shape");
  STS_CHECK(seq >= 1 && seq <= win_len, "need 1 <= seq (%u) <= win_len (%u)", seq, win_len);
  STS_CHECK(win_len <= max_len, "win_len %u > max_len %u", win_len, max_len);
  STS_CHECK(win_start < max_len, "win_start %u >= max_len %u", win_start, max_len);
  if (int rc = sts::check_prefill(seq, heads, head_dim, max_len, STS_PREC_BF16_MFMA)) return rc;
  STS_CHECK(head_dim == 64 || head_dim == 128, "bf16 K/V rows need head_dim 64 or 128 (got %u)",
            head_dim);
  STS_CHECK(aligned16(q) && aligned16(k16) && aligned16(v16) && aligned16(out),
            "pointers must be 16-byte aligned");
  STS_CHECK(std::isfinite(scale), "scale must be finite");
  sts::PrefillParams p;
  p.q = q;
  p.k16 = k16;
  p.v16 = v16;
  p.out = out;
  p.S = seq;
  p.H = heads;
  p.M = max_len;
  p.start = win_start;
  p.len = win_len;
  p.scale_log2 = sts::softmax_scale_log2(scale);
  return sts::launch_prefill(p, head_dim, STS_PREC_BF16_MFMA, as_stream(stream));
}

/* ---------------------------------------------------------------------- */
/* RoPE                                                                     */
/* ---------------------------------------------------------------------- */

int sts_rope_create(uint32_t head_dim, uint32_t max_seq_len, float theta, sts_rope** out) {
  sts::clear_error();
  STS_CHECK(out, "null out pointer");
  *out = nullptr;
  if (int rc = check_head_dim(head_dim)) return rc;
  STS_CHECK(max_seq_len >= 1, "max_seq_len must be >= 1");
  STS_CHECK(std::isfinite(theta) && theta > 0.f, "theta must be positive");
  const uint32_t half = head_dim / 2;
  // model.rs:49-60: f32 inverse frequencies and f32 angles.
  std::vector<float> inv(half);
  for (uint32_t i = 0; i < half; ++i)
    inv[i] = 1.0f / powf(theta, (float)(2 * i) / (float)head_dim);
  const size_t n = (size_t)max_seq_len * half;
  std::vector<float> c(n), s(n);
  for (uint32_t p = 0; p < max_seq_len; ++p) {
    const float pos = (float)p;
    for (uint32_t j = 0; j < half; ++j) {
      const float ang = pos * inv[j];
      c[(size_t)p * half + j] = (float)std::cos((double)ang);
      s[(size_t)p * half + j] = (float)std::sin((double)ang);
    }
  }
  sts_rope* r = new (std::nothrow) sts_rope;
  if (!r) return fail(STS_ERR_NOMEM, "host allocation failed");
  r->head_dim = head_dim;
  r->max_seq_len = max_seq_len;
  if (hipMalloc(&r->cos_t, n * sizeof(float)) != hipSuccess ||
      hipMalloc(&r->sin_t, n * sizeof(float)) != hipSuccess) {
    if (r->cos_t) (void)hipFree(r->cos_t);
    delete r;
    return fail(STS_ERR_NOMEM, "RoPE table allocation failed");
  }
  if (hipMemcpy(r->cos_t, c.data(), n * sizeof(float), hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(r->sin_t, s.data(), n * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) {
    (void)hipFree(r->cos_t);
    (void)hipFree(r->sin_t);
    delete r;
    return fail(STS_ERR_HIP, "RoPE table upload failed");
  }
  *out = r;
  return STS_OK;
}

int sts_rope_destroy(sts_rope* rope) {
  sts::clear_error();
  if (!rope) return STS_OK;
  if (rope->cos_t) (void)hipFree(rope->cos_t);
  if (rope->sin_t) (void)hipFree(rope->sin_t);
  delete rope;
  return STS_OK;
}

int sts_rope_apply(const sts_rope* rope, float* x, uint32_t batch, uint32_t seq, uint32_t heads,
                   uint32_t offset, void* stream) {
  sts::clear_error();
  STS_CHECK(rope && x, "null pointer argument");
  STS_CHECK((uint64_t)offset + seq <= rope->max_seq_len,
            "positions %u..%u exceed the RoPE table (%u rows)", offset, offset + seq,
            rope->max_seq_len);
  STS_CHECK(aligned16(x), "x must be 16-byte aligned");
  return sts::launch_rope(x, rope->cos_t, rope->sin_t, batch, seq, heads, rope->head_dim, offset,
                          as_stream(stream));
}

/* ---------------------------------------------------------------------- */
/* KV cache handle                                                          */
/* ---------------------------------------------------------------------- */

int sts_kv_create(uint64_t max_len, uint64_t heads, uint64_t head_dim, sts_kv_cache** out) {
  return sts_kv_create_ex(max_len, heads, head_dim, 0, out);
}

int sts_kv_create_ex(uint64_t max_len, uint64_t heads, uint64_t head_dim, uint32_t flags,
                     sts_kv_cache** out) {
  sts::clear_error();
  STS_CHECK((flags & ~(uint32_t)STS_KV_BF16_MIRROR) == 0, "unknown flags 0x%x", flags);
  STS_CHECK(out, "null out pointer");
  *out = nullptr;
  STS_CHECK(max_len >= 1 && max_len <= 0x7fffffffull, "max_len must be in 1..2^31-1");
  STS_CHECK(heads >= 1 && heads <= 65535, "heads must be in 1..65535");
  if (int rc = check_head_dim(head_dim)) return rc;
  sts_kv_cache* c = new (std::nothrow) sts_kv_cache;
  if (!c) return fail(STS_ERR_NOMEM, "host allocation failed");
  c->max_len = max_len;
  c->heads = heads;
  c->q_heads = heads;
  c->head_dim = head_dim;
  c->flags = flags;
  *out = c;
  return STS_OK;
}

int sts_kv_set_query_heads(sts_kv_cache* cache, uint64_t q_heads) {
  sts::clear_error();
  STS_CHECK(cache, "null cache handle");
  STS_CHECK(q_heads >= cache->heads && q_heads <= 65535 && q_heads % cache->heads == 0,
            "query heads %llu must be a multiple of the %llu K/V heads, at most 65535",
            (unsigned long long)q_heads, (unsigned long long)cache->heads);
  cache->q_heads = q_heads;
  return STS_OK;
}

int sts_kv_destroy(sts_kv_cache* cache) {
  sts::clear_error();
  if (!cache) return STS_OK;
  kv_free(cache);
  delete cache;
  return STS_OK;
}

int sts_kv_mirror(const sts_kv_cache* cache, uint16_t** k16, uint16_t** v16) {
  sts::clear_error();
  STS_CHECK(cache && k16 && v16, "null pointer argument");
  *k16 = cache->k16;
  *v16 = cache->v16;
  return STS_OK;
}

int sts_kv_sync_mirror(sts_kv_cache* cache, void* stream) {
  sts::clear_error();
  STS_CHECK(cache, "null cache handle");
  if (!cache->k16) return STS_OK;
  const uint64_t n = cache->batch * cache->heads * cache->max_len * cache->head_dim;
  if (int rc = sts::launch_to_bf16(cache->k, cache->k16, n, as_stream(stream))) return rc;
  return sts::launch_to_bf16(cache->v, cache->v16, n, as_stream(stream));
}

int sts_kv_ensure_allocated(sts_kv_cache* cache, uint64_t batch, float** k, float** v,
                            uint64_t* write_pos, void* stream) {
  sts::clear_error();
  STS_CHECK(cache, "null cache handle");
  if (int rc = kv_ensure(cache, batch, as_stream(stream))) return rc;
  if (k) *k = cache->k;
  if (v) *v = cache->v;
  if (write_pos) *write_pos = cache->write_pos;
  return STS_OK;
}

int sts_kv_get_state(const sts_kv_cache* cache, sts_kv_state* out) {
  sts::clear_error();
  STS_CHECK(cache && out, "null pointer argument");
  std::memset(out, 0, sizeof *out);
  out->offset = cache->offset;
  out->len = cache->len;
  out->write_pos = cache->write_pos;
  out->max_len = cache->max_len;
  out->heads = cache->heads;
  out->head_dim = cache->head_dim;
  out->batch = cache->batch;
  out->allocated = cache->k != nullptr;
  out->flags = (int32_t)cache->flags;
  out->q_heads = cache->q_heads;
  return STS_OK;
}

int sts_kv_window(const sts_kv_cache* cache, uint64_t* start, uint64_t* len) {
  sts::clear_error();
  STS_CHECK(cache && start && len, "null pointer argument");
  *start = kv_start(cache);
  *len = cache->len;
  return STS_OK;
}

int sts_kv_advance(sts_kv_cache* cache, uint64_t n) {
  sts::clear_error();
  STS_CHECK(cache, "null cache handle");
  kv_advance(cache, n);
  return STS_OK;
}

int sts_kv_update(sts_kv_cache* cache, const float* k_new, const float* v_new, uint64_t batch,
                  uint64_t seq, void* stream) {
  sts::clear_error();
  STS_CHECK(cache && k_new && v_new, "null pointer argument");
  STS_CHECK(seq >= 1 && seq <= cache->max_len, "seq %llu must be in 1..max_len",
            (unsigned long long)seq);
  hipStream_t s = as_stream(stream);
  if (int rc = kv_ensure(cache, batch, s)) return rc;
  // gpu_cache_write_v with pos_offset = offset (model.rs:747-749); write_pos
  // and offset agree modulo max_len under advance and rollback.
  const uint32_t pos = (uint32_t)(cache->offset % cache->max_len);
  if (aligned16(k_new) && aligned16(v_new)) {
    // K and V (and their bf16 mirror) in one launch.
    if (int rc = sts::launch_kv_append(k_new, v_new, cache->k, cache->v, pos, (uint32_t)batch,
                                       (uint32_t)seq, (uint32_t)cache->heads,
                                       (uint32_t)cache->head_dim, (uint32_t)cache->max_len,
                                       nullptr, nullptr, 0, cache->k16, cache->v16, s))
      return rc;
  } else if (cache->k16) {
    return fail(STS_ERR_INVALID, "a cache with a bf16 mirror needs 16-byte aligned k_new, v_new");
  } else {
    if (int rc = sts::launch_cache_write(k_new, cache->k, pos, (uint32_t)batch, (uint32_t)seq,
                                         (uint32_t)cache->heads, (uint32_t)cache->head_dim,
                                         (uint32_t)cache->max_len, s))
      return rc;
    if (int rc = sts::launch_cache_write(v_new, cache->v, pos, (uint32_t)batch, (uint32_t)seq,
                                         (uint32_t)cache->heads, (uint32_t)cache->head_dim,
                                         (uint32_t)cache->max_len, s))
      return rc;
  }
  kv_advance(cache, seq);
  return STS_OK;
}

int sts_kv_reset(sts_kv_cache* cache) {
  sts::clear_error();
  STS_CHECK(cache, "null cache handle");
  kv_free(cache);
  cache->batch = 0;
  cache->offset = cache->len = cache->write_pos = 0;
  return STS_OK;
}

int sts_kv_reset_keep_buffers(sts_kv_cache* cache, void* stream) {
  sts::clear_error();
  STS_CHECK(cache, "null cache handle");
  if (cache->k) {
    const uint64_t n = cache->batch * cache->heads * cache->max_len * cache->head_dim;
    STS_HIP(hipMemsetAsync(cache->k, 0, n * sizeof(float), as_stream(stream)));
    STS_HIP(hipMemsetAsync(cache->v, 0, n * sizeof(float), as_stream(stream)));
    if (cache->k16) {
      STS_HIP(hipMemsetAsync(cache->k16, 0, n * sizeof(uint16_t), as_stream(stream)));
      STS_HIP(hipMemsetAsync(cache->v16, 0, n * sizeof(uint16_t), as_stream(stream)));
    }
  }
  cache->offset = cache->len = cache->write_pos = 0;
  return STS_OK;
}

int sts_kv_rollback(sts_kv_cache* cache, uint64_t n) {
  sts::clear_error();
  STS_CHECK(cache, "null cache handle");
  // model.rs:352-362
  if (n > cache->len) n = cache->len;
  cache->offset -= n;
  cache->len -= n;
  if (cache->write_pos >= n)
    cache->write_pos -= n;
  else
    cache->write_pos = cache->max_len - (n - cache->write_pos);
  return STS_OK;
}

// q/out hold the handle's query heads; K/V head j serves query heads
// j * group .. j * group + group - 1 (model.rs:766-783's repeat of each K/V
// head), k_new/v_new the K/V heads.
static void fill_cache_decode(const sts_kv_cache* c, sts::DecodeParams& p) {
  p.k = c->k;
  p.v = c->v;
  p.M = (uint32_t)c->max_len;
  p.H = (uint32_t)c->q_heads;
  p.group = (uint32_t)(c->q_heads / c->heads);
  p.q_bstride = c->q_heads * c->head_dim;
  p.out_bstride = c->q_heads * c->head_dim;
  p.kn_bstride = c->heads * c->head_dim;
  p.kv_hstride = c->max_len * c->head_dim;
  p.kv_bstride = c->heads * c->max_len * c->head_dim;
}

int sts_kv_attend(sts_kv_cache* cache, const float* q, float* out, float scale, void* stream) {
  sts::clear_error();
  STS_CHECK(cache && q && out, "null pointer argument");
  if (!cache->k) return fail(STS_ERR_STATE, "cache has no buffers yet (nothing appended)");
  STS_CHECK(cache->len >= 1, "cache window is empty");
  STS_CHECK(aligned16(q) && aligned16(out), "q and out must be 16-byte aligned");
  STS_CHECK(std::isfinite(scale), "scale must be finite");
  sts::DecodeParams p;
  fill_cache_decode(cache, p);
  p.q = q;
  p.out = out;
  p.len = (uint32_t)cache->len;
  p.start = (uint32_t)kv_start(cache);
  p.scale_log2 = sts::softmax_scale_log2(scale);
  return sts::launch_decode(p, (uint32_t)cache->batch, (uint32_t)cache->head_dim, p.len,
                            as_stream(stream));
}

int sts_kv_decode_step(sts_kv_cache* cache, const sts_rope* rope, const float* q,
                       const float* k_new, const float* v_new, float* out, uint64_t batch,
                       float scale, void* stream) {
  sts::clear_error();
  STS_CHECK(cache && q && k_new && v_new && out, "null pointer argument");
  STS_CHECK(aligned16(q) && aligned16(k_new) && aligned16(v_new) && aligned16(out),
            "pointers must be 16-byte aligned");
  STS_CHECK(std::isfinite(scale), "scale must be finite");
  if (rope) {
    STS_CHECK(rope->head_dim == cache->head_dim, "RoPE head_dim %u != cache head_dim %llu",
              rope->head_dim, (unsigned long long)cache->head_dim);
    // RoPE::apply slices the table at offset..offset+1 (model.rs:92-95).
    STS_CHECK(cache->offset < rope->max_seq_len, "position %llu beyond the RoPE table (%u rows)",
              (unsigned long long)cache->offset, rope->max_seq_len);
  }
  hipStream_t s = as_stream(stream);
  if (int rc = kv_ensure(cache, batch, s)) return rc;
  const uint64_t pos = cache->offset;
  sts_kv_cache next = *cache;
  kv_advance(&next, 1);
  sts::DecodeParams p;
  fill_cache_decode(cache, p);
  p.q = q;
  p.out = out;
  p.k_new = k_new;
  p.v_new = v_new;
  p.k_wr = cache->k;
  p.v_wr = cache->v;
  p.k16_wr = cache->k16;
  p.v16_wr = cache->v16;
  p.len = (uint32_t)next.len;
  p.start = (uint32_t)kv_start(&next);
  if (rope) {
    p.rope_cos = rope->cos_t;
    p.rope_sin = rope->sin_t;
    p.rope_pos = (uint32_t)pos;
  }
  p.scale_log2 = sts::softmax_scale_log2(scale);
  if (int rc = sts::launch_decode(p, (uint32_t)batch, (uint32_t)cache->head_dim, p.len, s))
    return rc;
  *cache = next;
  return STS_OK;
}

int sts_kv_prefill(sts_kv_cache* cache, const sts_rope* rope, const float* q,
                   const float* k_new, const float* v_new, float* out, uint64_t seq,
                   float scale, int precision, void* stream) {
  sts::clear_error();
  // Every check runs before anything is written or the counters move, so a
  // rejected call leaves the cache as it was.
  STS_CHECK(cache && q && k_new && v_new && out, "null pointer argument");
  STS_CHECK(seq >= 1 && seq <= cache->max_len, "seq %llu must be in 1..max_len",
            (unsigned long long)seq);
  if (cache->k && cache->batch != 1)
    return fail(STS_ERR_STATE, "prefill needs a batch-1 cache (allocated with batch %llu)",
                (unsigned long long)cache->batch);
  if (int rc = sts::check_prefill((uint32_t)seq, (uint32_t)cache->q_heads,
                                  (uint32_t)cache->head_dim, (uint32_t)cache->max_len, precision))
    return rc;
  STS_CHECK(aligned16(q) && aligned16(k_new) && aligned16(v_new) && aligned16(out),
            "q, k_new, v_new, out must be 16-byte aligned");
  STS_CHECK(std::isfinite(scale), "scale must be finite");
  if (rope) {
    STS_CHECK(rope->head_dim == cache->head_dim, "RoPE head_dim %u != cache head_dim %llu",
              rope->head_dim, (unsigned long long)cache->head_dim);
    // RoPE::apply slices the table at offset..offset+seq (model.rs:92-95).
    STS_CHECK(cache->offset + seq <= rope->max_seq_len,
              "positions %llu..%llu beyond the RoPE table (%u rows)",
              (unsigned long long)cache->offset, (unsigned long long)(cache->offset + seq),
              rope->max_seq_len);
  }
  hipStream_t s = as_stream(stream);
  sts_kv_cache next = *cache;
  kv_advance(&next, seq);
  const bool bf16_rows = precision == STS_PREC_BF16_MFMA && (cache->flags & STS_KV_BF16_MIRROR);
  // Everything the attention launch needs is acquired before the append runs
  // and the counters move: a call refused here (workspace needed while the
  // stream is being captured, out of memory) leaves the cache as it was.
  if (int rc = sts::reserve_prefill((uint32_t)seq, (uint32_t)cache->q_heads, (uint32_t)next.len,
                                    (uint32_t)cache->head_dim, precision, bf16_rows, s))
    return rc;
  if (int rc = kv_ensure(cache, 1, s)) return rc;
  next.k = cache->k;
  next.v = cache->v;
  next.k16 = cache->k16;
  next.v16 = cache->v16;
  next.batch = cache->batch;
  const uint32_t pos = (uint32_t)(cache->offset % cache->max_len);
  // RoPE of k (at offset + s) fused into one append launch of K and V.
  if (int rc = sts::launch_kv_append(k_new, v_new, cache->k, cache->v, pos, 1, (uint32_t)seq,
                                     (uint32_t)cache->heads, (uint32_t)cache->head_dim,
                                     (uint32_t)cache->max_len, rope ? rope->cos_t : nullptr,
                                     rope ? rope->sin_t : nullptr, (uint32_t)cache->offset,
                                     cache->k16, cache->v16, s))
    return rc;
  const uint64_t q_pos0 = cache->offset;
  *cache = next;
  sts::PrefillParams p;
  p.q = q;
  p.k = cache->k;
  p.v = cache->v;
  p.out = out;
  p.S = (uint32_t)seq;
  p.H = (uint32_t)cache->q_heads;
  p.group = (uint32_t)(cache->q_heads / cache->heads);
  p.M = (uint32_t)cache->max_len;
  p.start = (uint32_t)kv_start(cache);
  p.len = (uint32_t)cache->len;
  p.scale_log2 = sts::softmax_scale_log2(scale);
  if (rope) {
    // q rotated in registers inside the attention kernel (table rows offset + i).
    p.rope_cos = rope->cos_t;
    p.rope_sin = rope->sin_t;
    p.rope_pos0 = (uint32_t)q_pos0;
  }
  if (precision == STS_PREC_BF16_MFMA && cache->k16) {
    // The mirror holds exactly the bf16 values the kernel would round the f32
    // rows to: same result, half the K/V bytes.
    p.k16 = cache->k16;
    p.v16 = cache->v16;
  }
  return sts::launch_prefill(p, (uint32_t)cache->head_dim, precision, s);
}

/* ---------------------------------------------------------------------- */
/* Device error word and wait bound                                         */
/* ---------------------------------------------------------------------- */

int sts_device_errors(void* stream, uint32_t* flags) {
  sts::clear_error();
  uint32_t f = 0;
  if (int rc = sts::take_device_errors(as_stream(stream), &f)) return rc;
  if (flags) *flags = f;
  if (f & STS_DEVERR_WAIT_TIMEOUT)
    return fail(STS_ERR_DEVICE,
                "a bounded wait inside a kernel gave up (flags 0x%x): an output written since "
                "the last check is invalid", f);
  if (f) return fail(STS_ERR_DEVICE, "device error flags 0x%x", f);
  return STS_OK;
}

int sts_debug_set_wait_limit(uint32_t polls) {
  sts::clear_error();
  sts::set_wait_limit(polls);
  return STS_OK;
}

}  // extern "C"

// ---- Q4_K ------------------------------------------------------------------

extern "C" int sts_q4k_matvec(const uint8_t* weights, const float* x, const float* residual,
                              float* y, uint32_t batch, uint32_t k, uint32_t n, void* stream) {
  sts::clear_error();
  STS_CHECK(weights && x && y, "null pointer argument");
  STS_CHECK(batch >= 1 && batch <= 65535, "batch %u out of range 1..65535", batch);
  STS_CHECK(n >= 1, "empty shape");
  STS_CHECK(k >= 256 && k % 256 == 0 && k <= 16384,
            "k = %u must be a multiple of 256 in 256..16384", k);
  STS_CHECK(aligned16(weights) && aligned16(x), "weights and x must be 16-byte aligned");
  sts::Q4kParams p;
  p.w = weights;
  p.x = x;
  p.res = residual;
  p.y = y;
  p.B = batch;
  p.K = k;
  p.N = n;
  return sts::launch_q4k_matvec(p, as_stream(stream));
}

extern "C" int sts_q4k_dequant(const uint8_t* weights, float* out, uint32_t k, uint32_t n,
                               void* stream) {
  sts::clear_error();
  STS_CHECK(weights && out, "null pointer argument");
  STS_CHECK(n >= 1, "empty shape");
  STS_CHECK(k >= 256 && k % 256 == 0, "k = %u must be a positive multiple of 256", k);
  STS_CHECK(aligned16(weights) && aligned16(out), "weights and out must be 16-byte aligned");
  return sts::launch_q4k_dequant(weights, out, n, k, as_stream(stream));
}
