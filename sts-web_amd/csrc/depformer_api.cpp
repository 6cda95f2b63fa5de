// depformer_api.cpp -- C ABI of the depformer step chain and its building blocks.
//
// sts_depformer_generate issues, on one stream, the launches of
// DepthEngine::generate (crates/sts-wasm/src/depth_engine.rs:884-1491) for a
// batch of streams: one GEMM for the input projections of every step, then
// per step an embedding + add, per layer the QKV GEMM (RMSNorm fused on its
// input), fused cache-write + attention, out_proj GEMM + residual, linear_in
// GEMM (RMSNorm on its input, SwiGLU on its output), linear_out GEMM +
// residual, and finally the output GEMM and the sampler.  Nothing is allocated or read back per call.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <vector>

#include "common.hpp"
#include "decode.hpp"
#include "depformer.hpp"
#include "sts_attn.h"

namespace {

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

struct sts_depformer {
  sts_depformer_config cfg{};
  std::vector<const uint8_t*> input_proj, attn_in_proj, attn_out_proj, ffn_in, ffn_out,
      output_linear, audio_emb;
  std::vector<const float*> norm1, norm2;
  const uint8_t* text_emb = nullptr;
  uint32_t max_batch = 0;
  float* mem = nullptr;
  float *proj = nullptr, *h = nullptr, *h2 = nullptr, *nrm = nullptr, *qkv = nullptr,
        *att = nullptr, *sw = nullptr, *logits = nullptr, *kc = nullptr, *vc = nullptr;
};

extern "C" {

int sts_q4k_gemm(const uint8_t* weights, const float* x, uint64_t ldx, const float* norm_alpha,
                 float norm_eps, const float* residual, uint64_t ldr, float* y, uint64_t ldy,
                 uint32_t rows, uint32_t k, uint32_t n, int swiglu, void* stream) {
  sts::clear_error();
  STS_CHECK(weights && x && y, "null pointer argument");
  STS_CHECK(rows >= 1 && n >= 1, "empty shape");
  STS_CHECK(ldx >= k && (rows == 1 || ldy >= (swiglu ? n / 2 : n)),
            "row strides smaller than the rows");
  STS_CHECK(!swiglu || (n % 2 == 0 && !residual), "SwiGLU needs an even n and no residual");
  STS_CHECK(!residual || rows == 1 || ldr >= n, "residual stride smaller than n");
  STS_CHECK(!norm_alpha || (aligned16(norm_alpha) && std::isfinite(norm_eps) && norm_eps >= 0.f),
            "norm_alpha must be 16-byte aligned and norm_eps finite and >= 0");
  sts::Q4kGemmParams p;
  p.w[0] = weights;
  p.x = x;
  p.res = residual;
  p.y = y;
  p.M = rows;
  p.N = n;
  p.K = k;
  p.ldx = ldx;
  p.ldy = ldy;
  p.ldr = ldr;
  p.swiglu_f = swiglu ? n / 2 : 0;
  p.norm_alpha = norm_alpha;
  p.norm_eps = norm_eps;
  return sts::launch_q4k_gemm(p, as_stream(stream));
}

int sts_rmsnorm(const float* x, const float* alpha, float* out, uint32_t rows, uint32_t dim,
                float eps, void* stream) {
  sts::clear_error();
  STS_CHECK(x && alpha && out, "null pointer argument");
  STS_CHECK(std::isfinite(eps) && eps >= 0.f, "eps must be finite and >= 0");
  return sts::launch_rmsnorm(x, alpha, out, rows, dim, eps, as_stream(stream));
}

int sts_embed_add_q4_0(const uint8_t* table, uint32_t vocab, const uint32_t* tokens,
                       uint64_t tok_stride, const float* proj, float* h, uint32_t batch,
                       uint32_t dim, void* stream) {
  sts::clear_error();
  STS_CHECK(table && tokens && proj && h, "null pointer argument");
  return sts::launch_embed_add(table, vocab, tokens, tok_stride, proj, h, batch, dim,
                               as_stream(stream));
}

int sts_sample_topk(const float* logits, uint64_t ld, uint32_t batch, uint32_t vocab,
                    uint32_t top_k, float temperature, float penalty, const float* rand,
                    const uint32_t* ptoks, uint64_t pt_stride, const uint32_t* num_penalty,
                    uint64_t rs_stride, uint32_t* out, uint64_t out_stride, void* stream) {
  sts::clear_error();
  STS_CHECK(logits && rand && ptoks && num_penalty && out, "null pointer argument");
  STS_CHECK(batch == 1 || ld >= vocab, "logits stride smaller than vocab");
  STS_CHECK(std::isfinite(temperature) && temperature != 0.f, "temperature must be finite, != 0");
  STS_CHECK(std::isfinite(penalty), "penalty must be finite");
  sts::SampleParams p;
  p.logits = logits;
  p.ld_logits = ld;
  p.B = batch;
  p.V = vocab;
  p.top_k = top_k;
  p.temperature = temperature;
  p.penalty = penalty;
  p.rand = rand;
  p.ptoks = ptoks;
  p.num_penalty = num_penalty;
  p.rs_stride = rs_stride;
  p.pt_stride = pt_stride;
  p.out = out;
  p.out_stride = out_stride;
  return sts::launch_sample_topk(p, as_stream(stream));
}

int sts_depformer_create(const sts_depformer_config* cfg, const sts_depformer_weights* w,
                         uint32_t max_batch, sts_depformer** out) {
  sts::clear_error();
  STS_CHECK(cfg && w && out, "null pointer argument");
  *out = nullptr;
  const sts_depformer_config& c = *cfg;
  STS_CHECK(c.num_steps >= 1 && c.num_steps <= (uint32_t)sts::kGemmMaxZ,
            "num_steps %u must be in 1..%d", c.num_steps, sts::kGemmMaxZ);
  STS_CHECK(c.num_layers >= 1 && c.num_heads >= 1 && c.dim % c.num_heads == 0,
            "bad layers/heads/dim");
  const uint32_t hd = c.dim / c.num_heads;
  STS_CHECK(hd == 64 || hd == 128, "head_dim %u must be 64 or 128", hd);
  STS_CHECK(c.dim % 256 == 0 && c.dim <= 4096 && c.ffn % 256 == 0 && c.ffn <= 4096 &&
                c.temporal_dim % 256 == 0 && c.temporal_dim <= 4096,
            "dim, ffn, temporal_dim must be multiples of 256 up to 4096");
  STS_CHECK(c.out_vocab >= 1 && c.out_vocab <= sts::kMaxVocab, "out_vocab %u must be <= %u",
            c.out_vocab, sts::kMaxVocab);
  STS_CHECK(c.kv_max_len >= c.num_steps, "kv_max_len %u < num_steps %u", c.kv_max_len,
            c.num_steps);
  STS_CHECK(c.num_audio_emb >= 1 || c.num_steps == 1, "no audio embedding tables");
  STS_CHECK(std::isfinite(c.rms_eps) && std::isfinite(c.attn_scale), "non-finite eps/scale");
  STS_CHECK(max_batch >= 1 && max_batch <= 65535u, "max_batch %u must be in 1..65535", max_batch);
  STS_CHECK(w->input_proj && w->attn_in_proj && w->attn_out_proj && w->ffn_linear_in &&
                w->ffn_linear_out && w->norm1_alpha && w->norm2_alpha && w->output_linear &&
                w->text_emb && (w->audio_emb || c.num_steps == 1),
            "null weight array");
  const uint32_t S = c.num_steps, L = c.num_layers;
  auto* d = new (std::nothrow) sts_depformer;
  if (!d) return sts::fail(STS_ERR_NOMEM, "host allocation failed");
  d->cfg = c;
  d->max_batch = max_batch;
  d->input_proj.assign(w->input_proj, w->input_proj + S);
  d->output_linear.assign(w->output_linear, w->output_linear + S);
  d->attn_in_proj.assign(w->attn_in_proj, w->attn_in_proj + L * S);
  d->attn_out_proj.assign(w->attn_out_proj, w->attn_out_proj + L * S);
  d->ffn_in.assign(w->ffn_linear_in, w->ffn_linear_in + L * S);
  d->ffn_out.assign(w->ffn_linear_out, w->ffn_linear_out + L * S);
  d->norm1.assign(w->norm1_alpha, w->norm1_alpha + L);
  d->norm2.assign(w->norm2_alpha, w->norm2_alpha + L);
  if (c.num_audio_emb) d->audio_emb.assign(w->audio_emb, w->audio_emb + c.num_audio_emb);
  d->text_emb = w->text_emb;
  bool ok = aligned16(d->text_emb);
  for (auto* v : {&d->input_proj, &d->output_linear, &d->attn_in_proj, &d->attn_out_proj,
                  &d->ffn_in, &d->ffn_out, &d->audio_emb})
    for (const uint8_t* p : *v) ok = ok && p && aligned16(p);
  for (auto* v : {&d->norm1, &d->norm2})
    for (const float* p : *v) ok = ok && p && aligned16(p);
  if (!ok) {
    delete d;
    return sts::fail(STS_ERR_INVALID, "weight pointers must be non-null and 16-byte aligned");
  }
  const size_t B = max_batch, D = c.dim;
  const size_t kv = (size_t)L * B * c.num_heads * c.kv_max_len * hd;
  const size_t sizes[] = {(size_t)S * B * D, B * D, B * D, B * D, 3 * B * D, B * D,
                          B * c.ffn, B * c.out_vocab, kv, kv};
  size_t total = 0;
  for (size_t s : sizes) total += (s + 63) / 64 * 64;
  if (hipMalloc(&d->mem, total * sizeof(float)) != hipSuccess) {
    delete d;
    return sts::fail(STS_ERR_NOMEM, "device allocation of %zu bytes failed", total * 4);
  }
  float** dst[] = {&d->proj, &d->h, &d->h2, &d->nrm, &d->qkv, &d->att,
                   &d->sw, &d->logits, &d->kc, &d->vc};
  size_t off = 0;
  for (int i = 0; i < 10; ++i) {
    *dst[i] = d->mem + off;
    off += (sizes[i] + 63) / 64 * 64;
  }
  *out = d;
  return STS_OK;
}

int sts_depformer_destroy(sts_depformer* d) {
  sts::clear_error();
  if (!d) return STS_OK;
  if (d->mem) STS_HIP(hipFree(d->mem));
  delete d;
  return STS_OK;
}

int sts_depformer_generate(sts_depformer* d, const float* temporal_hidden,
                           const uint32_t* text_token, uint32_t batch, uint32_t top_k,
                           float temperature, float penalty, const float* rand,
                           const uint32_t* penalty_tokens, const uint32_t* num_penalty,
                           uint32_t* tokens, float* logits, void* stream) {
  sts::clear_error();
  STS_CHECK(d && temporal_hidden && text_token && rand && penalty_tokens && num_penalty && tokens,
            "null pointer argument");
  STS_CHECK(batch >= 1 && batch <= d->max_batch, "batch %u must be in 1..%u", batch,
            d->max_batch);
  STS_CHECK(aligned16(temporal_hidden), "temporal_hidden must be 16-byte aligned");
  STS_CHECK(top_k <= sts::kMaxTopK, "top_k %u exceeds %u", top_k, sts::kMaxTopK);
  STS_CHECK(std::isfinite(temperature) && temperature != 0.f, "temperature must be finite, != 0");
  STS_CHECK(std::isfinite(penalty), "penalty must be finite");
  const sts_depformer_config& c = d->cfg;
  const hipStream_t st = as_stream(stream);
  const uint32_t S = c.num_steps, L = c.num_layers, D = c.dim, F = c.ffn, V = c.out_vocab;
  const uint32_t H = c.num_heads, hd = D / H, M = c.kv_max_len;
  const uint64_t B = batch;

  // Phase 1: the input projections of every step in one launch (:953-983).
  sts::Q4kGemmParams ip;
  for (uint32_t s = 0; s < S; ++s) ip.w[s] = d->input_proj[s];
  ip.Z = S;
  ip.x = temporal_hidden;
  ip.ldx = c.temporal_dim;
  ip.y = d->proj;
  ip.ldy = D;
  ip.y_zstride = B * D;
  ip.M = batch;
  ip.N = D;
  ip.K = c.temporal_dim;
  if (int rc = sts::launch_q4k_gemm(ip, st)) return rc;

  auto gemm = [&](const uint8_t* w, const float* x, uint32_t K, uint32_t N, const float* res,
                  float* y, uint64_t ldy, uint32_t swiglu_f, const float* norm = nullptr) {
    sts::Q4kGemmParams p;
    p.norm_alpha = norm;
    p.norm_eps = c.rms_eps;
    p.w[0] = w;
    p.x = x;
    p.ldx = K;
    p.res = res;
    p.ldr = ldy;
    p.y = y;
    p.ldy = ldy;
    p.M = batch;
    p.N = N;
    p.K = K;
    p.swiglu_f = swiglu_f;
    return sts::launch_q4k_gemm(p, st);
  };

  for (uint32_t s = 0; s < S; ++s) {
    // Embedding of the previous token plus the projection (:988-1057).
    const uint8_t* table = d->text_emb;
    uint32_t vocab = c.text_emb_vocab;
    const uint32_t* tok = text_token;
    uint64_t tok_stride = 1;
    if (s > 0) {
      table = d->audio_emb[std::min(s - 1, c.num_audio_emb - 1)];
      vocab = c.audio_emb_vocab;
      tok = tokens + (s - 1);
      tok_stride = S;
    }
    if (int rc = sts::launch_embed_add(table, vocab, tok, tok_stride, d->proj + s * B * D, d->h,
                                       batch, D, st))
      return rc;
    for (uint32_t l = 0; l < L; ++l) {
      const size_t wi = (size_t)l * S + s;
      float* kl = d->kc + (size_t)l * B * H * M * hd;
      float* vl = d->vc + (size_t)l * B * H * M * hd;
      // RMSNorm 1 fused into the QKV projection (:1069-1119).
      if (int rc = gemm(d->attn_in_proj[wi], d->h, D, 3 * D, nullptr, d->qkv, 3 * D, 0,
                        d->norm1[l]))
        return rc;
      // Cache write of K and V at slot s and attention over slots 0..s
      // (:1121-1209), one launch.
      sts::DecodeParams a;
      a.q = d->qkv;
      a.k_new = d->qkv + D;
      a.v_new = d->qkv + 2 * D;
      a.q_bstride = 3 * (uint64_t)D;
      a.k = a.k_wr = kl;
      a.v = a.v_wr = vl;
      a.out = d->att;
      a.out_bstride = D;
      a.len = s + 1;
      a.start = 0;
      a.M = M;
      a.H = H;
      a.kv_hstride = (uint64_t)M * hd;
      a.kv_bstride = (uint64_t)H * M * hd;
      a.scale_log2 = sts::softmax_scale_log2(c.attn_scale);
      if (int rc = sts::launch_decode(a, batch, hd, s + 1, st)) return rc;
      if (int rc = gemm(d->attn_out_proj[wi], d->att, D, D, d->h, d->h2, D, 0)) return rc;
      // RMSNorm 2 fused into linear_in, SwiGLU into its output (:1262-1332).
      if (int rc = gemm(d->ffn_in[wi], d->h2, D, 2 * F, nullptr, d->sw, F, F, d->norm2[l]))
        return rc;
      if (int rc = gemm(d->ffn_out[wi], d->sw, F, D, d->h2, d->h, D, 0)) return rc;
    }
    float* lg = logits ? logits + (size_t)s * B * V : d->logits;
    if (int rc = gemm(d->output_linear[s], d->h, D, V, nullptr, lg, V, 0)) return rc;
    sts::SampleParams sp;
    sp.logits = lg;
    sp.ld_logits = V;
    sp.B = batch;
    sp.V = V;
    sp.top_k = top_k;
    sp.temperature = temperature;
    sp.penalty = penalty;
    sp.rand = rand + s;
    sp.rs_stride = S;
    sp.ptoks = penalty_tokens + (size_t)s * sts::kMaxPenalty;
    sp.pt_stride = (uint64_t)S * sts::kMaxPenalty;
    sp.num_penalty = num_penalty + s;
    sp.out = tokens + s;
    sp.out_stride = S;
    if (int rc = sts::launch_sample_topk(sp, st)) return rc;
  }
  return STS_OK;
}

}  // extern "C"
