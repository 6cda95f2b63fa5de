/*
 * oracle.h -- CPU restatement of sts-web's attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this code, and only as the checker or
 * as the timed CPU baseline -- never as a product path.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * crates/sts-wasm/src/ of idle-intelligence/sts-web).  tests/test_oracle.py
 * pins each one against something independent of this code: closed forms,
 * scipy/torch routines, the reference's own KVCache unit-test sequences,
 * brute force on tiny inputs, and planted mistakes that must be caught.
 */
#ifndef STS_ORACLE_H
#define STS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- test-data RNG (our spec; no reference counterpart) ------------------ */

/* SplitMix64 output for counter i:  mix(seed + (i+1) * 0x9E3779B97F4A7C15). */
uint64_t orc_splitmix64(uint64_t seed, uint64_t i);

/*
 * out[j] = N(0,1) sample number (first + j) of stream `seed`, by Box-Muller on
 * SplitMix64 counters: pair k uses counters 2k and 2k+1,
 *   u1 = ((c0 >> 40) + 1) * 2^-24,  u2 = (c1 >> 40) * 2^-24,
 *   r = sqrt(-2 ln u1),  sample 2k = r cos(2 pi u2),  2k+1 = r sin(2 pi u2),
 * evaluated in double and rounded to f32.  OpenMP-parallel.
 */
void orc_fill_normal(uint64_t seed, uint64_t first, uint64_t n, float* out);

/* ---- RoPE (model.rs:38-122) ---------------------------------------------- */

/* RoPE::new tables (model.rs:46-66): cos_t, sin_t [max_seq_len][head_dim/2]. */
void orc_rope_tables(uint32_t head_dim, uint32_t max_seq_len, float theta,
                     float* cos_t, float* sin_t);

/* RoPE::apply_rope_to_tensor (model.rs:79-105), in place on x [B][S][H][D]. */
void orc_rope_apply(float* x, uint32_t B, uint32_t S, uint32_t H, uint32_t D,
                    uint32_t offset, const float* cos_t, const float* sin_t);

/* ---- KV append (shader_cache_write.wgsl:19-49, model.rs:143-188) -------- */

void orc_cache_write(const float* input, float* cache, uint32_t pos_offset,
                     uint32_t B, uint32_t S, uint32_t H, uint32_t D, uint32_t max_len);

/* ---- GQA expansion of K/V heads (model.rs:766-783) ----------------------- */

void orc_gqa_expand(const float* kv, float* out, uint32_t B, uint32_t nkv, uint32_t rep,
                    uint64_t rows);

/* ---- KV cache counters (model.rs:195-363) -------------------------------- */

typedef struct orc_kv {
  uint64_t offset, len, write_pos, max_len;
} orc_kv;

void orc_kv_init(orc_kv* c, uint64_t max_len);       /* KVCache::new      */
void orc_kv_advance(orc_kv* c, uint64_t n);          /* advance  :293-302 */
void orc_kv_update(orc_kv* c);                       /* update   :245-251 */
void orc_kv_reset(orc_kv* c);                        /* reset    :325-331 */
void orc_kv_rollback(orc_kv* c, uint64_t n);         /* rollback :352-362 */

/* ---- decode attention ---------------------------------------------------- */

/*
 * shader_attention.wgsl:43-156 in its exact f32 evaluation order: 256 lanes,
 * lane t takes rows t, t+256, ...; per-lane online softmax; tree merge of
 * (max, sum); per-dimension tree sum; divide by the sum.  One "workgroup" per
 * head; OpenMP over heads.  q/out [H][D]; k/v row p of head h at
 * h*kv_head_stride + p*D.
 */
void orc_attention_wgsl(const float* q, const float* k, const float* v, float* out,
                        uint32_t H, uint32_t D, uint32_t S, float scale,
                        uint64_t kv_head_stride);

/*
 * The same, over a wrapped ring window: row i of head h is slot
 * (start + i) % M of a [H][M][D] cache.  The window is gathered into order
 * and passed to orc_attention_wgsl (the reference's view is the unwrapped
 * special case start = 0, model.rs:252-258).
 */
void orc_attention_ring_wgsl(const float* q, const float* kc, const float* vc, float* out,
                             uint32_t H, uint32_t D, uint32_t M, uint32_t start,
                             uint32_t len, float scale);
/* A temporal decode frame: every (layer, head) over its ring window, shader
 * order, parallel over (layer, head). */
void orc_decode_frame_wgsl(const float* const* q, const float* const* kc,
                           const float* const* vc, float* const* out, uint32_t L, uint32_t H,
                           uint32_t D, uint32_t M, const uint32_t* starts, const uint32_t* lens,
                           float scale);

/*
 * Textbook softmax(scale * q K^T) V in double over the same ring window
 * (the closed form the shader computes).  out is double [H][D].
 */
void orc_attention_ring_f64(const float* q, const float* kc, const float* vc, double* out,
                            uint32_t H, uint32_t D, uint32_t M, uint32_t start,
                            uint32_t len, double scale);

/* ---- chunked prefill ----------------------------------------------------- */

/*
 * Causal prefill in double: q/out [S][H][D]; query i sits at window row
 * w_i = len - S + i and attends window rows 0..w_i (model.rs:551-557 mask
 * "j > offset + i", applied to softmax((Q K^T) * scale) V, model.rs:789-792).
 */
void orc_prefill_f64(const float* q, const float* kc, const float* vc, double* out,
                     uint32_t S, uint32_t H, uint32_t D, uint32_t M, uint32_t start,
                     uint32_t len, double scale);

/*
 * What the reference actually executes for a prefill (stream.rs:482-492):
 * S sequential decodes, query i over the first w_i + 1 window rows, each in
 * the shader's f32 order.  q/out [S][H][D].
 */
void orc_prefill_seq_wgsl(const float* q, const float* kc, const float* vc, float* out,
                          uint32_t S, uint32_t H, uint32_t D, uint32_t M, uint32_t start,
                          uint32_t len, float scale);

/* ---- Q4_K weights and matvec (gguf.rs, wgsl/shader_q4k_matvec.wgsl) ------
 * A Q4_K matrix [N][K] is N rows of K/256 super-blocks of 144 bytes:
 * d (f16), dmin (f16), 12 bytes of packed 6-bit sub-block scales and mins,
 * 128 bytes of 4-bit quants (shader_q4k_matvec.wgsl:13-19).  Weight k of
 * sub-block j is (d*scale_j)*q - (dmin*min_j). */

/* WGSL unpack2x16float as the Q4_K shaders use it (shader_q4k_matvec.wgsl:82):
 * exact binary16 -> binary32. */
float orc_f16_to_f32(uint16_t bits);

/* orc_f16_to_f32 over n values (elementwise; for tests). */
void orc_f16_to_f32_n(const uint16_t* bits, float* out, uint64_t n);

/* f32 -> f16 bits, round to nearest even (numpy's astype(float16), which
 * scripts/quantize.py:193-194 uses). */
uint16_t orc_f32_to_f16(float x);

/* shader_q4k_matvec.wgsl:85-113 (= shader_q4k.wgsl:48-63): 6-bit scale and
 * min of sub-block j (0..7) from the 12 packed bytes. */
void orc_q4k_scale_min(const uint8_t* scales12, uint32_t j, uint32_t* sc, uint32_t* mn);

/* Dequantised weights w[N][K], in the shader's f32 order
 * (shader_q4k_matvec.wgsl:117-136): d1 = d*scale, m1 = dmin*min, w = q*d1 - m1. */
void orc_q4k_dequant(const uint8_t* blocks, uint32_t N, uint32_t K, float* w);

/* scripts/quantize.py:162-253 quantize_q4_k, row by row (K % 256 == 0). */
void orc_q4k_quantize(const float* x, uint32_t N, uint32_t K, uint8_t* blocks);

/* shader_q4k_matvec.wgsl:48-356 for each output y[b][n] (x [B][K], y [B][N]):
 * acc over super-blocks in order; per block 4 iterations of 8 words; per
 * word acc += dot(lo) then acc += dot(hi), dot evaluated left to right
 * (WGSL leaves the order of dot() to the implementation). */
void orc_q4k_matvec_wgsl(const uint8_t* blocks, const float* x, float* y, uint32_t B,
                         uint32_t K, uint32_t N);

/* y = W x in double over the dequantised weights. */
void orc_q4k_matvec_f64(const uint8_t* blocks, const float* x, double* y, uint32_t B,
                        uint32_t K, uint32_t N);

/* ---- depformer step chain (depth_engine.rs:884-1491) ---------------------- */

/* shader_rmsnorm.wgsl:27-92 for one row of D: thread t (of 256) sums
 * x[t]^2, x[t+256]^2, ... in order; tree sum (t += t+128, ..., then s0 + s1);
 * rms = sqrt(sum / D + eps); out[i] = x[i] * (1 / rms) * alpha[i]. */
void orc_rmsnorm_wgsl(const float* x, const float* alpha, float* out, uint32_t D, float eps);

/* shader_swiglu.wgsl:24-35: out[i] = gate[i] / (1 + exp(-gate[i])) * value[i],
 * gate = in[0..F), value = in[F..2F). */
void orc_swiglu(const float* in, float* out, uint32_t F);

/* shader_embed_q4.wgsl:58-107: row `token` of a Q4_0 table [vocab][dim]
 * (18-byte blocks: f16 scale, 16 bytes of nibbles; element j < 16 is the low
 * nibble of byte j, j >= 16 the high nibble of byte j-16; value
 * (nibble - 8) * scale, an Inf/NaN scale reads as 0); zeros if
 * token >= vocab. */
void orc_embed_q4_0(const uint8_t* table, uint32_t vocab, uint32_t dim, uint32_t token,
                    float* out);

/* shader_sample_topk.wgsl:37-221 on one logits row (modified in place as the
 * shader does): repetition penalty on the listed tokens (a token listed twice
 * is penalised once: the shader's lanes read before they write), division by
 * the temperature, then argmax (top_k <= 1) or top-k selection, insertion
 * sort, softmax and the cumulative draw against `rand`.  Returns the token. */
uint32_t orc_sample_topk_wgsl(float* logits, uint32_t V, uint32_t top_k, float temperature,
                              float penalty, float rand, const uint32_t* penalty_tokens,
                              uint32_t num_penalty);
uint32_t orc_sample_topk_wgsl_ex(float* logits, uint32_t V, uint32_t top_k, float temperature,
                                 float penalty, float rand, const uint32_t* penalty_tokens,
                                 uint32_t num_penalty, uint32_t* idx_out, float* cum_out);

typedef struct orc_depformer_cfg {
  uint32_t num_steps, num_layers, dim, num_heads, ffn, temporal_dim;
  uint32_t out_vocab, text_emb_vocab, audio_emb_vocab, num_audio_emb, kv_max_len;
  float rms_eps, attn_scale;
} orc_depformer_cfg;

/* Weights: Q4_K matrices (input_proj[step] [dim][temporal_dim];
 * attn_in_proj, attn_out_proj, ffn_linear_in, ffn_linear_out indexed
 * layer * num_steps + step, shapes [3 dim][dim], [dim][dim], [2 ffn][dim],
 * [dim][ffn]; output_linear[step] [out_vocab][dim]), f32 norm alphas per
 * layer, Q4_0 embeddings (text_emb, audio_emb[i]). */
typedef struct orc_depformer_weights {
  const uint8_t* const* input_proj;
  const uint8_t* const* attn_in_proj;
  const uint8_t* const* attn_out_proj;
  const uint8_t* const* ffn_linear_in;
  const uint8_t* const* ffn_linear_out;
  const float* const* norm1_alpha;
  const float* const* norm2_alpha;
  const uint8_t* const* output_linear;
  const uint8_t* text_emb;
  const uint8_t* const* audio_emb;
} orc_depformer_weights;

/* DepthEngine::generate (depth_engine.rs:884-1491) for one stream, every op
 * in its shader's f32 order: input projections of the temporal hidden state,
 * then per step: embedding of the previous token (text_token at step 0,
 * audio_emb[min(step-1, n-1)] after) added to the projection, num_layers
 * blocks (rmsnorm, QKV projection, cache write at slot `step`, attention
 * over slots 0..step, out_proj + residual, rmsnorm, linear_in, SwiGLU,
 * linear_out + residual), output linear, top-k sampling.  rand
 * [num_steps], penalty_tokens [num_steps][30], num_penalty [num_steps];
 * tokens [num_steps].  logits [num_steps][out_vocab] (before sampling) and
 * hidden [num_steps][dim] (input of the output linear) may be NULL. */
void orc_depformer_generate(const orc_depformer_cfg* cfg, const orc_depformer_weights* w,
                            const float* temporal_hidden, uint32_t text_token, uint32_t top_k,
                            float temperature, float penalty, const float* rand,
                            const uint32_t* penalty_tokens, const uint32_t* num_penalty,
                            uint32_t* tokens, float* logits, float* hidden);

/* Number of OpenMP threads the oracle uses (for the CPU-baseline record). */
int orc_num_threads(void);
void orc_set_num_threads(int n);
int orc_bind_threads(const int* cpus, int n, int pin);

#ifdef __cplusplus
}
#endif

#endif
