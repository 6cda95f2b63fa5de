/*
 * sts_attn.h -- C ABI of the MI355X (gfx950) attention hot path of sts-web.
 *
 * This library replaces, behind plain C entry points, the attention op and the
 * ring-buffer KV cache of idle-intelligence/sts-web (paths below are relative
 * to crates/sts-wasm/src/ of that repository):
 *
 *   fused_attention          model.rs:598-668  + wgsl/shader_attention.wgsl
 *   gpu_cache_write_v        model.rs:143-188  + wgsl/shader_cache_write.wgsl
 *   KVCache / LayerCaches    model.rs:195-411
 *   RoPE                     model.rs:38-122
 *   prefill branch           model.rs:760-797, 837-873 (causal mask 539-563)
 *   depformer step attention depth.rs:79-273, depth_engine.rs:1121-1209
 *   Q4_K matmul              gguf.rs:808-905   + wgsl/shader_q4k*.wgsl
 *   depformer step chain     depth_engine.rs:884-1491 (RMSNorm, SwiGLU, Q4_0
 *                            embeddings, top-k sampling)
 *
 * Conventions (every entry point):
 *   - Returns int status: STS_OK (0) on success, a negative STS_ERR_* code
 *     otherwise.  sts_last_error() returns a message for the calling thread's
 *     last failure.  No entry point aborts the process.
 *   - Pointers named q/k/v/out/input/cache are DEVICE pointers (hipMalloc'd or
 *     owned by the caller's tensor library), f32, contiguous as documented.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).  All
 *     device work is enqueued asynchronously on it; nothing blocks the host
 *     except the one-time allocation of library workspace (see below).
 *   - head_dim is a multiple of 4 up to 128.  The model's two head sizes
 *     (temporal 4096/32 = 128, depformer 1024/16 = 64; lib.rs:128-140) run
 *     their own kernels; the others run a padded decode kernel, and their
 *     prefill is the chunk's queries as decodes over their causal windows, in
 *     f32 whatever precision is asked (the bf16-K/V prefill takes 64 and 128
 *     only).  The reference shader takes any head_dim up to 128 and silently
 *     overflows beyond (shader_attention.wgsl:36, :66); here that is an
 *     error, and so is a head_dim that is not a multiple of 4.
 *   - Attention entry points use a per-(device, stream) workspace owned by the
 *     library for split-KV partial results.  It is allocated (hipMalloc) on the
 *     first call on a stream that needs it and grown when a larger launch needs
 *     more; replaced buffers are retired, not freed, so graphs captured earlier
 *     stay valid.  A call that would allocate or grow it while its stream is
 *     being captured into a HIP graph fails with STS_ERR_STATE: run the largest
 *     call once on the stream before capturing it.  Calls issued on the same
 *     stream are ordered; calls on different streams use different workspaces.
 *   - Handles are not internally locked: use one handle from one host thread at
 *     a time (the reference's caches are !Sync, model.rs:483).
 */
#ifndef STS_ATTN_H
#define STS_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define STS_ATTN_ABI_VERSION 3

enum sts_status {
  STS_OK = 0,
  STS_ERR_INVALID = -1, /* bad argument: null pointer, size, head_dim, range */
  STS_ERR_HIP = -2,     /* a HIP runtime call failed (message has the code)  */
  STS_ERR_STATE = -3,   /* handle in the wrong state for the call            */
  STS_ERR_NOMEM = -4,   /* device or host allocation failed                  */
  STS_ERR_DEVICE = -5   /* a kernel raised a device error flag (sts_device_errors) */
};

/* Bits of the device error word (sts_device_errors). */
enum sts_device_error {
  STS_DEVERR_WAIT_TIMEOUT = 1 /* a bounded wait between the waves of a workgroup
                                 gave up (bf16 prefill kernels); outputs written
                                 since the last check are invalid               */
};

enum sts_precision {
  STS_PREC_F32 = 0,           /* f32 inputs, f32 arithmetic                  */
  STS_PREC_BF16_MFMA = 1,     /* f32 inputs rounded to bf16 for MFMA, f32 accumulate */
  STS_PREC_F32_SPLIT_BF16 = 2 /* f32 inputs split into bf16 hi + lo (16 significant
                                 bits), each product as three bf16 MFMAs
                                 (hi*hi + hi*lo + lo*hi), f32 accumulate, on the
                                 bf16 matrix rate.  The scores carry a relative
                                 error of ~2^-16, so the result error grows with
                                 the score range: within 1e-4 of f64 for scores of
                                 standard deviation up to ~4 (STS_PREC_F32 stays
                                 within 1e-4 far beyond).  Prefill only.         */
};

/* Message for the calling thread's most recent failed call ("" if none). */
const char* sts_last_error(void);

/* STS_ATTN_ABI_VERSION of the loaded library. */
int sts_abi_version(void);

/* ------------------------------------------------------------------------ */
/* Stateless ops (raw device pointers)                                       */
/* ------------------------------------------------------------------------ */

/*
 * Single-query attention over the first `seq_len` rows of a K/V buffer.
 * Replaces fused_attention (model.rs:598-668), which launches
 * shader_attention.wgsl with info [num_heads, head_dim, seq_len, scale_bits,
 * kv_head_stride] (model.rs:631-640).
 *   q   [num_heads][head_dim]                        (contiguous)
 *   k,v row p of head h at  h*kv_head_stride + p*head_dim   (p < seq_len)
 *   out [num_heads][head_dim]                        (caller-owned)
 *   out_h = sum_p softmax_p(scale * q_h . k_{h,p}) v_{h,p}
 * seq_len must be >= 1 and kv_head_stride >= seq_len*head_dim.
 */
int sts_fused_attention(const float* q, const float* k, const float* v, float* out,
                        uint32_t num_heads, uint32_t head_dim, uint32_t seq_len,
                        float scale, uint64_t kv_head_stride, void* stream);

/*
 * Ring-buffer append.  Replaces gpu_cache_write_v (model.rs:143-188) and
 * shader_cache_write.wgsl:19-49, bit for bit:
 *   cache[((b*H + h)*max_len + (pos_offset + s) % max_len)*D + d]
 *       = input[((b*S + s)*H + h)*D + d]
 *   input [B][S][H][D],  cache [B][H][max_len][D].
 * Any head_dim >= 1 is accepted here (pure copy).  Slots not addressed are
 * left untouched.  Writes from one call must not collide: S <= max_len.
 */
int sts_cache_write(const float* input, float* cache, uint32_t pos_offset,
                    uint32_t batch, uint32_t seq, uint32_t heads, uint32_t head_dim,
                    uint32_t max_len, void* stream);

/*
 * Decode attention over a wrapped ring window, batched over streams with
 * ragged lengths (the generalisation of fused_attention that the cache needs
 * once the ring wraps; the reference's view assumes the window starts at slot
 * 0, model.rs:252-258).
 *   q, out       [batch][heads][head_dim]
 *   k/v cache    [batch][heads][max_len][head_dim]
 *   lens[b]      valid rows of stream b, 0..max_len   (device int32 array)
 *   starts[b]    slot of stream b's oldest row, 0..max_len-1 (device int32)
 *   row i (0 <= i < lens[b]) of stream b lives in slot (starts[b]+i) % max_len
 * A stream with lens[b] == 0 gets out = 0.  lens/starts outside their ranges
 * are clamped on the device (len to max_len, start modulo max_len).
 */
int sts_decode_ring(const float* q, const float* k_cache, const float* v_cache,
                    float* out, const int32_t* lens, const int32_t* starts,
                    uint32_t batch, uint32_t heads, uint32_t head_dim, uint32_t max_len,
                    float scale, void* stream);

/*
 * sts_decode_ring without any allocation: no counterpart in the reference.
 * For callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, checks and results (bit for bit) as sts_decode_ring; the split
 * partial records and arrival counters live in a static device array of the
 * library (8 MiB of records and 16384 counters, per GPU, held until the
 * process ends) instead of the per-stream workspace.  It calls no hipMalloc,
 * hipFree or allocating routine.  A launch that needs more than that array
 * holds (batch * heads * nsplit * (head_dim + 4) floats, nsplit up to 64 and
 * chosen as sts_decode_ring chooses it; e.g. 64 streams x 32 heads x 3000
 * rows fits) fails with STS_ERR_INVALID.  Every call on a GPU shares that GPU's
 * array: calls that overlap in time on one GPU (two streams, or a replayed
 * graph beside an eager call) race and must not be issued.
 */
int sts_decode_ring_noalloc(const float* q, const float* k_cache, const float* v_cache,
                            float* out, const int32_t* lens, const int32_t* starts,
                            uint32_t batch, uint32_t heads, uint32_t head_dim,
                            uint32_t max_len, float scale, void* stream);

/*
 * Depformer step attention, batched over independent streams: appends the
 * step's K/V row at slot `step` and attends over slots 0..step (L = step+1),
 * in one launch.  Replaces the per-step cache-write K, cache-write V and
 * attention dispatches of depth_engine.rs:1121-1209 (info buffers
 * depth_engine.rs:626-645, 725-741) and the decode branch of
 * MultiLinearAttention (depth.rs:104-119, 203-217).
 *   q, k_new, v_new: stream b's rows at  ptr + b*qkv_stride  ([heads][head_dim]
 *                    each; qkv_stride = 3*heads*head_dim for a packed qkv_out)
 *   k/v cache        [batch][heads][max_len][head_dim]
 *   out              [batch][heads][head_dim]
 * Requires step < max_len.  No RoPE (depformer has none, depth.rs:100).
 */
int sts_depformer_step(const float* q, const float* k_new, const float* v_new,
                       uint64_t qkv_stride, float* k_cache, float* v_cache, float* out,
                       uint32_t batch, uint32_t heads, uint32_t head_dim,
                       uint32_t max_len, uint32_t step, float scale, void* stream);

/*
 * Chunked causal prefill attention over a ring window (batch 1).  The chunk's
 * `seq` rows must already be appended: they are the last `seq` rows of the
 * window.  Query i (0 <= i < seq) sits at window row w_i = win_len - seq + i
 * and attends window rows 0..w_i.  This is the semantics of the reference's
 * prefill branch (model.rs:784-792, mask model.rs:551-557: key j masked when
 * j > offset + i) and of the S sequential decodes the reference actually runs
 * (stream.rs:482-492).
 *   q, out     [seq][heads][head_dim]
 *   k/v cache  [heads][max_len][head_dim];  window row r in slot (win_start + r) % max_len
 * precision: STS_PREC_F32, STS_PREC_BF16_MFMA or STS_PREC_F32_SPLIT_BF16.
 */
int sts_prefill_attention(const float* q, const float* k_cache, const float* v_cache,
                          float* out, uint32_t seq, uint32_t heads, uint32_t head_dim,
                          uint32_t max_len, uint32_t win_start, uint32_t win_len,
                          float scale, int precision, void* stream);

/*
 * sts_prefill_attention at STS_PREC_BF16_MFMA over bf16 copies of the caches:
 * k16, v16 [heads][max_len][head_dim] hold the caches' values rounded to bf16
 * (nearest even, the rounding that precision applies to the f32 rows), so
 * the result equals sts_prefill_attention's bit for bit while the kernel
 * reads half the K/V bytes and converts nothing.  No counterpart in the
 * reference; the bf16 mirror of a KV handle (STS_KV_BF16_MIRROR) keeps such
 * copies.  All pointers 16-byte aligned.
 */
int sts_prefill_attention_bf16kv(const float* q, const uint16_t* k16, const uint16_t* v16,
                                 float* out, uint32_t seq, uint32_t heads, uint32_t head_dim,
                                 uint32_t max_len, uint32_t win_start, uint32_t win_len,
                                 float scale, void* stream);

/* ------------------------------------------------------------------------ */
/* RoPE (model.rs:38-122)                                                     */
/* ------------------------------------------------------------------------ */

typedef struct sts_rope sts_rope;

/*
 * Builds the cos/sin tables [max_seq_len][head_dim/2] of RoPE::new
 * (model.rs:46-66): inv_freq_j = 1 / theta^(2j/head_dim) and
 * angle = pos * inv_freq_j, both in f32 as the reference computes them; cos
 * and sin of each f32 angle are rounded to nearest f32.  Uploads them to the
 * current device (synchronous, once).
 */
int sts_rope_create(uint32_t head_dim, uint32_t max_seq_len, float theta, sts_rope** out);
/* Frees the tables (hipFree): not while a stream of the device is being
 * captured into a graph, which a free inside the capture would invalidate. */
int sts_rope_destroy(sts_rope* rope);

/*
 * In-place interleaved rotation of x [batch][seq][heads][head_dim] at
 * positions offset..offset+seq-1 (RoPE::apply_rope_to_tensor,
 * model.rs:79-105): pair (x0, x1) = (x[2j], x[2j+1]) becomes
 * (x0*c - x1*s, x0*s + x1*c).  offset+seq must not exceed max_seq_len
 * (the reference slices the table there, model.rs:92-95).
 */
int sts_rope_apply(const sts_rope* rope, float* x, uint32_t batch, uint32_t seq,
                   uint32_t heads, uint32_t offset, void* stream);

/* ------------------------------------------------------------------------ */
/* KV cache handle (KVCache, model.rs:195-363)                               */
/* ------------------------------------------------------------------------ */

typedef struct sts_kv_cache sts_kv_cache;

typedef struct sts_kv_state {
  uint64_t offset;    /* logical rows ever appended, minus rollbacks       */
  uint64_t len;       /* valid rows, min(count, max_len)                   */
  uint64_t write_pos; /* next slot to write, offset % max_len unless rolled */
  uint64_t max_len;
  uint64_t heads;
  uint64_t head_dim;
  uint64_t batch;     /* 0 until the buffers are allocated                 */
  int32_t allocated;  /* 1 when the K/V buffers exist                      */
  int32_t flags;      /* the sts_kv_create_ex flags (STS_KV_BF16_MIRROR)   */
  uint64_t q_heads;   /* query heads of q/out (sts_kv_set_query_heads)     */
} sts_kv_state;

/* sts_kv_create_ex flag: keep a bf16 copy of K and V (see sts_kv_create_ex). */
#define STS_KV_BF16_MIRROR 1u

/* KVCache::new (model.rs:207-219).  Allocates nothing on the device. */
int sts_kv_create(uint64_t max_len, uint64_t heads, uint64_t head_dim, sts_kv_cache** out);

/*
 * sts_kv_create with flags; no counterpart in the reference (its caches are
 * f32 only).  STS_KV_BF16_MIRROR: the handle also keeps K and V rounded to
 * bf16 (nearest even; same layout, half the bytes), written by every append
 * made through the handle (sts_kv_update, sts_kv_decode_step,
 * sts_kv_prefill) and cleared with the caches.  sts_kv_prefill with
 * STS_PREC_BF16_MFMA then reads the mirror: the same result bit for bit (it
 * holds exactly the values that kernel rounds the f32 rows to), half the K/V
 * bytes.  The f32 caches stay the reference's, bit for bit.  Rows written
 * into the f32 buffers by other means (sts_cache_write on the pointers of
 * sts_kv_ensure_allocated) reach the mirror only through sts_kv_sync_mirror.
 * A mirrored cache needs 16-byte aligned inputs in sts_kv_update.
 */
int sts_kv_create_ex(uint64_t max_len, uint64_t heads, uint64_t head_dim, uint32_t flags,
                     sts_kv_cache** out);

/* The bf16 mirror buffers [batch][heads][max_len][head_dim] (bf16 bits), or
 * NULL when the cache has none or is not allocated yet. */
int sts_kv_mirror(const sts_kv_cache* cache, uint16_t** k16, uint16_t** v16);

/* Rebuilds the bf16 mirror from the f32 caches (after direct writes). */
int sts_kv_sync_mirror(sts_kv_cache* cache, void* stream);

/*
 * Grouped-query attention (the prefill branch's K/V expansion,
 * model.rs:766-783, which the reference also takes for S = 1 when
 * n_heads != n_kv_heads, model.rs:739): the cache holds `heads` K/V heads and
 * q / out of sts_kv_attend, sts_kv_decode_step and sts_kv_prefill have
 * q_heads heads, a multiple of heads; query head h attends K/V head
 * h / (q_heads / heads), i.e. each K/V head repeated for q_heads / heads
 * consecutive query heads.  k_new / v_new keep `heads` heads.  The default
 * is q_heads = heads.
 */
int sts_kv_set_query_heads(sts_kv_cache* cache, uint64_t q_heads);
/* Frees the buffers (hipFree): not while a stream of the device is being
 * captured into a graph, which a free inside the capture would invalidate. */
int sts_kv_destroy(sts_kv_cache* cache);

/*
 * KVCache::ensure_allocated (model.rs:270-284): allocates zero-filled K and V
 * buffers [batch][heads][max_len][head_dim] on first use and returns them with
 * the current write position.  A later call with another batch fails.
 */
int sts_kv_ensure_allocated(sts_kv_cache* cache, uint64_t batch, float** k, float** v,
                            uint64_t* write_pos, void* stream);

/* Counters (model.rs:313-323), plus write_pos and allocation state. */
int sts_kv_get_state(const sts_kv_cache* cache, sts_kv_state* out);

/*
 * The logical window: row i (0 <= i < len) is in slot (start + i) % max_len,
 * start = (write_pos + max_len - len) % max_len.
 */
int sts_kv_window(const sts_kv_cache* cache, uint64_t* start, uint64_t* len);

/* KVCache::advance (model.rs:293-311), counters only. */
int sts_kv_advance(sts_kv_cache* cache, uint64_t n);

/*
 * Append `seq` rows and advance: KVCache::update (model.rs:221-268), with the
 * chunk written at slots (offset+s) % max_len as gpu_cache_write_v does (the
 * reference's update writes a single slot, model.rs:245-246).  k_new, v_new
 * are [batch][seq][heads][head_dim].  Allocates on first use.  seq <= max_len.
 */
int sts_kv_update(sts_kv_cache* cache, const float* k_new, const float* v_new,
                  uint64_t batch, uint64_t seq, void* stream);

/* KVCache::reset (model.rs:325-331): frees the buffers, zeroes counters. */
int sts_kv_reset(sts_kv_cache* cache);

/* KVCache::reset_keep_buffers (model.rs:333-345): zero-fills, zeroes counters. */
int sts_kv_reset_keep_buffers(sts_kv_cache* cache, void* stream);

/* KVCache::rollback (model.rs:352-362): n is clamped to len. */
int sts_kv_rollback(sts_kv_cache* cache, uint64_t n);

/*
 * Decode attention over the cache's current window for each stream of the
 * batch (equal lengths): q, out [batch][q_heads][head_dim] (q_heads = heads
 * unless set by sts_kv_set_query_heads).  This is fused_attention(q, k_all,
 * v_all) on the views advance() returns (model.rs:829-831), generalised to a
 * wrapped window.
 */
int sts_kv_attend(sts_kv_cache* cache, const float* q, float* out, float scale, void* stream);

/*
 * One fused decode step of the temporal (or depformer) attention: optional
 * RoPE of q and k_new at position `offset`, append of k_new/v_new at slot
 * write_pos, advance(1), and attention over the new window -- the decode
 * branch of Q4Attention::forward_with_cache (model.rs:739-758, 818-835) in one
 * launch.  q, out are [batch][q_heads][head_dim], k_new, v_new
 * [batch][heads][head_dim].  `rope` may be
 * NULL (depformer, depth.rs:100); when given, q and k_new are read unrotated
 * and the rotated q is not written back.  Allocates the cache on first use.
 */
int sts_kv_decode_step(sts_kv_cache* cache, const sts_rope* rope, const float* q,
                       const float* k_new, const float* v_new, float* out,
                       uint64_t batch, float scale, void* stream);

/*
 * Chunked prefill (batch 1): the prefill branch of
 * Q4Attention::forward_with_cache (model.rs:760-797) with a working
 * multi-row append.  With `rope` set, q and k_new are read unrotated and
 * rotated at positions offset..offset+seq-1 (RoPE::apply, model.rs:760-764):
 * k inside the append, which writes the K and V rows
 * ([seq][heads][head_dim]) at slots (offset+s) % max_len in one launch, and q
 * in registers inside the attention kernel (the rotated q is not written
 * back).  With rope NULL, q and k_new are taken as already rotated.  Then
 * causal attention of the `seq` queries q [seq][q_heads][head_dim] over the
 * grown window into out (with q_heads > heads, grouped-query attention as
 * sts_kv_set_query_heads describes).  Every argument is checked before anything is
 * written: a rejected call leaves the cache and its counters unchanged.
 * q, k_new, v_new, out 16-byte aligned; offset+seq must not exceed the RoPE
 * table.
 */
int sts_kv_prefill(sts_kv_cache* cache, const sts_rope* rope, const float* q,
                   const float* k_new, const float* v_new, float* out, uint64_t seq,
                   float scale, int precision, void* stream);

/* ---- device error word ---------------------------------------------------- */

/*
 * Synchronises `stream`, then reads and clears the current device's error
 * word (STS_DEVERR_* bits raised by kernels since the last call, on any
 * stream) into *flags (may be NULL).  Returns STS_ERR_DEVICE when a bit was
 * set.  No counterpart in the reference: its WGSL shaders have no bounded
 * waits.  The bf16 prefill kernels' waves hand over LDS stages through
 * bounded polls; a poll that gives up sets STS_DEVERR_WAIT_TIMEOUT instead of
 * hanging the GPU.
 */
int sts_device_errors(void* stream, uint32_t* flags);

/*
 * Test hook, no counterpart in the reference: the number of polls after which
 * the bounded waits give up (0 restores the default, 2^24).  A small value
 * makes the waits give up on purpose so that tests can check that the error
 * word reports it while every kernel still exits normally.
 */
int sts_debug_set_wait_limit(uint32_t polls);

/* ---- Q4_K projections (the matvecs on either side of attention) --------- */

/*
 * y = W x (+ residual) for a Q4_K weight matrix W [n][k]: q4k_matmul with
 * M = 1 and q4k_matmul_with_residual (gguf.rs:808-905, kernel
 * wgsl/shader_q4k_matvec.wgsl) -- the in_proj / out_proj (and FFN) products
 * of every decode step (model.rs:730, :834).  `weights` holds the tensor as
 * the GGUF file stores it (Q4KTensor::from_q4k_bytes, gguf.rs:530-563):
 * n rows of k/256 super-blocks of 144 bytes.  x is [batch][k] (the
 * reference's [B, 1, K] input), y [batch][n], residual [batch][n] or NULL.
 * k must be a multiple of 256 and at most 16384; weights and x 16-byte
 * aligned.  Each batch row reads the whole weight matrix once.
 */
int sts_q4k_matvec(const uint8_t* weights, const float* x, const float* residual, float* y,
                   uint32_t batch, uint32_t k, uint32_t n, void* stream);

/*
 * Dequantise a Q4_K matrix to f32 out [n][k], each weight rounded as the
 * reference shader computes it: d1 = d*scale, m1 = dmin*min, w = q*d1 - m1
 * (shader_q4k_matvec.wgsl:117-136).
 */
int sts_q4k_dequant(const uint8_t* weights, float* out, uint32_t k, uint32_t n, void* stream);

/* ---- depformer step chain (depth_engine.rs:884-1491), batched over streams -
 *
 * The reference's DepthEngine runs one stream per frame as ~360 WGSL
 * dispatches.  These entry points run B streams at once: every Q4_K product
 * becomes a GEMM with the streams as rows, so each weight byte is read once
 * per frame for the whole batch. */

/*
 * Y[m][n] = sum_k W[n][k] X[m][k] (+ residual[m][n]) for m < rows: the Q4_K
 * product for more than one row, which the reference runs with the
 * one-thread-per-output shader (q4k_matmul with M > 1, gguf.rs:810-897 and
 * wgsl/shader_q4k.wgsl; q4k_matmul_with_residual, gguf.rs:899-905).  The
 * weights are dequantised exactly as the shader rounds them and multiplied
 * in f32 on the matrix cores.  With swiglu != 0 the matrix has n = 2F rows and
 * y[m][j] = silu(G[m][j]) * G[m][j + F] for j < F (the SwiGLU of
 * wgsl/shader_swiglu.wgsl applied to the product; residual must be NULL).
 * With norm_alpha non-NULL each x row is first RMS-normalised,
 * x * (1/sqrt(mean(x^2) + norm_eps)) * norm_alpha (the RMSNorm that precedes
 * every projection of the depformer, depth_engine.rs:1069-1095, 1262-1282,
 * fused; its sum of squares is taken in this kernel's order, not the
 * shader's).  k must be a multiple of 256 in 256..16384; above 4096 (the
 * temporal FFN's linear_out, k = 11264) the product runs as slices of 4096
 * summed in slice order by a second kernel, through the stream's library
 * workspace (see the workspace rules above), without norm_alpha or swiglu.
 * x rows, norm_alpha and weights 16-byte aligned; ldx, ldy, ldr are row
 * strides in floats (ldx a multiple of 4).
 */
int sts_q4k_gemm(const uint8_t* weights, const float* x, uint64_t ldx, const float* norm_alpha,
                 float norm_eps, const float* residual, uint64_t ldr, float* y, uint64_t ldy,
                 uint32_t rows, uint32_t k, uint32_t n, int swiglu, void* stream);

/*
 * RMSNorm of each row of x [rows][dim]: out = x * (1/sqrt(mean(x^2) + eps)) * alpha,
 * summed in wgsl/shader_rmsnorm.wgsl's order (bit-identical results).
 */
int sts_rmsnorm(const float* x, const float* alpha, float* out, uint32_t rows, uint32_t dim,
                float eps, void* stream);

/*
 * h[b][e] = proj[b][e] + E[token_b][e] for a Q4_0 embedding table E [vocab][dim]
 * (wgsl/shader_embed_q4.wgsl + shader_vec_add.wgsl, depth_engine.rs:988-1057);
 * token_b = tokens[b * tok_stride] (device), out-of-vocab tokens embed as zeros.
 * The table is 2-byte aligned (each 18-byte block starts with its f16 scale).
 */
int sts_embed_add_q4_0(const uint8_t* table, uint32_t vocab, const uint32_t* tokens,
                       uint64_t tok_stride, const float* proj, float* h, uint32_t batch,
                       uint32_t dim, void* stream);

/*
 * Top-k sampling with repetition penalty and temperature for each stream b
 * (wgsl/shader_sample_topk.wgsl, depth_engine.rs:1411-1439): logits row b at
 * logits + b*ld (not modified), rand[b*rs_stride] in [0,1),
 * penalty tokens ptoks[b*pt_stride ..] (num_penalty[b*rs_stride] of them, at
 * most 30), token to out[b*out_stride].  top_k <= 1 is the argmax.
 * vocab <= 4096, top_k <= 256.  The top k and their order equal the
 * shader's for distinct logits (among equal logits, -0 and +0 included, this
 * build ranks lower indices first); the softmax sum and running total are
 * summed in a
 * different f32 order, so the draw can differ only where rand lies within
 * rounding of a cumulative boundary.
 */
int sts_sample_topk(const float* logits, uint64_t ld, uint32_t batch, uint32_t vocab,
                    uint32_t top_k, float temperature, float penalty, const float* rand,
                    const uint32_t* ptoks, uint64_t pt_stride, const uint32_t* num_penalty,
                    uint64_t rs_stride, uint32_t* out, uint64_t out_stride, void* stream);

/* DepthEngineConfig (depth_engine.rs:50-107). */
typedef struct sts_depformer_config {
  uint32_t num_steps;       /* depth steps per frame (8)                       */
  uint32_t num_layers;      /* 6                                               */
  uint32_t dim;             /* 1024                                            */
  uint32_t num_heads;       /* 16 (head_dim = dim / num_heads = 64)            */
  uint32_t ffn;             /* 2816 (linear_in has 2*ffn rows)                 */
  uint32_t temporal_dim;    /* 4096                                            */
  uint32_t out_vocab;       /* 2048                                            */
  uint32_t text_emb_vocab;  /* 32001                                           */
  uint32_t audio_emb_vocab; /* 2049                                            */
  uint32_t num_audio_emb;   /* audio tables; step s >= 1 reads min(s-1, n-1)   */
  uint32_t kv_max_len;      /* 9 (>= num_steps)                                */
  float rms_eps;            /* 1e-8                                            */
  float attn_scale;         /* (dim / num_heads)^-0.5                          */
} sts_depformer_config;

/*
 * Device pointers to the weights (LayerStepWeights / StepWeights,
 * depth_engine.rs:114-175), owned by the caller for the handle's lifetime.
 * Q4_K matrices: input_proj[step] [dim][temporal_dim]; attn_in_proj,
 * attn_out_proj, ffn_linear_in, ffn_linear_out indexed [layer*num_steps + step],
 * shapes [3 dim][dim], [dim][dim], [2 ffn][dim], [dim][ffn];
 * output_linear[step] [out_vocab][dim].  f32 alphas per layer.  Q4_0 tables
 * text_emb [text_emb_vocab][dim], audio_emb[i] [audio_emb_vocab][dim].  Every
 * pointer must be 16-byte aligned.  The pointer arrays themselves are host
 * memory and are copied at create.
 */
typedef struct sts_depformer_weights {
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
} sts_depformer_weights;

typedef struct sts_depformer sts_depformer;

/* Validates the shapes, copies the weight pointers and allocates activations
 * and KV caches for up to max_batch streams (DepthEngine::new). */
int sts_depformer_create(const sts_depformer_config* cfg, const sts_depformer_weights* w,
                         uint32_t max_batch, sts_depformer** out);
int sts_depformer_destroy(sts_depformer* d);

/*
 * DepthEngine::generate (depth_engine.rs:884-1491) for `batch` streams:
 * temporal_hidden [batch][temporal_dim], text_token [batch] (u32),
 * rand [batch][num_steps], penalty_tokens [batch][num_steps][30],
 * num_penalty [batch][num_steps] -> tokens [batch][num_steps]; optional
 * logits [num_steps][batch][out_vocab] receives each step's logits before
 * sampling.  All device pointers; nothing is read back, so the call can be
 * captured in a HIP graph.  The KV caches start empty every call (the
 * reference clears them per frame, depth_engine.rs:1497-1509).
 */
int sts_depformer_generate(sts_depformer* d, const float* temporal_hidden,
                           const uint32_t* text_token, uint32_t batch, uint32_t top_k,
                           float temperature, float penalty, const float* rand,
                           const uint32_t* penalty_tokens, const uint32_t* num_penalty,
                           uint32_t* tokens, float* logits, void* stream);

/* ---------------------------------------------------------------------- */
/* Measurement                                                              */
/* ---------------------------------------------------------------------- */

/*
 * Plain-read roofline probe: no counterpart in the reference.  Reads a_bytes
 * at a and b_bytes at b (multiples of 16, 16-byte aligned; b may be null
 * with b_bytes 0) once, with 16-byte nontemporal loads and nothing else,
 * `workgroups` workgroups of 256 threads each streaming a contiguous share of
 * both buffers; stores one float per workgroup to sink[0..workgroups).
 * Timed on a kernel's own bytes and grid, it measures what a read of those
 * bytes reaches on the device, the ceiling that kernel is compared with.
 */
int sts_probe_stream_read(const void* a, uint64_t a_bytes, const void* b, uint64_t b_bytes,
                          uint32_t workgroups, float* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* STS_ATTN_H */
