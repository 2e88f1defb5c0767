/*
 * lbt.h -- C ABI of the MI355X (gfx950) packed-ternary x int8 hot path and
 * BitNet b1.58 token loop.  Drop-in boundary for festeraeb/lemonade-burn:
 * every entry point names the reference interface it replaces.
 *
 * Conventions
 *   - Every function returns 0 on success or a negative LBT_E_* code; it never
 *     aborts.  lbt_last_error(ctx) holds a message for the last failure.
 *   - Host-pointer entry points copy inputs in and outputs out (the reference's
 *     slice API).  `_dev` entry points take device pointers and run
 *     asynchronously on the context's stream (call lbt_ctx_synchronize).
 *   - Packed weights use the reference's LB2 layout unchanged
 *     (crates/lb-ternary/src/pack.rs:1-16): row-major [rows, padded(cols)/4]
 *     bytes, 128-weight blocks of 32 bytes, bits 2k..2k+1 of byte j = code
 *     (w + 1) of weight k*32 + j, padding code 1.
 *   - One context per host thread (like the reference's single model worker
 *     thread, crates/lb-server/src/main.rs:92-100); a context is not
 *     thread-safe.
 *   - Sizes (rows, columns, token counts, config dimensions) above 2^30 are
 *     refused with LBT_E_INVALID; token and step counts past the cache's
 *     room (max_position_embeddings, or a batch slot's capacity) with
 *     LBT_E_RANGE.  Both before any memory behind the pointers is read.
 */
#ifndef LBT_H
#define LBT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LBT_OK 0
#define LBT_E_INVALID (-1)   /* bad argument / shape mismatch (reference: assert!) */
#define LBT_E_DEVICE (-2)    /* HIP runtime error */
#define LBT_E_NOMEM (-3)     /* device allocation failed */
#define LBT_E_IO (-4)        /* file missing or malformed */
#define LBT_E_RANGE (-5)     /* context length exceeded */

typedef struct lbt_ctx lbt_ctx;
typedef struct lbt_weight lbt_weight;
typedef struct lbt_bf16 lbt_bf16;
typedef struct lbt_model lbt_model;
typedef struct lbt_cache lbt_cache;

/* ---- context --------------------------------------------------------------
 * Replaces the process-wide Kernel::detect() + rayon pool
 * (crates/lb-ternary/src/gemm.rs:78-91): owns one HIP stream and workspace. */
int lbt_ctx_create(int device, lbt_ctx** out);
void lbt_ctx_destroy(lbt_ctx* ctx);
const char* lbt_last_error(const lbt_ctx* ctx);
int lbt_ctx_synchronize(lbt_ctx* ctx);
/* The context's hipStream_t, as an opaque pointer. */
void* lbt_ctx_stream(lbt_ctx* ctx);
/* Device allocation helpers for `_dev` callers and tests. */
int lbt_dev_alloc(lbt_ctx* ctx, size_t bytes, void** out);
int lbt_dev_free(lbt_ctx* ctx, void* p);
int lbt_memcpy_h2d(lbt_ctx* ctx, void* dst, const void* src, size_t bytes);
int lbt_memcpy_d2h(lbt_ctx* ctx, void* dst, const void* src, size_t bytes);
/* Device-to-device copy on the context's stream by the library's own
 * streaming kernel (16-byte loads/stores; asynchronous).  Also the known-size
 * reference kernel when HBM counters are calibrated.  No counterpart in the
 * reference (its tensors live in host memory). */
int lbt_memcpy_d2d(lbt_ctx* ctx, void* dst, const void* src, size_t bytes);
/* Library build id (version + arch). */
const char* lbt_version(void);

/* ---- packed ternary weights ------------------------------------------------
 * TernaryView::new / PackedTernary (crates/lb-ternary/src/pack.rs:28-81):
 * `packed` is rows * padded(cols)/4 bytes, `scale` = 1/mean|W| (WeightQuant). */
int lbt_weight_upload(lbt_ctx* ctx, const uint8_t* packed, size_t rows, size_t cols, float scale,
                      lbt_weight** out);
/* Same, from bytes already in device memory (copied; the caller keeps its buffer). */
int lbt_weight_upload_dev(lbt_ctx* ctx, const uint8_t* packed_dev, size_t rows, size_t cols,
                          float scale, lbt_weight** out);
void lbt_weight_free(lbt_weight* w);
size_t lbt_weight_rows(const lbt_weight* w);
size_t lbt_weight_cols(const lbt_weight* w);
const uint8_t* lbt_weight_device_ptr(const lbt_weight* w);

/* ---- activation quantization -----------------------------------------------
 * quantize_acts (crates/lb-ternary/src/quant.rs:38-75, ActQuant): per row
 * amax = max|x| (NaN ignored), s_a = 127/max(amax,1e-5),
 * q = clamp(round_half_even(x*s_a), -128, 127) (NaN -> 0), sum = sum(q).
 * q is [m, padded(k)] with zero padding (QuantActs::q, quant.rs:19-35). */
int lbt_quantize_acts(lbt_ctx* ctx, const float* x, size_t m, size_t k, int8_t* q, float* scale,
                      int32_t* sum);
int lbt_quantize_acts_dev(lbt_ctx* ctx, const float* x, size_t m, size_t k, int8_t* q, float* scale,
                          int32_t* sum);
/* The RMSNorm + ActQuant fusion (model.rs:267-272 feeding ops.rs:315):
 * x -> x * (mean(x^2)+eps).sqrt().recip() * w -> quantize_acts. */
int lbt_rmsnorm_quantize_dev(lbt_ctx* ctx, const float* x, const float* norm_w, float eps, size_t m,
                             size_t k, int8_t* q, float* scale, int32_t* sum);

/* ---- ternary GEMV / GEMM ----------------------------------------------------
 * ternary_gemm_i32 (crates/lb-ternary/src/gemm.rs:95-114): exact
 * out[t*rows + r] = sum_k w[r,k] * q[t,k] for quantized activations
 * (q [m, padded(cols)], sum [m] as from lbt_quantize_acts). */
int lbt_gemm_i32(lbt_ctx* ctx, const lbt_weight* w, const int8_t* q, const int32_t* sum, size_t m,
                 int32_t* out);
int lbt_gemm_i32_dev(lbt_ctx* ctx, const lbt_weight* w, const int8_t* q, const int32_t* sum, size_t m,
                     int32_t* out);
/* ternary_gemm_multi (gemm.rs:128-195): n (1..3) matrices sharing the same
 * activations; outs[i][t*rows_i + r] = (dot as f32) * (1 / (scale[t] * s_w_i)).
 * ternary_gemm (gemm.rs:117-119) is n = 1. */
int lbt_gemm_multi(lbt_ctx* ctx, const lbt_weight* const* ws, size_t n, const int8_t* q,
                   const float* scale, const int32_t* sum, size_t m, float* const* outs);
int lbt_gemm_multi_dev(lbt_ctx* ctx, const lbt_weight* const* ws, size_t n, const int8_t* q,
                       const float* scale, const int32_t* sum, size_t m, float* const* outs);
/* TernaryBackend::ternary_linear / ternary_linear2 / ternary_linear3
 * (crates/lb-model/src/ops.rs:20-40, Flex impl :116-136, :301-329):
 * f32 x [m, cols] is quantized once inside the op, then one fused GEMM over
 * the n matrices; each output equals the n = 1 call bit for bit. */
int lbt_ternary_linear(lbt_ctx* ctx, const lbt_weight* const* ws, size_t n, const float* x, size_t m,
                       size_t cols, float* const* outs);
int lbt_ternary_linear_dev(lbt_ctx* ctx, const lbt_weight* const* ws, size_t n, const float* x,
                           size_t m, size_t cols, float* const* outs);
/* lbt_ternary_linear_dev that allocates nothing.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc).  The
 * several-row paths keep their quantized activations in a static 4 MiB
 * scratch per device instead of the context's grow-only buffer, so
 * round256(m * padded(cols)) + 8 m must be <= 4 MiB (LBT_E_INVALID beyond,
 * e.g. about 600 rows at cols = 6912); profiling must be off.  Results equal
 * lbt_ternary_linear_dev's bit for bit.  Every call on a device shares that
 * device's scratch; calls are ordered per device (one at a time on the host,
 * each stream waiting on the device for the previous call of another
 * stream), except under stream capture, where no cross-stream wait is
 * recorded and captured calls overlapping other streams' calls race. */
int lbt_ternary_linear_dev_noalloc(lbt_ctx* ctx, const lbt_weight* const* ws, size_t n, const float* x,
                                   size_t m, size_t cols, float* const* outs);

/* ---- bf16 linear (tied LM head) ---------------------------------------------
 * bf16_gemv (crates/lb-ternary/src/bf16.rs:14-25) / TernaryBackend::bf16_linear
 * (ops.rs:75-76, :199-218): out[t*rows + r] = sum_k x[t,k] * bf16(W[r,k]),
 * f32 accumulation.  cols must be a multiple of 8. */
int lbt_bf16_upload(lbt_ctx* ctx, const uint16_t* w, size_t rows, size_t cols, lbt_bf16** out);
void lbt_bf16_free(lbt_bf16* w);
int lbt_bf16_linear(lbt_ctx* ctx, const lbt_bf16* w, const float* x, size_t m, float* out);
int lbt_bf16_linear_dev(lbt_ctx* ctx, const lbt_bf16* w, const float* x, size_t m, float* out);

/* ---- opt-in int8 LM head ------------------------------------------------------
 * Q8Head (crates/lb-ternary/src/q8head.rs:9-15): int8 [rows, cols] row-major
 * with one f32 scale per row; halves the head's weight bytes at the cost of
 * exact logits.  lbt_q8head_from_bf16 is Q8Head::from_bf16 (:18-32), run on the
 * device from an uploaded bf16 matrix: scale = amax / 127 (1.0 for an all-zero
 * row), q = round_ties_even(w / scale) clamped to [-127, 127]; bit-exact. */
typedef struct lbt_q8head lbt_q8head;
int lbt_q8head_from_bf16(lbt_ctx* ctx, const lbt_bf16* w, lbt_q8head** out);
void lbt_q8head_free(lbt_q8head* h);
/* Host copies of the quantized weights (q: rows*cols bytes, scale: rows). */
int lbt_q8head_read(lbt_ctx* ctx, const lbt_q8head* h, int8_t* q, float* scale);
/* Q8Head::gemv (q8head.rs:34-57) for m rows: out[t*rows + r] = scale[r] *
 * sum_k q[r,k] * x[t,k], f32 accumulation (device order; within the
 * reference's own 1e-4 * sum|terms| bound, q8head.rs:84-97). */
int lbt_q8head_linear(lbt_ctx* ctx, const lbt_q8head* h, const float* x, size_t m, float* out);
int lbt_q8head_linear_dev(lbt_ctx* ctx, const lbt_q8head* h, const float* x, size_t m, float* out);

/* ---- sampling -------------------------------------------------------------------
 * SamplingParams (crates/lb-model/src/sample.rs:3-15) without the seed: the
 * xorshift64 state is the caller's (Sampler::new sets it to seed.max(1),
 * sample.rs:33-35) and each sample at temperature > 0 advances it by one draw. */
typedef struct lbt_sample_params {
    float temperature; /* <= 0: argmax */
    float top_p;       /* >= 1 (or NaN): no cut */
    size_t top_k;      /* 0: no truncation */
} lbt_sample_params;

/* Sampler::sample (sample.rs:45-82) on the device for `rows` rows of logits
 * [rows][vocab]; states[r] is row r's sampler state (updated), out[r] its id.
 * The reference's steps in its order; the cumulative probabilities are exact
 * integer sums of floor(p * 2^45) (the reference's sequential f32 sums pick
 * the same id except where the draw lies within rounding of a boundary);
 * equal logits are ordered by ascending index (the reference's unstable sort
 * leaves it open). */
int lbt_sample(lbt_ctx* ctx, const float* logits, size_t rows, size_t vocab, const lbt_sample_params* p,
               uint64_t* states, uint32_t* out);
int lbt_sample_dev(lbt_ctx* ctx, const float* logits, size_t rows, size_t vocab, const lbt_sample_params* p,
                   uint64_t* states, uint32_t* out);

/* ---- BitNet b1.58 model ------------------------------------------------------
 * Config (crates/lb-model/src/model.rs:22-42). */
typedef struct lbt_config {
    int32_t hidden_size;
    int32_t intermediate_size;
    int32_t num_attention_heads;
    int32_t num_key_value_heads;
    int32_t num_hidden_layers;
    int32_t vocab_size;
    int32_t max_position_embeddings;
    uint32_t bos_token_id;
    double rms_norm_eps;
    double rope_theta;
} lbt_config;

/* BitNet::load (model.rs:149-232): reads DIR/config.json and the lb-convert v1
 * file DIR/model.lbt.safetensors (crates/lb-convert/src/lib.rs:1-16; metadata
 * format "lemonade-burn-ternary") and uploads everything to the device. */
int lbt_model_load(lbt_ctx* ctx, const char* dir, lbt_model** out);
/* A random-initialised model of the given shape, generated on the device from
 * `seed` (i.i.d. ternary P(-1,0,+1) = 0.3/0.4/0.3, bf16 uniform(-1,1) embedding,
 * norms uniform(0.5,1.5)). */
int lbt_model_create_synthetic(lbt_ctx* ctx, const lbt_config* cfg, uint64_t seed, lbt_model** out);
void lbt_model_free(lbt_model* m);
int lbt_model_get_config(const lbt_model* m, lbt_config* out);
/* Device weights of one layer's linear (which: 0..6 = q,k,v,o,gate,up,down). */
const lbt_weight* lbt_model_linear(const lbt_model* m, int layer, int which);

/* BitNet::new_cache (model.rs:234-236) / KvCache (:140-146): bf16 K/V,
 * [layers][kv_heads][cap][head_dim]; grows by doubling like ensure_cap
 * (:238-265). */
int lbt_cache_new(lbt_model* m, lbt_cache** out);
void lbt_cache_free(lbt_cache* c);
int lbt_cache_len(const lbt_cache* c);
/* Copy one layer's K or V ([kv_heads, len, head_dim] bf16 bits) to the host. */
int lbt_cache_read(lbt_cache* c, int layer, int is_v, uint16_t* out);

/* BitNet::forward (model.rs:305-374): runs `tokens` at positions cache.len..;
 * writes logits [all_logits ? m : 1, vocab] to host memory. */
int lbt_model_forward(lbt_model* m, const uint32_t* tokens, size_t n, lbt_cache* c, int all_logits,
                      float* logits);
/* forward + greedy argmax on the device (sample.rs:17-25): only the token id
 * crosses to the host. */
int lbt_model_forward_argmax(lbt_model* m, const uint32_t* tokens, size_t n, lbt_cache* c,
                             uint32_t* next);
/* The lb-run bench loop (crates/lb-model/src/bin/lb-run.rs:127-138): prefill
 * `prompt`, then `steps` greedy decode steps with token feedback on the
 * device.  out_tokens gets steps + 1 ids (the prefill's argmax first).
 * If ms_prefill / ms_decode are non-null they receive device-timed ms. */
int lbt_model_generate_greedy(lbt_model* m, const uint32_t* prompt, size_t n, size_t steps,
                              lbt_cache* c, uint32_t* out_tokens, float* ms_prefill, float* ms_decode);
/* Decode-only continuation of the loop above (the lb-server decode loop,
 * crates/lb-server/src/main.rs:141-160, greedy): feeds `first` at position
 * cache.len, then `steps - 1` more tokens chosen on the device; out_tokens
 * gets the `steps` argmax ids.  ms_decode (nullable) gets device-timed ms. */
int lbt_model_decode_greedy(lbt_model* m, lbt_cache* c, uint32_t first, size_t steps, uint32_t* out_tokens,
                            float* ms_decode);
/* The lb-server job loop with its Sampler (crates/lb-server/src/main.rs:102-160,
 * sample.rs:45-82) on the device: forward_sample runs the prompt and samples
 * the first token; decode_sample feeds `first` and samples `steps` tokens,
 * each fed back on the device.  *state is the sampler state (seed.max(1) for
 * a new job), updated.  Only token ids cross to the host. */
int lbt_model_forward_sample(lbt_model* m, const uint32_t* tokens, size_t n, lbt_cache* c,
                             const lbt_sample_params* p, uint64_t* state, uint32_t* next);
int lbt_model_decode_sample(lbt_model* m, lbt_cache* c, uint32_t first, size_t steps, const lbt_sample_params* p,
                            uint64_t* state, uint32_t* out_tokens, float* ms_decode);
/* LM head of the model's forwards: 0 = the exact tied bf16 head (default),
 * 1 = the opt-in int8 head (q8head.rs), quantized on the device from the
 * tied embedding when first selected, 2 = the tied bf16 head with heads of
 * 33..64 rows (batched steps, prefill logits) on the bf16 matrix cores
 * (activations as bf16 hi + lo parts, f32 accumulation: logits within
 * tolerance of kind 0; other heads exact).  A cached decode-step graph is
 * rebuilt.  No counterpart in the reference for kind 2: it serves batched
 * decode, which the reference does not have. */
int lbt_model_set_head(lbt_model* m, int kind);
/* Residual stream of the last forward ([n, hidden] f32) for layer-level tests. */
int lbt_model_read_hidden(lbt_model* m, float* out, size_t n);

/* ---- batched decode (several sequences per step) ------------------------------------
 * No counterpart in the reference, which decodes one sequence at a time
 * (lb-server main.rs:92-100).  `nseq` independent sequences, each with its own
 * bf16 KV cache of fixed capacity `cap` positions; a step appends one token to
 * every sequence with one pass over the weights (rows of the ternary GEMMs are
 * the sequences) and attention over each sequence's own cache.  Per-sequence
 * results equal those of the single-sequence API on the same tokens. */
typedef struct lbt_batch lbt_batch;
int lbt_batch_new(lbt_model* m, int nseq, int cap, lbt_batch** out);
void lbt_batch_free(lbt_batch* b);
int lbt_batch_len(const lbt_batch* b, int seq);
/* Prompt of sequence `seq` (n tokens after its current length); its greedy
 * next token in *next (nullable). */
int lbt_batch_prefill(lbt_batch* b, int seq, const uint32_t* tokens, size_t n, uint32_t* next);
/* Every sequence's cache holds `len` positions of seeded synthetic K/V
 * (approximately N(0,1), bf16) and its length becomes `len`. */
int lbt_batch_fill_synthetic(lbt_batch* b, int len, uint64_t seed);
/* One step: tokens[s] is appended to sequence s; logits [nseq][vocab]
 * (nullable) and greedy next[s] (nullable). */
int lbt_batch_forward(lbt_batch* b, const uint32_t* tokens, float* logits, uint32_t* next);
/* `steps` greedy steps of every sequence starting from first[s]:
 * out_tokens[i * nseq + s] is sequence s's token produced by step i;
 * *ms_decode (nullable) the device time of the steps. */
/* lbt_batch_prefill / lbt_batch_forward with the device sampler
 * (sample.rs:45-82): the first token of `seq` drawn with *p and its sampler
 * state *state; one step of every sequence, sequence s drawn with params[s]
 * and states[s] (host arrays of nseq; states updated; temperature 0 is the
 * argmax).  Only token ids return to the host. */
int lbt_batch_prefill_sample(lbt_batch* b, int seq, const uint32_t* tokens, size_t n, const lbt_sample_params* p,
                             uint64_t* state, uint32_t* next);
int lbt_batch_forward_sample(lbt_batch* b, const uint32_t* tokens, const lbt_sample_params* params,
                             uint64_t* states, uint32_t* next);
int lbt_batch_decode_greedy(lbt_batch* b, const uint32_t* first, size_t steps, uint32_t* out_tokens,
                            float* ms_decode);

/* Sequence `seq` starts over (length 0); its cache rows are overwritten by
 * the next prefill.  No counterpart in the reference (one cache per request). */
int lbt_batch_reset(lbt_batch* b, int seq);

/* ---- continuous batching (no counterpart in the reference,
 * whose server runs one request at a time, lb-server main.rs:92-100) ---------
 * Greedy requests share one lbt_batch of `slots` sequences: a queued request
 * takes a free slot (its prompt prefilled there), every step advances all
 * active slots by one token in one batched forward, and a finished request
 * (max_new tokens, or its stop token) frees its slot for the queue.  Each
 * request's tokens equal those of running it alone (greedy, same model). */
typedef struct lbt_sched lbt_sched;
int lbt_sched_new(lbt_model* m, int slots, int cap, lbt_sched** out);
void lbt_sched_free(lbt_sched* s);
/* Queue a request; stop = 0xFFFFFFFF for none; prompt length + max_new must
 * fit the slot capacity.  *id receives the request's id. */
int lbt_sched_submit(lbt_sched* s, const uint32_t* prompt, size_t n, size_t max_new, uint32_t stop,
                     uint64_t* id);
/* One step: admit queued requests into free slots (prefill, first token),
 * then one batched decode step of the active slots.  *pending (nullable):
 * requests still queued or active afterwards. */
/* lbt_sched_submit for a request sampled with *p (the job's SamplingParams,
 * lb-server/src/main.rs:102-109) from a sampler seeded with `seed`
 * (seed.max(1), sample.rs:33-35); requests of both kinds share the steps. */
int lbt_sched_submit_sample(lbt_sched* s, const uint32_t* prompt, size_t n, size_t max_new, uint32_t stop,
                            const lbt_sample_params* p, uint64_t seed, uint64_t* id);
int lbt_sched_step(lbt_sched* s, int* pending);
/* The tokens of request id so far (up to cap of them into tokens, nullable),
 * their count in *n and whether it is finished in *done. */
int lbt_sched_result(lbt_sched* s, uint64_t id, uint32_t* tokens, size_t cap, size_t* n, int* done);
/* Drop a finished request's record (its id becomes unknown). */
int lbt_sched_release(lbt_sched* s, uint64_t id);

/* ---- profiling (replaces the PROF_* counters, ops.rs:79-97) ----------------
 * When enabled, every ternary GEMV/GEMM launch of the model loop is bracketed
 * by HIP events on the context stream; totals are per kernel class
 * (0 = ternary decode GEMV, 1 = ternary prefill GEMM, 2 = bf16 LM head,
 * 3 = attention, 4 = other; slot 5 is unused). */
typedef struct lbt_prof {
    double ms[6];
    double bytes[6];
    uint64_t launches[6];
} lbt_prof;
int lbt_prof_enable(lbt_ctx* ctx, int on);
int lbt_prof_read(lbt_ctx* ctx, lbt_prof* out, int reset);

#ifdef __cplusplus
}
#endif
#endif
