/*
 * lbt_oracle.h -- CPU oracle for the packed-ternary x int8 hot path and the
 * BitNet b1.58 token loop.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or as the timed CPU baseline).  The product library (liblbt_hip.so) never
 * links, loads or calls anything here.
 *
 * Reference: festeraeb/lemonade-burn (Rust).  Each function cites the
 * reference file:line it restates.  Parity pins (what checks each function
 * against something other than itself) are listed in tests/test_oracle.py.
 */
#ifndef LBT_ORACLE_H
#define LBT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- layout (crates/lb-ternary/src/pack.rs) ---------------------------- */
size_t or_padded_cols(size_t cols);                          /* pack.rs:22-24 */
size_t or_row_bytes(size_t cols);                            /* pack.rs:83-85 */
void or_pack_row(const int8_t* vals, size_t cols, uint8_t* out); /* pack.rs:88-103 */
void or_unpack_row(const uint8_t* row, size_t padded, int8_t* out); /* pack.rs:106-116 */
void or_pack(const int8_t* vals, size_t rows, size_t cols, uint8_t* out);
float or_absmean(const float* w, size_t n);                  /* pack.rs:135-138 */
float or_ternarize_absmean(const float* w, size_t n, int8_t* t); /* pack.rs:129-142 */

/* ---- activation quantizer (crates/lb-ternary/src/quant.rs) ------------- */
/* quantize_row_scalar (quant.rs:100-118): returns scale, writes q[0..k) and *sum. */
float or_quantize_row(const float* x, size_t k, int8_t* q, int32_t* sum);
/* quantize_acts (quant.rs:45-75): q is [m, kp] zero padded. */
void or_quantize_acts(const float* x, size_t m, size_t k, int8_t* q, float* scale, int32_t* sum);

/* ---- ternary GEMV/GEMM (crates/lb-ternary/src/gemm.rs) ----------------- */
/* codes_dot_scalar (gemm.rs:329-343) for one row and one token. */
int32_t or_codes_dot(const uint8_t* row, size_t kp, const int8_t* x);
/* ternary_gemm_i32 (gemm.rs:95-114): out[t*rows + r] = sum_k w[r,k] q[t,k]. */
void or_gemm_i32(const uint8_t* packed, size_t rows, size_t cols, const int8_t* q,
                 const int32_t* qsum, size_t m, int32_t* out);
/* ternary_gemm (gemm.rs:117-119, :141, :150, :158): out = dot as f32 * (1/(s_a*s_w)). */
void or_gemm_f32(const uint8_t* packed, size_t rows, size_t cols, float s_w,
                 const int8_t* q, const float* s_a, const int32_t* qsum, size_t m, float* out);
/* gemv_i32_reference (crates/ternary-kernels/src/reference.rs:7-16): brute force
 * over unpacked weights, no code-offset trick. */
void or_gemm_i32_bruteforce(const uint8_t* packed, size_t rows, size_t cols,
                            const int8_t* q, size_t m, int32_t* out);

/* ---- bf16 GEMV (crates/lb-ternary/src/bf16.rs) ------------------------- */
float or_bf16_to_f32(uint16_t b);                            /* bf16.rs:9-11 */
uint16_t or_f32_to_bf16(float f);                            /* round to nearest even */
/* dot_scalar (bf16.rs:38-51): 8 lane accumulators. */
float or_bf16_dot_ref(const uint16_t* w, const float* x, size_t n);
/* The device LM-head order: 64 lanes, lane l takes 8-element chunks l, l+64, ...
 * with fused multiply-add, then an xor butterfly over the lanes. */
float or_bf16_dot_lanes(const uint16_t* w, const float* x, size_t n);
void or_bf16_gemv_lanes(const uint16_t* w, size_t rows, size_t cols, const float* x, float* out);

/* ---- opt-in int8 LM head (crates/lb-ternary/src/q8head.rs) ----------------- */
void or_q8head_from_bf16(const uint16_t* w, size_t rows, size_t cols, int8_t* q, float* scale); /* :18-32 */
void or_q8head_gemv_ref(const int8_t* q, const float* scale, size_t rows, size_t cols, const float* x,
                        float* out); /* :35-57, the reference's order */
void or_q8head_gemv_lanes(const int8_t* q, const float* scale, size_t rows, size_t cols, const float* x,
                          float* out); /* the device order */

/* ---- float building blocks in the device order ------------------------- */
float or_block_sum256(const float* partials);                 /* wave butterflies, then (w0+w1)+(w2+w3) */
float or_sumsq(const float* x, size_t n);                     /* canonical order (1024 virtual threads) */
/* rms_norm (crates/lb-model/src/model.rs:267-272): x * (mean(x^2)+eps).sqrt().recip() * w */
void or_rmsnorm(const float* x, const float* w, size_t n, float eps, float* out);
float or_expf(float x);                                       /* Cody-Waite + Taylor(7) */
uint32_t or_argmax(const float* v, size_t n);                 /* sample.rs:17-25 */
/* Sampler::sample (sample.rs:45-82) with exact integer masses; the helpers
 * are exported for the tests. */
uint32_t or_sample(const float* logits, size_t V, float temperature, float top_p, size_t top_k, uint64_t* state);
uint64_t or_sample_key(float x, uint32_t i);
uint64_t or_top_p_target(float top_p, uint64_t W);
uint32_t or_sample_uniform(uint64_t* state);

/* ---- RoPE tables (crates/lb-model/src/model.rs:213-230) ---------------- */
/* cos/sin are [max_pos, hd/2]: entry i serves dims i and i + hd/2. */
void or_rope_tables(size_t hd, size_t max_pos, double theta, float* cos_t, float* sin_t);

/* ---- synthetic weights (shared generator with the device) -------------- */
uint64_t or_splitmix64(uint64_t z);
uint64_t or_synth_hash(uint64_t seed, uint64_t tensor, uint64_t i);
int8_t or_synth_ternary(uint64_t seed, uint64_t tensor, uint64_t i);
void or_synth_packed(uint64_t seed, uint64_t tensor, size_t rows, size_t cols, uint8_t* out);
void or_synth_f32(uint64_t seed, uint64_t tensor, size_t n, float lo, float span, float* out);
void or_synth_bf16(uint64_t seed, uint64_t tensor, size_t n, uint16_t* out);
float or_synth_wscale(size_t cols);

/* ---- BitNet model (crates/lb-model/src/model.rs) ----------------------- */
typedef struct or_config {
    int hidden, intermediate, heads, kv_heads, layers, vocab, max_pos;
    double rms_norm_eps, rope_theta;
} or_config;

typedef struct or_model or_model;

/* Tensor ids of the synthetic generator (one namespace, shared with the device). */
#define OR_T_EMBED 1u
#define OR_T_FINAL_NORM 2u
#define OR_T_LAYER(l, k) (16u + (uint64_t)(l) * 16u + (k))
/* k: 0..6 = q,k,v,o,gate,up,down; 7..10 = input, post_attn, attn_sub, ffn_sub norms */

or_model* or_model_synthetic(const or_config* cfg, uint64_t seed);
/* Wrap caller-owned host arrays (lb-convert v1 contents); nothing is copied. */
or_model* or_model_wrap(const or_config* cfg, const uint8_t* const* packed /*[layers*7]*/,
                        const float* wscales /*[layers*7]*/, const float* const* norms /*[layers*4]*/,
                        const float* final_norm, const uint16_t* embed);
void or_model_free(or_model* m);
/* LM head of the forwards: 0 = bf16 (default), 1 = int8 head from the embedding. */
int or_model_set_head(or_model* m, int kind);
const uint8_t* or_model_packed(const or_model* m, int layer, int which);
float or_model_wscale(const or_model* m, int layer, int which);
const uint16_t* or_model_embed(const or_model* m);
void or_model_reset(or_model* m);       /* empty KV cache */
int or_model_len(const or_model* m);
/* BitNet::forward (model.rs:305-374), device reduction order.  Writes logits
 * [all_logits ? m : 1, vocab].  Returns 0, or -1 when the context is exceeded. */
int or_model_fill_synth_kv(or_model* m, uint64_t seed, int nseq, int seq, int len);
int or_model_forward(or_model* m, const uint32_t* tokens, size_t n, int all_logits, float* logits);
/* Internals exposed for layer-level parity: the residual stream after the last
 * forward ([n, hidden]) and the bf16 K/V cache of one layer ([kvh, cap, hd]). */
const float* or_model_hidden(const or_model* m);
const uint16_t* or_model_kcache(const or_model* m, int layer);
const uint16_t* or_model_vcache(const or_model* m, int layer);
int or_model_cap(const or_model* m);
/* 0: scalar codes_dot (the oracle).  1: the multi-threaded SIMD integer
 * kernels of lbt_port.c (exact, same integers, same logits).  2: also the
 * reference-order AVX-512 bf16 LM head (the CPU baseline; logits then differ
 * from the device order by float rounding).  Returns the previous setting. */
int or_set_fast(int fast);
int or_set_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
