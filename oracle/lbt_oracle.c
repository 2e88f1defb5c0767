/*
 * lbt_oracle.c -- CPU restatement of lemonade-burn's ternary hot path.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py, as the checker.  Never linked into the product.
 *
 * Build: see oracle/Makefile (gcc -O2 -ffp-contract=off: no contraction, so
 * every float operation below is one IEEE-754 binary32 operation; fmaf() is
 * used explicitly wherever the device kernels use a fused multiply-add).
 *
 * Reference files restated (paths relative to festeraeb/lemonade-burn):
 *   crates/lb-ternary/src/pack.rs, quant.rs, gemm.rs, bf16.rs
 *   crates/ternary-kernels/src/reference.rs
 *   crates/lb-model/src/model.rs, sample.rs
 *
 * Float reduction order.  The reference's non-GEMM float ops run inside Burn
 * Flex (burn-flex 0.22.1, not vendored); their summation order cannot be
 * restated.  The device kernels therefore use one fixed, documented order and
 * this oracle follows the same order, so the device path can be compared bit
 * for bit.  The order itself is pinned against an f64 evaluation of the same
 * formulas (tests/test_oracle.py) to the north-star tolerance.
 */
#include "lbt_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#include "lbt_port.h"

#define BLOCK 128
#define BLOCK_BYTES 32

/* ------------------------------------------------------------------------ */
/* pack.rs                                                                   */
/* ------------------------------------------------------------------------ */

/* pack.rs:22-24 */
size_t or_padded_cols(size_t cols) { return (cols + BLOCK - 1) / BLOCK * BLOCK; }

/* pack.rs:83-85 */
size_t or_row_bytes(size_t cols) { return or_padded_cols(cols) / 4; }

/* pack.rs:88-103: byte j of block b holds, in bits 2k..2k+1, code (w+1) of
 * weight b*128 + k*32 + j; columns past `cols` are weight 0 (code 1). */
void or_pack_row(const int8_t* vals, size_t cols, uint8_t* out) {
    size_t nb = or_padded_cols(cols) / BLOCK;
    for (size_t b = 0; b < nb; b++) {
        for (size_t j = 0; j < BLOCK_BYTES; j++) {
            uint8_t v = 0;
            for (size_t k = 0; k < 4; k++) {
                size_t idx = b * BLOCK + k * 32 + j;
                int w = idx < cols ? vals[idx] : 0;
                v |= (uint8_t)(((w + 1) & 3) << (2 * k));
            }
            out[b * BLOCK_BYTES + j] = v;
        }
    }
}

/* pack.rs:106-116 */
void or_unpack_row(const uint8_t* row, size_t padded, int8_t* out) {
    size_t nb = padded / BLOCK;
    for (size_t b = 0; b < nb; b++)
        for (size_t j = 0; j < BLOCK_BYTES; j++)
            for (size_t k = 0; k < 4; k++)
                out[b * BLOCK + k * 32 + j] = (int8_t)(((row[b * BLOCK_BYTES + j] >> (2 * k)) & 3) - 1);
}

/* PackedTernary::from_ternary (pack.rs:69-77) */
void or_pack(const int8_t* vals, size_t rows, size_t cols, uint8_t* out) {
    size_t rb = or_row_bytes(cols);
    for (size_t r = 0; r < rows; r++) or_pack_row(vals + r * cols, cols, out + r * rb);
}

/* absmean_f32 (pack.rs:135-138): f64 sum of |w|, one rounding to f32. */
float or_absmean(const float* w, size_t n) {
    double s = 0.0;
    for (size_t i = 0; i < n; i++) s += fabs((double)w[i]);
    return (float)(s / (double)n);
}

/* ternarize_absmean + ternarize_with_scale (pack.rs:129-142) */
float or_ternarize_absmean(const float* w, size_t n, int8_t* t) {
    float mean = or_absmean(w, n);
    float scale = 1.0f / fmaxf(mean, 1e-5f);
    for (size_t i = 0; i < n; i++) {
        float r = rintf(w[i] * scale); /* round_ties_even (default rounding mode) */
        if (r > 1.0f) r = 1.0f;
        if (r < -1.0f) r = -1.0f;
        t[i] = (int8_t)r;
    }
    return scale;
}

/* ------------------------------------------------------------------------ */
/* quant.rs                                                                  */
/* ------------------------------------------------------------------------ */

/* quant_one (quant.rs:116-118): (v*scale).round_ties_even().clamp(-128,127) as i8.
 * Rust's float->int `as` maps NaN to 0; clamp keeps +-inf at the bounds. */
static int8_t quant_one(float v, float scale) {
    float y = rintf(v * scale);
    if (y != y) return 0;
    if (y < -128.0f) y = -128.0f;
    if (y > 127.0f) y = 127.0f;
    return (int8_t)y;
}

/* quantize_row_scalar (quant.rs:100-113).  f32::max ignores a NaN operand,
 * as fmaxf does. */
float or_quantize_row(const float* x, size_t k, int8_t* q, int32_t* sum) {
    float amax = 0.0f;
    for (size_t i = 0; i < k; i++) amax = fmaxf(amax, fabsf(x[i]));
    float scale = 127.0f / fmaxf(amax, 1e-5f);
    int32_t s = 0;
    for (size_t i = 0; i < k; i++) {
        int8_t r = quant_one(x[i], scale);
        q[i] = r;
        s += r;
    }
    *sum = s;
    return scale;
}

/* quantize_acts_into (quant.rs:45-75): rows padded with zeros to kp. */
void or_quantize_acts(const float* x, size_t m, size_t k, int8_t* q, float* scale, int32_t* sum) {
    size_t kp = or_padded_cols(k);
    memset(q, 0, m * kp);
    for (size_t i = 0; i < m; i++) scale[i] = or_quantize_row(x + i * k, k, q + i * kp, sum + i);
}

/* ------------------------------------------------------------------------ */
/* gemm.rs                                                                   */
/* ------------------------------------------------------------------------ */

/* codes_dot_scalar (gemm.rs:329-343): sum of code * x over the padded row. */
int32_t or_codes_dot(const uint8_t* row, size_t kp, const int8_t* x) {
    int32_t acc = 0;
    size_t nb = kp / BLOCK;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = row + b * BLOCK_BYTES;
        for (size_t k = 0; k < 4; k++)
            for (size_t j = 0; j < BLOCK_BYTES; j++) {
                int32_t c = (blk[j] >> (2 * k)) & 3;
                acc += c * (int32_t)x[b * BLOCK + k * 32 + j];
            }
    }
    return acc;
}

/* ternary_gemm_i32 (gemm.rs:95-114) with dot_row's -sum(q) (gemm.rs:306-308). */
void or_gemm_i32(const uint8_t* packed, size_t rows, size_t cols, const int8_t* q,
                 const int32_t* qsum, size_t m, int32_t* out) {
    size_t kp = or_padded_cols(cols), rb = kp / 4;
#pragma omp parallel for schedule(static) if (rows * m * kp > (1u << 22))
    for (long r = 0; r < (long)rows; r++)
        for (size_t t = 0; t < m; t++)
            out[t * rows + r] = or_codes_dot(packed + r * rb, kp, q + t * kp) - qsum[t];
}

/* ternary_gemm / multi (gemm.rs:128-195): y = (dot as f32) * (1 / (s_a * s_w)). */
void or_gemm_f32(const uint8_t* packed, size_t rows, size_t cols, float s_w,
                 const int8_t* q, const float* s_a, const int32_t* qsum, size_t m, float* out) {
    int32_t* d = (int32_t*)malloc(rows * m * sizeof(int32_t));
    or_gemm_i32(packed, rows, cols, q, qsum, m, d);
    for (size_t t = 0; t < m; t++) {
        float inv = 1.0f / (s_a[t] * s_w);
        for (size_t r = 0; r < rows; r++) out[t * rows + r] = (float)d[t * rows + r] * inv;
    }
    free(d);
}

/* gemv_i32_reference (ternary-kernels/src/reference.rs:7-16) */
void or_gemm_i32_bruteforce(const uint8_t* packed, size_t rows, size_t cols,
                            const int8_t* q, size_t m, int32_t* out) {
    size_t kp = or_padded_cols(cols), rb = kp / 4;
    int8_t* w = (int8_t*)malloc(kp);
    for (size_t r = 0; r < rows; r++) {
        or_unpack_row(packed + r * rb, kp, w);
        for (size_t t = 0; t < m; t++) {
            int64_t acc = 0;
            for (size_t k = 0; k < kp; k++) acc += (int64_t)w[k] * q[t * kp + k];
            out[t * rows + r] = (int32_t)acc;
        }
    }
    free(w);
}

/* ------------------------------------------------------------------------ */
/* bf16.rs                                                                   */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* bf16_to_f32 (bf16.rs:9-11) */
float or_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* f32 -> bf16, round to nearest even; NaN -> canonical quiet NaN. */
uint16_t or_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* dot_scalar (bf16.rs:38-51) */
float or_bf16_dot_ref(const uint16_t* w, const float* x, size_t n) {
    float acc[8] = {0};
    size_t n8 = n / 8 * 8;
    for (size_t i = 0; i < n8; i += 8)
        for (int l = 0; l < 8; l++) acc[l] += or_bf16_to_f32(w[i + l]) * x[i + l];
    float s = 0.0f;
    for (int l = 0; l < 8; l++) s += acc[l];
    for (size_t i = n8; i < n; i++) s += or_bf16_to_f32(w[i]) * x[i];
    return s;
}

/* xor butterfly over 64 lane values, as the device reduces a wavefront:
 * step m: lane l takes v[l] + v[l ^ m] for m = 32, 16, ..., 1. */
static float butterfly64(float* v) {
    float t[64];
    for (int m = 32; m >= 1; m >>= 1) {
        for (int l = 0; l < 64; l++) t[l] = v[l] + v[l ^ m];
        memcpy(v, t, sizeof(t));
    }
    return v[0];
}

/* The device LM-head dot: n % 8 == 0; lane l accumulates chunks c = l + 64 i. */
float or_bf16_dot_lanes(const uint16_t* w, const float* x, size_t n) {
    float lane[64];
    size_t chunks = n / 8;
    for (int l = 0; l < 64; l++) {
        float acc = 0.0f;
        for (size_t c = (size_t)l; c < chunks; c += 64)
            for (int e = 0; e < 8; e++) acc = fmaf(or_bf16_to_f32(w[c * 8 + e]), x[c * 8 + e], acc);
        lane[l] = acc;
    }
    return butterfly64(lane);
}

void or_bf16_gemv_lanes(const uint16_t* w, size_t rows, size_t cols, const float* x, float* out) {
#pragma omp parallel for schedule(static) if (rows * cols > (1u << 22))
    for (long r = 0; r < (long)rows; r++) out[r] = or_bf16_dot_lanes(w + (size_t)r * cols, x, cols);
}

/* ------------------------------------------------------------------------ */
/* q8head.rs: opt-in int8 LM head                                            */
/* ------------------------------------------------------------------------ */

/* Q8Head::from_bf16 (q8head.rs:18-32): per row amax (f32::max ignores NaN),
 * scale = amax / 127 (1.0 when amax == 0), q = round_ties_even(w / scale)
 * clamped to [-127, 127]; a NaN quotient casts to 0 (Rust `as i8`). */
void or_q8head_from_bf16(const uint16_t* w, size_t rows, size_t cols, int8_t* q, float* scale) {
    for (size_t r = 0; r < rows; r++) {
        const uint16_t* wr = w + r * cols;
        float amax = 0.0f;
        for (size_t i = 0; i < cols; i++) {
            float a = fabsf(or_bf16_to_f32(wr[i]));
            if (a > amax) amax = a; /* a NaN never compares greater */
        }
        float s = amax == 0.0f ? 1.0f : amax / 127.0f;
        scale[r] = s;
        for (size_t i = 0; i < cols; i++) {
            float y = rintf(or_bf16_to_f32(wr[i]) / s); /* default rounding: ties to even */
            if (y != y) y = 0.0f;
            if (y < -127.0f) y = -127.0f;
            if (y > 127.0f) y = 127.0f;
            q[r * cols + i] = (int8_t)y;
        }
    }
}

/* Q8Head::gemv (q8head.rs:35-57), the reference's order: 8 lane accumulators
 * over k in steps of 8 (unfused multiply, add), their sequential sum, the
 * scalar tail, then scale[r] * sum. */
void or_q8head_gemv_ref(const int8_t* q, const float* scale, size_t rows, size_t cols, const float* x, float* out) {
    size_t n8 = cols / 8 * 8;
    for (size_t r = 0; r < rows; r++) {
        const int8_t* row = q + r * cols;
        float acc[8] = {0};
        for (size_t k = 0; k < n8; k += 8)
            for (int j = 0; j < 8; j++) {
                float p = (float)row[k + j] * x[k + j];
                acc[j] = acc[j] + p;
            }
        float sum = 0.0f;
        for (int j = 0; j < 8; j++) sum = sum + acc[j];
        for (size_t k = n8; k < cols; k++) {
            float p = (float)row[k] * x[k];
            sum = sum + p;
        }
        out[r] = scale[r] * sum;
    }
}

/* The device int8 head: cols % 8 == 0; lane l accumulates the 8-byte chunks
 * c = l + 64 i with fused multiply-adds in element order, the xor butterfly,
 * then scale[r] * sum. */
void or_q8head_gemv_lanes(const int8_t* q, const float* scale, size_t rows, size_t cols, const float* x, float* out) {
    size_t chunks = cols / 8;
#pragma omp parallel for schedule(static) if (rows * cols > (1u << 22))
    for (long r = 0; r < (long)rows; r++) {
        const int8_t* row = q + (size_t)r * cols;
        float lane[64];
        for (int l = 0; l < 64; l++) {
            float acc = 0.0f;
            for (size_t c = (size_t)l; c < chunks; c += 64)
                for (int e = 0; e < 8; e++) acc = fmaf((float)row[c * 8 + e], x[c * 8 + e], acc);
            lane[l] = acc;
        }
        out[r] = scale[r] * butterfly64(lane);
    }
}

/* ------------------------------------------------------------------------ */
/* device-order float building blocks                                        */
/* ------------------------------------------------------------------------ */

/* Block sum of 256 per-thread partials as the device reduces them: each
 * wavefront of 64 reduces with the xor butterfly, then the four wave sums are
 * added as (w0 + w1) + (w2 + w3). */
float or_block_sum256(const float* partials) {
    float w[4];
    for (int k = 0; k < 4; k++) {
        float v[64];
        memcpy(v, partials + 64 * k, sizeof(v));
        w[k] = butterfly64(v);
    }
    return (w[0] + w[1]) + (w[2] + w[3]);
}

/* Canonical sum of squares of a row, the device order for any workgroup size
 * (lemonade-burn_amd/csrc/lbt_device.h row_sumsq): element group gi (elements
 * 4gi..4gi+3) belongs to virtual thread vt = gi mod 1024, which accumulates
 * x^2 by fused multiply-adds over its elements in ascending order; each of the
 * 16 virtual wavefronts (vt / 64) reduces with the xor butterfly, and the 16
 * wavefront sums are added as a full binary tree. */
float or_sumsq(const float* x, size_t n) {
    float w[16];
    for (int wv = 0; wv < 16; wv++) {
        float v[64];
        for (int l = 0; l < 64; l++) {
            size_t vt = (size_t)(64 * wv + l);
            float a = 0.0f;
            for (size_t gi = vt; 4 * gi < n; gi += 1024)
                for (size_t i = 4 * gi; i < 4 * gi + 4 && i < n; i++) a = fmaf(x[i], x[i], a);
            v[l] = a;
        }
        w[wv] = butterfly64(v);
    }
    float a = ((w[0] + w[1]) + (w[2] + w[3])) + ((w[4] + w[5]) + (w[6] + w[7]));
    float b = ((w[8] + w[9]) + (w[10] + w[11])) + ((w[12] + w[13]) + (w[14] + w[15]));
    return a + b;
}

/* rms_norm (model.rs:267-272): x * (mean(x^2) + eps).sqrt().recip() * w */
void or_rmsnorm(const float* x, const float* w, size_t n, float eps, float* out) {
    float mean = or_sumsq(x, n) / (float)n;
    float r = 1.0f / sqrtf(mean + eps);
    for (size_t i = 0; i < n; i++) out[i] = (x[i] * r) * w[i];
}

/* exp(x) for the softmax: Cody & Waite (1980) two-constant reduction
 * x = n ln2 + r, |r| <= ln2/2, then the degree-7 Taylor polynomial of e^r in
 * Horner form (truncation error < 2e-9 relative), scaled by 2^n through the
 * exponent bits.  Results below 2^-126 flush to zero. */
#define EXP_LOG2E 1.44269504088896341f
#define EXP_LN2_HI 0.693145751953125f
#define EXP_LN2_LO 1.42860682030941723212e-6f
float or_expf(float x) {
    if (x != x) return x;
    if (x > 88.5f) return INFINITY;
    if (x < -87.0f) return 0.0f;
    float n = rintf(x * EXP_LOG2E);
    float r = fmaf(-n, EXP_LN2_HI, x);
    r = fmaf(-n, EXP_LN2_LO, r);
    float p = 1.98412698412698e-4f;          /* 1/5040 */
    p = fmaf(p, r, 1.38888888888889e-3f);    /* 1/720 */
    p = fmaf(p, r, 8.33333333333333e-3f);    /* 1/120 */
    p = fmaf(p, r, 4.16666666666667e-2f);    /* 1/24 */
    p = fmaf(p, r, 1.66666666666667e-1f);    /* 1/6 */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    int ni = (int)n;
    if (ni > 127) return (p * 2.0f) * u2f(0x7f000000u); /* n = 128 */
    if (ni < -126) return 0.0f;
    return p * u2f((uint32_t)(ni + 127) << 23);
}

/* argmax (sample.rs:17-25): first index of the maximum (strict >). */
uint32_t or_argmax(const float* v, size_t n) {
    size_t best = 0;
    for (size_t i = 0; i < n; i++)
        if (v[i] > v[best]) best = i;
    return (uint32_t)best;
}

/* ------------------------------------------------------------------------ */
/* Sampler::sample (sample.rs:45-82) as the device sampler computes it        */
/* ------------------------------------------------------------------------ */
/* Order of sort_unstable_by(total_cmp, descending) made total: larger logit
 * first (IEEE total order, so -0.0 after +0.0 and NaNs by sign), equal logits
 * by ascending index.  Ascending keys give that order. */
uint64_t or_sample_key(float x, uint32_t i) {
    uint32_t b;
    memcpy(&b, &x, 4);
    uint32_t asc = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)(~asc) << 32) | i;
}

static int cmp_u64(const void* a, const void* b) {
    uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
    return x < y ? -1 : x > y;
}

/* ceil(top_p * W) for 0 < top_p < 1, exactly (top_p = M 2^-sh, M < 2^24). */
uint64_t or_top_p_target(float top_p, uint64_t W) {
    if (!(top_p > 0.0f)) return 0;
    int e;
    float m = frexpf(top_p, &e);
    uint64_t M = (uint64_t)ldexpf(m, 24);
    int sh = 24 - e;
    if (sh >= 128) return 1;
    unsigned __int128 x = (unsigned __int128)M * W;
    uint64_t q = (uint64_t)(x >> sh);
    return q + (((x & ((((unsigned __int128)1) << sh) - 1)) != 0) ? 1 : 0);
}

/* The step of sample.rs:36-43 (xorshift64, seed.max(1) initially); returns
 * the 24-bit draw, r = draw / 2^24. */
uint32_t or_sample_uniform(uint64_t* state) {
    uint64_t s = *state;
    s ^= s << 13;
    s ^= s >> 7;
    s ^= s << 17;
    *state = s;
    return (uint32_t)(s >> 40);
}

/* temperature <= 0: argmax (state untouched).  Otherwise the reference's
 * steps in its order -- sort, top-k truncation, p = exp((l - max) / t), top-p
 * cut, one uniform draw, first cumulative mass above the draw -- with the
 * masses in exact integers: w = floor(p 2^45) (p <= 1, so any 2^17 of them
 * sum below 2^62), c >= top_p as sum(w) >= ceil(top_p W), r < c as
 * sum(w) > draw W_keep / 2^24.  The reference sums f32 in sorted order; the
 * two agree except where the draw lies within rounding of a boundary.  A NaN
 * among the top-k p (a NaN logit in the set, max = +inf, all -inf, a NaN
 * temperature) makes every reference comparison false: the last element of
 * the set is returned, as there. */
uint32_t or_sample(const float* logits, size_t V, float temperature, float top_p, size_t top_k, uint64_t* state) {
    if (temperature <= 0.0f) return or_argmax(logits, V);
    uint64_t* s = (uint64_t*)malloc(V * sizeof(uint64_t));
    for (size_t i = 0; i < V; i++) s[i] = or_sample_key(logits[i], (uint32_t)i);
    qsort(s, V, sizeof(uint64_t), cmp_u64);
    const size_t k = (top_k > 0 && top_k < V) ? top_k : V;
    const float mx = logits[(uint32_t)s[0]];
    uint64_t* w = (uint64_t*)malloc(k * sizeof(uint64_t));
    int bad = 0;
    for (size_t j = 0; j < k; j++) {
        float p = or_expf((logits[(uint32_t)s[j]] - mx) / temperature);
        if (p != p) bad = 1;
        w[j] = p != p ? 0 : (uint64_t)(p * 0x1p45f);
    }
    const uint64_t u = or_sample_uniform(state);
    uint32_t out = (uint32_t)s[k - 1];
    if (!bad) {
        uint64_t W = 0;
        for (size_t j = 0; j < k; j++) W += w[j];
        size_t keep = k;
        if (top_p < 1.0f) {
            const uint64_t T = or_top_p_target(top_p, W);
            uint64_t c = 0;
            for (size_t j = 0; j < k; j++) {
                c += w[j];
                if (c >= T) {
                    keep = j + 1;
                    break;
                }
            }
        }
        uint64_t WK = 0;
        for (size_t j = 0; j < keep; j++) WK += w[j];
        const uint64_t Td = (uint64_t)(((unsigned __int128)u * WK) >> 24) + 1;
        uint64_t c = 0;
        out = (uint32_t)s[keep - 1];
        for (size_t j = 0; j < keep; j++) {
            c += w[j];
            if (c >= Td) {
                out = (uint32_t)s[j];
                break;
            }
        }
    }
    free(w);
    free(s);
    return out;
}

/* ------------------------------------------------------------------------ */
/* RoPE tables (model.rs:213-230)                                            */
/* ------------------------------------------------------------------------ */
void or_rope_tables(size_t hd, size_t max_pos, double theta, float* cos_t, float* sin_t) {
    size_t h2 = hd / 2;
    float* inv = (float*)malloc(h2 * sizeof(float));
    for (size_t i = 0; i < h2; i++) inv[i] = (float)(1.0 / pow(theta, (double)(2 * i) / (double)hd));
    for (size_t p = 0; p < max_pos; p++)
        for (size_t i = 0; i < h2; i++) {
            float f = (float)p * inv[i];
            cos_t[p * h2 + i] = (float)cos((double)f);
            sin_t[p * h2 + i] = (float)sin((double)f);
        }
    free(inv);
}

/* ------------------------------------------------------------------------ */
/* synthetic weights                                                         */
/* ------------------------------------------------------------------------ */
uint64_t or_splitmix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

uint64_t or_synth_hash(uint64_t seed, uint64_t tensor, uint64_t i) {
    return or_splitmix64(or_splitmix64(seed ^ (tensor << 40)) + i);
}

/* i.i.d. ternary with P(-1, 0, +1) = (0.3, 0.4, 0.3): bucket = hi32 * 10 >> 32. */
int8_t or_synth_ternary(uint64_t seed, uint64_t tensor, uint64_t i) {
    uint64_t b = ((or_synth_hash(seed, tensor, i) >> 32) * 10u) >> 32;
    return b < 3 ? -1 : (b < 7 ? 0 : 1);
}

void or_synth_packed(uint64_t seed, uint64_t tensor, size_t rows, size_t cols, uint8_t* out) {
    size_t rb = or_row_bytes(cols);
#pragma omp parallel for schedule(static) if (rows * cols > (1u << 20))
    for (long r = 0; r < (long)rows; r++)
        for (size_t byte = 0; byte < rb; byte++) {
            size_t b = byte / BLOCK_BYTES, j = byte % BLOCK_BYTES;
            uint8_t v = 0;
            for (size_t k = 0; k < 4; k++) {
                size_t c = b * BLOCK + k * 32 + j;
                int w = c < cols ? or_synth_ternary(seed, tensor, (uint64_t)r * cols + c) : 0;
                v |= (uint8_t)((w + 1) << (2 * k));
            }
            out[(size_t)r * rb + byte] = v;
        }
}

/* u = (hash >> 40) * 2^-24 in [0, 1) (exact), value = lo + span * u. */
void or_synth_f32(uint64_t seed, uint64_t tensor, size_t n, float lo, float span, float* out) {
    for (size_t i = 0; i < n; i++) {
        float u = (float)(or_synth_hash(seed, tensor, i) >> 40) * 5.9604644775390625e-8f;
        out[i] = lo + span * u;
    }
}

/* bf16 of uniform [-1, 1). */
void or_synth_bf16(uint64_t seed, uint64_t tensor, size_t n, uint16_t* out) {
#pragma omp parallel for schedule(static) if (n > (1u << 20))
    for (long i = 0; i < (long)n; i++) {
        float u = (float)(or_synth_hash(seed, tensor, (uint64_t)i) >> 40) * 5.9604644775390625e-8f;
        out[i] = or_f32_to_bf16(u * 2.0f - 1.0f);
    }
}

/* Per-tensor weight scale of a synthetic matrix: sqrt(0.6 cols) keeps the
 * scaled outputs O(1) for O(1) activations. */
float or_synth_wscale(size_t cols) { return (float)sqrt(0.6 * (double)cols); }

/* ------------------------------------------------------------------------ */
/* BitNet forward (model.rs)                                                 */
/* ------------------------------------------------------------------------ */
struct or_model {
    or_config c;
    int owns;
    const uint8_t* packed[7 * 64];
    float wscale[7 * 64];
    const float* norm[4 * 64];
    const float* final_norm;
    const uint16_t* embed;
    float *cos_t, *sin_t;
    uint16_t* kc; /* [layers][kvh][cap][hd] */
    uint16_t* vc;
    int cap, len;
    float* hidden; /* residual stream of the last forward, [n, hidden] */
    size_t hidden_rows;
    int head_kind; /* 0 = bf16 head, 1 = int8 head (q8, q8s from embed) */
    int8_t* q8;
    float* q8s;
};

static int g_fast = 0;
int or_set_fast(int fast) { int o = g_fast; g_fast = fast; return o; }
static int g_threads = 0; /* 0: every OpenMP thread */
/* Thread count of every parallel loop here and of the SIMD port's kernels
 * (0 = all); returns the previous setting.  Used to time the CPU baseline on
 * one core and on all cores in one process. */
int or_set_threads(int n) {
    int o = g_threads;
    g_threads = n > 0 ? n : 0;
#ifdef _OPENMP
    static int all = 0;
    if (!all) all = omp_get_max_threads();
    omp_set_num_threads(n > 0 ? n : all);
#endif
    return o;
}

static const int kLinRows[7] = {0, 1, 1, 0, 2, 2, 0}; /* rows: 0=hidden 1=kv 2=inter */

static void lin_shape(const or_config* c, int which, size_t* rows, size_t* cols) {
    size_t kv = (size_t)c->kv_heads * (c->hidden / c->heads);
    size_t r = which == 1 || which == 2 ? kv : (which == 4 || which == 5 ? (size_t)c->intermediate : (size_t)c->hidden);
    (void)kLinRows;
    *rows = r;
    *cols = which == 6 ? (size_t)c->intermediate : (size_t)c->hidden;
}

static void model_alloc_runtime(or_model* m) {
    const or_config* c = &m->c;
    size_t hd = (size_t)(c->hidden / c->heads);
    m->cos_t = (float*)malloc((size_t)c->max_pos * hd / 2 * sizeof(float));
    m->sin_t = (float*)malloc((size_t)c->max_pos * hd / 2 * sizeof(float));
    or_rope_tables(hd, (size_t)c->max_pos, c->rope_theta, m->cos_t, m->sin_t);
    m->cap = c->max_pos;
    size_t kvn = (size_t)c->layers * c->kv_heads * (size_t)m->cap * hd;
    m->kc = (uint16_t*)calloc(kvn, 2);
    m->vc = (uint16_t*)calloc(kvn, 2);
    m->len = 0;
}

or_model* or_model_synthetic(const or_config* cfg, uint64_t seed) {
    or_model* m = (or_model*)calloc(1, sizeof(or_model));
    m->c = *cfg;
    m->owns = 1;
    for (int l = 0; l < cfg->layers; l++) {
        for (int w = 0; w < 7; w++) {
            size_t rows, cols;
            lin_shape(cfg, w, &rows, &cols);
            uint8_t* p = (uint8_t*)malloc(rows * or_row_bytes(cols));
            or_synth_packed(seed, OR_T_LAYER(l, w), rows, cols, p);
            m->packed[l * 7 + w] = p;
            m->wscale[l * 7 + w] = or_synth_wscale(cols);
        }
        for (int k = 0; k < 4; k++) {
            size_t n = k == 3 ? (size_t)cfg->intermediate : (size_t)cfg->hidden;
            float* v = (float*)malloc(n * sizeof(float));
            or_synth_f32(seed, OR_T_LAYER(l, 7 + k), n, 0.5f, 1.0f, v);
            m->norm[l * 4 + k] = v;
        }
    }
    float* fnorm = (float*)malloc((size_t)cfg->hidden * sizeof(float));
    or_synth_f32(seed, OR_T_FINAL_NORM, (size_t)cfg->hidden, 0.5f, 1.0f, fnorm);
    m->final_norm = fnorm;
    uint16_t* e = (uint16_t*)malloc((size_t)cfg->vocab * cfg->hidden * 2);
    or_synth_bf16(seed, OR_T_EMBED, (size_t)cfg->vocab * cfg->hidden, e);
    m->embed = e;
    model_alloc_runtime(m);
    return m;
}

or_model* or_model_wrap(const or_config* cfg, const uint8_t* const* packed, const float* wscales,
                        const float* const* norms, const float* final_norm, const uint16_t* embed) {
    or_model* m = (or_model*)calloc(1, sizeof(or_model));
    m->c = *cfg;
    m->owns = 0;
    for (int i = 0; i < cfg->layers * 7; i++) { m->packed[i] = packed[i]; m->wscale[i] = wscales[i]; }
    for (int i = 0; i < cfg->layers * 4; i++) m->norm[i] = norms[i];
    m->final_norm = final_norm;
    m->embed = embed;
    model_alloc_runtime(m);
    return m;
}

void or_model_free(or_model* m) {
    if (!m) return;
    if (m->owns) {
        for (int i = 0; i < m->c.layers * 7; i++) free((void*)m->packed[i]);
        for (int i = 0; i < m->c.layers * 4; i++) free((void*)m->norm[i]);
        free((void*)m->final_norm);
        free((void*)m->embed);
    }
    free(m->cos_t); free(m->sin_t); free(m->kc); free(m->vc); free(m->hidden);
    free(m->q8); free(m->q8s);
    free(m);
}

int or_model_set_head(or_model* m, int kind) {
    if (kind != 0 && kind != 1) return -1;
    if (kind == 1 && !m->q8) {
        size_t V = (size_t)m->c.vocab, H = (size_t)m->c.hidden;
        m->q8 = (int8_t*)malloc(V * H);
        m->q8s = (float*)malloc(V * sizeof(float));
        or_q8head_from_bf16(m->embed, V, H, m->q8, m->q8s);
    }
    m->head_kind = kind;
    return 0;
}

const uint8_t* or_model_packed(const or_model* m, int layer, int which) { return m->packed[layer * 7 + which]; }
float or_model_wscale(const or_model* m, int layer, int which) { return m->wscale[layer * 7 + which]; }
const uint16_t* or_model_embed(const or_model* m) { return m->embed; }
void or_model_reset(or_model* m) { m->len = 0; }
int or_model_len(const or_model* m) { return m->len; }
const float* or_model_hidden(const or_model* m) { return m->hidden; }
int or_model_cap(const or_model* m) { return m->cap; }
const uint16_t* or_model_kcache(const or_model* m, int layer) {
    size_t hd = (size_t)(m->c.hidden / m->c.heads);
    return m->kc + (size_t)layer * m->c.kv_heads * m->cap * hd;
}
const uint16_t* or_model_vcache(const or_model* m, int layer) {
    size_t hd = (size_t)(m->c.hidden / m->c.heads);
    return m->vc + (size_t)layer * m->c.kv_heads * m->cap * hd;
}

/* Quantize each of n rows (width k), then y[t, r] = dot * (1/(s_a s_w)) for
 * each matrix sharing the input (ops.rs:301-329: quantize once, fused GEMM). */
static void linear(const or_model* m, const float* x, size_t n, size_t k, int layer, int which, float* y) {
    size_t rows, cols;
    lin_shape(&m->c, which, &rows, &cols);
    size_t kp = or_padded_cols(k);
    int8_t* q = (int8_t*)calloc(n * kp, 1);
    float* sa = (float*)malloc(n * sizeof(float));
    int32_t* qs = (int32_t*)malloc(n * sizeof(int32_t));
    or_quantize_acts(x, n, k, q, sa, qs);
    int32_t* d = (int32_t*)malloc(n * rows * sizeof(int32_t));
    if (g_fast) port_gemm_i32(m->packed[layer * 7 + which], rows, cols, q, qs, n, d, g_threads);
    else or_gemm_i32(m->packed[layer * 7 + which], rows, cols, q, qs, n, d);
    float sw = m->wscale[layer * 7 + which];
    for (size_t t = 0; t < n; t++) {
        float inv = 1.0f / (sa[t] * sw);
        for (size_t r = 0; r < rows; r++) y[t * rows + r] = (float)d[t * rows + r] * inv;
    }
    free(q); free(sa); free(qs); free(d);
}

/* xor butterfly over n values (n a power of two): step m = n/2 .. 1 adds
 * v[l ^ m] to v[l]; returns v[0]. */
static float butterfly_n(float* v, int n) {
    float t[64];
    for (int m = n / 2; m >= 1; m >>= 1) {
        for (int l = 0; l < n; l++) t[l] = v[l] + v[l ^ m];
        memcpy(v, t, (size_t)n * sizeof(float));
    }
    return v[0];
}

/* q.k in the device order: LK = hd/8 lanes, lane c sums dims 8c..8c+7 by
 * fused multiply-adds, lanes combine by butterfly_n. */
static float attn_score(const float* q, const uint16_t* k, size_t hd) {
    int lk = (int)(hd / 8);
    float part[64];
    for (int c = 0; c < lk; c++) {
        float a = 0.0f;
        for (int e = 0; e < 8; e++) a = fmaf(q[8 * c + e], or_bf16_to_f32(k[8 * c + e]), a);
        part[c] = a;
    }
    return butterfly_n(part, lk);
}

/* probs @ V in the device order: 256/LK key groups, group g accumulates keys
 * j = g, g + 256/LK, ... by fused multiply-adds; the 64/LK groups of each
 * wavefront combine by xor over the group index (m = 1, 2, ...), then the four
 * wave sums as (w0 + w1) + (w2 + w3). */
static void attn_pv(const float* p, const uint16_t* V, size_t vis, size_t hd, float* out) {
    int lk = (int)(hd / 8), gw = 64 / lk, ng = 256 / lk;
    float acc[256];
    for (size_t d = 0; d < hd; d++) {
        for (int g = 0; g < ng; g++) {
            float a = 0.0f;
            for (size_t j = (size_t)g; j < vis; j += (size_t)ng) a = fmaf(p[j], or_bf16_to_f32(V[j * hd + d]), a);
            acc[g] = a;
        }
        float wsum[4];
        for (int w = 0; w < 4; w++) {
            float v[64], t[64];
            memcpy(v, acc + w * gw, (size_t)gw * sizeof(float));
            for (int m = 1; m < gw; m <<= 1) {
                for (int l = 0; l < gw; l++) t[l] = v[l] + v[l ^ m];
                memcpy(v, t, (size_t)gw * sizeof(float));
            }
            wsum[w] = v[0];
        }
        out[d] = (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
    }
}

/* apply_rope (model.rs:295-301): x*cos + rot*sin, rot = cat(-x2, x1). */
static void rope(float* v, size_t hd, const float* c, const float* s) {
    size_t h2 = hd / 2;
    float tmp[512];
    for (size_t d = 0; d < hd; d++) {
        size_t i = d % h2;
        float rot = d < h2 ? -v[d + h2] : v[d - h2];
        tmp[d] = v[d] * c[i] + rot * s[i];
    }
    memcpy(v, tmp, hd * sizeof(float));
}

/* Split-key attention of the gh query heads that read one KV head, in the
 * device's float order (lemonade-burn_amd/csrc/attn_common.h):
 * ks = max(64, ceil(vis/16)) keys per split; per split and head the max m_s,
 * l_s = block sum of per-thread sums of exp(s_u - m_s) (thread t: u = t, t+256,
 * ...), o_s = attn_pv of the exponentials; then in split order
 * f_s = exp(m_s - M), L = xor butterfly over 16 split slots of l_s f_s,
 * O = fma(o_s, f_s, O) in split order, out = O * (1 / L). */
#define ATTN_SPLITS 16
#define ATTN_MIN_KEYS 64
static void attn_split_group(const float* qg, const uint16_t* K, const uint16_t* V, size_t vis, size_t hd,
                             size_t gh, float scaling, float* out) {
    size_t ks = (vis + ATTN_SPLITS - 1) / ATTN_SPLITS;
    if (ks < ATTN_MIN_KEYS) ks = ATTN_MIN_KEYS;
    size_t ns = (vis + ks - 1) / ks;
    float* ms = (float*)malloc(ns * gh * sizeof(float));
    float* ls = (float*)malloc(ns * gh * sizeof(float));
    float* os = (float*)malloc(ns * gh * hd * sizeof(float));
    float* e = (float*)malloc(ks * sizeof(float));
    for (size_t s = 0; s < ns; s++) {
        size_t j0 = s * ks, cnt = vis - j0 < ks ? vis - j0 : ks;
        for (size_t h = 0; h < gh; h++) {
            const float* qh = qg + h * hd;
            float mx = -INFINITY;
            for (size_t u = 0; u < cnt; u++) {
                e[u] = attn_score(qh, K + (j0 + u) * hd, hd) * scaling;
                mx = fmaxf(mx, e[u]);
            }
            for (size_t u = 0; u < cnt; u++) e[u] = or_expf(e[u] - mx);
            float part[256];
            for (int th = 0; th < 256; th++) {
                float a = 0.0f;
                for (size_t u = (size_t)th; u < cnt; u += 256) a = a + e[u];
                part[th] = a;
            }
            ms[s * gh + h] = mx;
            ls[s * gh + h] = or_block_sum256(part);
            attn_pv(e, V + j0 * hd, cnt, hd, os + (s * gh + h) * hd);
        }
    }
    for (size_t h = 0; h < gh; h++) {
        float M = -INFINITY;
        for (size_t s = 0; s < ns; s++) M = fmaxf(M, ms[s * gh + h]);
        float f[ATTN_SPLITS], lf[ATTN_SPLITS];
        for (size_t s = 0; s < ATTN_SPLITS; s++) {
            f[s] = s < ns ? or_expf(ms[s * gh + h] - M) : 0.0f;
            lf[s] = s < ns ? ls[s * gh + h] * f[s] : 0.0f;
        }
        float L = butterfly_n(lf, ATTN_SPLITS);
        float rl = 1.0f / L;
        for (size_t d = 0; d < hd; d++) {
            float O = 0.0f;
            for (size_t s = 0; s < ns; s++) O = fmaf(os[(s * gh + h) * hd + d], f[s], O);
            out[h * hd + d] = O * rl;
        }
    }
    free(ms); free(ls); free(os); free(e);
}

/* The synthetic KV fill of a batch of nseq sequences (the device's
 * lbt_batch_fill_synthetic, a test fixture with no reference counterpart),
 * restated for sequence `seq` of such a batch: cache rows r = (layer * nseq +
 * seq) * kv_heads + head hold, at flat index i = (r * len + pos) * hd + d of
 * the [rows][len][hd] values, bf16((sum of the four 16-bit fields of
 * splitmix64(splitmix64(s) + i), each / 65536) - 2) * sqrt(3)) with s =
 * 2 seed + 1 for K and 2 seed + 2 for V.  The model's length becomes len. */
static uint16_t synth_kv_value(uint64_t base, uint64_t i) {
    const uint64_t z = or_splitmix64(base + i);
    float acc = 0.0f;
    for (int k = 0; k < 4; k++) acc += (float)((z >> (16 * k)) & 0xffffu) * (1.0f / 65536.0f);
    return or_f32_to_bf16((acc - 2.0f) * 1.7320508075688772f);
}

int or_model_fill_synth_kv(or_model* m, uint64_t seed, int nseq, int seq, int len) {
    const or_config* c = &m->c;
    if (len < 0 || len > m->cap || seq < 0 || seq >= nseq) return -1;
    const size_t hd = (size_t)(c->hidden / c->heads), kvh = (size_t)c->kv_heads, cap = (size_t)m->cap;
    const uint64_t bk = or_splitmix64(seed * 2 + 1), bv = or_splitmix64(seed * 2 + 2);
    for (int l = 0; l < c->layers; l++)
        for (size_t g = 0; g < kvh; g++) {
            const uint64_t r = ((uint64_t)l * (uint64_t)nseq + (uint64_t)seq) * kvh + g;
            uint16_t* K = m->kc + ((size_t)l * kvh + g) * cap * hd;
            uint16_t* V = m->vc + ((size_t)l * kvh + g) * cap * hd;
            for (size_t p = 0; p < (size_t)len; p++)
                for (size_t d = 0; d < hd; d++) {
                    const uint64_t i = (r * (uint64_t)len + p) * hd + d;
                    K[p * hd + d] = synth_kv_value(bk, i);
                    V[p * hd + d] = synth_kv_value(bv, i);
                }
        }
    m->len = len;
    return 0;
}

int or_model_forward(or_model* m, const uint32_t* tokens, size_t n, int all_logits, float* logits) {
    const or_config* c = &m->c;
    size_t H = (size_t)c->hidden, I = (size_t)c->intermediate;
    size_t nh = (size_t)c->heads, kvh = (size_t)c->kv_heads, hd = H / nh, group = nh / kvh;
    size_t h2 = hd / 2, cap = (size_t)m->cap;
    size_t pos0 = (size_t)m->len, total = pos0 + n;
    float eps = (float)c->rms_norm_eps;
    if (total > (size_t)c->max_pos) return -1;
    float scaling = powf((float)hd, -0.5f);

    float* x = (float*)malloc(n * H * sizeof(float));
    float* nrm = (float*)malloc(n * (I > H ? I : H) * sizeof(float)); /* normed rows of either width */
    float* q = (float*)malloc(n * H * sizeof(float));
    float* kk = (float*)malloc(n * kvh * hd * sizeof(float));
    float* vv = (float*)malloc(n * kvh * hd * sizeof(float));
    float* att = (float*)malloc(n * H * sizeof(float));
    float* y = (float*)malloc(n * H * sizeof(float));
    float* g = (float*)malloc(n * I * sizeof(float));
    float* u = (float*)malloc(n * I * sizeof(float));

    /* embed (model.rs:274-282) */
    for (size_t t = 0; t < n; t++)
        for (size_t i = 0; i < H; i++) x[t * H + i] = or_bf16_to_f32(m->embed[(size_t)tokens[t] * H + i]);

    for (int l = 0; l < c->layers; l++) {
        const float* const* nw = &m->norm[l * 4]; /* input, post_attn, attn_sub, ffn_sub */
        uint16_t* K = m->kc + (size_t)l * kvh * cap * hd;
        uint16_t* V = m->vc + (size_t)l * kvh * cap * hd;
        for (size_t t = 0; t < n; t++) or_rmsnorm(x + t * H, nw[0], H, eps, nrm + t * H);
        linear(m, nrm, n, H, l, 0, q);
        linear(m, nrm, n, H, l, 1, kk);
        linear(m, nrm, n, H, l, 2, vv);
        for (size_t t = 0; t < n; t++) {
            size_t p = pos0 + t;
            const float* cs = m->cos_t + p * h2;
            const float* sn = m->sin_t + p * h2;
            for (size_t h = 0; h < nh; h++) rope(q + t * H + h * hd, hd, cs, sn);
            for (size_t h = 0; h < kvh; h++) {
                rope(kk + (t * kvh + h) * hd, hd, cs, sn);
                for (size_t d = 0; d < hd; d++) {
                    K[(h * cap + p) * hd + d] = or_f32_to_bf16(kk[(t * kvh + h) * hd + d]);
                    V[(h * cap + p) * hd + d] = or_f32_to_bf16(vv[(t * kvh + h) * hd + d]);
                }
            }
        }
        /* GQA attention (model.rs:349-357): q head h reads kv head h / group. */
        for (size_t t = 0; t < n; t++) {
            size_t vis = pos0 + t + 1;
            if (g_fast >= 2) { /* reference order, SIMD, heads over threads (timed CPU baseline only) */
                port_attention(q + t * H, K, V, nh, group, cap, vis, hd, scaling, att + t * H, g_threads);
                continue;
            }
            for (size_t h = 0; h < nh; h++)
                attn_split_group(q + t * H + h * hd, K + (h / group) * cap * hd, V + (h / group) * cap * hd, vis, hd,
                                 1, scaling, att + t * H + h * hd);
        }
        for (size_t t = 0; t < n; t++) or_rmsnorm(att + t * H, nw[2], H, eps, nrm + t * H);
        linear(m, nrm, n, H, l, 3, y);
        for (size_t i = 0; i < n * H; i++) x[i] = x[i] + y[i];
        for (size_t t = 0; t < n; t++) or_rmsnorm(x + t * H, nw[1], H, eps, nrm + t * H);
        linear(m, nrm, n, H, l, 4, g);
        linear(m, nrm, n, H, l, 5, u);
        /* relu(g)^2 * u (model.rs:363) */
        for (size_t i = 0; i < n * I; i++) {
            float r = g[i] > 0.0f ? g[i] : 0.0f;
            g[i] = (r * r) * u[i];
        }
        for (size_t t = 0; t < n; t++) or_rmsnorm(g + t * I, nw[3], I, eps, nrm + t * I);
        linear(m, nrm, n, I, l, 6, y);
        for (size_t i = 0; i < n * H; i++) x[i] = x[i] + y[i];
    }
    m->len = (int)total;
    free(m->hidden);
    m->hidden = (float*)malloc(n * H * sizeof(float));
    memcpy(m->hidden, x, n * H * sizeof(float));
    m->hidden_rows = n;

    /* final norm + tied bf16 LM head (model.rs:368-373) */
    size_t first = all_logits ? 0 : n - 1;
    for (size_t t = first; t < n; t++) {
        or_rmsnorm(x + t * H, m->final_norm, H, eps, nrm);
        float* lt = logits + (t - first) * (size_t)c->vocab;
        if (m->head_kind == 1) or_q8head_gemv_lanes(m->q8, m->q8s, (size_t)c->vocab, H, nrm, lt);
        else if (g_fast >= 2) port_bf16_gemv(m->embed, (size_t)c->vocab, H, nrm, lt, g_threads); /* reference order */
        else or_bf16_gemv_lanes(m->embed, (size_t)c->vocab, H, nrm, lt);
    }
    free(x); free(nrm); free(q); free(kk); free(vv); free(att); free(y); free(g); free(u);
    return 0;
}
