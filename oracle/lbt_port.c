/*
 * lbt_port.c -- SIMD CPU restatement of lemonade-burn's kernels (the timed
 * CPU baseline).  TEST INFRASTRUCTURE ONLY; see lbt_port.h.
 *
 * The integer kernels follow the reference's arithmetic: codes c = w + 1 in
 * {0,1,2} are multiplied with the int8 activations (u8 x i8), summed exactly
 * in i32, and the caller subtracts sum(q) (gemm.rs:3-17, :306-308).
 */
#include "lbt_port.h"

#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "lbt_oracle.h"

enum { ISA_SCALAR, ISA_AVX2, ISA_AVX512BW, ISA_AVX512VNNI };

static int detect_isa(void) {
    static int isa = -1;
    if (isa >= 0) return isa;
    __builtin_cpu_init();
    int best = ISA_SCALAR;
    if (__builtin_cpu_supports("avx2")) best = ISA_AVX2;
    if (__builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw")) {
        best = ISA_AVX512BW;
        if (__builtin_cpu_supports("avx512vnni")) best = ISA_AVX512VNNI;
    }
    const char* env = getenv("LB_KERNEL");
    if (env) {
        int want = -1;
        if (!strcmp(env, "scalar")) want = ISA_SCALAR;
        else if (!strcmp(env, "avx2")) want = ISA_AVX2;
        else if (!strcmp(env, "avx512") || !strcmp(env, "avx512bw")) want = ISA_AVX512BW;
        else if (!strcmp(env, "avx512vnni") || !strcmp(env, "vnni")) want = ISA_AVX512VNNI;
        if (want >= 0 && want <= best) best = want;
    }
    isa = best;
    return isa;
}

const char* port_isa(void) {
    static const char* names[] = {"scalar", "avx2", "avx512bw", "avx512vnni"};
    return names[detect_isa()];
}

int port_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ---- AVX2 (gemm.rs:361-407) -------------------------------------------- */
__attribute__((target("avx2"))) static inline int32_t hsum256(__m256i v) {
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4e));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xb1));
    return _mm_cvtsi128_si32(s);
}

/* One 128-weight block: 32 packed bytes against 128 activations. */
__attribute__((target("avx2"))) static inline __m256i block_avx2(const uint8_t* p, const int8_t* xb) {
    const __m256i mask = _mm256_set1_epi8(3);
    __m256i v = _mm256_loadu_si256((const __m256i*)p);
    __m256i s = _mm256_maddubs_epi16(_mm256_and_si256(v, mask), _mm256_loadu_si256((const __m256i*)xb));
    s = _mm256_add_epi16(s, _mm256_maddubs_epi16(_mm256_and_si256(_mm256_srli_epi16(v, 2), mask),
                                                 _mm256_loadu_si256((const __m256i*)(xb + 32))));
    s = _mm256_add_epi16(s, _mm256_maddubs_epi16(_mm256_and_si256(_mm256_srli_epi16(v, 4), mask),
                                                 _mm256_loadu_si256((const __m256i*)(xb + 64))));
    s = _mm256_add_epi16(s, _mm256_maddubs_epi16(_mm256_and_si256(_mm256_srli_epi16(v, 6), mask),
                                                 _mm256_loadu_si256((const __m256i*)(xb + 96))));
    return _mm256_madd_epi16(s, _mm256_set1_epi16(1));
}

__attribute__((target("avx2"))) static int32_t dot_avx2(const uint8_t* row, size_t nb, const int8_t* x) {
    __m256i a = _mm256_setzero_si256();
    for (size_t b = 0; b < nb; b++) a = _mm256_add_epi32(a, block_avx2(row + b * 32, x + b * 128));
    return hsum256(a);
}

/* ---- AVX-512 (gemm.rs:409-469, :553-588): two blocks per 64-byte load ---- */
__attribute__((target("avx512f,avx512bw"))) static inline __m512i xpair(const int8_t* xb, int k) {
    __m256i lo = _mm256_loadu_si256((const __m256i*)(xb + k * 32));
    __m256i hi = _mm256_loadu_si256((const __m256i*)(xb + 128 + k * 32));
    return _mm512_inserti64x4(_mm512_castsi256_si512(lo), hi, 1);
}

__attribute__((target("avx512f,avx512bw,avx2"))) static int32_t dot_avx512bw(const uint8_t* row, size_t nb,
                                                                             const int8_t* x) {
    const __m512i mask = _mm512_set1_epi8(3), ones = _mm512_set1_epi16(1);
    __m512i a = _mm512_setzero_si512();
    size_t pairs = nb / 2;
    for (size_t bb = 0; bb < pairs; bb++) {
        __m512i v = _mm512_loadu_si512((const void*)(row + bb * 64));
        const int8_t* xb = x + bb * 256;
        __m512i s = _mm512_maddubs_epi16(_mm512_and_si512(v, mask), xpair(xb, 0));
        s = _mm512_add_epi16(s, _mm512_maddubs_epi16(_mm512_and_si512(_mm512_srli_epi16(v, 2), mask), xpair(xb, 1)));
        s = _mm512_add_epi16(s, _mm512_maddubs_epi16(_mm512_and_si512(_mm512_srli_epi16(v, 4), mask), xpair(xb, 2)));
        s = _mm512_add_epi16(s, _mm512_maddubs_epi16(_mm512_and_si512(_mm512_srli_epi16(v, 6), mask), xpair(xb, 3)));
        a = _mm512_add_epi32(a, _mm512_madd_epi16(s, ones));
    }
    int32_t r = _mm512_reduce_add_epi32(a);
    if (nb % 2) r += hsum256(block_avx2(row + (nb - 1) * 32, x + (nb - 1) * 128));
    return r;
}

__attribute__((target("avx512f,avx512bw,avx512vnni,avx2"))) static int32_t dot_avx512vnni(const uint8_t* row,
                                                                                           size_t nb,
                                                                                           const int8_t* x) {
    const __m512i mask = _mm512_set1_epi8(3);
    __m512i a = _mm512_setzero_si512();
    size_t pairs = nb / 2;
    for (size_t bb = 0; bb < pairs; bb++) {
        __m512i v = _mm512_loadu_si512((const void*)(row + bb * 64));
        const int8_t* xb = x + bb * 256;
        a = _mm512_dpbusd_epi32(a, _mm512_and_si512(v, mask), xpair(xb, 0));
        a = _mm512_dpbusd_epi32(a, _mm512_and_si512(_mm512_srli_epi16(v, 2), mask), xpair(xb, 1));
        a = _mm512_dpbusd_epi32(a, _mm512_and_si512(_mm512_srli_epi16(v, 4), mask), xpair(xb, 2));
        a = _mm512_dpbusd_epi32(a, _mm512_and_si512(_mm512_srli_epi16(v, 6), mask), xpair(xb, 3));
    }
    int32_t r = _mm512_reduce_add_epi32(a);
    if (nb % 2) r += hsum256(block_avx2(row + (nb - 1) * 32, x + (nb - 1) * 128));
    return r;
}

static int32_t codes_dot(int isa, const uint8_t* row, size_t kp, const int8_t* x) {
    size_t nb = kp / 128;
    switch (isa) {
        case ISA_AVX512VNNI: return dot_avx512vnni(row, nb, x);
        case ISA_AVX512BW: return dot_avx512bw(row, nb, x);
        case ISA_AVX2: return dot_avx2(row, nb, x);
        default: return or_codes_dot(row, kp, x);
    }
}

void port_gemm_i32(const uint8_t* packed, size_t rows, size_t cols, const int8_t* q,
                   const int32_t* qsum, size_t m, int32_t* out, int threads) {
    int isa = detect_isa();
    size_t kp = or_padded_cols(cols), rb = kp / 4;
    int nt = threads > 0 ? threads : port_threads();
    /* ~8 row chunks per thread (chunk_rows, gemm.rs:204-209) */
    long chunk = (long)((rows + (size_t)nt * 8 - 1) / ((size_t)nt * 8));
    if (chunk < 8) chunk = 8;
#pragma omp parallel for schedule(dynamic) num_threads(nt)
    for (long c0 = 0; c0 < (long)rows; c0 += chunk) {
        long c1 = c0 + chunk < (long)rows ? c0 + chunk : (long)rows;
        for (long r = c0; r < c1; r++)
            for (size_t t = 0; t < m; t++)
                out[t * rows + (size_t)r] = codes_dot(isa, packed + (size_t)r * rb, kp, q + t * kp) - qsum[t];
    }
}

void port_gemm_f32(const uint8_t* packed, size_t rows, size_t cols, float s_w, const int8_t* q,
                   const float* s_a, const int32_t* qsum, size_t m, float* out, int threads) {
    int32_t* d = (int32_t*)malloc(rows * m * sizeof(int32_t));
    port_gemm_i32(packed, rows, cols, q, qsum, m, d, threads);
    for (size_t t = 0; t < m; t++) {
        float inv = 1.0f / (s_a[t] * s_w);
        for (size_t r = 0; r < rows; r++) out[t * rows + r] = (float)d[t * rows + r] * inv;
    }
    free(d);
}

/* ---- quantize_row_avx2 (quant.rs:141-193) ------------------------------- */
__attribute__((target("avx2"))) static float quant_avx2(const float* x, size_t n, int8_t* q, int32_t* sum) {
    const __m256 absmask = _mm256_castsi256_ps(_mm256_set1_epi32(0x7fffffff));
    __m256 mx = _mm256_setzero_ps();
    size_t n8 = n / 8 * 8;
    for (size_t i = 0; i < n8; i += 8) mx = _mm256_max_ps(_mm256_and_ps(_mm256_loadu_ps(x + i), absmask), mx);
    float lanes[8];
    _mm256_storeu_ps(lanes, mx);
    float amax = 0.0f;
    for (int l = 0; l < 8; l++) amax = fmaxf(amax, lanes[l]);
    for (size_t i = n8; i < n; i++) amax = fmaxf(amax, fabsf(x[i]));
    float scale = 127.0f / fmaxf(amax, 1e-5f);
    const __m256 s = _mm256_set1_ps(scale), lo = _mm256_set1_ps(-128.0f), hi = _mm256_set1_ps(127.0f);
    __m256i acc = _mm256_setzero_si256();
    size_t i = 0;
    for (; i + 8 <= n; i += 8) {
        __m256 y = _mm256_mul_ps(_mm256_loadu_ps(x + i), s);
        __m256 r = _mm256_round_ps(y, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
        __m256 c = _mm256_min_ps(_mm256_max_ps(r, lo), hi);
        c = _mm256_and_ps(c, _mm256_cmp_ps(y, y, _CMP_ORD_Q)); /* NaN -> 0 */
        __m256i v = _mm256_cvtps_epi32(c);
        acc = _mm256_add_epi32(acc, v);
        int32_t tmp[8];
        _mm256_storeu_si256((__m256i*)tmp, v);
        for (int l = 0; l < 8; l++) q[i + l] = (int8_t)tmp[l];
    }
    int32_t s32 = hsum256(acc);
    for (; i < n; i++) {
        float y = rintf(x[i] * scale);
        int8_t r = y != y ? 0 : (int8_t)(y < -128.0f ? -128.0f : (y > 127.0f ? 127.0f : y));
        q[i] = r;
        s32 += r;
    }
    *sum = s32;
    return scale;
}

float port_quantize_row(const float* x, size_t k, int8_t* q, int32_t* sum) {
    if (detect_isa() >= ISA_AVX2) return quant_avx2(x, k, q, sum);
    return or_quantize_row(x, k, q, sum);
}

/* ---- bf16 GEMV (bf16.rs:14-105) ---------------------------------------- */
__attribute__((target("avx512f"))) static float bdot_avx512(const uint16_t* w, const float* x, size_t n) {
    size_t n64 = n / 64 * 64;
    __m512 a[4] = {_mm512_setzero_ps(), _mm512_setzero_ps(), _mm512_setzero_ps(), _mm512_setzero_ps()};
    for (size_t i = 0; i < n64; i += 64)
        for (int u = 0; u < 4; u++) {
            __m512i wi = _mm512_cvtepu16_epi32(_mm256_loadu_si256((const __m256i*)(w + i + u * 16)));
            __m512 wf = _mm512_castsi512_ps(_mm512_slli_epi32(wi, 16));
            a[u] = _mm512_fmadd_ps(wf, _mm512_loadu_ps(x + i + u * 16), a[u]);
        }
    __m512 s = _mm512_add_ps(_mm512_add_ps(a[0], a[1]), _mm512_add_ps(a[2], a[3]));
    float r = _mm512_reduce_add_ps(s);
    for (size_t j = n64; j < n; j++) r += or_bf16_to_f32(w[j]) * x[j];
    return r;
}

__attribute__((target("avx2,fma"))) static float bdot_avx2(const uint16_t* w, const float* x, size_t n) {
    size_t n32 = n / 32 * 32;
    __m256 a[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
    for (size_t i = 0; i < n32; i += 32)
        for (int u = 0; u < 4; u++) {
            __m256i wi = _mm256_cvtepu16_epi32(_mm_loadu_si128((const __m128i*)(w + i + u * 8)));
            __m256 wf = _mm256_castsi256_ps(_mm256_slli_epi32(wi, 16));
            a[u] = _mm256_fmadd_ps(wf, _mm256_loadu_ps(x + i + u * 8), a[u]);
        }
    __m256 s = _mm256_add_ps(_mm256_add_ps(a[0], a[1]), _mm256_add_ps(a[2], a[3]));
    float buf[8];
    _mm256_storeu_ps(buf, s);
    float r = 0.0f;
    for (int l = 0; l < 8; l++) r += buf[l];
    for (size_t j = n32; j < n; j++) r += or_bf16_to_f32(w[j]) * x[j];
    return r;
}

void port_bf16_gemv(const uint16_t* w, size_t rows, size_t cols, const float* x, float* out, int threads) {
    int isa = detect_isa();
    int nt = threads > 0 ? threads : port_threads();
#pragma omp parallel for schedule(static, 256) num_threads(nt)
    for (long r = 0; r < (long)rows; r++) {
        const uint16_t* wr = w + (size_t)r * cols;
        out[r] = isa >= ISA_AVX512BW ? bdot_avx512(wr, x, cols)
                 : isa == ISA_AVX2   ? bdot_avx2(wr, x, cols)
                                     : or_bf16_dot_ref(wr, x, cols);
    }
}

/* ---- attention over the bf16 cache (model.rs:349-357) ----------------------
 * One query row per head: scores = q.K^T * scaling, softmax, probs @ V, as the
 * reference's Flex backend computes them (f32 dot products, max-subtracted
 * expf, a normalised sum of value rows), with the cache rows read in order. */
__attribute__((target("avx2,fma"))) static inline __m256 bf16x8_avx2(const uint16_t* p) {
    __m128i h = _mm_loadu_si128((const __m128i*)p);
    return _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(h), 16));
}

__attribute__((target("avx2,fma"))) static void attn_head_avx2(const float* q, const uint16_t* K,
                                                                const uint16_t* V, size_t vis, size_t hd,
                                                                float scaling, float* e, float* out) {
    float mx = -INFINITY;
    for (size_t j = 0; j < vis; j++) {
        const uint16_t* kr = K + j * hd;
        __m256 a = _mm256_setzero_ps();
        for (size_t d = 0; d < hd; d += 8) a = _mm256_fmadd_ps(_mm256_loadu_ps(q + d), bf16x8_avx2(kr + d), a);
        __m128 s4 = _mm_add_ps(_mm256_castps256_ps128(a), _mm256_extractf128_ps(a, 1));
        s4 = _mm_add_ps(s4, _mm_movehl_ps(s4, s4));
        s4 = _mm_add_ss(s4, _mm_shuffle_ps(s4, s4, 1));
        e[j] = _mm_cvtss_f32(s4) * scaling;
        if (e[j] > mx) mx = e[j];
    }
    float sum = 0.0f;
    for (size_t j = 0; j < vis; j++) {
        e[j] = expf(e[j] - mx);
        sum += e[j];
    }
    float acc[512];
    for (size_t d = 0; d < hd; d++) acc[d] = 0.0f;
    for (size_t j = 0; j < vis; j++) {
        const uint16_t* vr = V + j * hd;
        __m256 p = _mm256_set1_ps(e[j]);
        for (size_t d = 0; d < hd; d += 8)
            _mm256_storeu_ps(acc + d, _mm256_fmadd_ps(p, bf16x8_avx2(vr + d), _mm256_loadu_ps(acc + d)));
    }
    float inv = 1.0f / sum;
    for (size_t d = 0; d < hd; d++) out[d] = acc[d] * inv;
}

void port_attention(const float* q, const uint16_t* K, const uint16_t* V, size_t nh, size_t group,
                    size_t cap, size_t vis, size_t hd, float scaling, float* out, int threads) {
    int nt = threads > 0 ? threads : port_threads();
    int fast = detect_isa() >= ISA_AVX2 && hd % 8 == 0 && hd <= 512;
#pragma omp parallel num_threads(nt)
    {
        float* e = (float*)malloc(vis * sizeof(float));
#pragma omp for schedule(static)
        for (long h = 0; h < (long)nh; h++) {
            const uint16_t* Kh = K + (size_t)(h / (long)group) * cap * hd;
            const uint16_t* Vh = V + (size_t)(h / (long)group) * cap * hd;
            const float* qh = q + (size_t)h * hd;
            float* oh = out + (size_t)h * hd;
            if (fast) {
                attn_head_avx2(qh, Kh, Vh, vis, hd, scaling, e, oh);
                continue;
            }
            float mx = -INFINITY, sum = 0.0f;
            for (size_t j = 0; j < vis; j++) {
                float a = 0.0f;
                for (size_t d = 0; d < hd; d++) a += qh[d] * or_bf16_to_f32(Kh[j * hd + d]);
                e[j] = a * scaling;
                if (e[j] > mx) mx = e[j];
            }
            for (size_t j = 0; j < vis; j++) {
                e[j] = expf(e[j] - mx);
                sum += e[j];
            }
            for (size_t d = 0; d < hd; d++) oh[d] = 0.0f;
            for (size_t j = 0; j < vis; j++)
                for (size_t d = 0; d < hd; d++) oh[d] += e[j] * or_bf16_to_f32(Vh[j * hd + d]);
            for (size_t d = 0; d < hd; d++) oh[d] /= sum;
        }
        free(e);
    }
}
