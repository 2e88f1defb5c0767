/*
 * lbt_port.h -- multi-threaded SIMD restatement of the reference's CPU kernels
 * (crates/lb-ternary/src/gemm.rs, quant.rs, bf16.rs).
 *
 * TEST INFRASTRUCTURE ONLY: it is the timed CPU baseline of bench.py and a
 * fast exact integer kernel for the model oracle.  Checked bit for bit against
 * the scalar oracle (tests/test_oracle.py) before it is trusted.
 */
#ifndef LBT_PORT_H
#define LBT_PORT_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* Best ISA on this CPU: "avx512vnni", "avx512bw", "avx2" or "scalar"
 * (Kernel::detect, gemm.rs:78-91); LB_KERNEL overrides as in the reference. */
const char* port_isa(void);
/* ternary_gemm_i32 (gemm.rs:95-114) with the SIMD codes_dot kernels
 * (gemm.rs:387-407 avx2, :433-469 avx512bw, :553-588 avx512vnni), rows split
 * over `threads` OpenMP threads (0 = all). */
void port_gemm_i32(const uint8_t* packed, size_t rows, size_t cols, const int8_t* q,
                   const int32_t* qsum, size_t m, int32_t* out, int threads);
/* ternary_gemm f32 epilogue (gemm.rs:141,150). */
void port_gemm_f32(const uint8_t* packed, size_t rows, size_t cols, float s_w, const int8_t* q,
                   const float* s_a, const int32_t* qsum, size_t m, float* out, int threads);
/* quantize_row_avx2 (quant.rs:141-193); falls back to scalar without AVX2. */
float port_quantize_row(const float* x, size_t k, int8_t* q, int32_t* sum);
/* bf16_gemv (bf16.rs:14-25) with dot_avx512 (bf16.rs:84-105) / dot_avx2 (:58-81). */
void port_bf16_gemv(const uint16_t* w, size_t rows, size_t cols, const float* x, float* out, int threads);
/* GQA attention of one token (model.rs:349-357): head h of nh reads kv head
 * h / group of K/V [kv_heads][cap][hd] (bf16) over positions 0..vis-1. */
void port_attention(const float* q, const uint16_t* K, const uint16_t* V, size_t nh, size_t group,
                    size_t cap, size_t vis, size_t hd, float scaling, float* out, int threads);
int port_threads(void);

#ifdef __cplusplus
}
#endif
#endif
