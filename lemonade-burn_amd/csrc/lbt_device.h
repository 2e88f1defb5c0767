// lbt_device.h -- device helpers shared by the gfx950 kernels.
//
// Float reduction order is fixed and documented here; the CPU oracle
// (oracle/lbt_oracle.c) follows the same order so results compare bit for bit.
//   * wavefront sums: xor butterfly, lane l takes v[l] + v[l ^ m] for
//     m = 32, ..., 1;
//   * block sums (256 threads): wavefront sums, then (w0 + w1) + (w2 + w3);
//   * max and integer sums are order independent.
// All code is compiled with -ffp-contract=off; fused multiply-adds are written
// explicitly with __builtin_fmaf.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lbt {

constexpr int kBlock = 128;      // weights per LB2 block (pack.rs:18)
constexpr int kBlockBytes = 32;  // bytes per LB2 block (pack.rs:19)
constexpr int kThreads = 256;    // threads per workgroup everywhere

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16-byte streaming load (nontemporal: the weights are read once per token).
__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
    const u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// Round to nearest even; NaN -> canonical quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// quant_one (crates/lb-ternary/src/quant.rs:116-118):
// (v*scale).round_ties_even().clamp(-128, 127) as i8, NaN -> 0.
__device__ __forceinline__ int quant_one(float v, float scale) {
    float y = __builtin_rintf(v * scale);
    if (y != y) return 0;
    y = y < -128.0f ? -128.0f : y;
    y = y > 127.0f ? 127.0f : y;
    return (int)y;
}

// exp(x) for the softmax: Cody & Waite two-constant reduction x = n ln2 + r,
// degree-7 Taylor polynomial of e^r (Horner, fused multiply-adds), scale by
// 2^n through the exponent bits; below 2^-126 flushes to zero.
__device__ __forceinline__ float lbt_expf(float x) {
    if (x != x) return x;
    if (x > 88.5f) return __uint_as_float(0x7f800000u);
    if (x < -87.0f) return 0.0f;
    float n = __builtin_rintf(x * 1.44269504088896341f);
    float r = __builtin_fmaf(-n, 0.693145751953125f, x);
    r = __builtin_fmaf(-n, 1.42860682030941723212e-6f, r);
    float p = 1.98412698412698e-4f;
    p = __builtin_fmaf(p, r, 1.38888888888889e-3f);
    p = __builtin_fmaf(p, r, 8.33333333333333e-3f);
    p = __builtin_fmaf(p, r, 4.16666666666667e-2f);
    p = __builtin_fmaf(p, r, 1.66666666666667e-1f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    int ni = (int)n;
    if (ni > 127) return (p * 2.0f) * __uint_as_float(0x7f000000u);
    if (ni < -126) return 0.0f;
    return p * __uint_as_float((uint32_t)(ni + 127) << 23);
}

// xor butterfly over the 64 lanes of a wavefront: every lane ends with the
// same value, lane l having added v[l] + v[l ^ m] for m = 32, 16, ..., 1.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = v + __shfl_xor(v, m);
    return v;
}

// Block sum of one value per thread (blockDim.x == 256): wave butterflies,
// then (w0 + w1) + (w2 + w3).  `red` >= 16 floats of LDS (workgroups of up
// to 1024 threads; only the first four waves' sums are used).
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float r = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m));
    return v;
}

__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    return v;
}

// Block max over the first 256 threads; `red` >= 16 floats of LDS.
__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float r = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    return r;
}

__device__ __forceinline__ int block_sum_i(int v, int* red) {
    v = wave_sum_i(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    int r = red[0] + red[1] + red[2] + red[3];
    __syncthreads();
    return r;
}

// Hides a uniform pointer's value from the optimizer, so per-element
// addresses derived from it are recomputed where they are used instead of
// being hoisted out of long loops (which exhausts registers in the
// persistent decode kernel).
// The pointer must be uniform across the wavefront.
template <typename T>
__device__ __forceinline__ T* launder(T* p) {
    const unsigned long long v = (unsigned long long)p;
    unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)v);
    unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(v >> 32));
    asm volatile("" : "+s"(lo), "+s"(hi));
    return (T*)(((unsigned long long)hi << 32) | lo);
}

// threadIdx.x hidden from the optimizer (same purpose as launder: per-lane
// values are recomputed in each phase instead of living across a long loop).
__device__ __forceinline__ int fresh_tid() {
    int t = (int)threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

// Row sources for the activation prologues: f32 rows, or bf16 rows (the
// embedding, widened exactly).
struct SrcF32 {
    const float* p;
    __device__ __forceinline__ float operator()(int i) const { return p[i]; }
    __device__ __forceinline__ SrcF32 fresh() const { return SrcF32{launder(p)}; }
};
struct SrcBf16 {
    const uint16_t* p;
    __device__ __forceinline__ float operator()(int i) const { return bf16_to_f32(p[i]); }
    __device__ __forceinline__ SrcBf16 fresh() const { return SrcBf16{launder(p)}; }
};

// Loads row x[0..cols) into registers, v[e] = x[threadIdx.x + 256 e] (0 past
// cols), and if norm_w is set applies rms_norm (crates/lb-model/src/model.rs:
// 267-272) in place: r = 1 / sqrt(sum(x^2)/cols + eps) with the sum of squares
// accumulated per thread by fused multiply-adds in ascending i and combined by
// block_sum; v = (x * r) * w.  Requires cols <= 256 * EPT.  One global pass.
// Only the first 256 threads of the workgroup take part; larger workgroups
// call it with all threads (the barriers are shared) and get zeros elsewhere.
template <int EPT, typename Src>
__device__ __forceinline__ void load_norm_row(Src x, int cols, const float* norm_w, float eps, float (&v)[EPT],
                                              float* red) {
    const bool act = threadIdx.x < kThreads;
    float nw[EPT];
#pragma unroll
    for (int e = 0; e < EPT; e++) {
        const int i = threadIdx.x + e * kThreads;
        v[e] = (act && i < cols) ? x(i) : 0.0f;
        nw[e] = (act && norm_w && i < cols) ? norm_w[i] : 0.0f;
    }
    if (!norm_w) return;
    float p = 0.0f;
#pragma unroll
    for (int e = 0; e < EPT; e++)
        if (act && threadIdx.x + e * kThreads < cols) p = __builtin_fmaf(v[e], v[e], p);
    const float ss = block_sum(p, red);
    const float r = 1.0f / __builtin_sqrtf(ss / (float)cols + eps);
#pragma unroll
    for (int e = 0; e < EPT; e++) v[e] = (v[e] * r) * nw[e];
}

// Same result for rows longer than 256 * EPT, re-reading x from memory.
template <typename Src>
__device__ __forceinline__ float norm_factor_global(Src x, int cols, const float* norm_w, float eps, float* red) {
    if (!norm_w) return 1.0f;
    float p = 0.0f;
    if (threadIdx.x < kThreads)
        for (int i = threadIdx.x; i < cols; i += kThreads) p = __builtin_fmaf(x(i), x(i), p);
    const float ss = block_sum(p, red);
    return 1.0f / __builtin_sqrtf(ss / (float)cols + eps);
}

// Ordered key for an f32 so that unsigned comparison follows float order; NaN
// gets the lowest key (never selected, as in sample.rs:17-25 where `v > best`
// is false for NaN).
__device__ __forceinline__ uint32_t float_key(float v) {
    uint32_t u = __float_as_uint(v);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Argmax key: larger value wins, ties go to the lower index (first max).
__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t idx) {
    return ((unsigned long long)float_key(v) << 32) | (unsigned long long)(0xffffffffu - idx);
}

// Position of activation element i of a padded row (kp = 64 * C) inside the
// permuted LDS image used by the ternary kernels: group kk = (i/32)%4 major,
// then 16-byte chunk c = 2*(i/128) + (i/16)%2, then byte i%16.  Chunk c of a
// packed row (bytes 16c..16c+15) pairs with the 16 bytes at (kk*C + c)*16.
__device__ __forceinline__ int perm_pos(int i, int C) {
    const int kk = (i >> 5) & 3;
    const int c = ((i >> 7) << 1) | ((i >> 4) & 1);
    return ((kk * C + c) << 4) | (i & 15);
}

}  // namespace lbt
