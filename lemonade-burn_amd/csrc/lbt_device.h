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

#define LBT_GLOBAL __attribute__((address_space(1)))

// Load through the global address space (global_load rather than flat_load,
// which also occupies the LDS counter); p must point to device memory.
template <typename T>
__device__ __forceinline__ T gload(const T* p) {
    return *(const LBT_GLOBAL T*)p;
}

// 16-byte streaming load (nontemporal: the weights are read once per token).
__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
    const u32x4 v = __builtin_nontemporal_load((const LBT_GLOBAL u32x4*)p);
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

// Cross-lane exchange without LDS: xor_pair<M>(v) returns (a, b) with
// {a, b} = {v[l], v[l ^ M]} at every lane l (the order within the pair may
// differ between lanes, which commutative combines do not see).
//   M = 1, 2:  DPP quad_perm;      M = 4: two DPP row rotates (row_ror:n
//   reads lane (i - n) mod 16: by 12 for lane banks 0 and 2, by 4 for banks
//   1 and 3);   M = 8: DPP row_ror:8;
//   M = 16, 32: v_permlane16_swap / v_permlane32_swap (gfx950).
// Every lane of the wavefront must be active.
template <int M>
__device__ __forceinline__ void xor_pair(uint32_t v, uint32_t& a, uint32_t& b) {
    static_assert(M == 1 || M == 2 || M == 4 || M == 8 || M == 16 || M == 32, "xor distance");
    if constexpr (M == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        a = r[0];
        b = r[1];
    } else if constexpr (M == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        a = r[0];
        b = r[1];
    } else {
        const int iv = (int)v;
        int p;
        if constexpr (M == 1) p = __builtin_amdgcn_update_dpp(0, iv, 0xB1, 0xf, 0xf, false);
        else if constexpr (M == 2) p = __builtin_amdgcn_update_dpp(0, iv, 0x4E, 0xf, 0xf, false);
        else if constexpr (M == 8) p = __builtin_amdgcn_update_dpp(0, iv, 0x128, 0xf, 0xf, false);
        else {
            p = __builtin_amdgcn_update_dpp(0, iv, 0x12C, 0xf, 0x5, false);
            p = __builtin_amdgcn_update_dpp(p, iv, 0x124, 0xf, 0xA, false);
        }
        a = v;
        b = (uint32_t)p;
    }
}

// v[l] + v[l ^ M] (bit-identical to v + __shfl_xor(v, M)).
template <int M>
__device__ __forceinline__ float xor_add(float v) {
    uint32_t a, b;
    xor_pair<M>(__float_as_uint(v), a, b);
    return __uint_as_float(a) + __uint_as_float(b);
}
template <int M>
__device__ __forceinline__ int xor_add_i(int v) {
    uint32_t a, b;
    xor_pair<M>((uint32_t)v, a, b);
    return (int)a + (int)b;
}
template <int M>
__device__ __forceinline__ float xor_max(float v) {
    uint32_t a, b;
    xor_pair<M>(__float_as_uint(v), a, b);
    return fmaxf(__uint_as_float(a), __uint_as_float(b));
}

// Butterfly steps M, M/2, ..., 1 (descending), as
// `for (m = M; m >= 1; m >>= 1) v = v + __shfl_xor(v, m)`.
template <int M>
__device__ __forceinline__ float xor_sum_down(float v) {
    if constexpr (M >= 1) {
        v = xor_add<M>(v);
        return xor_sum_down<M / 2>(v);
    }
    return v;
}
template <int M>
__device__ __forceinline__ int xor_sum_down_i(int v) {
    if constexpr (M >= 1) {
        v = xor_add_i<M>(v);
        return xor_sum_down_i<M / 2>(v);
    }
    return v;
}

// Butterfly steps M, 2M, ..., 32 (ascending), as
// `for (m = M; m <= 32; m <<= 1) v = v + __shfl_xor(v, m)`.
template <int M>
__device__ __forceinline__ float xor_sum_up(float v) {
    if constexpr (M <= 32) {
        v = xor_add<M>(v);
        return xor_sum_up<M * 2>(v);
    }
    return v;
}

// xor butterfly over the 64 lanes of a wavefront: every lane ends with the
// same value, lane l having added v[l] + v[l ^ m] for m = 32, 16, ..., 1.
__device__ __forceinline__ float wave_sum(float v) { return xor_sum_down<32>(v); }

__device__ __forceinline__ float wave_max(float v) {
    v = xor_max<32>(v);
    v = xor_max<16>(v);
    v = xor_max<8>(v);
    v = xor_max<4>(v);
    v = xor_max<2>(v);
    return xor_max<1>(v);
}

__device__ __forceinline__ int wave_sum_i(int v) { return xor_sum_down_i<32>(v); }

// Block reductions over the first 256 threads (four wavefronts): wavefront
// results of waves 0..3 go to red[4*slot .. 4*slot+3], one barrier, then
// sum (w0 + w1) + (w2 + w3) / max / integer sum.  No trailing barrier: a slot
// may be written again only after two further barriers, which holds when
// successive reductions rotate through slots 0, 1, 2 or a barrier separates
// them from the next use.  `red` >= 16 floats of LDS; larger workgroups call
// with all threads (the barrier is shared) and get the first four waves'
// result.
__device__ __forceinline__ float block_sum_slot(float v, float* red, int slot) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0 && w < 4) red[4 * slot + w] = v;
    __syncthreads();
    const float* r = red + 4 * slot;
    return (r[0] + r[1]) + (r[2] + r[3]);
}
__device__ __forceinline__ float block_max_slot(float v, float* red, int slot) {
    v = wave_max(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0 && w < 4) red[4 * slot + w] = v;
    __syncthreads();
    const float* r = red + 4 * slot;
    return fmaxf(fmaxf(r[0], r[1]), fmaxf(r[2], r[3]));
}
__device__ __forceinline__ int block_sum_i_slot(int v, int* red, int slot) {
    v = wave_sum_i(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0 && w < 4) red[4 * slot + w] = v;
    __syncthreads();
    const int* r = red + 4 * slot;
    return r[0] + r[1] + r[2] + r[3];
}

// The same reductions followed by a barrier, so `red` is free on return.
__device__ __forceinline__ float block_sum(float v, float* red) {
    const float r = block_sum_slot(v, red, 0);
    __syncthreads();
    return r;
}
__device__ __forceinline__ float block_max(float v, float* red) {
    const float r = block_max_slot(v, red, 0);
    __syncthreads();
    return r;
}
__device__ __forceinline__ int block_sum_i(int v, int* red) {
    const int r = block_sum_i_slot(v, red, 0);
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
    __device__ __forceinline__ float operator()(int i) const { return gload(p + i); }
    __device__ __forceinline__ SrcF32 fresh() const { return SrcF32{launder(p)}; }
};
struct SrcBf16 {
    const uint16_t* p;
    __device__ __forceinline__ float operator()(int i) const { return bf16_to_f32(gload(p + i)); }
    __device__ __forceinline__ SrcBf16 fresh() const { return SrcBf16{launder(p)}; }
};

// Loads row x[0..cols) into registers, v[e] = x[threadIdx.x + 256 e] (0 past
// cols), and if norm_w is set applies rms_norm (crates/lb-model/src/model.rs:
// 267-272) in place: r = 1 / sqrt(sum(x^2)/cols + eps) with the sum of squares
// accumulated per thread by fused multiply-adds in ascending i and combined by
// block_sum; v = (x * r) * w.  Requires cols <= 256 * EPT.  One global pass.
// Uses reduction slot 0 of `red` (see block_sum_slot).
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
        nw[e] = (act && norm_w && i < cols) ? gload(norm_w + i) : 0.0f;
    }
    if (!norm_w) return;
    float p = 0.0f;
#pragma unroll
    for (int e = 0; e < EPT; e++)
        if (act && threadIdx.x + e * kThreads < cols) p = __builtin_fmaf(v[e], v[e], p);
    const float ss = block_sum_slot(p, red, 0);
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
