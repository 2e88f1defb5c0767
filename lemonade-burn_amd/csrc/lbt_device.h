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
constexpr int kThreads = 256;    // threads per workgroup of most kernels
constexpr int kRedFloats = 48;   // LDS floats of a row prologue's reductions (16-byte aligned)

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

#define LBT_GLOBAL __attribute__((address_space(1)))

// Load through the global address space (global_load rather than flat_load,
// which also occupies the LDS counter); p must point to device memory.
template <typename T>
__device__ __forceinline__ T gload(const T* p) {
    return *(const LBT_GLOBAL T*)p;
}
// Store through the global address space (a flat store also counts on the
// LDS counter, and waits for it then wait for every store in flight).
template <typename T>
__device__ __forceinline__ void gstore(T* p, T v) {
    *(LBT_GLOBAL T*)p = v;
}

// Buffer resource over [base, base + bytes): raw buffer loads past the end
// return zeros, so bounded loads need no branch (and no register merge that
// would make the compiler wait for them early).  Word 3 is the gfx9-family
// raw-buffer format.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ f32x4 buf_load_f4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}
__device__ __forceinline__ f32x2 buf_load_f2(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, 0));
}

// Loads the compiler does not track (inline asm), waited for with explicit
// counts (vm_wait<N>: at most N vector-memory operations still outstanding;
// loads complete in issue order, stores count too).  For loops that keep the
// next iteration's loads in flight: the compiler's own tracking of
// loop-carried loads falls back to waiting for everything.  Rules: every use
// of a result comes after a vm_wait that covers it, followed by pin() on the
// value (so no use is scheduled above the wait), and every result stays live
// until such a wait (a dead result's register could be handed to another
// value while the load is still to write it).
__device__ __forceinline__ u32x4 ld_u4_async_nt(const void* p) {
    u32x4 v;
    asm volatile("global_load_dwordx4 %0, %1, off nt" : "=v"(v) : "v"(p) : "memory");
    return v;
}
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u32x2 ld_u2_async_nt(const void* p) {
    u32x2 v;
    asm volatile("global_load_dwordx2 %0, %1, off nt" : "=v"(v) : "v"(p) : "memory");
    return v;
}
__device__ __forceinline__ float ld_f32_async(const float* p) {
    float v;
    asm volatile("global_load_dword %0, %1, off" : "=v"(v) : "v"(p) : "memory");
    return v;
}
template <int N>
__device__ __forceinline__ void vm_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
template <typename T>
__device__ __forceinline__ void pin(T& v) {
    asm volatile("" : "+v"(v));
}
template <typename T>
__device__ __forceinline__ void keep(const T& v) {
    asm volatile("" ::"v"(v));
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
    const float y = __builtin_rintf(v * scale);
    if (y != y) return 0;
    return (int)__builtin_amdgcn_fmed3f(y, -128.0f, 127.0f);
}

// Four quant_one values of consecutive elements, packed little-endian into
// one word; *sum += their sum.  v_cvt_i32_f32 saturates out-of-range values
// and converts NaN to 0, so rint -> convert -> clamp to [-128, 127] equals
// quant_one for every input.
__device__ __forceinline__ uint32_t quant4(const float* v, float scale, int& sum) {
    uint32_t word = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        int q;
        asm("v_cvt_i32_f32 %0, %1" : "=v"(q) : "v"(__builtin_rintf(v[k] * scale)));
        q = q < -128 ? -128 : (q > 127 ? 127 : q);
        word |= ((uint32_t)q & 0xffu) << (8 * k);
    }
    sum = __builtin_amdgcn_sdot4((int)word, 0x01010101, sum, false);
    return word;
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

// Recursive halving of K per-lane partial sums over the wavefront: step M
// pairs accumulator j with j + K/2, the lanes with bit M set keep the upper
// one and receive the partner lanes' values of it, the others the lower one;
// each kept sum is v[l] + v[l ^ M], the same pairwise sums (bit for bit, the
// adds being commutative) as a full butterfly of that accumulator.  After
// steps 32, 16, ..., 2, lane l holds accumulator (l >> 1) & 31 (K = 32);
// in general the lane bits of the steps taken, high to low, index it.
template <int M, int K>
__device__ __forceinline__ void halve(const float (&v)[K], float (&o)[K / 2]) {
    const int lane = (int)threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < K / 2; j++) {
        const uint32_t lo = __float_as_uint(v[j]), hi = __float_as_uint(v[j + K / 2]);
        if constexpr (M == 32) {
            // lanes 0-31 get (lo[l], lo[l+32]), lanes 32-63 (hi[l-32], hi[l])
            const auto r = __builtin_amdgcn_permlane32_swap(lo, hi, false, false);
            o[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
        } else if constexpr (M == 16) {
            // rows 0, 2 get (lo, lo of the next row), rows 1, 3 (hi of the previous row, hi)
            const auto r = __builtin_amdgcn_permlane16_swap(lo, hi, false, false);
            o[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
        } else {
            const bool up = (lane & M) != 0;
            const uint32_t keep = up ? hi : lo, send = up ? lo : hi;
            uint32_t a, b;
            xor_pair<M>(send, a, b);  // b: the partner's `send` (a is own)
            o[j] = __uint_as_float(keep) + __uint_as_float(b);
        }
    }
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

// Max / integer sum over the first NT threads (NT/64 wavefronts, values at
// w[0 .. NT/64)); one barrier, no trailing barrier (order independent).
template <int NT>
__device__ __forceinline__ float block_max_n(float v, float* w) {
    v = wave_max(v);
    const int wi = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0 && wi < NT / 64) w[wi] = v;
    __syncthreads();
    float r = w[0];
#pragma unroll
    for (int i = 1; i < NT / 64; i++) r = fmaxf(r, w[i]);
    return r;
}
template <int NT>
__device__ __forceinline__ int block_sum_i_n(int v, int* w) {
    v = wave_sum_i(v);
    const int wi = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0 && wi < NT / 64) w[wi] = v;
    __syncthreads();
    int r = 0;
#pragma unroll
    for (int i = 0; i < NT / 64; i++) r += w[i];
    return r;
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
    // four elements i..i+3 at once when vec_ok (16-byte aligned groups)
    __device__ __forceinline__ bool vec_ok(int cols) const {
        return (cols & 3) == 0 && ((uintptr_t)p & 15) == 0;
    }
    __device__ __forceinline__ void load4(int i, float* o) const {
        const f32x4 v = gload((const f32x4*)(p + i));
        o[0] = v.x;
        o[1] = v.y;
        o[2] = v.z;
        o[3] = v.w;
    }
    __device__ __forceinline__ SrcF32 fresh() const { return SrcF32{launder(p)}; }
};
struct SrcBf16 {
    const uint16_t* p;
    __device__ __forceinline__ float operator()(int i) const { return bf16_to_f32(gload(p + i)); }
    __device__ __forceinline__ bool vec_ok(int cols) const {
        return (cols & 3) == 0 && ((uintptr_t)p & 7) == 0;
    }
    __device__ __forceinline__ void load4(int i, float* o) const {
        const u32x2 v = gload((const u32x2*)(p + i));
        o[0] = __uint_as_float(v.x << 16);
        o[1] = __uint_as_float(v.x & 0xffff0000u);
        o[2] = __uint_as_float(v.y << 16);
        o[3] = __uint_as_float(v.y & 0xffff0000u);
    }
    __device__ __forceinline__ SrcBf16 fresh() const { return SrcBf16{launder(p)}; }
};

// Element layout of the row prologues with NT participating threads (256,
// 512 or 1024; threads past NT take no part): thread t holds EPT/4 groups of
// four consecutive elements, v[4g + k] = x[4*NT*g + 4t + k].  Rows of up to
// NT * EPT elements are held in registers (one global pass).
template <int NT = kThreads>
__device__ __forceinline__ int row_elem(int tid, int e) {
    return 4 * NT * (e >> 2) + 4 * tid + (e & 3);
}

template <int EPT>
struct RowRegs {
    static_assert(EPT % 4 == 0, "groups of four");
    float v[EPT];
    float nw[EPT];
};

// Issues the loads of row x[0..cols) (0 past cols) and, if norm_w is set, of
// the norm weights, into r.
template <int EPT, int NT = kThreads, typename Src>
__device__ __forceinline__ void row_load(Src x, int cols, const float* norm_w, RowRegs<EPT>& r) {
    const int tid = (int)threadIdx.x;
    const bool act = tid < NT;
    const bool vec = x.vec_ok(cols) && (!norm_w || ((uintptr_t)norm_w & 15) == 0);
#pragma unroll
    for (int g = 0; g < EPT / 4; g++) {
        const int i0 = 4 * NT * g + 4 * tid;
        if (vec && act && i0 < cols) {
            x.load4(i0, &r.v[4 * g]);
            if (norm_w) {
                const f32x4 w = gload((const f32x4*)(norm_w + i0));
                r.nw[4 * g] = w.x;
                r.nw[4 * g + 1] = w.y;
                r.nw[4 * g + 2] = w.z;
                r.nw[4 * g + 3] = w.w;
            }
        } else {
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int i = i0 + k;
                r.v[4 * g + k] = (!vec && act && i < cols) ? x(i) : 0.0f;
                r.nw[4 * g + k] = (!vec && act && norm_w && i < cols) ? gload(norm_w + i) : 0.0f;
            }
        }
        if (!norm_w) {
#pragma unroll
            for (int k = 0; k < 4; k++) r.nw[4 * g + k] = 0.0f;
        }
    }
}

// row_load for a 16-byte aligned f32 row with cols % 4 == 0, through
// bounded buffer loads (branch-free; threads past NT load nothing).
template <int EPT, int NT>
__device__ __forceinline__ void row_load_buf(const float* x, int cols, const float* norm_w, RowRegs<EPT>& r) {
    const int tid = (int)threadIdx.x;
    const auto rx = buf_rsrc(x, (uint32_t)cols * 4u);
    const auto rw = buf_rsrc(norm_w ? norm_w : x, norm_w ? (uint32_t)cols * 4u : 0u);
#pragma unroll
    for (int g = 0; g < EPT / 4; g++) {
        const uint32_t off = tid < NT ? (uint32_t)(4 * NT * g + 4 * tid) * 4u : 0xfffffff0u;
        const f32x4 v = buf_load_f4(rx, off);
        const f32x4 w = buf_load_f4(rw, off);
        r.v[4 * g] = v.x;
        r.v[4 * g + 1] = v.y;
        r.v[4 * g + 2] = v.z;
        r.v[4 * g + 3] = v.w;
        r.nw[4 * g] = w.x;
        r.nw[4 * g + 1] = w.y;
        r.nw[4 * g + 2] = w.z;
        r.nw[4 * g + 3] = w.w;
    }
}

// Sum of the 16 per-wavefront partial sums w[0..15] as a full binary tree.
__device__ __forceinline__ float tree16(const float* w) {
    const float a = ((w[0] + w[1]) + (w[2] + w[3])) + ((w[4] + w[5]) + (w[6] + w[7]));
    const float b = ((w[8] + w[9]) + (w[10] + w[11])) + ((w[12] + w[13]) + (w[14] + w[15]));
    return a + b;
}

// Canonical sum of squares of a row (the same bits for any thread count):
// element groups gi (elements 4gi .. 4gi+3) belong to virtual thread
// vt = gi mod 1024, which accumulates x^2 by fused multiply-adds over its
// elements in ascending order; the 16 virtual wavefronts (vt / 64) reduce
// by xor butterflies, then tree16.  A kernel with NT threads holds
// A = 1024 / NT virtual threads per thread (vt = t + NT*j).  Uses red[0..15]
// (reduction slots 0..3).  row_sumsq_part leaves the 16 virtual-wavefront
// sums in red[0..15] (threads past NT take no part; no barrier).
template <int EPT, int NT = kThreads>
__device__ __forceinline__ void row_sumsq_part(const RowRegs<EPT>& r, int cols, float* red) {
    static_assert(NT == 256 || NT == 512 || NT == 1024, "threads of a row prologue");
    constexpr int A = 1024 / NT;
    const int tid = (int)threadIdx.x, lane = tid & 63;
    const bool act = tid < NT;
    float acc[A];
#pragma unroll
    for (int j = 0; j < A; j++) acc[j] = 0.0f;
#pragma unroll
    for (int g = 0; g < EPT / 4; g++)
#pragma unroll
        for (int k = 0; k < 4; k++)
            if (act && row_elem<NT>(tid, 4 * g + k) < cols)
                acc[g % A] = __builtin_fmaf(r.v[4 * g + k], r.v[4 * g + k], acc[g % A]);
    if constexpr (A == 4) {
        // the four wavefront sums together: recursive halving over lane bits
        // 5 and 4 (each kept sum is v[l] + v[l^m], the butterfly's sums), then
        // the butterfly's last four steps; accumulator 2*b5 + b4 ends in the
        // lanes with those bits (lanes 0, 16, 32, 48 write them)
        float h2[2], h1[1];
        halve<32, 4>(acc, h2);
        halve<16, 2>(h2, h1);
        const float s = xor_sum_down<8>(h1[0]);
        if ((lane & 15) == 0 && act) red[(tid >> 6) + (lane >> 4) * (NT / 64)] = s;
    } else {
#pragma unroll
        for (int j = 0; j < A; j++) {
            const float s = wave_sum(acc[j]);
            if (lane == 0 && act) red[(tid >> 6) + j * (NT / 64)] = s;
        }
    }
}
// The partials of row_sumsq_part, published by a barrier, summed.
template <int EPT, int NT = kThreads>
__device__ __forceinline__ float row_sumsq(const RowRegs<EPT>& r, int cols, float* red) {
    row_sumsq_part<EPT, NT>(r, cols, red);
    __syncthreads();
    return tree16(red);
}

// rms_norm (crates/lb-model/src/model.rs:267-272) of the loaded row, in place,
// when norm_w is set: f = 1 / sqrt(row_sumsq/cols + eps); v = (x * f) * w.
// NORM: 1 norm present, 0 absent, -1 decided at run time by norm_w (a
// compile-time choice keeps the caller's code free of a merge point).
template <int EPT, int NT = kThreads, int NORM = -1>
__device__ __forceinline__ void row_norm(RowRegs<EPT>& r, int cols, const float* norm_w, float eps, float* red) {
    if constexpr (NORM == 0) return;
    if (NORM < 0 && !norm_w) return;
    const float ss = row_sumsq<EPT, NT>(r, cols, red);
    const float f = 1.0f / __builtin_sqrtf(ss / (float)cols + eps);
#pragma unroll
    for (int e = 0; e < EPT; e++) r.v[e] = (r.v[e] * f) * r.nw[e];
}

// row_load + row_norm: v[e] = normed x[row_elem(threadIdx.x, e)].  Requires
// cols <= 256 * EPT.  Only the first 256 threads of the workgroup take part;
// larger workgroups call it with all threads (the barriers are shared) and get
// zeros elsewhere.
template <int EPT, typename Src>
__device__ __forceinline__ void load_norm_row(Src x, int cols, const float* norm_w, float eps, float (&v)[EPT],
                                              float* red) {
    RowRegs<EPT> r;
    row_load<EPT>(x, cols, norm_w, r);
    row_norm<EPT>(r, cols, norm_w, eps, red);
#pragma unroll
    for (int e = 0; e < EPT; e++) v[e] = r.v[e];
}

// The same norm factor for rows longer than the register path, re-reading x
// from memory (first 256 threads, four virtual threads each).
template <typename Src>
__device__ __forceinline__ float norm_factor_global(Src x, int cols, const float* norm_w, float eps, float* red) {
    if (!norm_w) return 1.0f;
    const int tid = (int)threadIdx.x, lane = tid & 63;
    const bool act = tid < kThreads;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        float p = 0.0f;
        if (act)
            for (int gi = tid + kThreads * j; 4 * gi < cols; gi += 1024)
                for (int i = 4 * gi; i < 4 * gi + 4 && i < cols; i++) p = __builtin_fmaf(x(i), x(i), p);
        const float s = wave_sum(p);
        if (lane == 0 && act) red[(tid >> 6) + 4 * j] = s;
    }
    __syncthreads();
    const float ss = tree16(red);
    __syncthreads();
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
