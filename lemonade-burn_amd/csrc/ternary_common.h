// ternary_common.h -- shared by the ternary decode GEMV and the int8-MFMA
// prefill GEMM: kernel arguments, the virtual-row mapping of the fused
// matrices, and the output epilogues, so both kernels write identical values.
#pragma once
#include "lbt_device.h"
#include "lbt_internal.h"

namespace lbt {

struct GemvArgs {
    const uint8_t* w[3];
    int rows[3];
    float sw[3];
    int total_rows;  // virtual rows (2*rows for the gate/up interleave)
    int cols, kp, C;
    int m;
    const int8_t* q;
    const float* qscale;
    const int32_t* qsum;
    const float* x;
    const float* norm_w;
    float eps;
    const float* att_o;  // kInAttn
    const float* att_ml;
    int att_nh;
    void* out[3];
    // kOutQKV: RoPE at positions pos0 + token and bf16 K/V cache append
    int hd, pos0, cap;
    const int* pos_dev;  // if set, *pos_dev replaces pos0 (graph-replayed steps)
    const int* tok_pos;  // if set, token t is sequence t at position tok_pos[t]
    size_t seq_stride;   // its cache rows start t * seq_stride elements in
    const float* cos_t;
    const float* sin_t;
    uint16_t* kc;
    uint16_t* vc;
    // split-k GEMM: the k steps are cut into ksplit ranges (gridDim.z); each
    // workgroup stores its int32 partial tile to kpart and the last of a
    // tile's workgroups (counter kcnt[tile], left at zero) adds them up and
    // runs the epilogue
    int ksplit;
    int* kcnt;
    int* kpart;
};

// Element i (0..2) of a 3-array of uniform values by selects between scalar
// registers.  A runtime index into a local struct would put the struct in
// scratch memory, and a plain select of kernel-argument fields is turned into
// a vector load from the argument segment (one memory round trip before the
// first weight load); the elements are pinned to scalar registers first.
__device__ __forceinline__ uint32_t pin_s(uint32_t v) {
    v = __builtin_amdgcn_readfirstlane(v);
    asm volatile("" : "+s"(v));
    return v;
}
template <typename T>
__device__ __forceinline__ T* sel3(T* const (&v)[3], int i) {
    T* a = launder(v[0]);
    T* b = launder(v[1]);
    T* c = launder(v[2]);
    return i == 0 ? a : (i == 1 ? b : c);
}
__device__ __forceinline__ int sel3(const int (&v)[3], int i) {
    const int a = (int)pin_s((uint32_t)v[0]), b = (int)pin_s((uint32_t)v[1]), c = (int)pin_s((uint32_t)v[2]);
    return i == 0 ? a : (i == 1 ? b : c);
}
__device__ __forceinline__ float sel3(const float (&v)[3], int i) {
    const float a = __uint_as_float(pin_s(__float_as_uint(v[0])));
    const float b = __uint_as_float(pin_s(__float_as_uint(v[1])));
    const float c = __uint_as_float(pin_s(__float_as_uint(v[2])));
    return i == 0 ? a : (i == 1 ? b : c);
}

// Virtual row -> (matrix, row).  kOutRelu2 interleaves gate/up rows
// (2r, 2r+1) = (gate r, up r).  kOutQKV interleaves RoPE partners: for q and
// k, virtual rows (2p, 2p+1) are rows (d, d + hd/2) of one head; v keeps its
// order.  Otherwise rows of the matrices follow one another.
template <int OUT>
__device__ __forceinline__ void resolve_row(const GemvArgs& a, int vr, int& mat, int& r) {
    if (OUT == kOutRelu2) {
        mat = vr & 1;
        r = vr >> 1;
        return;
    }
    if (OUT == kOutQKV) {
        int p = vr >> 1;
        const int s = vr & 1, h2 = a.hd >> 1;
        mat = 0;
        if (p >= a.rows[0] >> 1) {
            p -= a.rows[0] >> 1;
            mat = 1;
            if (p >= a.rows[1] >> 1) {
                p -= a.rows[1] >> 1;
                mat = 2;
            }
        }
        r = mat == 2 ? 2 * p + s : (p / h2) * a.hd + (p % h2) + s * h2;
        return;
    }
    mat = 0;
    r = vr;
    if (r >= a.rows[0]) {
        r -= a.rows[0];
        mat = 1;
        if (r >= a.rows[1]) {
            r -= a.rows[1];
            mat = 2;
        }
    }
}

// Output of one (token, virtual row) for the unpaired modes:
// i32 dot; f32 y = dot * (1/(s_a*s_w)) (gemm.rs:141,150); or the residual
// x += y (model.rs:359,365).
template <int OUT>
__device__ __forceinline__ void store_single(const GemvArgs& a, int tok, int v, int dot, float sa) {
    int mt, ro;
    resolve_row<OUT>(a, v, mt, ro);
    const size_t o = (size_t)tok * sel3(a.rows, mt) + ro;
    if (OUT == kOutI32) {
        gstore((int32_t*)sel3(a.out, mt) + o, (int32_t)dot);
    } else {
        const float y = (float)dot * (1.0f / (sa * sel3(a.sw, mt)));
        float* dst = (float*)sel3(a.out, mt) + o;
        gstore(dst, OUT == kOutF32Add ? gload(dst) + y : y);
    }
}

// Output of the virtual-row pair (v0, v0 + 1) for the paired modes:
// kOutRelu2: relu(gate)^2 * up (model.rs:362-363);
// kOutQKV:   q/k get apply_rope (model.rs:295-301) at the token's position, q is
//            stored f32, k and v are rounded to bf16 into the cache.
template <int OUT>
__device__ __forceinline__ void store_pair(const GemvArgs& a, int tok, int v0, int d0, int d1, float sa) {
    int mat, r0;
    resolve_row<OUT>(a, v0, mat, r0);
    const float inv = 1.0f / (sa * sel3(a.sw, mat));
    const float y0 = (float)d0 * inv;
    if (OUT == kOutRelu2) {
        const float u = (float)d1 * (1.0f / (sa * a.sw[1]));
        const float rl = y0 > 0.0f ? y0 : 0.0f;
        gstore((float*)a.out[0] + (size_t)tok * a.rows[0] + r0, (rl * rl) * u);
        return;
    }
    const float y1 = (float)d1 * inv;
    const int pos = a.tok_pos ? gload(a.tok_pos + tok) : (a.pos_dev ? gload(a.pos_dev) : a.pos0) + tok;
    const size_t coff = a.tok_pos ? (size_t)tok * a.seq_stride : 0;
    if (mat == 2) {  // v: rows r0, r0 + 1 of head r0 / hd
        const int g = r0 / a.hd, d = r0 % a.hd;
        uint16_t* dst = a.vc + coff + ((size_t)g * a.cap + pos) * a.hd + d;
        gstore(dst, f32_to_bf16(y0));
        gstore(dst + 1, f32_to_bf16(y1));
        return;
    }
    const int h2 = a.hd >> 1, g = r0 / a.hd, d = r0 % a.hd;
    const float c = gload(a.cos_t + (size_t)pos * h2 + d), sn = gload(a.sin_t + (size_t)pos * h2 + d);
    const float z0 = y0 * c + (-y1) * sn;
    const float z1 = y1 * c + y0 * sn;
    if (mat == 0) {
        float* q = (float*)a.out[0] + (size_t)tok * a.rows[0];
        gstore(q + r0, z0);
        gstore(q + r0 + h2, z1);
    } else {
        uint16_t* dst = a.kc + coff + ((size_t)g * a.cap + pos) * a.hd + d;
        gstore(dst, f32_to_bf16(z0));
        gstore(dst + h2, f32_to_bf16(z1));
    }
}

// amax over the (normed) row, then s_a = 127 / max(amax, 1e-5) (quant.rs:100-113).
template <typename Src>
__device__ __forceinline__ float act_scale(Src x, int cols, const float* norm_w, float rr, float* red) {
    float am = 0.0f;
    if (threadIdx.x < kThreads)
        for (int i = threadIdx.x; i < cols; i += kThreads)
            am = fmaxf(am, fabsf(norm_w ? (x(i) * rr) * norm_w[i] : x(i)));
    am = block_max(am, red);
    return 127.0f / fmaxf(am, 1e-5f);
}

// ActQuant (quant.rs:100-118) of a row already in registers (row_load, and
// row_norm applied here when norm_w is set) into `dst` at positions pos(i),
// four bytes per store (pos keeps each 4-aligned group contiguous); zeros
// fill [cols, kp).  s_a and sum(q) go to *sa / *qs (written by thread 0).
// Requires kp <= NT * EPT.  Work is done by the first NT threads; every
// thread must call it (shared barriers).  `red` holds kRedFloats floats
// (16-byte aligned): [0, 16) sum of squares, [16, 32) max, [32, 48) integer
// sum, each in use until two more barriers have passed (successive calls are
// safe).  DEFER_QS: sum(q) is not reduced;
// wavefront w's partial is left at ((int*)(red + 32))[w] for the caller to
// add up after its next barrier (integer sum: any order), and *qs is unused.
template <int EPT, int NT = kThreads, int NORM = -1, bool DEFER_QS = false, typename Pos>
__device__ __forceinline__ void quantize_row_regs(RowRegs<EPT>& r, int cols, int kp, const float* norm_w, float eps,
                                                  int8_t* dst, Pos pos, float* sa, int* qs, float* red) {
    const int tid = (int)threadIdx.x;
    const bool act = tid < NT;
    row_norm<EPT, NT, NORM>(r, cols, norm_w, eps, red);
    float am = 0.0f;
#pragma unroll
    for (int e = 0; e < EPT; e++) am = fmaxf(am, fabsf(r.v[e]));
    am = block_max_n<NT>(am, red + 16);
    const float scale = 127.0f / fmaxf(am, 1e-5f);
    int s = 0;
#pragma unroll
    for (int g = 0; g < EPT / 4; g++) {
        const int i0 = 4 * NT * g + 4 * tid;
        if (act && i0 < kp) {
            // elements past cols hold 0 and quantize to 0
            *(uint32_t*)(dst + pos(i0)) = quant4(&r.v[4 * g], scale, s);
        }
    }
    if constexpr (DEFER_QS) {
        s = wave_sum_i(s);
        if ((tid & 63) == 0 && act) ((int*)(red + 32))[tid >> 6] = s;
        if (tid == 0) *sa = scale;
        return;
    }
    s = block_sum_i_n<NT>(s, (int*)(red + 32));
    if (tid == 0) {
        *sa = scale;
        *qs = s;
    }
}

// RMSNorm (optional) + ActQuant of one row (loads it first).  Rows of up to
// 256 * EPT values take one global pass with the values in registers; longer
// rows re-read x (same arithmetic, same results).  Same contract as
// quantize_row_regs.
template <int EPT, typename Src, typename Pos>
__device__ __forceinline__ void quantize_row_block(Src x0, int cols, int kp, const float* norm_w0, float eps,
                                                   int8_t* dst, Pos pos, float* sa, int* qs, float* red) {
    const Src x = x0.fresh();
    const float* norm_w = norm_w0 ? launder(norm_w0) : nullptr;
    if (kp <= EPT * kThreads) {
        RowRegs<EPT> r;
        row_load<EPT>(x, cols, norm_w, r);
        quantize_row_regs<EPT>(r, cols, kp, norm_w, eps, dst, pos, sa, qs, red);
        return;
    }
    const bool act = threadIdx.x < kThreads;
    int s = 0;
    const float rr = norm_factor_global(x, cols, norm_w, eps, red);
    const float scale = act_scale(x, cols, norm_w, rr, red);
    if (act)
        for (int i = threadIdx.x; i < kp; i += kThreads) {
            const int qv = i < cols ? quant_one(norm_w ? (x(i) * rr) * norm_w[i] : x(i), scale) : 0;
            dst[pos(i)] = (int8_t)qv;
            s += qv;
        }
    s = block_sum_i_n<kThreads>(s, (int*)(red + 32));
    if (threadIdx.x == 0) {
        *sa = scale;
        *qs = s;
    }
}

// Fills GemvArgs from a TernaryOp (shared host-side setup).
int make_gemv_args(lbt_ctx* ctx, const TernaryOp& op, GemvArgs& a);

}  // namespace lbt
