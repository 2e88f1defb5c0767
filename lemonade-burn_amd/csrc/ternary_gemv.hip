// ternary_gemv.hip -- packed 2-bit ternary x int8 decode GEMV for gfx950.
//
// Replaces the reference's CPU decode path: quantize_acts_into
// (crates/lb-ternary/src/quant.rs:45-75) + ternary_gemm_multi decode branch
// (crates/lb-ternary/src/gemm.rs:137-154) + dot_row / codes_dot_*
// (gemm.rs:292-343, :387-469, :553-588).
//
// Work mapping (HBM-bound, no MFMA):
//   * a workgroup is 4 wavefronts on the same R = 64/L rows; inside a wave,
//     L consecutive lanes share a row and the 4 waves split its 16-byte chunks
//     (chunk c = (i*4 + wave)*L + lane%L), so each row's bytes are read once
//     with 128-bit loads, 16*L contiguous bytes per row per instruction;
//   * the weight loads of the first round are issued before the activation
//     prologue, so HBM traffic starts at kernel entry;
//   * the prologue quantizes (and optionally RMS-normalises) the f32
//     activations into LDS in a permuted image where the 64 activations that
//     pair with one 16-byte chunk are four 16-byte runs (lbt::perm_pos);
//   * codes c = w+1 in {0,1,2} are unpacked with one shift and one mask per
//     dword and multiplied with v_dot4_i32_i8; the integer result
//     acc - sum(q) is exact (gemm.rs:3-17), lanes reduce with xor shuffles and
//     waves through LDS (integer, order independent);
//   * epilogues: i32 out, f32 y = dot * (1/(s_a*s_w)) (gemm.rs:141,150),
//     residual add (model.rs:359,365), and relu(g)^2 * u for interleaved
//     gate/up rows (model.rs:362-363).
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
    void* out[3];
};

// Per-row prep shared by the GEMV prologue and the standalone quantizer:
// returns the RMSNorm factor r (1 when no norm) and the ActQuant scale.
// rms_norm (model.rs:267-272): r = 1 / sqrt(sum(x^2)/n + eps), tree256 order.
__device__ __forceinline__ float norm_factor(const float* xr, int cols, const float* norm_w, float eps,
                                             float* red) {
    if (!norm_w) return 1.0f;
    float p = 0.0f;
    for (int i = threadIdx.x; i < cols; i += kThreads) p = __builtin_fmaf(xr[i], xr[i], p);
    float ss = block_tree256(p, red);
    float mean = ss / (float)cols;
    return 1.0f / __builtin_sqrtf(mean + eps);
}

__device__ __forceinline__ float normed(const float* xr, const float* norm_w, float rr, int i) {
    return norm_w ? (xr[i] * rr) * norm_w[i] : xr[i];
}

// amax over the (normed) row, then s_a = 127 / max(amax, 1e-5) (quant.rs:100-113).
__device__ __forceinline__ float act_scale(const float* xr, int cols, const float* norm_w, float rr, float* red) {
    float am = 0.0f;
    for (int i = threadIdx.x; i < cols; i += kThreads) am = fmaxf(am, fabsf(normed(xr, norm_w, rr, i)));
    am = block_max(am, red);
    return 127.0f / fmaxf(am, 1e-5f);
}

template <int T, int IN>
__device__ __forceinline__ void build_acts(const GemvArgs& a, int t0, int8_t* xq, float* sa, int* qs,
                                           float* red) {
    const int kp = a.kp, C = a.C;
    for (int t = 0; t < T; t++) {
        const int tok = t0 + t;
        int8_t* dst = xq + t * kp;
        if (tok >= a.m) {
            for (int u = threadIdx.x; u < kp / 16; u += kThreads)
                *(int4*)(dst + (u << 4)) = make_int4(0, 0, 0, 0);
            if (threadIdx.x == 0) { sa[t] = 1.0f; qs[t] = 0; }
            continue;
        }
        if (IN == kInPreQ) {
            const int8_t* src = a.q + (size_t)tok * kp;
            for (int u = threadIdx.x; u < kp / 16; u += kThreads)
                *(int4*)(dst + perm_pos(u << 4, C)) = *(const int4*)(src + (u << 4));
            if (threadIdx.x == 0) { sa[t] = a.qscale ? a.qscale[tok] : 1.0f; qs[t] = a.qsum[tok]; }
        } else {
            const float* xr = a.x + (size_t)tok * a.cols;
            const float rr = norm_factor(xr, a.cols, a.norm_w, a.eps, red);
            const float scale = act_scale(xr, a.cols, a.norm_w, rr, red);
            int s = 0;
            for (int i = threadIdx.x; i < kp; i += kThreads) {
                int qv = i < a.cols ? quant_one(normed(xr, a.norm_w, rr, i), scale) : 0;
                dst[perm_pos(i, C)] = (int8_t)qv;
                s += qv;
            }
            s = block_sum_i(s, (int*)red);
            if (threadIdx.x == 0) { sa[t] = scale; qs[t] = s; }
        }
    }
}

__device__ __forceinline__ void resolve_row(const GemvArgs& a, int vr, bool pair, int& mat, int& r) {
    if (pair) {
        mat = vr & 1;
        r = vr >> 1;
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

template <int L, int T, int NCH, int IN, int OUT>
__global__ __launch_bounds__(kThreads) void tgemv_kernel(GemvArgs a) {
    constexpr int R = 64 / L;
    extern __shared__ __align__(16) int8_t xq[];  // T * kp, permuted
    __shared__ float red[kThreads];
    __shared__ float sa[T];
    __shared__ int qs[T];
    __shared__ int part[4][R][T];

    const int tid = threadIdx.x, w = tid >> 6, ln = tid & 63;
    const int rg = ln / L, j = ln % L;
    const int vr = blockIdx.x * R + rg;
    const int t0 = blockIdx.y * T;
    const int C = a.C;
    const bool valid = vr < a.total_rows;
    int mat, r;
    resolve_row(a, valid ? vr : 0, OUT == kOutRelu2, mat, r);
    const uint4* rowp = (const uint4*)(a.w[mat] + (size_t)r * (size_t)(a.kp >> 2));

    // First round of weight loads goes out before the prologue.
    uint4 wv[NCH];
#pragma unroll
    for (int i = 0; i < NCH; i++) {
        const int c = (i * 4 + w) * L + j;
        wv[i] = (valid && c < C) ? rowp[c] : make_uint4(0, 0, 0, 0);
    }

    build_acts<T, IN>(a, t0, xq, sa, qs, red);
    __syncthreads();

    int acc[T];
#pragma unroll
    for (int t = 0; t < T; t++) acc[t] = 0;

    for (int base = 0;; base += NCH * 4 * L) {
#pragma unroll
        for (int i = 0; i < NCH; i++) {
            const int c = base + (i * 4 + w) * L + j;
            if (c < C) {
                const uint32_t d0 = wv[i].x, d1 = wv[i].y, d2 = wv[i].z, d3 = wv[i].w;
#pragma unroll
                for (int kk = 0; kk < 4; kk++) {
                    const int off = (kk * C + c) << 4;
                    const int s = 2 * kk;
                    const int c0 = (int)((d0 >> s) & 0x03030303u);
                    const int c1 = (int)((d1 >> s) & 0x03030303u);
                    const int c2 = (int)((d2 >> s) & 0x03030303u);
                    const int c3 = (int)((d3 >> s) & 0x03030303u);
#pragma unroll
                    for (int t = 0; t < T; t++) {
                        const int4 xv = *(const int4*)(xq + t * a.kp + off);
                        int s0 = __builtin_amdgcn_sdot4(c0, xv.x, acc[t], false);
                        s0 = __builtin_amdgcn_sdot4(c1, xv.y, s0, false);
                        s0 = __builtin_amdgcn_sdot4(c2, xv.z, s0, false);
                        acc[t] = __builtin_amdgcn_sdot4(c3, xv.w, s0, false);
                    }
                }
            }
        }
        const int nbase = base + NCH * 4 * L;
        if (nbase >= C) break;
#pragma unroll
        for (int i = 0; i < NCH; i++) {
            const int c = nbase + (i * 4 + w) * L + j;
            wv[i] = (valid && c < C) ? rowp[c] : make_uint4(0, 0, 0, 0);
        }
    }

#pragma unroll
    for (int t = 0; t < T; t++) {
#pragma unroll
        for (int o = L / 2; o >= 1; o >>= 1) acc[t] += __shfl_xor(acc[t], o);
    }
    if (j == 0) {
#pragma unroll
        for (int t = 0; t < T; t++) part[w][rg][t] = acc[t];
    }
    __syncthreads();

    if (OUT == kOutRelu2) {
        if (tid < (R / 2) * T) {
            const int p = tid / T, t = tid % T;
            const int vg = blockIdx.x * R + 2 * p;
            const int tok = t0 + t;
            if (vg < a.total_rows && tok < a.m) {
                const int dg = part[0][2 * p][t] + part[1][2 * p][t] + part[2][2 * p][t] + part[3][2 * p][t] - qs[t];
                const int du = part[0][2 * p + 1][t] + part[1][2 * p + 1][t] + part[2][2 * p + 1][t] +
                               part[3][2 * p + 1][t] - qs[t];
                const float g = (float)dg * (1.0f / (sa[t] * a.sw[0]));
                const float u = (float)du * (1.0f / (sa[t] * a.sw[1]));
                const float rl = g > 0.0f ? g : 0.0f;
                ((float*)a.out[0])[(size_t)tok * a.rows[0] + (vg >> 1)] = (rl * rl) * u;
            }
        }
        return;
    }
    if (tid < R * T) {
        const int rr = tid / T, t = tid % T;
        const int v = blockIdx.x * R + rr;
        const int tok = t0 + t;
        if (v < a.total_rows && tok < a.m) {
            int mt, ro;
            resolve_row(a, v, false, mt, ro);
            const int dot = part[0][rr][t] + part[1][rr][t] + part[2][rr][t] + part[3][rr][t] - qs[t];
            const size_t o = (size_t)tok * a.rows[mt] + ro;
            if (OUT == kOutI32) {
                ((int32_t*)a.out[mt])[o] = dot;
            } else {
                const float y = (float)dot * (1.0f / (sa[t] * a.sw[mt]));
                float* dst = (float*)a.out[mt];
                if (OUT == kOutF32Add) dst[o] = dst[o] + y;
                else dst[o] = y;
            }
        }
    }
}

// Standalone quantizer: one workgroup per row, writes q [m, kp] (zero padded),
// scale [m], sum [m].
__global__ __launch_bounds__(kThreads) void quantize_kernel(const float* x, const float* norm_w, float eps,
                                                            int k, int kp, int8_t* q, float* scale,
                                                            int32_t* sum) {
    __shared__ float red[kThreads];
    const int row = blockIdx.x;
    const float* xr = x + (size_t)row * k;
    const float rr = norm_factor(xr, k, norm_w, eps, red);
    const float s = act_scale(xr, k, norm_w, rr, red);
    int acc = 0;
    for (int i = threadIdx.x; i < kp; i += kThreads) {
        int qv = i < k ? quant_one(normed(xr, norm_w, rr, i), s) : 0;
        q[(size_t)row * kp + i] = (int8_t)qv;
        acc += qv;
    }
    acc = block_sum_i(acc, (int*)red);
    if (threadIdx.x == 0) {
        scale[row] = s;
        sum[row] = acc;
    }
}

namespace {

constexpr int kL = 8;

template <int T, int NCH, int IN>
hipError_t launch_out(const GemvArgs& a, int out_mode, dim3 grid, size_t lds, hipStream_t s) {
    switch (out_mode) {
        case kOutI32:
            hipLaunchKernelGGL((tgemv_kernel<kL, T, NCH, IN, kOutI32>), grid, dim3(kThreads), lds, s, a);
            break;
        case kOutF32:
            hipLaunchKernelGGL((tgemv_kernel<kL, T, NCH, IN, kOutF32>), grid, dim3(kThreads), lds, s, a);
            break;
        case kOutF32Add:
            hipLaunchKernelGGL((tgemv_kernel<kL, T, NCH, IN, kOutF32Add>), grid, dim3(kThreads), lds, s, a);
            break;
        default:
            hipLaunchKernelGGL((tgemv_kernel<kL, T, NCH, IN, kOutRelu2>), grid, dim3(kThreads), lds, s, a);
            break;
    }
    return hipGetLastError();
}

template <int T, int NCH>
hipError_t launch_in(const GemvArgs& a, int in_mode, int out_mode, dim3 grid, size_t lds, hipStream_t s) {
    return in_mode == kInPreQ ? launch_out<T, NCH, kInPreQ>(a, out_mode, grid, lds, s)
                              : launch_out<T, NCH, kInF32>(a, out_mode, grid, lds, s);
}

}  // namespace

int launch_ternary_gemv(lbt_ctx* ctx, const TernaryOp& op) {
    GemvArgs a{};
    const int nmat = op.nmat;
    if (nmat < 1 || nmat > 3 || op.cols <= 0 || op.m <= 0) return set_err(ctx, LBT_E_INVALID, "ternary: bad shape");
    if (op.out_mode == kOutRelu2 && (nmat != 2 || op.rows[0] != op.rows[1]))
        return set_err(ctx, LBT_E_INVALID, "ternary: gate/up fusion needs two matrices of equal rows");
    if (op.out_mode == kOutF32Add && nmat != 1)
        return set_err(ctx, LBT_E_INVALID, "ternary: residual epilogue takes one matrix");
    int total = 0;
    for (int i = 0; i < 3; i++) {
        a.w[i] = i < nmat ? op.w[i] : op.w[0];
        a.rows[i] = i < nmat ? op.rows[i] : 0;
        a.sw[i] = i < nmat ? op.sw[i] : 1.0f;
        a.out[i] = i < nmat ? op.out[i] : nullptr;
        total += a.rows[i];
    }
    a.total_rows = total;
    a.cols = op.cols;
    a.kp = (int)padded_cols((size_t)op.cols);
    a.C = a.kp / 64;
    a.m = op.m;
    a.q = op.q;
    a.qscale = op.qscale;
    a.qsum = op.qsum;
    a.x = op.x;
    a.norm_w = op.norm_w;
    a.eps = op.eps;
    constexpr int R = 64 / kL;
    const int T = op.m == 1 ? 1 : 4;
    const int per_lane = (a.C + 4 * kL - 1) / (4 * kL);
    const int nch = per_lane <= 2 ? 2 : 4;
    dim3 grid((unsigned)((total + R - 1) / R), (unsigned)((op.m + T - 1) / T));
    const size_t lds = (size_t)T * a.kp;
    if (lds > 64 * 1024) return set_err(ctx, LBT_E_INVALID, "ternary: activation image exceeds LDS budget");
    hipEvent_t ev = nullptr;
    prof_begin(ctx, &ev);
    hipError_t e;
    if (T == 1)
        e = nch == 2 ? launch_in<1, 2>(a, op.in_mode, op.out_mode, grid, lds, ctx->stream)
                     : launch_in<1, 4>(a, op.in_mode, op.out_mode, grid, lds, ctx->stream);
    else
        e = nch == 2 ? launch_in<4, 2>(a, op.in_mode, op.out_mode, grid, lds, ctx->stream)
                     : launch_in<4, 4>(a, op.in_mode, op.out_mode, grid, lds, ctx->stream);
    if (e != hipSuccess) return hip_err(ctx, e, "tgemv_kernel launch");
    const double bytes = (double)total * (a.kp / 4);
    prof_end(ctx, ev, kProfGemv, bytes);
    return LBT_OK;
}

int launch_quantize(lbt_ctx* ctx, const float* x, const float* norm_w, float eps, int m, int k, int8_t* q,
                    float* scale, int32_t* sum) {
    if (m <= 0) return LBT_OK;
    const int kp = (int)padded_cols((size_t)k);
    hipLaunchKernelGGL(quantize_kernel, dim3(m), dim3(kThreads), 0, ctx->stream, x, norm_w, eps, k, kp, q, scale,
                       sum);
    LBT_HIP(ctx, hipGetLastError());
    return LBT_OK;
}

int launch_ternary(lbt_ctx* ctx, const TernaryOp& op) {
    return launch_ternary_gemv(ctx, op);
}

}  // namespace lbt
