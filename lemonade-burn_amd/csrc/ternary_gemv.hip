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
#include <hip/hip_runtime.h>


#include "lbt_device.h"
#include "lbt_internal.h"
#include "ternary_common.h"
#include "attn_common.h"

#include <stdlib.h>


namespace lbt {


template <int T, int IN, int EPT>
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
            quantize_row_block<EPT>(SrcF32{a.x + (size_t)tok * a.cols}, a.cols, kp, a.norm_w, a.eps, dst,
                                    [C](int i) { return perm_pos(i, C); }, &sa[t], &qs[t], red);
        }
    }
}

template <int R, int T>
__device__ __forceinline__ int row_dot(const int (&part)[4][R][T], int rr, int t, int qsum) {
    return part[0][rr][t] + part[1][rr][t] + part[2][rr][t] + part[3][rr][t] - qsum;
}

// Outputs of one tile; thread `tid` (0 .. R*T-1, others return) writes one
// (row, token) or one row pair.
template <int R, int T, int OUT>
__device__ __forceinline__ void epilogue(const GemvArgs& a, int vr0, int t0, const int (&part)[4][R][T],
                                         const float* sa, const int* qs, int tid) {
    if (tid < 0) return;
    if (OUT == kOutRelu2 || OUT == kOutQKV) {
        if (tid >= (R / 2) * T) return;
        const int p = tid / T, t = tid % T;
        const int v0 = vr0 + 2 * p, tok = t0 + t;
        if (v0 >= a.total_rows || tok >= a.m) return;
        store_pair<OUT>(a, tok, v0, row_dot(part, 2 * p, t, qs[t]), row_dot(part, 2 * p + 1, t, qs[t]), sa[t]);
        return;
    }
    if (tid >= R * T) return;
    const int rr = tid / T, t = tid % T;
    const int v = vr0 + rr, tok = t0 + t;
    if (v >= a.total_rows || tok >= a.m) return;
    store_single<OUT>(a, tok, v, row_dot(part, rr, t, qs[t]), sa[t]);
}

// One workgroup handles TILES consecutive tiles of R rows; the loads of a
// single f32 input row go out first, then all weight loads, then the
// activation prologue runs while the weights are in flight.  Rows longer than one
// round (NCH * 4 * L chunks) reload per round (TILES == 1 only).
template <int L, int T, int NCH, int TILES, int IN, int OUT>
__global__ __launch_bounds__(kThreads) void tgemv_kernel(GemvArgs a) {
    constexpr int R = 64 / L;
    extern __shared__ __align__(16) int8_t xq[];  // T * kp, permuted
    __shared__ __align__(16) float red[kRedFloats];
    __shared__ float sa[T];
    __shared__ int qs[T];
    __shared__ int part[TILES][4][R][T];

    const int tid = threadIdx.x, w = tid >> 6, ln = tid & 63;
    const int rg = ln / L, j = ln % L;
    const int t0 = blockIdx.y * T;
    const int C = a.C;

    // Single-token f32 input held in registers: its loads go out first, so the
    // prologue waits for them without waiting for the weight loads behind.
    // kInAttn: the row is the combine of the attention splits (same order).
    constexpr int EPT = NCH * 8;
    constexpr bool kAttn = IN == kInAttn;
    constexpr bool kRegs = T == 1 && (IN == kInF32 || kAttn);
    static_assert(!kAttn || T == 1, "attention rows are single tokens");
    const bool regs = kRegs && (kAttn || a.kp <= EPT * kThreads);
    RowRegs<kRegs ? EPT : 4> rrow;
    AttnRegs<kAttn ? EPT : 4, kAttn ? 4 : 1> arow;
    AttnRow attn{a.att_o, a.att_ml, 0, a.att_nh, a.hd, a.cols};
    const float* norm_w = a.norm_w ? launder(a.norm_w) : nullptr;
    if constexpr (kAttn) {
        attn_row_issue(attn, norm_w, arow, rrow);
    } else {
        if (regs) row_load(SrcF32{launder(a.x) + (size_t)t0 * a.cols}, a.cols, norm_w, rrow);
    }

    const uint4* rowp[TILES];
    bool valid[TILES];
    uint4 wv[TILES][NCH];
#pragma unroll
    for (int k = 0; k < TILES; k++) {
        const int vr = (blockIdx.x * TILES + k) * R + rg;
        valid[k] = vr < a.total_rows;
        int mat, r;
        resolve_row<OUT>(a, valid[k] ? vr : 0, mat, r);
        rowp[k] = (const uint4*)(sel3(a.w, mat) + (size_t)r * (size_t)(a.kp >> 2));
#pragma unroll
        for (int i = 0; i < NCH; i++) {
            const int c = (i * 4 + w) * L + j;
            wv[k][i] = (valid[k] && c < C) ? ld_stream(rowp[k] + c) : make_uint4(0, 0, 0, 0);
        }
    }

    if constexpr (kAttn) {
        __shared__ AttnTab tab;
        attn.ns = attn_splits((a.pos_dev ? *a.pos_dev : a.pos0) + 1);
        attn_row_finish(attn, arow, rrow, tab);
        quantize_row_regs(rrow, a.cols, a.kp, norm_w, a.eps, xq, [C](int i) { return perm_pos(i, C); }, &sa[0],
                          &qs[0], red);
    } else if constexpr (kRegs) {
        if (regs)
            quantize_row_regs(rrow, a.cols, a.kp, norm_w, a.eps, xq, [C](int i) { return perm_pos(i, C); }, &sa[0],
                              &qs[0], red);
        else
            build_acts<T, IN, EPT>(a, t0, xq, sa, qs, red);
    } else {
        build_acts<T, IN, EPT>(a, t0, xq, sa, qs, red);
    }
    __syncthreads();

#pragma unroll
    for (int k = 0; k < TILES; k++) {
        int acc[T];
#pragma unroll
        for (int t = 0; t < T; t++) acc[t] = 0;
        for (int base = 0;; base += NCH * 4 * L) {
#pragma unroll
            for (int i = 0; i < NCH; i++) {
                const int c = base + (i * 4 + w) * L + j;
                if (c < C) {
                    const uint32_t d0 = wv[k][i].x, d1 = wv[k][i].y, d2 = wv[k][i].z, d3 = wv[k][i].w;
#pragma unroll
                    for (int kk = 0; kk < 4; kk++) {
                        const int off = (kk * C + c) << 4;
                        const int sh = 2 * kk;
                        const int c0 = (int)((d0 >> sh) & 0x03030303u);
                        const int c1 = (int)((d1 >> sh) & 0x03030303u);
                        const int c2 = (int)((d2 >> sh) & 0x03030303u);
                        const int c3 = (int)((d3 >> sh) & 0x03030303u);
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
            if (TILES > 1 || nbase >= C) break;
#pragma unroll
            for (int i = 0; i < NCH; i++) {
                const int c = nbase + (i * 4 + w) * L + j;
                wv[k][i] = (valid[k] && c < C) ? ld_stream(rowp[k] + c) : make_uint4(0, 0, 0, 0);
            }
        }
#pragma unroll
        for (int t = 0; t < T; t++) acc[t] = xor_sum_down_i<L / 2>(acc[t]);
        if (j == 0) {
#pragma unroll
            for (int t = 0; t < T; t++) part[k][w][rg][t] = acc[t];
        }
    }
    __syncthreads();
    // one barrier for all tiles: tile k's outputs go to wavefront k, so the
    // tiles' epilogues run side by side
    static_assert(TILES <= 4 && R * T <= 64, "one wavefront per tile epilogue");
#pragma unroll
    for (int k = 0; k < TILES; k++)
        epilogue<R, T, OUT>(a, (blockIdx.x * TILES + k) * R, t0, part[k], sa, qs, tid - k * 64);
}

// Standalone quantizer: one workgroup per row, writes q [m, kp] (zero padded),
// scale [m], sum [m].
__global__ __launch_bounds__(kThreads) void quantize_kernel(const float* x, const float* norm_w, float eps,
                                                            int k, int kp, int8_t* q, float* scale,
                                                            int32_t* sum) {
    __shared__ __align__(16) float red[kRedFloats];
    const int row = blockIdx.x;
    quantize_row_block<32>(SrcF32{x + (size_t)row * k}, k, kp, norm_w, eps, q + (size_t)row * kp, [](int i) { return i; },
                           &scale[row], &sum[row], red);
}

// The same quantizer for 16-byte aligned rows with k % 4 == 0, on 1024
// threads with EPT (4 or 8) elements each: short dependent chains per thread
// (the same float order: the norm's virtual-thread layout does not depend on
// the thread count) and branch-free buffer loads of the row.
template <int EPT>
__global__ __launch_bounds__(1024) void quantize_wide_kernel(const float* x, const float* norm_w, float eps, int k,
                                                            int kp, int8_t* q, float* scale, int32_t* sum) {
    __shared__ __align__(16) float red[kRedFloats];
    const int row = blockIdx.x;
    RowRegs<EPT> r;
    const float* nw = norm_w ? launder(norm_w) : nullptr;
    row_load_buf<EPT, 1024>(x + (size_t)row * k, k, nw, r);
    quantize_row_regs<EPT, 1024>(r, k, kp, nw, eps, q + (size_t)row * kp, [](int i) { return i; }, &scale[row],
                                 &sum[row], red);
}

namespace {

constexpr int kL = 8;

template <int T, int NCH, int TILES, int IN>
hipError_t launch_out(const GemvArgs& a, int out_mode, dim3 grid, size_t lds, hipStream_t s, hipEvent_t e0,
                      hipEvent_t e1) {
    switch (out_mode) {
        case kOutI32:
            hipExtLaunchKernelGGL((tgemv_kernel<kL, T, NCH, TILES, IN, kOutI32>), grid, dim3(kThreads), lds, s, e0, e1, 0, a);
            break;
        case kOutF32:
            hipExtLaunchKernelGGL((tgemv_kernel<kL, T, NCH, TILES, IN, kOutF32>), grid, dim3(kThreads), lds, s, e0, e1, 0, a);
            break;
        case kOutF32Add:
            hipExtLaunchKernelGGL((tgemv_kernel<kL, T, NCH, TILES, IN, kOutF32Add>), grid, dim3(kThreads), lds, s, e0, e1, 0, a);
            break;
        case kOutRelu2:
            hipExtLaunchKernelGGL((tgemv_kernel<kL, T, NCH, TILES, IN, kOutRelu2>), grid, dim3(kThreads), lds, s, e0, e1, 0, a);
            break;
        default:
            hipExtLaunchKernelGGL((tgemv_kernel<kL, T, NCH, TILES, IN, kOutQKV>), grid, dim3(kThreads), lds, s, e0, e1, 0, a);
            break;
    }
    return hipGetLastError();
}

template <int T, int NCH, int TILES>
hipError_t launch_in(const GemvArgs& a, int in_mode, int out_mode, dim3 grid, size_t lds, hipStream_t s,
                     hipEvent_t e0, hipEvent_t e1) {
    if (in_mode == kInAttn) {
        if constexpr (T == 1) {
            hipExtLaunchKernelGGL((tgemv_kernel<kL, 1, NCH, TILES, kInAttn, kOutF32Add>), grid, dim3(kThreads), lds, s,
                                  e0, e1, 0, a);
            return hipGetLastError();
        }
        return hipErrorInvalidValue;
    }
    return in_mode == kInPreQ ? launch_out<T, NCH, TILES, kInPreQ>(a, out_mode, grid, lds, s, e0, e1)
                              : launch_out<T, NCH, TILES, kInF32>(a, out_mode, grid, lds, s, e0, e1);
}

template <int T>
hipError_t launch_t(const GemvArgs& a, int nch, int tiles, int in_mode, int out_mode, dim3 grid, size_t lds,
                    hipStream_t s, hipEvent_t e0, hipEvent_t e1) {
    if (nch == 2) {
        if (tiles == 4) return launch_in<T, 2, 4>(a, in_mode, out_mode, grid, lds, s, e0, e1);
        if (tiles == 2) return launch_in<T, 2, 2>(a, in_mode, out_mode, grid, lds, s, e0, e1);
        return launch_in<T, 2, 1>(a, in_mode, out_mode, grid, lds, s, e0, e1);
    }
    if (tiles == 2) return launch_in<T, 4, 2>(a, in_mode, out_mode, grid, lds, s, e0, e1);
    return launch_in<T, 4, 1>(a, in_mode, out_mode, grid, lds, s, e0, e1);
}

}  // namespace

int make_gemv_args(lbt_ctx* ctx, const TernaryOp& op, GemvArgs& a) {
    a = GemvArgs{};
    a.ksplit = 1;
    const int nmat = op.nmat;
    if (nmat < 1 || nmat > 3 || op.cols <= 0 || op.m <= 0) return set_err(ctx, LBT_E_INVALID, "ternary: bad shape");
    if (op.out_mode == kOutRelu2 && (nmat != 2 || op.rows[0] != op.rows[1]))
        return set_err(ctx, LBT_E_INVALID, "ternary: gate/up fusion needs two matrices of equal rows");
    if (op.out_mode == kOutF32Add && nmat != 1)
        return set_err(ctx, LBT_E_INVALID, "ternary: residual epilogue takes one matrix");
    if (op.out_mode == kOutQKV &&
        (nmat != 3 || op.hd <= 0 || op.hd % 2 || op.rows[0] % op.hd || op.rows[1] % op.hd || op.rows[1] != op.rows[2]))
        return set_err(ctx, LBT_E_INVALID, "ternary: q/k/v fusion needs head-aligned q, k, v");
    if (op.in_mode == kInAttn &&
        (op.m != 1 || op.tok_pos || op.out_mode != kOutF32Add || !op.att_o || !op.att_ml || op.att_nh <= 0 ||
         op.att_nh > kAttnMaxHeads || op.hd <= 0 || op.hd % 4 || op.att_nh * op.hd != op.cols || op.cols % 4 ||
         op.cols > 4096))
        return set_err(ctx, LBT_E_INVALID, "ternary: attention-combine input needs one token, nh*hd = cols <= 4096");
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
    a.att_o = op.att_o;
    a.att_ml = op.att_ml;
    a.att_nh = op.att_nh;
    a.hd = op.hd;
    a.pos0 = op.pos0;
    a.pos_dev = op.pos_dev;
    a.tok_pos = op.tok_pos;
    a.seq_stride = op.seq_stride;
    a.cap = op.cap;
    a.cos_t = op.cos_t;
    a.sin_t = op.sin_t;
    a.kc = op.kc;
    a.vc = op.vc;
    return LBT_OK;
}

int launch_ternary_gemv(lbt_ctx* ctx, const TernaryOp& op) {
    if (op.m == 1 && op.in_mode != kInPreQ) {
        const int rc = launch_ternary_gemv_cu(ctx, op);
        if (rc != 1) return rc;  // launched, or an error
    }
    GemvArgs a;
    int rc = make_gemv_args(ctx, op, a);
    if (rc) return rc;
    const int total = a.total_rows;
    constexpr int R = 64 / kL;
    const int T = op.m == 1 ? 1 : 4;
    const int per_lane = (a.C + 4 * kL - 1) / (4 * kL);
    const int nch = per_lane <= 2 ? 2 : 4;
    const int ntiles = (total + R - 1) / R;
    // several tiles per workgroup amortise the activation prologue once the
    // grid already covers the chip (rows > 1 round only with one tile)
    int tiles = 1;
    if (per_lane <= 4) {
        while (tiles < (nch == 2 ? 4 : 2) && ntiles / (tiles * 2) >= 384) tiles *= 2;
    }
    dim3 grid((unsigned)((ntiles + tiles - 1) / tiles), (unsigned)((op.m + T - 1) / T));
    const size_t lds = (size_t)T * a.kp;
    if (lds > 64 * 1024) return set_err(ctx, LBT_E_INVALID, "ternary: activation image exceeds LDS budget");
    hipEvent_t e0, e1;
    prof_pair(ctx, &e0, &e1);
    hipError_t e = T == 1 ? launch_t<1>(a, nch, tiles, op.in_mode, op.out_mode, grid, lds, ctx->stream, e0, e1)
                          : launch_t<4>(a, nch, tiles, op.in_mode, op.out_mode, grid, lds, ctx->stream, e0, e1);
    if (e != hipSuccess) return hip_err(ctx, e, "tgemv_kernel launch");
    const double bytes = (double)total * (a.kp / 4) + (double)op.m * op.cols * 4.0;
    prof_commit(ctx, e0, e1, kProfGemv, bytes);
    return LBT_OK;
}

int launch_quantize(lbt_ctx* ctx, const float* x, const float* norm_w, float eps, int m, int k, int8_t* q,
                    float* scale, int32_t* sum) {
    if (m <= 0) return LBT_OK;
    const int kp = (int)padded_cols((size_t)k);
    const bool wide = k % 4 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)norm_w & 15) == 0 && kp <= 8 * 1024;
    if (wide && kp <= 256 * 28 && !ctx->tune.quant_wide)
        return launch_quantize_pw(ctx, x, norm_w, eps, m, k, kp, q, scale, sum);
    if (wide && kp <= 4 * 1024)
        hipLaunchKernelGGL(quantize_wide_kernel<4>, dim3(m), dim3(1024), 0, ctx->stream, x, norm_w, eps, k, kp, q,
                           scale, sum);
    else if (wide)
        hipLaunchKernelGGL(quantize_wide_kernel<8>, dim3(m), dim3(1024), 0, ctx->stream, x, norm_w, eps, k, kp, q,
                           scale, sum);
    else
        hipLaunchKernelGGL(quantize_kernel, dim3(m), dim3(kThreads), 0, ctx->stream, x, norm_w, eps, k, kp, q, scale,
                           sum);
    LBT_HIP(ctx, hipGetLastError());
    return LBT_OK;
}

// Decode GEMV for one token (the VALU few-token GEMV on request), the int8-MFMA
// GEMM from kMfmaMinTokens up.
// Combine of row blockIdx.x's splits, then RMSNorm + ActQuant of the row
// into q (the GEMM input of the o projection for several rows): the combine
// of attn_combine_kernel and the quantizer of quantize_kernel on the same
// element layout, so the same q, s_a and sum(q).
template <int EPT>
__global__ __launch_bounds__(1024) void attn_quantize_kernel(const float* o, const float* ml, int nh, int hd,
                                                                 RowPos rp, const float* norm_w, float eps, int kp,
                                                                 int8_t* q, float* scale, int32_t* sum) {
    __shared__ AttnTab tab;
    __shared__ __align__(16) float red[kRedFloats];
    const int t = blockIdx.x, H = nh * hd;
    AttnRow a{o + (size_t)t * kAttnSplits * H, ml + (size_t)t * kAttnSplits * nh * 2, 0, nh, hd, H};
    RowRegs<EPT> r;
    AttnRegs<EPT, 4, 1024> ar;
    const float* nw = norm_w ? launder(norm_w) : nullptr;
    attn_row_issue<EPT, 4, 1024>(a, nw, ar, r);
    a.ns = attn_splits(row_position(rp, t) + 1);
    attn_row_finish<EPT, 4, 1024>(a, ar, r, tab);
    quantize_row_regs<EPT, 1024>(r, H, kp, nw, eps, q + (size_t)t * kp, [](int i) { return i; }, &scale[t], &sum[t],
                                 red);
}

int launch_attn_quantize(lbt_ctx* ctx, const float* o, const float* ml, int m, int nh, int hd, const RowPos& rp,
                         const float* norm_w, float eps, int kp, int8_t* q, float* scale, int32_t* sum) {
    const int H = nh * hd;
    if (nh <= 0 || nh > kAttnMaxHeads || hd % 4 || H > 4 * 1024 || kp < H || kp > 4 * 1024)
        return set_err(ctx, LBT_E_INVALID, "attention quantize: at most 64 heads and 4096 columns");
    hipLaunchKernelGGL(attn_quantize_kernel<4>, dim3(m), dim3(1024), 0, ctx->stream, o, ml, nh, hd, rp, norm_w, eps,
                       kp, q, scale, sum);
    LBT_HIP(ctx, hipGetLastError());
    return LBT_OK;
}

int launch_ternary(lbt_ctx* ctx, const TernaryOp& op_in) {
    TernaryOp op = op_in;
    if (op.in_mode == kInAttn && (op.m > 1 || op.tok_pos)) {
        // several rows: combine + norm + quantize in one kernel, then the
        // pre-quantized GEMV / GEMM (one token keeps the combine in the GEMV
        // prologue)
        const size_t kp = padded_cols((size_t)op.cols);
        const size_t qb = ((size_t)op.m * kp + 255) & ~(size_t)255;
        void* q;
        int rc = act_scratch(ctx, op, qb + (size_t)op.m * 8, &q);
        if (rc) return rc;
        float* sd = (float*)((char*)q + qb);
        int32_t* ud = (int32_t*)(sd + op.m);
        RowPos rp;
        rp.pos0 = op.pos0;
        rp.pos_dev = op.pos_dev;
        rp.tok_pos = op.tok_pos;
        if ((rc = launch_attn_quantize(ctx, op.att_o, op.att_ml, op.m, op.att_nh, op.hd, rp, op.norm_w, op.eps,
                                       (int)kp, (int8_t*)q, sd, ud)))
            return rc;
        op.in_mode = kInPreQ;
        op.q = (const int8_t*)q;
        op.qscale = sd;
        op.qsum = ud;
        op.tok_pos = nullptr;
        op.pos_dev = nullptr;
    }
    if (op.m >= ctx->tune.mfma_min && !ctx->tune.no_mfma) return launch_ternary_mfma(ctx, op);
    return launch_ternary_gemv(ctx, op);
}

}  // namespace lbt
