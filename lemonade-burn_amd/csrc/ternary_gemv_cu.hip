// ternary_gemv_cu.hip -- single-token decode GEMV, one 1024-thread workgroup
// per compute unit.
//
// Same arithmetic as the decode GEMV of ternary_gemv.hip (the reference's
// quantize_acts_into + ternary_gemm_multi decode branch, quant.rs:45-75,
// gemm.rs:137-154, with the model's fused epilogues), laid out for a
// batch-1 decode step, where the time goes to latency rather than to HBM:
//   * about one workgroup per CU (rows per workgroup = rows / CUs, even), so
//     the activation prologue (RMSNorm + ActQuant, or the attention combine)
//     runs once per CU, spread over 16 wavefronts: 4x fewer elements per
//     thread than a 256-thread workgroup;
//   * each row lives inside one wavefront (L = 16, 32 or 64 lanes per row,
//     lane j takes 16-byte chunks j, j+L, ...), so a row reduces with lane
//     butterflies only;
//   * the activation loads go out first (unconditional buffer loads), then
//     every weight load of the workgroup (CPL 16-byte chunks per lane)
//     without waiting for the row, then the prologue runs while the weights
//     are in flight;
//   * epilogues are the shared ones of ternary_common.h.
#include <hip/hip_runtime.h>


#include "lbt_device.h"
#include "lbt_internal.h"
#include "ternary_common.h"
#include "attn_common.h"

namespace lbt {

constexpr int kCuThreads = 1024;
constexpr int kCuEPT = 8;       // row elements per thread: rows up to 8192 (4: rows up to 4096)
constexpr int kCuMaxRows = 64;  // rows per workgroup (16 wavefronts x 64 / L, L >= 16)

// RMSNorm + ActQuant of a row held by the first PW wavefronts only (the
// element layout of row_elem<64 * PW>), the other wavefronts skipping every
// step but the barriers: the reductions' per-wavefront work (butterflies,
// the divisions and square root of the norm factor and scale) then runs
// once per SIMD instead of four times.  The same values as quantize_row_regs
// (canonical sum-of-squares order; max and integer sums are order
// independent).  s_a goes to *sa; wavefront w < PW leaves its sum(q)
// partial at ((int*)(red + 32))[w], published by the caller's next barrier.
template <int EPT, int PW, int NORM, typename Pos>
__device__ __forceinline__ void quant_row_waves(RowRegs<EPT>& r, int cols, int kp, const float* norm_w, float eps,
                                                int8_t* dst, Pos pos, float* sa, float* red) {
    constexpr int NT = 64 * PW;
    const int tid = (int)threadIdx.x, w = tid >> 6;
    const bool part = w < PW;  // uniform per wavefront
    if constexpr (NORM != 0) {
        if (part) row_sumsq_part<EPT, NT>(r, cols, red);
        __syncthreads();
    }
    if (part) {
        if constexpr (NORM != 0) {
            const float f = 1.0f / __builtin_sqrtf(tree16(red) / (float)cols + eps);
#pragma unroll
            for (int e = 0; e < EPT; e++) r.v[e] = (r.v[e] * f) * r.nw[e];
        }
        float am = 0.0f;
#pragma unroll
        for (int e = 0; e < EPT; e++) am = fmaxf(am, fabsf(r.v[e]));
        am = wave_max(am);
        if ((tid & 63) == 0) red[16 + w] = am;
    }
    __syncthreads();
    if (part) {
        float am = red[16];
#pragma unroll
        for (int i = 1; i < PW; i++) am = fmaxf(am, red[16 + i]);
        const float scale = 127.0f / fmaxf(am, 1e-5f);
        int s = 0;
#pragma unroll
        for (int g = 0; g < EPT / 4; g++) {
            const int i0 = 4 * NT * g + 4 * tid;
            if (i0 < kp) *(uint32_t*)(dst + pos(i0)) = quant4(&r.v[4 * g], scale, s);
        }
        s = wave_sum_i(s);
        if ((tid & 63) == 0) ((int*)(red + 32))[w] = s;
        if (tid == 0) *sa = scale;
    }
}

// RMSNorm (norm_w set) + ActQuant of row blockIdx.x into q / scale / sum on
// one 256-thread workgroup: the GEMV prologue's quant_row_waves on its four
// wavefronts, so the values of quantize_wide_kernel (canonical sum of
// squares; max and integer sums order free) with shorter reduction chains.
template <int EPT>
__global__ __launch_bounds__(256) void quantize_pw_kernel(const float* x, const float* norm_w, float eps, int k,
                                                          int kp, int8_t* q, float* scale, int32_t* sum) {
    __shared__ __align__(16) float red[kRedFloats];
    const int row = blockIdx.x;
    RowRegs<EPT> r;
    const float* nw = norm_w ? launder(norm_w) : nullptr;
    row_load_buf<EPT, 256>(x + (size_t)row * k, k, nw, r);
    if (nw)
        quant_row_waves<EPT, 4, 1>(r, k, kp, nw, eps, q + (size_t)row * kp, [](int i) { return i; }, &scale[row], red);
    else
        quant_row_waves<EPT, 4, 0>(r, k, kp, nw, eps, q + (size_t)row * kp, [](int i) { return i; }, &scale[row], red);
    __syncthreads();
    if (threadIdx.x == 0) {
        const int* ps = (const int*)(red + 32);
        sum[row] = (ps[0] + ps[1]) + (ps[2] + ps[3]);
    }
}

int launch_quantize_pw(lbt_ctx* ctx, const float* x, const float* norm_w, float eps, int m, int k, int kp,
                       int8_t* q, float* scale, int32_t* sum) {
    if (kp <= 256 * 12)
        hipLaunchKernelGGL(quantize_pw_kernel<12>, dim3(m), dim3(256), 0, ctx->stream, x, norm_w, eps, k, kp, q,
                           scale, sum);
    else if (kp <= 256 * 28)
        hipLaunchKernelGGL(quantize_pw_kernel<28>, dim3(m), dim3(256), 0, ctx->stream, x, norm_w, eps, k, kp, q,
                           scale, sum);
    else
        return set_err(ctx, LBT_E_INVALID, "quantize: row too long for the four-wavefront quantizer");
    LBT_HIP(ctx, hipGetLastError());
    return LBT_OK;
}

// PW: wavefronts of the activation prologue (16: all, EPT elements per
// thread; 4: the first four, EPT elements per thread of 256).
template <int L, int CPL, int IN, int OUT, int EPT, int PW>
__global__ __launch_bounds__(kCuThreads) void tgemv_cu_kernel(GemvArgs a, int rpw) {
    static_assert(PW == 16 || PW == 4, "prologue wavefronts");
    constexpr int RPWV = 64 / L;  // rows per wavefront
    constexpr int PNT = 64 * PW;  // threads of the prologue
    __shared__ __align__(16) int8_t xq[EPT * PNT];
    __shared__ __align__(16) float red[kRedFloats];
    __shared__ float sa_s;
    const int tid = (int)threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int rs = w * RPWV + lane / L, j = lane % L;
    const int C = a.C;
    const int vr0 = blockIdx.x * rpw;
    const bool rvalid = rs < rpw && vr0 + rs < a.total_rows;

    // the activation row's loads first
    RowRegs<EPT> row;
    AttnRegs<IN == kInAttn ? EPT : 4, IN == kInAttn ? 4 : 1, PNT> arow;
    AttnRow attn{a.att_o, a.att_ml, 0, a.att_nh, a.hd, a.cols};
    const float* norm_w = a.norm_w ? launder(a.norm_w) : nullptr;
    // the decode position (attention splits): an untracked load issued first,
    // waited for with the row (below), so no wait on it covers the weights
    float posf = 0.0f;
    // (without a device position, a harmless word of the partials is read)
    if constexpr (IN == kInAttn) {
        if (PW == 16 || w < PW) {
            posf = ld_f32_async(a.pos_dev ? (const float*)a.pos_dev : a.att_ml);
            attn_row_issue<EPT, 4, PNT>(attn, norm_w, arow, row);
        }
    } else if (PW == 16 || w < PW)
        row_load_buf<EPT, PNT>(launder(a.x), a.cols, norm_w, row);

    // then every weight load of this workgroup, once every wavefront's row
    // loads are queued ahead of them (a bare barrier: no wait for the data)
    __builtin_amdgcn_s_barrier();
    uint4 wv[CPL];
    {
        int mat, r;
        resolve_row<OUT>(a, rvalid ? vr0 + rs : 0, mat, r);
        const uint4* rowp = (const uint4*)(sel3(a.w, mat) + (size_t)r * (size_t)(a.kp >> 2));
        // unconditional (chunks past the row re-read its last one; rows past
        // the matrix read row 0), so the compiler's wait for the activation
        // row counts every weight load as issued; unused chunks are skipped
        // in the dot loop and unused rows are not stored
#pragma unroll
        for (int i = 0; i < CPL; i++) {
            const int c = j + L * i;
            wv[i] = ld_stream(rowp + (c < C ? c : C - 1));
        }
    }

    // prologue: (attention combine,) RMSNorm + ActQuant into the permuted LDS image
    if constexpr (IN == kInAttn) {
        __shared__ AttnTab tab;
        if (PW == 16 || w < PW) {
            vm_wait<CPL>();  // all but the weight loads: the position and the row
            pin(posf);
            attn.ns = attn_splits((a.pos_dev ? __float_as_int(posf) : a.pos0) + 1);
            attn_row_tab<EPT, 4, PNT>(attn, arow, tab);
        }
        __syncthreads();
        if (PW == 16 || w < PW) attn_row_combine<EPT, 4, PNT>(attn, arow, row, tab);
    }
    if constexpr (PW == 16)
        quantize_row_regs<EPT, kCuThreads, -1, true>(row, a.cols, a.kp, norm_w, a.eps, xq,
                                                        [C](int i) { return perm_pos(i, C); }, &sa_s, nullptr, red);
    else if (norm_w)
        quant_row_waves<EPT, PW, 1>(row, a.cols, a.kp, norm_w, a.eps, xq, [C](int i) { return perm_pos(i, C); },
                                    &sa_s, red);
    else
        quant_row_waves<EPT, PW, 0>(row, a.cols, a.kp, norm_w, a.eps, xq, [C](int i) { return perm_pos(i, C); },
                                    &sa_s, red);
    __syncthreads();
    // sum(q): the wavefronts' partials left by the quantizer
    int qsum = 0;
    {
        const int4* qp = (const int4*)(red + 32);
#pragma unroll
        for (int i = 0; i < PW / 4; i++) {
            const int4 v = qp[i];
            qsum += (v.x + v.y) + (v.z + v.w);
        }
    }

    // codes . q over this lane's chunks, one accumulator per 2-bit plane kk.
    // Planes 0..2 are masked in place, without the shift: their bytes hold
    // code << 2kk (at most 32, a valid signed byte), so accs[kk] is exactly
    // 4^kk times the plane's dot and is divided back exactly at the end;
    // plane 3 would reach 128 and is shifted down first.
    int accs[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < CPL; i++) {
        const int c = j + L * i;
        if (c < C) {
            const uint32_t d[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                const int4 xv = *(const int4*)(xq + ((kk * C + c) << 4));
                const uint32_t m = 0x03030303u << (2 * kk);
                int& acc = accs[kk];
                if (kk < 3) {
                    acc = __builtin_amdgcn_sdot4((int)(d[0] & m), xv.x, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)(d[1] & m), xv.y, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)(d[2] & m), xv.z, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)(d[3] & m), xv.w, acc, false);
                } else {
                    acc = __builtin_amdgcn_sdot4((int)((d[0] >> 6) & 0x03030303u), xv.x, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)((d[1] >> 6) & 0x03030303u), xv.y, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)((d[2] >> 6) & 0x03030303u), xv.z, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)((d[3] >> 6) & 0x03030303u), xv.w, acc, false);
                }
            }
        }
    }
    int acc = (accs[0] + (accs[1] >> 2)) + ((accs[2] >> 4) + accs[3]);
    acc = xor_sum_down_i<L / 2>(acc);  // every lane of the row holds its sum
    const int dot = acc - qsum;

    // epilogue by the row's first lane, no LDS pass: a row pair (2p, 2p + 1)
    // lies in one wavefront (L <= 32 for the paired outputs), the odd row's
    // dot L lanes up
    const bool out_row = j == 0 && rs < rpw && vr0 + rs < a.total_rows;
    if constexpr (OUT == kOutRelu2 || OUT == kOutQKV) {
        static_assert(L <= 32, "row pairs within a wavefront");
        const int d1 = __shfl_down(dot, L);
        if (out_row && (rs & 1) == 0) store_pair<OUT>(a, 0, vr0 + rs, dot, d1, sa_s);
    } else {
        if (out_row) store_single<OUT>(a, 0, vr0 + rs, dot, sa_s);
    }
}

namespace {

template <int L, int CPL, int EPT, int PW>
hipError_t launch_cu(const GemvArgs& a, int in_mode, int out_mode, int rpw, dim3 grid, hipStream_t s, hipEvent_t e0,
                     hipEvent_t e1) {
#define LBT_CU_LAUNCH(IN, OUT)                                                                                       \
    hipExtLaunchKernelGGL((tgemv_cu_kernel<L, CPL, IN, OUT, EPT, PW>), grid, dim3(kCuThreads), 0, s, e0, e1, 0, a, \
                          rpw)
    if (in_mode == kInAttn) {
        if constexpr (PW == 16 || EPT <= 16) {
            LBT_CU_LAUNCH(kInAttn, kOutF32Add);
            return hipGetLastError();
        } else {
            return hipErrorInvalidValue;
        }
    }
    switch (out_mode) {
        case kOutI32: LBT_CU_LAUNCH(kInF32, kOutI32); break;
        case kOutF32: LBT_CU_LAUNCH(kInF32, kOutF32); break;
        case kOutF32Add: LBT_CU_LAUNCH(kInF32, kOutF32Add); break;
        default:
            if constexpr (L <= 32) {  // the host picks L <= 32 for the paired outputs
                if (out_mode == kOutRelu2) LBT_CU_LAUNCH(kInF32, kOutRelu2);
                else LBT_CU_LAUNCH(kInF32, kOutQKV);
            } else {
                return hipErrorInvalidValue;
            }
            break;
    }
#undef LBT_CU_LAUNCH
    return hipGetLastError();
}

// Rows of up to 4096 elements take 4 per thread (half the prologue's
// instructions of the 8-per-thread build; the same float order: element
// groups beyond the row are skipped either way).
template <int L, int CPL>
hipError_t launch_cu_e(const GemvArgs& a, int in_mode, int out_mode, int rpw, dim3 grid, hipStream_t s,
                       hipEvent_t e0, hipEvent_t e1, int pw) {
    if (pw == 4) {
        if (a.kp <= 12 * 256) return launch_cu<L, CPL, 12, 4>(a, in_mode, out_mode, rpw, grid, s, e0, e1);
        if (in_mode == kInAttn) return launch_cu<L, CPL, 16, 4>(a, in_mode, out_mode, rpw, grid, s, e0, e1);
        if (a.kp <= 28 * 256) return launch_cu<L, CPL, 28, 4>(a, in_mode, out_mode, rpw, grid, s, e0, e1);
        return launch_cu<L, CPL, 32, 4>(a, in_mode, out_mode, rpw, grid, s, e0, e1);
    }
    if (a.kp <= 4 * kCuThreads) return launch_cu<L, CPL, 4, 16>(a, in_mode, out_mode, rpw, grid, s, e0, e1);
    return launch_cu<L, CPL, 8, 16>(a, in_mode, out_mode, rpw, grid, s, e0, e1);
}

template <int L>
hipError_t launch_cu_l(const GemvArgs& a, int cpl, int in_mode, int out_mode, int rpw, dim3 grid, hipStream_t s,
                       hipEvent_t e0, hipEvent_t e1, int pw) {
    switch (cpl) {
        case 1: return launch_cu_e<L, 1>(a, in_mode, out_mode, rpw, grid, s, e0, e1, pw);
        case 2: return launch_cu_e<L, 2>(a, in_mode, out_mode, rpw, grid, s, e0, e1, pw);
        case 4: return launch_cu_e<L, 4>(a, in_mode, out_mode, rpw, grid, s, e0, e1, pw);
        default: return launch_cu_e<L, 8>(a, in_mode, out_mode, rpw, grid, s, e0, e1, pw);
    }
}

}  // namespace

int launch_ternary_gemv_cu(lbt_ctx* ctx, const TernaryOp& op) {
    if (op.m != 1 || (op.in_mode != kInF32 && op.in_mode != kInAttn)) return 1;
    GemvArgs a;
    int rc = make_gemv_args(ctx, op, a);
    if (rc) return rc;
    if (a.kp > kCuEPT * kCuThreads) return 1;
    // the f32 row is read with bounded 16-byte buffer loads (branch-free, so
    // the weight loads behind them are issued before the row has arrived)
    if (op.in_mode == kInF32 &&
        (op.cols % 4 || ((uintptr_t)op.x & 15) || ((uintptr_t)op.norm_w & 15)))
        return 1;
    const int total = a.total_rows;
    int rpw = (total + ctx->cus - 1) / ctx->cus;
    rpw = (rpw + 1) & ~1;  // row pairs never straddle workgroups
    if (rpw > kCuMaxRows) rpw = kCuMaxRows;
    const bool paired = op.in_mode != kInAttn && (op.out_mode == kOutRelu2 || op.out_mode == kOutQKV);
    const int L = rpw <= 16 && !paired ? 64 : (rpw <= 32 ? 32 : 16);
    const int need = (a.C + L - 1) / L;
    if (need > 8) return 1;
    const int cpl = need <= 1 ? 1 : (need <= 2 ? 2 : (need <= 4 ? 4 : 8));
    dim3 grid((unsigned)((total + rpw - 1) / rpw));
    hipEvent_t e0, e1;
    prof_pair(ctx, &e0, &e1);
    hipError_t e;
    const int pw = op.in_mode == kInAttn ? ctx->tune.gemv_pwo : ctx->tune.gemv_pw;
    if (L == 64) e = launch_cu_l<64>(a, cpl, op.in_mode, op.out_mode, rpw, grid, ctx->stream, e0, e1, pw);
    else if (L == 32) e = launch_cu_l<32>(a, cpl, op.in_mode, op.out_mode, rpw, grid, ctx->stream, e0, e1, pw);
    else e = launch_cu_l<16>(a, cpl, op.in_mode, op.out_mode, rpw, grid, ctx->stream, e0, e1, pw);
    if (e != hipSuccess) return hip_err(ctx, e, "tgemv_cu_kernel launch");
    const double bytes = (double)total * (a.kp / 4) + (double)op.cols * 4.0;
    prof_commit(ctx, e0, e1, kProfGemv, bytes);
    return LBT_OK;
}

}  // namespace lbt
