// ternary_mfma.hip -- packed 2-bit ternary x int8 prefill GEMM on the gfx950
// int8 matrix cores (v_mfma_i32_16x16x64_i8).
//
// Replaces the reference's prefill branch of ternary_gemm_multi
// (crates/lb-ternary/src/gemm.rs:155-194) and its AVX-512 2x4 register tile
// (tile_rows / tile_avx512bw, gemm.rs:245-268, :483-550).
//
// Layout of one MFMA (16 tokens x 16 rows x 64 k): lane l = 16*g + i holds
// A = 16 int8 activations of token i and B = 16 weight codes of row i for the
// same 16 k values (chunk g).  The 64 k values of one MFMA are taken straight
// from the LB2 layout: lane group g owns packed chunk c = 4p + g (16 bytes =
// 64 weights of one 32-byte block half) of super step p (256 k), and MFMA
// number kk = 0..3 of the step uses code group kk of those bytes, i.e. the 16
// weights (b*128 + kk*32 + h*16 + e) with the 16 activations at the same
// positions.  The codes c = w + 1 are unpacked with one shift and one mask per
// dword (no table, no LDS expansion) and fed as int8; the exact i32 result
// sum(c*q) - sum(q) is the reference's dot (gemm.rs:3-17, :306-308).
//
// Tiling: 4 wavefronts (2 x 2), each 16*MS tokens x 16*NS rows; activations
// are staged through LDS in 256-byte k-slices (double-buffered, rows padded to
// 272 bytes so each 16-lane group reads distinct banks), weights go from HBM
// straight into registers one super step ahead.  The epilogues are those of
// the decode GEMV (ternary_common.h), so outputs are identical.
#include <stdlib.h>

#include "ternary_common.h"

namespace lbt {

typedef int v4i __attribute__((ext_vector_type(4)));

template <int MS, int NS, int OUT>
__global__ __launch_bounds__(kThreads) void tgemm_kernel(GemvArgs a) {
    constexpr int BM = 32 * MS, BN = 32 * NS, AST = 256 + 16, APT = BM / 16;
    __shared__ __align__(16) int8_t As[2][BM * AST];
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int wm = w & 1, wn = w >> 1;
    const int li = lane & 15, lg = lane >> 4;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int C = a.C, kp = a.kp, M = a.m;
    const int nsteps = (C + 3) / 4;

    const uint4* brow[NS];
    bool bval[NS];
#pragma unroll
    for (int s = 0; s < NS; s++) {
        const int vr = n0 + wn * (BN / 2) + s * 16 + li;
        bval[s] = vr < a.total_rows;
        int mat, r;
        resolve_row<OUT>(a, bval[s] ? vr : 0, mat, r);
        brow[s] = (const uint4*)(sel3(a.w, mat) + (size_t)r * (size_t)(kp >> 2));
    }

    int4 ast[APT];
    uint4 bw[NS];
    auto a_load = [&](int p) {
#pragma unroll
        for (int e = 0; e < APT; e++) {
            const int idx = tid + kThreads * e, row = idx >> 4, col = idx & 15;
            const int tok = m0 + row, kb = p * 256 + col * 16;
            ast[e] = (tok < M && kb < kp) ? *(const int4*)(a.q + (size_t)tok * kp + kb) : make_int4(0, 0, 0, 0);
        }
    };
    auto a_store = [&](int buf) {
#pragma unroll
        for (int e = 0; e < APT; e++) {
            const int idx = tid + kThreads * e, row = idx >> 4, col = idx & 15;
            *(int4*)(As[buf] + row * AST + col * 16) = ast[e];
        }
    };
    auto b_load = [&](int p) {
#pragma unroll
        for (int s = 0; s < NS; s++) {
            const int c = 4 * p + lg;
            bw[s] = (bval[s] && c < C) ? ld_stream(brow[s] + c) : make_uint4(0, 0, 0, 0);
        }
    };

    v4i acc[MS][NS];
#pragma unroll
    for (int ms = 0; ms < MS; ms++)
#pragma unroll
        for (int s = 0; s < NS; s++) acc[ms][s] = v4i{0, 0, 0, 0};

    a_load(0);
    b_load(0);
    a_store(0);
    __syncthreads();
    for (int p = 0; p < nsteps; p++) {
        const int buf = p & 1;
        uint4 bcur[NS];
#pragma unroll
        for (int s = 0; s < NS; s++) bcur[s] = bw[s];
        if (p + 1 < nsteps) {
            a_load(p + 1);
            b_load(p + 1);
        }
        const int8_t* Ab = As[buf] + (wm * (BM / 2) + li) * AST + (lg >> 1) * 128 + (lg & 1) * 16;
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            const int sh = 2 * kk;
            v4i bop[NS];
#pragma unroll
            for (int s = 0; s < NS; s++)
                bop[s] = v4i{(int)((bcur[s].x >> sh) & 0x03030303u), (int)((bcur[s].y >> sh) & 0x03030303u),
                             (int)((bcur[s].z >> sh) & 0x03030303u), (int)((bcur[s].w >> sh) & 0x03030303u)};
#pragma unroll
            for (int ms = 0; ms < MS; ms++) {
                const v4i aop = *(const v4i*)(Ab + ms * 16 * AST + kk * 32);
#pragma unroll
                for (int s = 0; s < NS; s++)
                    acc[ms][s] = __builtin_amdgcn_mfma_i32_16x16x64_i8(aop, bop[s], acc[ms][s], 0, 0, 0);
            }
        }
        if (p + 1 < nsteps) a_store(buf ^ 1);
        __syncthreads();
    }

    // D layout: lane (g, i) holds tokens 4g..4g+3 of the 16-token block, row i.
#pragma unroll
    for (int ms = 0; ms < MS; ms++)
#pragma unroll
        for (int s = 0; s < NS; s++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int tok = m0 + wm * (BM / 2) + ms * 16 + 4 * lg + r;
                const int vr = n0 + wn * (BN / 2) + s * 16 + li;
                const bool ok = tok < M && vr < a.total_rows;
                const int d = acc[ms][s][r] - (tok < M ? a.qsum[tok] : 0);
                const float sa = (tok < M && a.qscale) ? a.qscale[tok] : 1.0f;
                if (OUT == kOutRelu2 || OUT == kOutQKV) {
                    const int dp = __shfl_xor(d, 1);
                    if (ok && (li & 1) == 0) store_pair<OUT>(a, tok, vr, d, dp, sa);
                } else if (ok) {
                    store_single<OUT>(a, tok, vr, d, sa);
                }
            }
}

namespace {

template <int MS, int NS>
hipError_t launch_tiles(const GemvArgs& a, int out_mode, dim3 grid, hipStream_t s, hipEvent_t e0, hipEvent_t e1) {
    switch (out_mode) {
        case kOutI32: hipExtLaunchKernelGGL((tgemm_kernel<MS, NS, kOutI32>), grid, dim3(kThreads), 0, s, e0, e1, 0, a); break;
        case kOutF32: hipExtLaunchKernelGGL((tgemm_kernel<MS, NS, kOutF32>), grid, dim3(kThreads), 0, s, e0, e1, 0, a); break;
        case kOutF32Add: hipExtLaunchKernelGGL((tgemm_kernel<MS, NS, kOutF32Add>), grid, dim3(kThreads), 0, s, e0, e1, 0, a); break;
        case kOutRelu2: hipExtLaunchKernelGGL((tgemm_kernel<MS, NS, kOutRelu2>), grid, dim3(kThreads), 0, s, e0, e1, 0, a); break;
        default: hipExtLaunchKernelGGL((tgemm_kernel<MS, NS, kOutQKV>), grid, dim3(kThreads), 0, s, e0, e1, 0, a); break;
    }
    return hipGetLastError();
}

int qws_reserve(lbt_ctx* ctx, size_t bytes, void** out) {
    if (bytes > ctx->qws_bytes) {
        if (ctx->qws) {
            hipStreamSynchronize(ctx->stream);
            hipFree(ctx->qws);
            ctx->qws = nullptr;
            ctx->qws_bytes = 0;
        }
        LBT_HIP(ctx, hipMalloc(&ctx->qws, bytes));
        ctx->qws_bytes = bytes;
    }
    *out = ctx->qws;
    return LBT_OK;
}

}  // namespace

int launch_ternary_mfma(lbt_ctx* ctx, const TernaryOp& op_in) {
    TernaryOp op = op_in;
    if (op.in_mode == kInF32) {
        // RMSNorm + ActQuant once per token row (the same arithmetic as the
        // GEMV prologue), then the GEMM reads int8 activations.
        const size_t kp = padded_cols((size_t)op.cols);
        void* q;
        const size_t qb = ((size_t)op.m * kp + 255) & ~(size_t)255;
        int rc = qws_reserve(ctx, qb + (size_t)op.m * 8, &q);
        if (rc) return rc;
        int8_t* qd = (int8_t*)q;
        float* sd = (float*)((char*)q + qb);
        int32_t* ud = (int32_t*)(sd + op.m);
        if ((rc = launch_quantize(ctx, op.x, op.norm_w, op.eps, op.m, op.cols, qd, sd, ud))) return rc;
        op.in_mode = kInPreQ;
        op.q = qd;
        op.qscale = sd;
        op.qsum = ud;
    }
    GemvArgs a;
    int rc = make_gemv_args(ctx, op, a);
    if (rc) return rc;
    const int total = a.total_rows;
    const bool big = (long)((total + 127) / 128) * ((op.m + 127) / 128) >= 240;
    hipEvent_t e0, e1;
    prof_pair(ctx, &e0, &e1);
    hipError_t e;
    if (big) {
        dim3 grid((unsigned)((total + 127) / 128), (unsigned)((op.m + 127) / 128));
        e = launch_tiles<4, 4>(a, op.out_mode, grid, ctx->stream, e0, e1);
    } else {
        dim3 grid((unsigned)((total + 63) / 64), (unsigned)((op.m + 63) / 64));
        e = launch_tiles<2, 2>(a, op.out_mode, grid, ctx->stream, e0, e1);
    }
    if (e != hipSuccess) return hip_err(ctx, e, "tgemm_kernel launch");
    prof_commit(ctx, e0, e1, kProfGemm, 2.0 * op.m * (double)total * a.kp);
    return LBT_OK;
}

}  // namespace lbt
