// ternary_mfma.hip -- packed 2-bit ternary x int8 GEMMs on the gfx950 int8
// matrix cores: the few-token kernel (v_mfma_i32_16x16x64_i8, batched decode
// and short prefills) and the pipelined prefill GEMM
// (v_mfma_i32_32x32x32_i8).
//
// Replaces the reference's prefill branch of ternary_gemm_multi
// (crates/lb-ternary/src/gemm.rs:155-194) and its AVX-512 2x4 register tile
// (tile_rows / tile_avx512bw, gemm.rs:245-268, :483-550).
//
// Layout of one 16 x 16 x 64 MFMA (16 tokens x 16 rows x 64 k): lane l = 16*g + i holds
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
// The epilogues are those of the decode GEMV (ternary_common.h), so outputs
// are identical.
#include <stdlib.h>

#include <type_traits>
#include <utility>

#include "ternary_common.h"


namespace lbt {

typedef int v4i __attribute__((ext_vector_type(4)));

typedef int v16i __attribute__((ext_vector_type(16)));

// MFMA D layouts.  16 x 16 tiles (v4i): lane l holds row l & 15 and tokens
// 4 (l >> 4) + r, r = 0..3.  32 x 32 tiles (v16i): lane l holds row l & 31
// and tokens 8 (r >> 2) + 4 (l >> 5) + (r & 3), r = 0..15.
template <int TM>
struct DLayout;
template <>
struct DLayout<16> {
    static constexpr int R = 4;
    __device__ static int tok(int lane, int r) { return 4 * (lane >> 4) + r; }
    __device__ static int row(int lane) { return lane & 15; }
};
template <>
struct DLayout<32> {
    static constexpr int R = 16;
    __device__ static int tok(int lane, int r) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }
    __device__ static int row(int lane) { return lane & 31; }
};

// Output stage of one wave's MS x NS block of TM x TM MFMA tiles (tokens
// from tok0, virtual rows from row0), in the D layout above.  Values are
// those of store_single / store_pair: dot = acc - sum(q) and the same float
// expressions.  Every load comes first, with clamped (always valid)
// indices, so the loads are in flight together; the stores follow under the
// bounds checks.
// Per-token values of the 16 x 16 epilogue loaded ahead of the main loop
// (epi_prefetch): sum(q), s_a and, for the residual add, the old outputs.
template <int MS, int NS>
struct EpiPre {
    int qs[MS][4];
    float sa[MS][4];
    float old[MS][NS][4];
};

template <int OUT, int TM, int MS, int NS, typename AccT>
__device__ __forceinline__ void mfma_epilogue(const GemvArgs& a, AccT (&acc)[MS][NS], int tok0, int row0,
                                              const EpiPre<MS, NS>* pre = nullptr) {
    using L = DLayout<TM>;
    constexpr int R = L::R;
    const int lane = (int)threadIdx.x & 63, lr = L::row(lane);
    const int M = a.m;
    int qs[MS][R];
    float sa[MS][R];
#pragma unroll
    for (int ms = 0; ms < MS; ms++)
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int tok = tok0 + ms * TM + L::tok(lane, r);
            const int tc = tok < M ? tok : M - 1;
            if constexpr (TM == 16) {
                if (pre) {
                    qs[ms][r] = pre->qs[ms][r];
                    sa[ms][r] = pre->sa[ms][r];
                    continue;
                }
            }
            qs[ms][r] = gload(a.qsum + tc);
            sa[ms][r] = a.qscale ? gload(a.qscale + tc) : 1.0f;
        }
    if (OUT == kOutRelu2) {
        // store_pair's relu(gate)^2 * up with the two scale divisions once
        // per token: even lanes hold gate row r, odd lanes up row r
        float* out0 = (float*)a.out[0];
        const int ld0 = a.rows[0];
#pragma unroll
        for (int ms = 0; ms < MS; ms++)
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int tok = tok0 + ms * TM + L::tok(lane, r);
                const float ig = 1.0f / (sa[ms][r] * a.sw[0]);
                const float iu = 1.0f / (sa[ms][r] * a.sw[1]);
#pragma unroll
                for (int s = 0; s < NS; s++) {
                    const int vr = row0 + s * TM + lr;
                    const int d = acc[ms][s][r] - qs[ms][r];
                    const int dp = __shfl_xor(d, 1);
                    if (tok < M && vr < a.total_rows && (lr & 1) == 0) {
                        const float y0 = (float)d * ig;
                        const float u = (float)dp * iu;
                        const float rl = y0 > 0.0f ? y0 : 0.0f;
                        gstore(out0 + (size_t)tok * ld0 + (vr >> 1), (rl * rl) * u);
                    }
                }
            }
        return;
    }
    if (OUT == kOutQKV) {
#pragma unroll
        for (int ms = 0; ms < MS; ms++)
#pragma unroll
            for (int s = 0; s < NS; s++)
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const int tok = tok0 + ms * TM + L::tok(lane, r);
                    const int vr = row0 + s * TM + lr;
                    const int d = acc[ms][s][r] - qs[ms][r];
                    const int dp = __shfl_xor(d, 1);
                    if (tok < M && vr < a.total_rows && (lr & 1) == 0) store_pair<OUT>(a, tok, vr, d, dp, sa[ms][r]);
                }
        return;
    }
    // unpaired modes: row -> (matrix, row) once per row block
    void* base[NS];
    int ld[NS];
    float sw[NS];
    bool okr[NS];
#pragma unroll
    for (int s = 0; s < NS; s++) {
        const int vr = row0 + s * TM + lr;
        okr[s] = vr < a.total_rows;
        int mt, ro;
        resolve_row<OUT>(a, okr[s] ? vr : 0, mt, ro);
        ld[s] = sel3(a.rows, mt);
        sw[s] = sel3(a.sw, mt);
        base[s] = OUT == kOutI32 ? (void*)((int32_t*)sel3(a.out, mt) + ro) : (void*)((float*)sel3(a.out, mt) + ro);
    }
    // residual add: the old values, at most 32 loads in flight at a time
    constexpr int MH = (MS * NS * R > 32 && MS > 1) ? MS / 2 : MS;
#pragma unroll
    for (int h = 0; h < MS; h += MH) {
        float old[MH][NS][R];
        if (OUT == kOutF32Add) {
#pragma unroll
            for (int mi = 0; mi < MH; mi++)
#pragma unroll
                for (int s = 0; s < NS; s++)
#pragma unroll
                    for (int r = 0; r < R; r++) {
                        const int tok = tok0 + (h + mi) * TM + L::tok(lane, r);
                        const int tc = tok < M ? tok : M - 1;
                        if constexpr (TM == 16) {
                            if (pre) {
                                old[mi][s][r] = pre->old[h + mi][s][r];
                                continue;
                            }
                        }
                        old[mi][s][r] = gload((const float*)base[s] + (size_t)tc * ld[s]);
                    }
        }
#pragma unroll
        for (int mi = 0; mi < MH; mi++)
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int ms = h + mi;
                const int tok = tok0 + ms * TM + L::tok(lane, r);
                // 1/(s_a*s_w): one correctly rounded division per token while
                // the row blocks share one matrix scale
                const float inv0 = OUT == kOutI32 ? 0.0f : 1.0f / (sa[ms][r] * sw[0]);
#pragma unroll
                for (int s = 0; s < NS; s++) {
                    if (tok >= M || !okr[s]) continue;
                    const int d = acc[ms][s][r] - qs[ms][r];
                    const size_t o = (size_t)tok * ld[s];
                    if (OUT == kOutI32) {
                        gstore((int32_t*)base[s] + o, (int32_t)d);
                    } else {
                        const float inv = sw[s] == sw[0] ? inv0 : 1.0f / (sa[ms][r] * sw[s]);
                        const float y = (float)d * inv;
                        const float v = OUT == kOutF32Add ? old[mi][s][r] + y : y;
                        // the prefill GEMM's output streams past L2 (nontemporal):
                        // measured 2-10% faster on the config-3 shapes
                        if constexpr (TM == 32)
                            __builtin_nontemporal_store(v, (LBT_GLOBAL float*)((float*)base[s] + o));
                        else
                            gstore((float*)base[s] + o, v);
                    }
                }
            }
    }
}

// The same values for a wavefront block whose rows all lie in one matrix
// and whose tokens are all below M (every full tile of an unpaired output):
// no per-store bounds branch, one division per token (the per-row-block
// scale is the block's one matrix scale), 32-bit offsets from the matrix's
// base (the compiler then uses scalar-base stores), the residual's old
// values loaded half a tile ahead of its stores.  Instruction count, not
// memory, bounds the epilogue of a 128 x 128 tile (2088 instructions per
// wavefront in the general form).
// Per-token values of a wavefront block's 32 MS tokens: lane j holds token
// tok0 + j's sum(q) and 1/(s_a*s_w) of matrix mt (one load pair and one
// division per lane, instead of one per lane and D-tile element); the
// epilogue fetches them across lanes.  Loaded ahead of the main loop
// (divide = false), divided once the first slices' loads are out.
// A block of 32 MS tokens: lane j holds tokens tok0 + j + 64 i, i < (MS + 1) / 2.
template <int MS>
struct Epi32Tok {
    static constexpr int N = (MS + 1) / 2;
    int qs[N];
    float inv[N];
    int pos[N];  // the token's position (q/k/v outputs only)
};

template <int OUT, int MS>
__device__ __forceinline__ void epi32_pre(const GemvArgs& a, int tok0, float swm, Epi32Tok<MS>& t, bool divide) {
    const int lane = (int)threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < Epi32Tok<MS>::N; i++) {
        const int j = 64 * i + lane;
        const int tok = tok0 + (j < 32 * MS ? j : 0);
        if (!divide) {
            t.qs[i] = gload(a.qsum + tok);
            t.inv[i] = a.qscale ? gload(a.qscale + tok) : 1.0f;  // s_a until divided
            if constexpr (OUT == kOutQKV)
                t.pos[i] = a.tok_pos ? gload(a.tok_pos + tok) : (a.pos_dev ? gload(a.pos_dev) : a.pos0) + tok;
        } else {
            t.inv[i] = OUT == kOutI32 ? 0.0f : 1.0f / (t.inv[i] * swm);
        }
    }
}

template <int OUT, int MS, int NS>
__device__ __forceinline__ void epi32_full(const GemvArgs& a, v16i (&acc)[MS][NS], int tok0, int mt_v, int ro0_v,
                                           const Epi32Tok<MS>& t) {
    using L = DLayout<32>;
    constexpr int R = L::R;
    const int lane = (int)threadIdx.x & 63, lr = L::row(lane);
    // wavefront-uniform: scalar registers, scalar selects
    const int mt = __builtin_amdgcn_readfirstlane(mt_v), ro0 = __builtin_amdgcn_readfirstlane(ro0_v);
    const int ld = mt == 0 ? a.rows[0] : (mt == 1 ? a.rows[1] : a.rows[2]);
    const float swm = mt == 0 ? a.sw[0] : (mt == 1 ? a.sw[1] : a.sw[2]);
    void* const outv = mt == 0 ? a.out[0] : (mt == 1 ? a.out[1] : a.out[2]);
    // stores through a buffer resource: the matrix base in scalar registers,
    // a 32-bit byte offset per lane (the caller checks M * ld < 2^30)
    const __amdgpu_buffer_rsrc_t ob = buf_rsrc(outv, 0xffffffffu);
    (void)swm;
#pragma unroll
    for (int ms = 0; ms < MS; ms++) {
        // this block's tokens 32 ms .. 32 ms + 31 sit in slot ms / 2 of lanes 32 (ms & 1) + ..
        int qs[R];
        float inv[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int src = (ms & 1) * 32 + L::tok(lane, r);
            qs[r] = __shfl(t.qs[ms >> 1], src, 64);
            inv[r] = __shfl(t.inv[ms >> 1], src, 64);
        }
        float old[NS][R];
        if (OUT == kOutF32Add) {
#pragma unroll
            for (int s = 0; s < NS; s++)
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const int tok = tok0 + ms * 32 + L::tok(lane, r);
                    const uint32_t off = (uint32_t)(tok * ld + ro0 + s * 32 + lr) * 4u;
                    old[s][r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ob, off, 0, 0));
                }
        }
#pragma unroll
        for (int s = 0; s < NS; s++)
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int tok = tok0 + ms * 32 + L::tok(lane, r);
                const uint32_t off = (uint32_t)(tok * ld + ro0 + s * 32 + lr) * 4u;
                const int d = acc[ms][s][r] - qs[r];
                if (OUT == kOutI32) {
                    __builtin_amdgcn_raw_buffer_store_b32((uint32_t)d, ob, off, 0, 0);
                } else {
                    const float y = (float)d * inv[r];
                    const float v = OUT == kOutF32Add ? old[s][r] + y : y;
                    // nontemporal: the output streams past L2
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), ob, off, 0, 2);
                }
            }
    }
}

// The q/k/v output (RoPE on q and k, bf16 K/V cache append) of a wavefront
// block whose 32 NS virtual rows lie in one matrix and whose tokens are all
// below M: store_pair's values and float expressions, with its per-element
// work hoisted -- sum(q), 1/(s_a*s_w) and the position come per token from
// t (loaded and divided before the main loop), the row's matrix, head and
// dim once per lane, and every cos / sin load of a 32-token block issued
// before that block's stores (store_pair's loads wait behind the previous
// pair's stores, which might alias them).  A V pair (rows r, r + 1) goes out
// as one 32-bit store of the two bf16 values.
template <int MS, int NS>
__device__ __forceinline__ void epi32_qkv(const GemvArgs& a, v16i (&acc)[MS][NS], int tok0, int row0,
                                          const Epi32Tok<MS>& t) {
    using L = DLayout<32>;
    constexpr int R = L::R;
    const int lane = (int)threadIdx.x & 63, lr = L::row(lane);
    const bool even = (lr & 1) == 0;
    const int hd = a.hd, h2 = hd >> 1;
    int mat[NS], r0[NS];
#pragma unroll
    for (int s = 0; s < NS; s++) resolve_row<kOutQKV>(a, row0 + s * 32 + (lr & ~1), mat[s], r0[s]);
#pragma unroll
    for (int ms = 0; ms < MS; ms++) {
        int qs[R], pos[R];
        float inv[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int src = (ms & 1) * 32 + L::tok(lane, r);
            qs[r] = __shfl(t.qs[ms >> 1], src, 64);
            inv[r] = __shfl(t.inv[ms >> 1], src, 64);
            pos[r] = __shfl(t.pos[ms >> 1], src, 64);
        }
#pragma unroll
        for (int s = 0; s < NS; s++) {
            float y0[R], y1[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int d0 = acc[ms][s][r] - qs[r];
                const int d1 = __shfl_xor(d0, 1);
                y0[r] = (float)d0 * inv[r];
                y1[r] = (float)d1 * inv[r];
            }
            if (!even) continue;
            const int g = r0[s] / hd, dd = r0[s] % hd;
            if (mat[s] == 2) {
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const int tok = tok0 + ms * 32 + L::tok(lane, r);
                    const size_t coff = a.tok_pos ? (size_t)tok * a.seq_stride : 0;
                    uint16_t* dst = a.vc + coff + ((size_t)g * a.cap + pos[r]) * hd + dd;
                    gstore((uint32_t*)dst, (uint32_t)f32_to_bf16(y0[r]) | ((uint32_t)f32_to_bf16(y1[r]) << 16));
                }
                continue;
            }
            float c[R], sn[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                c[r] = gload(a.cos_t + (size_t)pos[r] * h2 + dd);
                sn[r] = gload(a.sin_t + (size_t)pos[r] * h2 + dd);
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int tok = tok0 + ms * 32 + L::tok(lane, r);
                const float z0 = y0[r] * c[r] + (-y1[r]) * sn[r];
                const float z1 = y1[r] * c[r] + y0[r] * sn[r];
                if (mat[s] == 0) {
                    float* q = (float*)a.out[0] + (size_t)tok * a.rows[0];
                    gstore(q + r0[s], z0);
                    gstore(q + r0[s] + h2, z1);
                } else {
                    const size_t coff = a.tok_pos ? (size_t)tok * a.seq_stride : 0;
                    uint16_t* dst = a.kc + coff + ((size_t)g * a.cap + pos[r]) * hd + dd;
                    gstore(dst, f32_to_bf16(z0));
                    gstore(dst + h2, f32_to_bf16(z1));
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Few-token GEMM (batched decode and short prefills, 2..32 tokens, and up to
// 64 for the shapes with few 64 x 64 tiles): the
// weight stream is the whole cost, so the grid is cut as finely as the
// 16 x 16 x 64 MFMA allows -- one workgroup per 16 rows (o/down of the 2B
// model: 160 workgroups instead of 40 tiles of 64 rows; 32 rows, NS = 2, where
// that still leaves >= 256 workgroups, halving the activation re-reads) --
// and its 4 wavefronts split K into contiguous step ranges.  Each wavefront
// issues every weight load of its range at once (at most kSmallMaxSteps uint4
// per lane and row tile), reads the activations (L2-resident, 16 MS tokens)
// straight from global memory one step ahead, and the three partial int32
// tiles are added to wavefront 0's through LDS (exact, any order) before the
// shared epilogue.  Operand layout: lane (li, lg) takes chunk
// 4p + lg of row li and, for MFMA kk of step p, the 16 activations of token
// li at k = 256 p + 128 (lg >> 1) + 32 kk + 16 (lg & 1).
// Loads of mfma_epilogue's per-token values (16 x 16 tiles), the same
// addresses it would use.
template <int OUT, int MS, int NS>
__device__ __forceinline__ void epi_prefetch(const GemvArgs& a, int tok0, int row0, EpiPre<MS, NS>& p) {
    using L = DLayout<16>;
    const int lane = (int)threadIdx.x & 63, lr = L::row(lane);
    const int M = a.m;
#pragma unroll
    for (int ms = 0; ms < MS; ms++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int tok = tok0 + ms * 16 + L::tok(lane, r);
            const int tc = tok < M ? tok : M - 1;
            p.qs[ms][r] = gload(a.qsum + tc);
            p.sa[ms][r] = a.qscale ? gload(a.qscale + tc) : 1.0f;
        }
    if (OUT != kOutF32Add) return;
#pragma unroll
    for (int s = 0; s < NS; s++) {
        const int vr = row0 + s * 16 + lr;
        int mt, ro;
        resolve_row<OUT>(a, vr < a.total_rows ? vr : 0, mt, ro);
        const float* base = (const float*)sel3(a.out, mt) + ro;
        const int ld = sel3(a.rows, mt);
#pragma unroll
        for (int ms = 0; ms < MS; ms++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int tok = tok0 + ms * 16 + L::tok(lane, r);
                const int tc = tok < M ? tok : M - 1;
                p.old[ms][s][r] = gload(base + (size_t)tc * ld);
            }
    }
}

constexpr int kSmallMaxSteps = 8;  // 256-k steps per wavefront: K <= 8192
constexpr int kSmallWideGroups = 256;  // 32-row tiles from 256 workgroups of them

template <int OUT, int MS, int NS, bool PF = false>
__global__ __launch_bounds__(kThreads) void tgemm_small_kernel(GemvArgs a) {
    __shared__ __align__(16) v4i part[3][MS][NS][64];
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int li = lane & 15, lg = lane >> 4;
    const int m0 = blockIdx.y * (16 * MS), n0 = blockIdx.x * (16 * NS);
    const int C = a.C, kp = a.kp, M = a.m;
    const int nsteps = (C + 3) / 4;
    const int p0 = (nsteps * w) >> 2, p1 = (nsteps * (w + 1)) >> 2;

    uint4 bw[NS][kSmallMaxSteps];
#pragma unroll
    for (int ns = 0; ns < NS; ns++) {
        const int vr = n0 + ns * 16 + li;
        const bool bval = vr < a.total_rows;
        int mat, r;
        resolve_row<OUT>(a, bval ? vr : 0, mat, r);
        const uint4* brow = (const uint4*)(sel3(a.w, mat) + (size_t)r * (size_t)(kp >> 2));
#pragma unroll
        for (int i = 0; i < kSmallMaxSteps; i++) {
            const int c = 4 * (p0 + i) + lg;
            bw[ns][i] = (bval && p0 + i < p1 && c < C) ? ld_stream(brow + c) : make_uint4(0, 0, 0, 0);
        }
    }

    const int8_t* arow[MS];
#pragma unroll
    for (int ms = 0; ms < MS; ms++) {
        const int tok = m0 + ms * 16 + li;
        arow[ms] = a.q + (size_t)(tok < M ? tok : M - 1) * kp + (lg >> 1) * 128 + (lg & 1) * 16;
    }
    // activation operands of one step; k beyond kp only meets zero weights,
    // so its address is clamped to the row's last step
    auto a_load = [&](int p, v4i (&dst)[MS][4]) {
        const int pc = 256 * p < kp ? p : (kp - 1) / 256;
#pragma unroll
        for (int ms = 0; ms < MS; ms++)
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                const int off = 256 * pc + 32 * kk + (lg >> 1) * 128 + (lg & 1) * 16;
                dst[ms][kk] = off + 16 <= kp ? *(const v4i*)(arow[ms] + 256 * pc + 32 * kk) : v4i{0, 0, 0, 0};
            }
    };

    EpiPre<MS, NS> pre;
    if (PF && w == 0) epi_prefetch<OUT, MS, NS>(a, m0, n0, pre);
    v4i acc[MS][NS];
#pragma unroll
    for (int ms = 0; ms < MS; ms++)
#pragma unroll
        for (int ns = 0; ns < NS; ns++) acc[ms][ns] = v4i{0, 0, 0, 0};
    v4i aop[2][MS][4];
    if (p0 < p1) a_load(p0, aop[0]);
#pragma unroll
    for (int i = 0; i < kSmallMaxSteps; i++) {
        if (p0 + i >= p1) break;
        if (p0 + i + 1 < p1) a_load(p0 + i + 1, aop[(i + 1) & 1]);
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            const int sh = 2 * kk;
#pragma unroll
            for (int ns = 0; ns < NS; ns++) {
                const uint4 b = bw[ns][i];
                const v4i bop = v4i{(int)((b.x >> sh) & 0x03030303u), (int)((b.y >> sh) & 0x03030303u),
                                    (int)((b.z >> sh) & 0x03030303u), (int)((b.w >> sh) & 0x03030303u)};
#pragma unroll
                for (int ms = 0; ms < MS; ms++)
                    acc[ms][ns] = __builtin_amdgcn_mfma_i32_16x16x64_i8(aop[i & 1][ms][kk], bop, acc[ms][ns], 0, 0, 0);
            }
        }
    }
    if (w > 0) {
#pragma unroll
        for (int ms = 0; ms < MS; ms++)
#pragma unroll
            for (int ns = 0; ns < NS; ns++) part[w - 1][ms][ns][lane] = acc[ms][ns];
    }
    __syncthreads();
    if (w > 0) return;
#pragma unroll
    for (int ms = 0; ms < MS; ms++)
#pragma unroll
        for (int ns = 0; ns < NS; ns++)
            acc[ms][ns] += (part[0][ms][ns][lane] + part[1][ms][ns][lane]) + part[2][ms][ns][lane];
    mfma_epilogue<OUT, 16>(a, acc, m0, n0, PF ? &pre : nullptr);
}

// ---------------------------------------------------------------------------
// Pipelined prefill GEMM on the full-rate int8 MFMA of gfx950
// (v_mfma_i32_32x32x32_i8: 32768 MACs in 8 passes, twice the rate of the
// 16x16x64 form).  A workgroup of 4 wavefronts (2 x 2) computes BM = 64 MS
// tokens x BN = 64 NS rows, each wavefront MS x NS tiles of 32 x 32.  A step
// covers KB 128-k blocks (8 KB MFMAs per tile).
//
// Activations go HBM -> LDS with global_load_lds_dwordx4 (no registers) into
// a ring of ST stages of one step's slice each, ST slices ahead; the MFMA A
// operands of slice p+1 are read from LDS while the MFMAs of slice p run.
// Packed weights go to registers ST steps ahead and are unpacked per MFMA.
// One barrier per step.  With KB = 1, MS = NS = 2 and three stages the ring
// is 48 KB, so two workgroups (register-bound) share a CU and one's prologue
// and epilogue overlap the other's MFMAs.
//
// LDS slice layout: token T of the tile owns RB = 128 KB bytes; its 16-byte
// chunk c sits at T*RB + ((c ^ swz(T)) * 16), swz(T) = T & 15 for 256-byte
// rows and (T >> 1) & 7 for 128-byte rows, so the 16 lanes of an operand
// read (16 consecutive tokens, same c) hit 16 different 16-byte bank groups.
//
// MFMA operands (32 x 32 x 32): lane l supplies, for A, token (l & 31) and
// for B, row (l & 31), the 16 k values 16 (l >> 5) .. 16 (l >> 5) + 15 of the
// 32-k chunk.  Chunk kc of a step (k = 32 kc .. 32 kc + 31) lies in 128-k
// block kc >> 2, 2-bit field kc & 3; its bytes 16 g .. 16 g + 15 (g = l >> 5)
// hold k = 32 (kc & 3) + 16 g + j: packed uint4 number 2 (kc >> 2) + g of the
// step, shifted right by 2 (kc & 3).
typedef __attribute__((address_space(3))) void lds_void_t;

// LDS ring stages of tgemm2_kernel (slices in flight ahead of the MFMAs):
// 3 measured 1-3% faster than 4 at M = 2048 (one stage less of LDS per
// workgroup) and as fast below; 2 is slower at M = 512.
constexpr int kG2Stages = 3;

// f(integral_constant<I>) for I = 0, 1, ... while it returns true.
template <int... I, class F>
__device__ __forceinline__ void seq_while(std::integer_sequence<int, I...>, F&& f) {
    (f(std::integral_constant<int, I>{}) && ...);
}

template <int KB>
__device__ __forceinline__ int g2_swz(int T) {
    return KB == 2 ? (T & 15) : ((T >> 1) & 7);
}

// XCD-aware tile order.  Workgroups are dispatched round-robin over the 8
// XCDs (workgroup b to XCD b % 8), each XCD with its own L2, and every tile
// re-reads its token tile and row tile from L2.  So the grid's tiles are
// listed in bands of kG2Group token tiles (row tiles of a band in order,
// the band's token tiles fastest) and XCD k takes the k-th contiguous
// eighth of that list: at M = 2048 on 6912 rows, 4 token tiles x 27 row
// tiles per XCD, whose operands (3.5 MB) fit its L2 (config 3: 2-3% at
// M = 2048, 8% on 2560 x 6912 at M = 512).  A bijection of the grid, so
// results do not depend on the dispatch order.
constexpr int kG2Group = 4;  // measured against 1, 2, 8 and the plain grid order

__device__ __forceinline__ void g2_tile(int& tx, int& ty) {
    const int TX = (int)gridDim.x, TY = (int)gridDim.y, n = TX * TY;
    const int b = (int)blockIdx.y * TX + (int)blockIdx.x;
    const int k = b & 7, j = b >> 3;
    const int base = n >> 3, rem = n & 7;
    const int t = k * base + (k < rem ? k : rem) + j;
    const int G = kG2Group < TY ? kG2Group : TY;
    const int band = t / (G * TX), r = t - band * G * TX;
    const int gsz = TY - band * G < G ? TY - band * G : G;
    tx = r / gsz;
    ty = band * G + r % gsz;
}

// Split-k: the partial int32 tile of every workgroup goes to kpart with
// device-coherent stores ([tile][range][wavefront][ms][s][r][lane], so each
// store instruction writes 256 contiguous bytes); once they are acknowledged
// the workgroup counts itself in at kcnt[tile].  The last one to arrive
// resets the counter, reads the other ranges' partials (device-coherent
// loads) and adds them to its own: integer sums, so the result has the same
// bits in any arrival order.  Returns whether this workgroup is the last.
template <int MS, int NS>
__device__ __forceinline__ bool split_reduce(const GemvArgs& a, v16i (&acc)[MS][NS], int tx, int ty, int w, int lane) {
    constexpr int CW = MS * NS * 1024;  // ints per wavefront
    __shared__ int last;
    const int tile = ty * (int)gridDim.x + tx, zs = (int)blockIdx.z, ks = a.ksplit;
    int* base = a.kpart + (size_t)tile * ks * (4 * CW) + w * CW + lane;
    int* mine = base + (size_t)zs * (4 * CW);
#pragma unroll
    for (int ms = 0; ms < MS; ms++)
#pragma unroll
        for (int s = 0; s < NS; s++)
#pragma unroll
            for (int r = 0; r < 16; r++)
                __hip_atomic_store(mine + ((ms * NS + s) * 16 + r) * 64, acc[ms][s][r], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        const int old = __hip_atomic_fetch_add(a.kcnt + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = old == ks - 1;
        if (old == ks - 1) __hip_atomic_store(a.kcnt + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last) return false;
    for (int z = 0; z < ks; z++) {
        if (z == zs) continue;
        const int* src = base + (size_t)z * (4 * CW);
#pragma unroll
        for (int ms = 0; ms < MS; ms++)
#pragma unroll
            for (int s = 0; s < NS; s++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                    acc[ms][s][r] += __hip_atomic_load(src + ((ms * NS + s) * 16 + r) * 64, __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT);
    }
    return true;
}

template <int OUT, int MS, int NS, int KB, int ST = kG2Stages>
// Two wavefronts per SIMD: without the bound the compiler moved the
// accumulators to AGPRs beyond 256 registers (one wavefront per SIMD, 20%
// slower); three per SIMD needs a single-buffered A operand (164 VGPRs),
// measured no faster.
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void tgemm2_kernel(GemvArgs a) {
    constexpr int TM = 32, BM = 2 * TM * MS, BN = 2 * TM * NS;
    constexpr int RB = 128 * KB;                 // LDS bytes per token per stage
    constexpr int KC = 4 * KB;                   // 32-k chunks per step
    constexpr int kSlice = BM * RB;              // bytes of one LDS stage
    constexpr int NA = kSlice / 16 / kThreads;   // A chunks per lane per step
    constexpr int NB = NS * KB;                  // weight uint4 loads per lane per step
    constexpr int TPB = 1024 / RB;               // tokens per 1 KB DMA block
    extern __shared__ __align__(16) int8_t As[];  // [ST][kSlice]
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int wm = w & 1, wn = w >> 1;
    const int l32 = lane & 31, g = lane >> 5;
    int tx, ty;
    g2_tile(tx, ty);
    const int m0 = ty * BM, n0 = tx * BN;
    const int kp = a.kp, M = a.m;
    // this workgroup's k steps: range blockIdx.z of a.ksplit
    const int nk = kp / RB, zs = (int)blockIdx.z;
    const int ps0 = (int)((long)nk * zs / a.ksplit), ps1 = (int)((long)nk * (zs + 1) / a.ksplit);
    // a full wavefront block of one matrix takes the lean epilogue; its
    // per-token values are loaded now and divided once the loads of the
    // first slices are out (they arrive during the main loop's prologue)
    const int tok0 = m0 + wm * (BM / 2), row0 = n0 + wn * (BN / 2);
    bool fast = false;
    int mt0 = 0, ro0 = 0;
    float swm = 1.0f;
    Epi32Tok<MS> et{};
    if constexpr (OUT == kOutF32 || OUT == kOutF32Add || OUT == kOutI32) {
        int mt1, ro1;
        resolve_row<OUT>(a, row0, mt0, ro0);
        resolve_row<OUT>(a, row0 + NS * TM - 1, mt1, ro1);
        const int ldm = mt0 == 0 ? a.rows[0] : (mt0 == 1 ? a.rows[1] : a.rows[2]);
        swm = mt0 == 0 ? a.sw[0] : (mt0 == 1 ? a.sw[1] : a.sw[2]);
        fast = tok0 + MS * TM <= M && row0 + NS * TM <= a.total_rows && mt0 == mt1 && (long)M * ldm < (1L << 30);
        if (fast) epi32_pre<OUT, MS>(a, tok0, swm, et, false);
    } else if constexpr (OUT == kOutQKV) {
        int mt1, ro1;
        resolve_row<OUT>(a, row0, mt0, ro0);
        resolve_row<OUT>(a, row0 + NS * TM - 1, mt1, ro1);
        swm = mt0 == 0 ? a.sw[0] : (mt0 == 1 ? a.sw[1] : a.sw[2]);
        fast = tok0 + MS * TM <= M && row0 + NS * TM <= a.total_rows && mt0 == mt1;
        if (fast) epi32_pre<OUT, MS>(a, tok0, swm, et, false);
    }

    // weights: row tile s of this wave, row l32; packed uint4 2b + g of a step
    const uint4* brow[NS];
#pragma unroll
    for (int s = 0; s < NS; s++) {
        const int vr = n0 + wn * (BN / 2) + s * TM + l32;
        int mat, r;
        resolve_row<OUT>(a, vr < a.total_rows ? vr : 0, mat, r);
        brow[s] = (const uint4*)(sel3(a.w, mat) + (size_t)r * (size_t)(kp >> 2)) + g;
    }
    // activations: this lane's NA chunks of a slice (LDS slot fixed by the
    // lane, global chunk chosen to realise the swizzle)
    const int8_t* asrc[NA];
    int adst[NA];
#pragma unroll
    for (int j = 0; j < NA; j++) {
        const int blk = w * NA + j;  // 1 KB block of the slice
        const int T = blk * TPB + lane / (RB / 16), cs = lane % (RB / 16);
        const int c = cs ^ g2_swz<KB>(T);
        const int tok = m0 + T < M ? m0 + T : M - 1;  // past M: any valid row, never stored
        asrc[j] = a.q + (size_t)tok * kp + c * 16;
        adst[j] = blk * 1024;
    }
    auto a_issue = [&](int p, int stage) {
        int8_t* dst = As + stage * kSlice;
#pragma unroll
        for (int j = 0; j < NA; j++)
            __builtin_amdgcn_global_load_lds((const void*)(asrc[j] + p * RB), (lds_void_t*)(dst + adst[j]), 16, 0, 0);
    };
    // Rows past total_rows load row 0 of matrix 0 (never stored), so every
    // load is unconditional and the outstanding-load count is the same on
    // every step.  The weight loads are issued as inline asm: the compiler
    // does not track them, so it adds no waits of its own (its tracking of
    // loop-carried loads falls back to waiting for everything); the step's
    // explicit s_waitcnt covers them, and pin() after it keeps every use of
    // the registers below the wait.
    u32x4 bw[ST][NB];  // [slot][s * KB + 128-k block]
    auto b_issue = [&](int p, u32x4 (&dst)[NB]) {
#pragma unroll
        for (int s = 0; s < NS; s++)
#pragma unroll
            for (int b = 0; b < KB; b++)
                asm volatile("global_load_dwordx4 %0, %1, off"
                             : "=v"(dst[s * KB + b])
                             : "v"(brow[s] + 2 * (KB * p + b))
                             : "memory");
    };
    auto pin = [](u32x4& v) { asm volatile("" : "+v"(v)); };
    // vector-memory count n, and the LDS counter 0 (this wave's operand reads
    // of a stage are done before any wave passes the barrier and refills it)
    auto wait_vm = [](auto n_c) {
        constexpr int n = decltype(n_c)::value;
        __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4) | (0 << 8));
    };

    v16i acc[MS][NS];
#pragma unroll
    for (int ms = 0; ms < MS; ms++)
#pragma unroll
        for (int s = 0; s < NS; s++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[ms][s][r] = 0;

    // A operand of (kc, ms): token wm*64 + ms*32 + l32 (its swizzle depends
    // on l32 only), chunk 2 kc + g of the slice
    const int arow = (wm * (BM / 2) + l32) * RB;
    int axo[KC];
#pragma unroll
    for (int kc = 0; kc < KC; kc++) axo[kc] = ((2 * kc + g) ^ g2_swz<KB>(l32)) << 4;
    v4i aop[2][KC][MS];  // A operands of the current and the next step
    auto a_read = [&](int stage, v4i (&dst)[KC][MS]) {
        const int8_t* Ab = As + stage * kSlice + arow;
#pragma unroll
        for (int kc = 0; kc < KC; kc++)
#pragma unroll
            for (int ms = 0; ms < MS; ms++) dst[kc][ms] = *(const v4i*)(Ab + axo[kc] + ms * TM * RB);
    };

    // Prologue: slices and weights of steps 0..3 in flight (steps past the
    // end re-load the last one: cache hits into a stage nobody reads, so the
    // count of loads in flight is the same on every step), then the A
    // operands of step 0.
    const int plast = ps1 - 1;
#pragma unroll
    for (int p = 0; p < ST; p++) {
        const int pi = ps0 + p < plast ? ps0 + p : plast;
        a_issue(pi, p);
        b_issue(pi, bw[p]);
    }
    if constexpr (OUT == kOutF32 || OUT == kOutF32Add || OUT == kOutI32 || OUT == kOutQKV)
        if (fast) epi32_pre<OUT, MS>(a, tok0, swm, et, true);
    wait_vm(std::integral_constant<int, NB + (ST - 1) * (NA + NB)>{});
    __builtin_amdgcn_s_barrier();
    a_read(0, aop[0]);

    // Step p (ring slot p % ST and operand buffer p % 2 as constants: no
    // register rotation, which would wait for every load in flight):
    //   wait for slice p+1 (own chunks) and weights p, barrier (all chunks of
    //   slice p+1; every wave has read slice p into registers);
    //   slice p+ST -> stage p % ST; LDS reads of slice p+1 into the other
    //   operand buffer while the MFMAs of step p run; weights p+ST into the
    //   registers of weights p once they are unpacked.  Loads are issued in
    //   the order A_0 B_0 A_1 B_1 ..., so "slice p+1 and weights p done"
    //   leaves B_{p+1} and the ST-2 later pairs in flight.
    auto step = [&](int p, auto slot_c, auto cur_c) {
        constexpr int slot = decltype(slot_c)::value;
        constexpr int cur = decltype(cur_c)::value;
        wait_vm(std::integral_constant<int, NB + (ST - 2) * (NA + NB)>{});
#pragma unroll
        for (int i = 0; i < NB; i++) pin(bw[slot][i]);
        __builtin_amdgcn_s_barrier();
        const int pn = p + ST < plast ? p + ST : plast;
        a_issue(pn, slot);
        a_read((slot + 1) % ST, aop[cur ^ 1]);
#pragma unroll
        for (int kc = 0; kc < KC; kc++) {
            const int sh = 2 * (kc & 3), b = kc >> 2;
            v4i bop[NS];
#pragma unroll
            for (int s = 0; s < NS; s++) {
                const u32x4 v = bw[slot][s * KB + b];
                bop[s] = v4i{(int)((v.x >> sh) & 0x03030303u), (int)((v.y >> sh) & 0x03030303u),
                             (int)((v.z >> sh) & 0x03030303u), (int)((v.w >> sh) & 0x03030303u)};
            }
#pragma unroll
            for (int ms = 0; ms < MS; ms++)
#pragma unroll
                for (int s = 0; s < NS; s++)
                    acc[ms][s] = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop[cur][kc][ms], bop[s], acc[ms][s], 0, 0, 0);
        }
        b_issue(pn, bw[slot]);
    };
    // unrolled over a multiple of both the ring (slot) and the operand
    // double buffer (cur), so both are constants in every step
    constexpr int U = ST % 2 == 0 ? ST : 2 * ST;
    for (int p = ps0; p < ps1; p += U)
        seq_while(std::make_integer_sequence<int, U>{}, [&](auto ic) {
            constexpr int i = decltype(ic)::value;
            if (p + i >= ps1) return false;
            step(p + i, std::integral_constant<int, i % ST>{}, std::integral_constant<int, i & 1>{});
            return true;
        });
    // No load in flight past this point.  The weight registers of the last
    // steps are never read, so each is used here, after the wait: until then
    // the compiler cannot give a register to anything else while a load
    // untracked by it is still to write it.
    __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
    for (int k = 0; k < ST; k++)
#pragma unroll
        for (int i = 0; i < NB; i++) asm volatile("" ::"v"(bw[k][i]));

    if (a.ksplit > 1 && !split_reduce<MS, NS>(a, acc, tx, ty, w, lane)) return;
    if constexpr (OUT == kOutF32 || OUT == kOutF32Add || OUT == kOutI32) {
        if (fast) {
            epi32_full<OUT, MS, NS>(a, acc, tok0, mt0, ro0, et);
            return;
        }
    } else if constexpr (OUT == kOutQKV) {
        if (fast) {
            epi32_qkv<MS, NS>(a, acc, tok0, row0, et);
            return;
        }
    }
    mfma_epilogue<OUT, TM>(a, acc, tok0, row0);
}

// Prefill GEMM with one workgroup per CU of 8 or more wavefronts (at least
// two per SIMD, what keeps the matrix pipe fed): WM x WN wavefronts of
// (32 MS) x (32 NS) each, so a tile is BM = 32 MS WM tokens x BN = 32 NS WN
// rows.  The product uses <WM, WN, MS, NS, KB> = <1, 8, 4, 1, 1>: 128 tokens
// x 256 rows, every wavefront all 128 tokens of 32 rows of its own, so each
// weight row is unpacked by one wavefront only (the unpacking -- a shift and
// a mask per dword and 32-k chunk -- is most of the main loop's VALU work;
// with 2 x 4 wavefronts of 64 x 64 every row was unpacked twice); and
// <1, 10, 2, 1, 1>: 64 tokens x 320 rows from 10 wavefronts (at most three
// per SIMD, 2 MFMA tiles each: 6 per SIMD and step against 8), for the
// matrices whose 128 x 256 tiles leave CUs idle -- 2560 rows at M = 2048
// give 256 tiles of 64 x 320 (44.0 -> 36.8 us, 39% of the int8 peak)
// against 160 of 128 x 256.  Workgroups of more than 8 wavefronts load each
// activation slice from the first LW of them only.
// Operands as in tgemm2_kernel (the same LDS slice layout and swizzle, the
// weights unpacked in registers); the ring holds ST slices and slice
// p + ST - 1 is issued once every wavefront has passed the barrier of step
// p, so ST - 1 slices are in flight during a step.  A operands are read from
// LDS one 32-k chunk ahead of the MFMAs.  Same accumulators, same epilogues:
// the same bits as every other GEMM path.  Measured against the 128 x 128
// tiles of tgemm2_kernel (two workgroups per CU), config-3 shapes: 2560 x
// 6912 at M = 2048 44.6 -> 42.5 us (160 tiles, one round), 6912 x 2560 at
// M = 1024 23.1 -> 22.0 us and at M = 2048 44.9 -> 43.1 us; slower where
// it leaves fewer than ~150 tiles (M = 512: 15.4 -> 19.4 us and 19.1 ->
// 39.2 us in the 2 x 4 form).  Measured and not kept: 2 x 4 wavefronts of
// 64 x 64 (3-5% slower), with the next slice's A operands read a whole
// step ahead as in tgemm2_kernel (2 x 4: 1-4% faster than per chunk; 1 x 8:
// 3-5% slower), ring depths of 4 and 6 slices (no faster), 256 x 256 tiles
// (216 tiles on 6912 x 2560 at M = 2048 in one round: 44.9 us; 74-79 us on
// the 2560-row matrix), 128 x 192 and 256 x 128 tiles, and 256-k steps
// (KB = 2: 2-10% slower).
constexpr int kG3MinTiles = 150;
constexpr int kG3Stages = 3;

// waves_per_eu bound of a workgroup of NW wavefronts, one workgroup per CU
template <int NW>
constexpr int g3_wpe = (NW + 3) / 4 < 2 ? 2 : (NW + 3) / 4;
// wavefronts that load the activation slices: the largest count <= NW that
// divides the slice's 1 KB blocks
template <int NW, int NBLK>
constexpr int g3_loaders() {
    int l = NW < NBLK ? NW : NBLK;
    while (NBLK % l) l--;
    return l;
}

template <int OUT, int WM, int WN, int MS, int NS, int KB, int ST>
__global__ __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(g3_wpe<WM * WN>, g3_wpe<WM * WN>)))
void tgemm3_kernel(GemvArgs a) {
    constexpr int NT = 64 * WM * WN;
    static_assert(NT >= 512, "at least two wavefronts per SIMD from one workgroup");
    constexpr int TM = 32, BM = TM * MS * WM, BN = TM * NS * WN;
    constexpr int RB = 128 * KB, KC = 4 * KB;
    constexpr int kSlice = BM * RB;
    constexpr int LW = g3_loaders<WM * WN, kSlice / 1024>();  // loading wavefronts
    constexpr int NA = kSlice / 1024 / LW;  // A chunks per lane per step (loading wavefronts)
    static_assert(NA * 1024 * LW == kSlice, "slice splits into whole 1 KB blocks per loading wavefront");
    constexpr int NB = NS * KB;           // weight uint4 loads per lane per step
    constexpr int TPB = 1024 / RB;
    extern __shared__ __align__(16) int8_t As[];  // [ST][kSlice]
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int wm = w % WM, wn = w / WM;
    const bool loader = __builtin_amdgcn_readfirstlane(w) < LW;
    const int l32 = lane & 31, g = lane >> 5;
    int tx, ty;
    g2_tile(tx, ty);
    const int m0 = ty * BM, n0 = tx * BN;
    const int kp = a.kp, M = a.m;
    const int nsteps = kp / RB;
    const int tok0 = m0 + wm * (TM * MS), row0 = n0 + wn * (TM * NS);
    bool fast = false;
    int mt0 = 0, ro0 = 0;
    float swm = 1.0f;
    Epi32Tok<MS> et{};
    if constexpr (OUT == kOutF32 || OUT == kOutF32Add || OUT == kOutI32) {
        int mt1, ro1;
        resolve_row<OUT>(a, row0, mt0, ro0);
        resolve_row<OUT>(a, row0 + NS * TM - 1, mt1, ro1);
        const int ldm = mt0 == 0 ? a.rows[0] : (mt0 == 1 ? a.rows[1] : a.rows[2]);
        swm = mt0 == 0 ? a.sw[0] : (mt0 == 1 ? a.sw[1] : a.sw[2]);
        fast = tok0 + MS * TM <= M && row0 + NS * TM <= a.total_rows && mt0 == mt1 && (long)M * ldm < (1L << 30);
        if (fast) epi32_pre<OUT, MS>(a, tok0, swm, et, false);
    } else if constexpr (OUT == kOutQKV) {
        int mt1, ro1;
        resolve_row<OUT>(a, row0, mt0, ro0);
        resolve_row<OUT>(a, row0 + NS * TM - 1, mt1, ro1);
        swm = mt0 == 0 ? a.sw[0] : (mt0 == 1 ? a.sw[1] : a.sw[2]);
        fast = tok0 + MS * TM <= M && row0 + NS * TM <= a.total_rows && mt0 == mt1;
        if (fast) epi32_pre<OUT, MS>(a, tok0, swm, et, false);
    }
    const uint4* brow[NS];
#pragma unroll
    for (int s = 0; s < NS; s++) {
        const int vr = row0 + s * TM + l32;
        int mat, r;
        resolve_row<OUT>(a, vr < a.total_rows ? vr : 0, mat, r);
        brow[s] = (const uint4*)(sel3(a.w, mat) + (size_t)r * (size_t)(kp >> 2)) + g;
    }
    const int8_t* asrc[NA];
    int adst[NA];
#pragma unroll
    for (int j = 0; j < NA; j++) {
        const int blk = (loader ? w : 0) * NA + j;
        const int T = blk * TPB + lane / (RB / 16), cs = lane % (RB / 16);
        const int c = cs ^ g2_swz<KB>(T);
        const int tok = m0 + T < M ? m0 + T : M - 1;  // past M: any valid row, never stored
        asrc[j] = a.q + (size_t)tok * kp + c * 16;
        adst[j] = blk * 1024;
    }
    auto a_issue = [&](int p, int stage) {
        if (!loader) return;
        int8_t* dst = As + stage * kSlice;
#pragma unroll
        for (int j = 0; j < NA; j++)
            __builtin_amdgcn_global_load_lds((const void*)(asrc[j] + p * RB), (lds_void_t*)(dst + adst[j]), 16, 0, 0);
    };
    // untracked weight loads (inline asm), covered by the explicit waits
    u32x4 bw[ST][NB];
    auto b_issue = [&](int p, u32x4 (&dst)[NB]) {
#pragma unroll
        for (int s = 0; s < NS; s++)
#pragma unroll
            for (int b = 0; b < KB; b++)
                asm volatile("global_load_dwordx4 %0, %1, off"
                             : "=v"(dst[s * KB + b])
                             : "v"(brow[s] + 2 * (KB * p + b))
                             : "memory");
    };
    auto pin = [](u32x4& v) { asm volatile("" : "+v"(v)); };
    auto wait_vm = [](auto n_c) {
        constexpr int n = decltype(n_c)::value;
        __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4) | (0 << 8));
    };
    v16i acc[MS][NS];
#pragma unroll
    for (int ms = 0; ms < MS; ms++)
#pragma unroll
        for (int s = 0; s < NS; s++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[ms][s][r] = 0;
    const int arow = (wm * (TM * MS) + l32) * RB;
    int axo[KC];
#pragma unroll
    for (int kc = 0; kc < KC; kc++) axo[kc] = ((2 * kc + g) ^ g2_swz<KB>(l32)) << 4;

const int plast = nsteps - 1;
#pragma unroll
    for (int p = 0; p < ST - 1; p++) {
        const int pi = p < plast ? p : plast;
        a_issue(pi, p);
        b_issue(pi, bw[p]);
    }
    if constexpr (OUT == kOutF32 || OUT == kOutF32Add || OUT == kOutI32 || OUT == kOutQKV)
        if (fast) epi32_pre<OUT, MS>(a, tok0, swm, et, true);

    // Step p: slice p and weights p landed (own loads), barrier (every
    // wavefront's chunks of slice p; every wavefront done with slice p - 1),
    // slice and weights p + ST - 1 into the slots of p - 1, then the MFMAs of
    // slice p with each chunk's A operands read one chunk ahead.
    auto step = [&](int p, auto slot_c) {
        constexpr int slot = decltype(slot_c)::value;
        constexpr int nslot = (slot + ST - 1) % ST;
        if (loader)
            wait_vm(std::integral_constant<int, (ST - 2) * (NA + NB)>{});
        else
            wait_vm(std::integral_constant<int, (ST - 2) * NB>{});
#pragma unroll
        for (int i = 0; i < NB; i++) pin(bw[slot][i]);
        __builtin_amdgcn_s_barrier();
        const int pn = p + ST - 1 < plast ? p + ST - 1 : plast;
        a_issue(pn, nslot);
        const int8_t* Ab = As + slot * kSlice + arow;
        v4i aop[2][MS];
#pragma unroll
        for (int ms = 0; ms < MS; ms++) aop[0][ms] = *(const v4i*)(Ab + axo[0] + ms * TM * RB);
#pragma unroll
        for (int kc = 0; kc < KC; kc++) {
            if (kc + 1 < KC) {
#pragma unroll
                for (int ms = 0; ms < MS; ms++)
                    aop[(kc + 1) & 1][ms] = *(const v4i*)(Ab + axo[kc + 1] + ms * TM * RB);
            }
            const int sh = 2 * (kc & 3), b = kc >> 2;
#pragma unroll
            for (int s = 0; s < NS; s++) {
                const u32x4 v = bw[slot][s * KB + b];
                const v4i bop = v4i{(int)((v.x >> sh) & 0x03030303u), (int)((v.y >> sh) & 0x03030303u),
                                    (int)((v.z >> sh) & 0x03030303u), (int)((v.w >> sh) & 0x03030303u)};
#pragma unroll
                for (int ms = 0; ms < MS; ms++)
                    acc[ms][s] = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop[kc & 1][ms], bop, acc[ms][s], 0, 0, 0);
            }
        }
        b_issue(pn, bw[nslot]);
    };
    for (int p = 0; p < nsteps; p += ST)
        seq_while(std::make_integer_sequence<int, ST>{}, [&](auto ic) {
            constexpr int i = decltype(ic)::value;
            if (p + i >= nsteps) return false;
            step(p + i, std::integral_constant<int, i>{});
            return true;
        });

    __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
    for (int k = 0; k < ST; k++)
#pragma unroll
        for (int i = 0; i < NB; i++) asm volatile("" ::"v"(bw[k][i]));
    if constexpr (OUT == kOutF32 || OUT == kOutF32Add || OUT == kOutI32) {
        if (fast) {
            epi32_full<OUT, MS, NS>(a, acc, tok0, mt0, ro0, et);
            return;
        }
    } else if constexpr (OUT == kOutQKV) {
        if (fast) {
            epi32_qkv<MS, NS>(a, acc, tok0, row0, et);
            return;
        }
    }
    // the general epilogue in blocks of at most two token tiles (its
    // per-token tables for four would not fit beside the accumulators)
    constexpr int EH = MS > 2 ? 2 : MS;
#pragma unroll
    for (int h = 0; h < MS; h += EH) {
        v16i part[EH][NS];
#pragma unroll
        for (int i = 0; i < EH; i++)
#pragma unroll
            for (int s = 0; s < NS; s++) part[i][s] = acc[h + i][s];
        mfma_epilogue<OUT, TM>(a, part, tok0 + h * TM, row0);
    }
}

namespace {

template <int MS, int NS, int KB, int ST = kG2Stages>
hipError_t launch_tiles2(const GemvArgs& a, int out_mode, dim3 grid, hipStream_t s, hipEvent_t e0, hipEvent_t e1) {
    constexpr size_t lds = (size_t)ST * (64 * MS) * (128 * KB);
    static bool attr = false;
    if (!attr) {
        const void* fns[] = {(const void*)tgemm2_kernel<kOutI32, MS, NS, KB, ST>, (const void*)tgemm2_kernel<kOutF32, MS, NS, KB, ST>,
                             (const void*)tgemm2_kernel<kOutF32Add, MS, NS, KB, ST>,
                             (const void*)tgemm2_kernel<kOutRelu2, MS, NS, KB, ST>,
                             (const void*)tgemm2_kernel<kOutQKV, MS, NS, KB, ST>};
        for (const void* f : fns) (void)hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        (void)hipGetLastError();
        attr = true;
    }
    switch (out_mode) {
        case kOutI32: hipExtLaunchKernelGGL((tgemm2_kernel<kOutI32, MS, NS, KB, ST>), grid, dim3(kThreads), lds, s, e0, e1, 0, a); break;
        case kOutF32: hipExtLaunchKernelGGL((tgemm2_kernel<kOutF32, MS, NS, KB, ST>), grid, dim3(kThreads), lds, s, e0, e1, 0, a); break;
        case kOutF32Add: hipExtLaunchKernelGGL((tgemm2_kernel<kOutF32Add, MS, NS, KB, ST>), grid, dim3(kThreads), lds, s, e0, e1, 0, a); break;
        case kOutRelu2: hipExtLaunchKernelGGL((tgemm2_kernel<kOutRelu2, MS, NS, KB, ST>), grid, dim3(kThreads), lds, s, e0, e1, 0, a); break;
        default: hipExtLaunchKernelGGL((tgemm2_kernel<kOutQKV, MS, NS, KB, ST>), grid, dim3(kThreads), lds, s, e0, e1, 0, a); break;
    }
    return hipGetLastError();
}


template <int WM, int WN, int MS, int NS, int KB, int ST>
hipError_t launch_tiles3(const GemvArgs& a, int out_mode, dim3 grid, hipStream_t s, hipEvent_t e0, hipEvent_t e1) {
    constexpr int NT = 64 * WM * WN;
    constexpr size_t lds = (size_t)ST * (32 * MS * WM) * (128 * KB);
    static bool attr = false;
    if (!attr) {
        const void* fns[] = {(const void*)tgemm3_kernel<kOutI32, WM, WN, MS, NS, KB, ST>,
                             (const void*)tgemm3_kernel<kOutF32, WM, WN, MS, NS, KB, ST>,
                             (const void*)tgemm3_kernel<kOutF32Add, WM, WN, MS, NS, KB, ST>,
                             (const void*)tgemm3_kernel<kOutRelu2, WM, WN, MS, NS, KB, ST>,
                             (const void*)tgemm3_kernel<kOutQKV, WM, WN, MS, NS, KB, ST>};
        for (const void* f : fns) (void)hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        (void)hipGetLastError();
        attr = true;
    }
    switch (out_mode) {
        case kOutI32: hipExtLaunchKernelGGL((tgemm3_kernel<kOutI32, WM, WN, MS, NS, KB, ST>), grid, dim3(NT), lds, s, e0, e1, 0, a); break;
        case kOutF32: hipExtLaunchKernelGGL((tgemm3_kernel<kOutF32, WM, WN, MS, NS, KB, ST>), grid, dim3(NT), lds, s, e0, e1, 0, a); break;
        case kOutF32Add: hipExtLaunchKernelGGL((tgemm3_kernel<kOutF32Add, WM, WN, MS, NS, KB, ST>), grid, dim3(NT), lds, s, e0, e1, 0, a); break;
        case kOutRelu2: hipExtLaunchKernelGGL((tgemm3_kernel<kOutRelu2, WM, WN, MS, NS, KB, ST>), grid, dim3(NT), lds, s, e0, e1, 0, a); break;
        default: hipExtLaunchKernelGGL((tgemm3_kernel<kOutQKV, WM, WN, MS, NS, KB, ST>), grid, dim3(NT), lds, s, e0, e1, 0, a); break;
    }
    return hipGetLastError();
}

template <int MS, int NS, bool PF>
hipError_t launch_small_pf(const GemvArgs& a, int out_mode, dim3 grid, hipStream_t s, hipEvent_t e0, hipEvent_t e1) {
    switch (out_mode) {
        case kOutI32: hipExtLaunchKernelGGL((tgemm_small_kernel<kOutI32, MS, NS, PF>), grid, dim3(kThreads), 0, s, e0, e1, 0, a); break;
        case kOutF32: hipExtLaunchKernelGGL((tgemm_small_kernel<kOutF32, MS, NS, PF>), grid, dim3(kThreads), 0, s, e0, e1, 0, a); break;
        case kOutF32Add: hipExtLaunchKernelGGL((tgemm_small_kernel<kOutF32Add, MS, NS, PF>), grid, dim3(kThreads), 0, s, e0, e1, 0, a); break;
        case kOutRelu2: hipExtLaunchKernelGGL((tgemm_small_kernel<kOutRelu2, MS, NS, PF>), grid, dim3(kThreads), 0, s, e0, e1, 0, a); break;
        default: hipExtLaunchKernelGGL((tgemm_small_kernel<kOutQKV, MS, NS, PF>), grid, dim3(kThreads), 0, s, e0, e1, 0, a); break;
    }
    return hipGetLastError();
}

template <int MS, int NS>
hipError_t launch_small(const GemvArgs& a, int out_mode, bool pf, dim3 grid, hipStream_t s, hipEvent_t e0,
                        hipEvent_t e1) {
    // 16-token tiles: the epilogue's per-token loads go out with the weight
    // stream (measured +1.5-2% at B = 8..64)
    if constexpr (MS == 1) {
        if (pf) return launch_small_pf<MS, NS, true>(a, out_mode, grid, s, e0, e1);
    }
    return launch_small_pf<MS, NS, false>(a, out_mode, grid, s, e0, e1);
}

}  // namespace

// Grow-only per-context scratch for quantized activations.
int qws_reserve(lbt_ctx* ctx, size_t bytes, void** out) {
    if (bytes > ctx->qws_bytes) {
        if (ctx->qws) {
            (void)hipStreamSynchronize(ctx->stream);
            (void)hipFree(ctx->qws);
            ctx->qws = nullptr;
            ctx->qws_bytes = 0;
        }
        LBT_HIP(ctx, hipMalloc(&ctx->qws, bytes));
        ctx->qws_bytes = bytes;
    }
    *out = ctx->qws;
    return LBT_OK;
}

namespace {
constexpr int kKsplitTiles = 1024;  // tile counters of the split-k scratch
constexpr int kKsplitMax = 3;        // k ranges per tile
constexpr int kKsplitMinSteps = 16;  // 128-k steps per range
// The split-k scratch, allocated once per context at this size and never
// moved (a captured graph may hold its address): the counters and the
// partial tiles of up to 512 workgroups of 128 x 128 tiles, what the
// automatic split asks for at most (two workgroups per CU).
constexpr size_t kKsplitBytes = (size_t)kKsplitTiles * 4 + (size_t)512 * 16384 * 4;

// k ranges for a pipelined-GEMM grid of `tiles` workgroups of `tile_ints`
// int32 accumulators over nk steps: as many as the two workgroup slots of
// every CU hold, at most kKsplitMax and at least kKsplitMinSteps steps each
// (the partials' hand-off costs ~2-3 us, so only long k pays: 2560 x 6912
// at M = 128 14.0 -> 10.6 us with 3 ranges, at M = 256 14.6 -> 12.6 us;
// 6912 x 2560 at M = 128, 20 steps, 8.4 -> 10.2 us with 2, so 1 there;
// wavefront groups splitting k inside a workgroup were no faster), and no
// more than the scratch holds; 1 where the call brings its own scratch (the
// allocation-free entry point), or the scratch is not there yet and a stream
// capture is under way or the allocation fails (the split is only a
// speed-up).  Sets a.ksplit / kcnt / kpart.
void pick_ksplit(lbt_ctx* ctx, const TernaryOp& op, GemvArgs& a, long tiles, int tile_ints, int nk) {
    a.ksplit = 1;
    if (op.scratch || tiles > kKsplitTiles) return;
    int ks = ctx->tune.gemm_ksplit;
    if (ks == 0) {
        const long fill = 2L * ctx->cus / tiles;
        ks = (int)(fill < kKsplitMax ? fill : kKsplitMax);
        if (ks > nk / kKsplitMinSteps) ks = nk / kKsplitMinSteps;
    }
    if (ks > nk) ks = nk;
    while (ks > 1 && (size_t)kKsplitTiles * 4 + (size_t)tiles * ks * tile_ints * 4 > kKsplitBytes) ks--;
    if (ks < 2) return;
    if (!ctx->kws) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(ctx->stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return;
        void* p = nullptr;
        if (hipMalloc(&p, kKsplitBytes) != hipSuccess) {
            (void)hipGetLastError();
            return;
        }
        if (hipMemsetAsync(p, 0, (size_t)kKsplitTiles * 4, ctx->stream) != hipSuccess) {
            (void)hipGetLastError();
            (void)hipFree(p);
            return;
        }
        ctx->kws = p;
    }
    a.ksplit = ks;
    a.kcnt = (int*)ctx->kws;
    a.kpart = (int*)ctx->kws + kKsplitTiles;
}
}  // namespace

int act_scratch(lbt_ctx* ctx, const TernaryOp& op, size_t bytes, void** out) {
    if (!op.scratch) return qws_reserve(ctx, bytes, out);
    if (bytes > op.scratch_bytes) return set_err(ctx, LBT_E_INVALID, "ternary: activations exceed the given scratch");
    *out = op.scratch;
    return LBT_OK;
}

int launch_ternary_mfma(lbt_ctx* ctx, const TernaryOp& op_in) {
    TernaryOp op = op_in;
    if (op.in_mode == kInF32) {
        // RMSNorm + ActQuant once per token row (the same arithmetic as the
        // GEMV prologue), then the GEMM reads int8 activations.
        const size_t kp = padded_cols((size_t)op.cols);
        void* q;
        const size_t qb = ((size_t)op.m * kp + 255) & ~(size_t)255;
        int rc = act_scratch(ctx, op, qb + (size_t)op.m * 8, &q);
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
    hipEvent_t e0, e1;
    prof_pair(ctx, &e0, &e1);
    hipError_t e;
    // path (LBT_GEMM_MODE forces one, for tests and measurements): 6 = the
    // few-token kernel, 4 / 5 = 64 / 128 tiles of the pipelined GEMM, 7 / 8 =
    // the 128 x 256 / 64 x 320 tiles of one workgroup per CU; by default the
    // few-token kernel up to tune.small_max tokens, then the one-workgroup-
    // per-CU tiles as picked below, else 128 x 128 tiles when there are
    // >= 200, else 64 x 64
    const LbtTuning& tu = ctx->tune;
    const int gmode = tu.gemm_mode;
    const long t128 = (long)((total + 127) / 128) * ((op.m + 127) / 128);
    const dim3 g128((unsigned)((total + 127) / 128), (unsigned)((op.m + 127) / 128));
    const dim3 g64((unsigned)((total + 63) / 64), (unsigned)((op.m + 63) / 64));
    // the 8-wavefront kernel: 128 x 256 tiles (two wavefronts of 4 MFMA
    // tiles per SIMD) or 64 x 320 tiles from 10 wavefronts (at most three of
    // 2 tiles per SIMD), whichever needs fewer rounds x MFMA tiles per SIMD
    // over the 256 CUs; only where the chosen one has >= kG3MinTiles tiles
    const dim3 g3((unsigned)((total + 255) / 256), (unsigned)((op.m + 127) / 128));
    const dim3 g3n((unsigned)((total + 319) / 320), (unsigned)((op.m + 63) / 64));
    const long t3 = (long)g3.x * g3.y, t3n = (long)g3n.x * g3n.y;
    // MFMA tiles per SIMD on the busiest CU: 8 per round of 128 x 256, 6 per
    // round of 64 x 320, 4 per 128 x 128 tile of tgemm2_kernel (one wavefront
    // of 2 x 2 per SIMD, two workgroups per CU), 1 per 64 x 64 tile; ties go
    // to the one-workgroup-per-CU kernel
    const long c3 = (t3 + 255) / 256 * 8, c3n = (t3n + 255) / 256 * 6;
    const long c2 = t128 >= 200 ? (t128 + 255) / 256 * 4 : ((long)g64.x * g64.y + 255) / 256;
    int g3pick = c3n < c3 ? (t3n >= kG3MinTiles ? 2 : 0) : (t3 >= kG3MinTiles ? 1 : 0);
    if (g3pick != 0 && (g3pick == 2 ? c3n : c3) > c2) g3pick = 0;
    const bool small_ok = a.kp <= 256 * 4 * kSmallMaxSteps;
    // up to 64 tokens the few-token kernel also serves the shapes the 64 x 64
    // tiling would give fewer than tune.small_tiles tiles (q/k/v, o, down of
    // the 2B model at B = 33..64)
    const long t64 = (long)((total + 63) / 64) * ((op.m + 63) / 64);
    const bool few_tiles = op.m <= 64 && t64 < tu.small_tiles;
    if (small_ok && (gmode == 6 || (gmode == 0 && (op.m <= tu.small_max || few_tiles)))) {
        // 16-token tiles (more workgroups) measured faster than 32..64-token
        // ones at every batch served here; tune.small_ms = 2..4 allows the
        // wider tiles
        int ms = op.m <= 16 ? 1 : op.m <= 32 ? 2 : op.m <= 48 ? 3 : 4;
        if (ms > tu.small_ms) ms = tu.small_ms;
        // 32-row tiles (half the activation and weight re-reads) where they
        // still give >= kSmallWideGroups workgroups over all token tiles
        // (measured at 2B, 64 tokens: q/k/v 9.4 -> 7.6 us, o 8.1 -> 7.4,
        // down 14.2 -> 12.0; 16 tokens keep 16-row tiles there);
        // tune.small_ns = 1 / 2 forces
        const long tt = (op.m + 16 * ms - 1) / (16 * ms);
        const int ns = tu.small_ns ? (tu.small_ns == 2 ? 2 : 1)
                                   : ((long)((total + 31) / 32) * tt >= kSmallWideGroups ? 2 : 1);
        const dim3 g((unsigned)((total + 16 * ns - 1) / (16 * ns)), (unsigned)((op.m + 16 * ms - 1) / (16 * ms)));
        const bool pf = tu.small_pf;
        if (ns == 2)
            e = ms == 1   ? launch_small<1, 2>(a, op.out_mode, pf, g, ctx->stream, e0, e1)
                : ms == 2 ? launch_small<2, 2>(a, op.out_mode, pf, g, ctx->stream, e0, e1)
                : ms == 3 ? launch_small<3, 2>(a, op.out_mode, pf, g, ctx->stream, e0, e1)
                          : launch_small<4, 2>(a, op.out_mode, pf, g, ctx->stream, e0, e1);
        else
            e = ms == 1   ? launch_small<1, 1>(a, op.out_mode, pf, g, ctx->stream, e0, e1)
                : ms == 2 ? launch_small<2, 1>(a, op.out_mode, pf, g, ctx->stream, e0, e1)
                : ms == 3 ? launch_small<3, 1>(a, op.out_mode, pf, g, ctx->stream, e0, e1)
                          : launch_small<4, 1>(a, op.out_mode, pf, g, ctx->stream, e0, e1);
    } else if (gmode == 7 || gmode == 8 || (gmode == 0 && g3pick != 0)) {
        if (gmode == 8 || (gmode == 0 && g3pick == 2))
            e = launch_tiles3<1, 10, 2, 1, 1, kG3Stages>(a, op.out_mode, g3n, ctx->stream, e0, e1);
        else
            e = launch_tiles3<1, 8, 4, 1, 1, kG3Stages>(a, op.out_mode, g3, ctx->stream, e0, e1);
    } else if (gmode != 4 && (t128 >= 200 || gmode == 5)) {
        // grids that leave workgroup slots idle split k (gridDim.z ranges)
        dim3 g = g128;
        pick_ksplit(ctx, op, a, t128, 4 * 4 * 1024, a.kp / 128);
        g.z = (unsigned)a.ksplit;
        e = launch_tiles2<2, 2, 1>(a, op.out_mode, g, ctx->stream, e0, e1);
    } else {
        dim3 g = g64;
        pick_ksplit(ctx, op, a, (long)g64.x * g64.y, 4 * 1024, a.kp / 128);
        g.z = (unsigned)a.ksplit;
        e = launch_tiles2<1, 1, 1>(a, op.out_mode, g, ctx->stream, e0, e1);
    }
    if (e != hipSuccess) return hip_err(ctx, e, "ternary GEMM launch");
    prof_commit(ctx, e0, e1, kProfGemm, 2.0 * op.m * (double)total * a.kp);
    return LBT_OK;
}

}  // namespace lbt
