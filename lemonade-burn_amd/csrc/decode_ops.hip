// decode_ops.hip -- the non-GEMM pieces of the BitNet b1.58 step on gfx950:
// token embedding, RoPE + bf16 KV append, GQA attention over the bf16 cache,
// the tied bf16 LM head with fused final RMSNorm and device argmax, and the
// synthetic-weight generator.
//
// Reference: crates/lb-model/src/model.rs (embed :274-282, rope :284-301,
// KV cache :340-347, GQA attention :349-357, final norm + head :368-373),
// crates/lb-ternary/src/bf16.rs (bf16_gemv :14-25), sample.rs:17-25 (argmax).
// Float order follows lbt_device.h; the oracle mirrors it.
#include <hip/hip_runtime.h>


#include "lbt_device.h"
#include "lbt_internal.h"
#include "attn_common.h"

#include <stdlib.h>

namespace lbt {

// ---------------------------------------------------------------------------
// embedding (model.rs:274-282).  Token ids come from `tokens`, or, when it is
// null, from the argmax key of the previous step (device-side feedback).  The
// key is cleared for the next LM head.
__global__ __launch_bounds__(kThreads) void embed_kernel(const uint16_t* embed, int hidden, int vocab,
                                                         const uint32_t* tokens, unsigned long long* key,
                                                         uint32_t* tok_out, float* x, int* state) {
    __shared__ uint32_t tok_s;
    const int t = blockIdx.x;
    if (threadIdx.x == 0) {
        uint32_t tok = tokens ? tokens[t] : 0xffffffffu - (uint32_t)(key[t] & 0xffffffffull);
        // a key that was never written (no finite logit) must not index past the table
        if (tok >= (uint32_t)vocab) tok = 0;
        tok_s = tok;
        if (state) {  // graph-replayed decode step (one token): next position, next output slot
            state[0] += 1;
            tok_out[state[1]++] = tok;
        } else if (tok_out) {
            tok_out[t] = tok;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0 && key) key[t] = 0ull;
    const uint16_t* row = embed + (size_t)tok_s * hidden;
    float* dst = x + (size_t)t * hidden;
    for (int i = threadIdx.x; i < hidden; i += kThreads) dst[i] = bf16_to_f32(row[i]);
}

// ---------------------------------------------------------------------------
// GQA attention splits, one workgroup per (query head, key split, query
// row); see attn_common.h.  Grid (nh * splits, m); splits past a row's
// last one exit at once.
template <int LK>
__global__ __launch_bounds__(kThreads) void attention_kernel(const float* q, int nh, int kvh, RowPos rp,
                                                             const uint16_t* kc, const uint16_t* vc, int cap,
                                                             float scaling, float* o, float* ml) {
    extern __shared__ float sc[];  // [attn_split_keys(visible keys)]
    __shared__ AttnShared<LK> sh;
    const int nsg = (int)gridDim.x / nh;  // splits in the grid (the most any row has)
    const int h = blockIdx.x / nsg, s = blockIdx.x % nsg, t = blockIdx.y;
    const int H = nh * LK * 8, g = h / (nh / kvh);
    const size_t kvoff = row_cache_offset(rp, t) + (size_t)g * cap * LK * 8;
    float* ot = o + (size_t)t * kAttnSplits * H;
    float* mlt = ml + (size_t)t * kAttnSplits * nh * 2;
    constexpr bool kGuess = 4 * (kThreads / LK) >= kAttnMinKeys;  // one key pass covers a guessed split
    if (kGuess && (rp.tok_pos || rp.pos_dev))  // the position is read after the first K/V loads
        attention_split_ku<LK, 4, kGuess>(q + (size_t)t * H, h, nh, s, rp.tok_pos ? 0 : t, kc + kvoff, vc + kvoff,
                                        scaling, ot, mlt, sc, sh, rp.tok_pos ? rp.tok_pos + t : rp.pos_dev, cap);
    else  // the row's position (a graph-replayed step reads it from the device)
        attention_split<LK>(q + (size_t)t * H, h, nh, s, row_position(rp, t), kc + kvoff, vc + kvoff, scaling, ot,
                            mlt, sc, sh);
}

// One wavefront per (query row, KV head, key split), four per workgroup:
// attention_split_wave, the grouped kernel's partials bit for bit without a
// barrier.  Task i = blockIdx.x * 4 + wavefront is (row, KV head, split)
// with the row fastest: neighbouring wavefronts read the same split's K/V
// rows, from L1 / L2 (measured against the split fastest: 2048-token
// prefill attention 22.1 -> 18.6-19.4 ms; nontemporal K/V loads were slower,
// 28.8 ms, and so was giving each XCD a contiguous eighth of the tasks,
// 21.5 ms).  nsg splits per (row, KV head) in the grid (the most any row
// has); scw floats of LDS scores per wavefront.
template <int LK, int GH>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) void attention_wave_kernel(const float* q, int nh, int kvh, RowPos rp,
                                                                  const uint16_t* kc, const uint16_t* vc, int cap,
                                                                  float scaling, float* o, float* ml, int m, int nsg,
                                                                  int scw) {
    extern __shared__ __align__(16) float sc[];  // [4][scw]
    // uniform per wavefront, and known to be: the task's row, KV head and
    // split then sit in scalar registers, and so do the K / V buffer
    // descriptors built from them (a descriptor the compiler cannot prove
    // uniform turns every buffer load into a waterfall loop)
    const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const long i = (long)blockIdx.x * 4 + w;
    if (i >= (long)m * kvh * nsg) return;  // the last workgroup's spare wavefronts
    const int t = (int)(i % m);
    const long r = i / m;
    const int g = (int)(r % kvh), s = (int)(r / kvh);
    const int H = nh * LK * 8;
    const size_t kvoff = row_cache_offset(rp, t) + (size_t)g * cap * LK * 8;
    attention_split_wave<LK, GH>(q + (size_t)t * H, g, nh, s, row_position(rp, t), kc + kvoff, vc + kvoff, scaling,
                                 o + (size_t)t * kAttnSplits * H, ml + (size_t)t * kAttnSplits * nh * 2, sc + w * scw);
}

// The same splits with one workgroup per (KV head, key split, query row)
// taking all GH query heads of the KV head.  Grid (kvh * splits, m).
// wide: eight key passes in flight per split of more than 64 keys (grids of
// many workgroups, where occupancy is not the limit); same partials.
template <int LK, int GH, bool WIDE>
__global__ __launch_bounds__(kThreads) void attention_group_kernel(const float* q, int nh, int kvh, RowPos rp,
                                                                   const uint16_t* kc, const uint16_t* vc, int cap,
                                                                   float scaling, float* o, float* ml) {
    extern __shared__ __align__(16) float sc[];  // [attn_group_score_keys(split keys)][GH]
    __shared__ AttnGroupShared<LK, GH> sh;
    const int nsg = (int)gridDim.x / kvh;  // splits in the grid (the most any row has)
    const int g = blockIdx.x / nsg, s = blockIdx.x % nsg, t = blockIdx.y;
    const int H = nh * LK * 8;
    const size_t kvoff = row_cache_offset(rp, t) + (size_t)g * cap * LK * 8;
    const int p = row_position(rp, t);
    // the eight-pass path is its own instantiation: its register buffers
    // would otherwise set the occupancy of the narrower paths too
    if (attn_split_keys(p + 1) <= 2 * (kThreads / LK))
        attention_split_group<LK, GH, 2>(q + (size_t)t * H, g, nh, s, p, kc + kvoff, vc + kvoff, scaling,
                                         o + (size_t)t * kAttnSplits * H, ml + (size_t)t * kAttnSplits * nh * 2, sc,
                                         sh);
    else if (!WIDE || attn_split_keys(p + 1) <= 4 * (kThreads / LK))
        attention_split_group<LK, GH, 4>(q + (size_t)t * H, g, nh, s, p, kc + kvoff, vc + kvoff, scaling,
                                         o + (size_t)t * kAttnSplits * H, ml + (size_t)t * kAttnSplits * nh * 2, sc,
                                         sh);
    else
        attention_split_group<LK, GH, 8>(q + (size_t)t * H, g, nh, s, p, kc + kvoff, vc + kvoff, scaling,
                                         o + (size_t)t * kAttnSplits * H, ml + (size_t)t * kAttnSplits * nh * 2, sc,
                                         sh);
}

// Combine of the attention splits of row blockIdx.x into out (attn_common.h).
template <int EPT>
__global__ __launch_bounds__(kThreads) void attn_combine_kernel(const float* o, const float* ml, int nh, int hd,
                                                                RowPos rp, float* out) {
    __shared__ AttnTab tab;
    const int t = blockIdx.x, H = nh * hd;
    AttnRow a{o + (size_t)t * kAttnSplits * H, ml + (size_t)t * kAttnSplits * nh * 2, 0, nh, hd, H};
    RowRegs<EPT> r;
    AttnRegs<EPT, 4> ar;
    attn_row_issue(a, nullptr, ar, r);
    a.ns = attn_splits(row_position(rp, t) + 1);
    attn_row_finish(a, ar, r, tab);
    float* dst = out + (size_t)t * H;
#pragma unroll
    for (int g = 0; g < EPT / 4; g++) {
        const int i0 = 1024 * g + 4 * (int)threadIdx.x;
        if (i0 < H) *(float4*)(dst + i0) = make_float4(r.v[4 * g], r.v[4 * g + 1], r.v[4 * g + 2], r.v[4 * g + 3]);
    }
}

// ---------------------------------------------------------------------------
// bf16 GEMV / tied LM head (bf16.rs:14-25, model.rs:369-373) with the final
// RMSNorm fused as a prologue.  One wavefront per output row; lane l takes
// the 16-byte chunks l, l+64, ... (8 bf16 each), fused multiply-adds in
// element order, then an xor butterfly.  The first-max key of each row t is
// atomically maxed into key[t] (argmax, sample.rs:17-25).
__device__ __forceinline__ float bf_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }

// acc += sum over e of bf16(w[e]) * x[e] for the 8 bf16 of one 16-byte chunk, in order.
__device__ __forceinline__ float dot8(uint4 wv, const float* x, float acc) {
    const float4 x0 = *(const float4*)x;
    const float4 x1 = *(const float4*)(x + 4);
    acc = __builtin_fmaf(bf_lo(wv.x), x0.x, acc);
    acc = __builtin_fmaf(bf_hi(wv.x), x0.y, acc);
    acc = __builtin_fmaf(bf_lo(wv.y), x0.z, acc);
    acc = __builtin_fmaf(bf_hi(wv.y), x0.w, acc);
    acc = __builtin_fmaf(bf_lo(wv.z), x1.x, acc);
    acc = __builtin_fmaf(bf_hi(wv.z), x1.y, acc);
    acc = __builtin_fmaf(bf_lo(wv.w), x1.z, acc);
    acc = __builtin_fmaf(bf_hi(wv.w), x1.w, acc);
    return acc;
}

// Signed byte k (0..3) of v as f32 (int8 head weights).
__device__ __forceinline__ float i8_at(uint32_t v, int k) { return (float)((int32_t)(v << (24 - 8 * k)) >> 24); }

// acc += sum over e of q[e] * x[e] for the 8 int8 of one 8-byte chunk, in order.
__device__ __forceinline__ float dot8_i8(uint2 wv, const float* x, float acc) {
    const float4 x0 = *(const float4*)x;
    const float4 x1 = *(const float4*)(x + 4);
    acc = __builtin_fmaf(i8_at(wv.x, 0), x0.x, acc);
    acc = __builtin_fmaf(i8_at(wv.x, 1), x0.y, acc);
    acc = __builtin_fmaf(i8_at(wv.x, 2), x0.z, acc);
    acc = __builtin_fmaf(i8_at(wv.x, 3), x0.w, acc);
    acc = __builtin_fmaf(i8_at(wv.y, 0), x1.x, acc);
    acc = __builtin_fmaf(i8_at(wv.y, 1), x1.y, acc);
    acc = __builtin_fmaf(i8_at(wv.y, 2), x1.z, acc);
    acc = __builtin_fmaf(i8_at(wv.y, 3), x1.w, acc);
    return acc;
}

__device__ __forceinline__ uint2 ld_stream8(const uint2* p) {
    const u32x2 v = __builtin_nontemporal_load((const LBT_GLOBAL u32x2*)p);
    return make_uint2(v.x, v.y);
}

constexpr int kLmChunks = 5;  // 16-byte chunks per lane per row (hidden <= 2560 on the fast path)

__global__ __launch_bounds__(kThreads) void lmhead_kernel(const uint16_t* W, int rows, int cols, const float* x,
                                                          const float* norm_w, float eps, float* logits,
                                                          unsigned long long* key) {
    extern __shared__ __align__(16) float xs[];  // cols
    __shared__ __align__(16) float red[kRedFloats];
    const int t = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
    const float* xr = x + (size_t)t * cols;
    if (cols <= 16 * kThreads) {
        float v[16];
        load_norm_row<16>(SrcF32{xr}, cols, norm_w, eps, v, red);
#pragma unroll
        for (int e = 0; e < 16; e++)
            if (tid < kThreads && row_elem(tid, e) < cols) xs[row_elem(tid, e)] = v[e];
    } else {
        const float rr = norm_factor_global(SrcF32{xr}, cols, norm_w, eps, red);
        for (int i = tid; i < cols; i += kThreads) xs[i] = norm_w ? (xr[i] * rr) * norm_w[i] : xr[i];
    }
    __syncthreads();
    const int nchunks = cols >> 3;
    const int gw = blockIdx.x * 4 + (tid >> 6), nw = gridDim.x * 4;
    unsigned long long best = 0ull;
    if (nchunks == 64 * kLmChunks) {
        // Row pairs (r, r + nw), r = gw + 2 nw p, with the next pair's loads in
        // flight while a pair computes (untracked loads, explicit waits; pairs
        // past the end load row 0 and are not used).  Same per-row order as
        // the loop below.
        constexpr int NL = 2 * kLmChunks;
        const int np = gw < rows ? (rows - gw + 2 * nw - 1) / (2 * nw) : 0;
        u32x4 A[2][kLmChunks], B[2][kLmChunks];
        auto issue = [&](int p, u32x4 (&a)[kLmChunks], u32x4 (&b)[kLmChunks]) {
            const int r0 = gw + 2 * nw * p, r1 = r0 + nw;
            const uint4* w0 = (const uint4*)(W + (size_t)(r0 < rows ? r0 : 0) * cols);
            const uint4* w1 = (const uint4*)(W + (size_t)(r1 < rows ? r1 : 0) * cols);
#pragma unroll
            for (int i = 0; i < kLmChunks; i++) {
                a[i] = ld_u4_async_nt(w0 + lane + 64 * i);
                b[i] = ld_u4_async_nt(w1 + lane + 64 * i);
            }
        };
        auto land = [&](u32x4 (&a)[kLmChunks], u32x4 (&b)[kLmChunks]) {
            vm_wait<NL>();  // all but the pair issued last
#pragma unroll
            for (int i = 0; i < kLmChunks; i++) {
                pin(a[i]);
                pin(b[i]);
            }
        };
        auto consume = [&](int p, u32x4 (&a)[kLmChunks], u32x4 (&b)[kLmChunks]) {
            const int r0 = gw + 2 * nw * p, r1 = r0 + nw;
            float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
            for (int i = 0; i < kLmChunks; i++) {
                const int c = lane + 64 * i;
                acc0 = dot8(make_uint4(a[i].x, a[i].y, a[i].z, a[i].w), xs + 8 * c, acc0);
                acc1 = dot8(make_uint4(b[i].x, b[i].y, b[i].z, b[i].w), xs + 8 * c, acc1);
            }
            acc0 = wave_sum(acc0);
            acc1 = wave_sum(acc1);
            if (lane == 0) {
                if (r0 < rows) {
                    if (logits) logits[(size_t)t * rows + r0] = acc0;
                    const unsigned long long k = argmax_key(acc0, (uint32_t)r0);
                    best = k > best ? k : best;
                }
                if (r1 < rows) {
                    if (logits) logits[(size_t)t * rows + r1] = acc1;
                    const unsigned long long k = argmax_key(acc1, (uint32_t)r1);
                    best = k > best ? k : best;
                }
            }
        };
        // loads, waits and pins are unconditional (no register copies of a
        // result still in flight); only the use of the last odd pair is not
        issue(0, A[0], B[0]);
        for (int p = 0; p < np; p += 2) {
            issue(p + 1, A[1], B[1]);
            land(A[0], B[0]);
            consume(p, A[0], B[0]);
            issue(p + 2, A[0], B[0]);
            land(A[1], B[1]);
            if (p + 1 < np) consume(p + 1, A[1], B[1]);
        }
        vm_wait<0>();
#pragma unroll
        for (int i = 0; i < kLmChunks; i++) {
            keep(A[0][i]);
            keep(B[0][i]);
            keep(A[1][i]);
            keep(B[1][i]);
        }
    } else if (nchunks <= 64 * kLmChunks) {
        // two rows per iteration, all their chunk loads in flight at once
        for (int r = gw; r < rows; r += 2 * nw) {
            const int r1 = r + nw;
            const bool has1 = r1 < rows;
            const uint4* w0 = (const uint4*)(W + (size_t)r * cols);
            const uint4* w1 = (const uint4*)(W + (size_t)(has1 ? r1 : r) * cols);
            uint4 a0[kLmChunks], a1[kLmChunks];
#pragma unroll
            for (int i = 0; i < kLmChunks; i++) {
                const int c = lane + 64 * i;
                a0[i] = c < nchunks ? ld_stream(w0 + c) : make_uint4(0, 0, 0, 0);
                a1[i] = (has1 && c < nchunks) ? ld_stream(w1 + c) : make_uint4(0, 0, 0, 0);
            }
            float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
            for (int i = 0; i < kLmChunks; i++) {
                const int c = lane + 64 * i;
                if (c < nchunks) {
                    acc0 = dot8(a0[i], xs + 8 * c, acc0);
                    acc1 = dot8(a1[i], xs + 8 * c, acc1);
                }
            }
            acc0 = wave_sum(acc0);
            acc1 = wave_sum(acc1);
            if (lane == 0) {
                if (logits) logits[(size_t)t * rows + r] = acc0;
                unsigned long long k = argmax_key(acc0, (uint32_t)r);
                best = k > best ? k : best;
                if (has1) {
                    if (logits) logits[(size_t)t * rows + r1] = acc1;
                    k = argmax_key(acc1, (uint32_t)r1);
                    best = k > best ? k : best;
                }
            }
        }
    } else {
        for (int r = gw; r < rows; r += nw) {
            const uint4* wr = (const uint4*)(W + (size_t)r * cols);
            float acc = 0.0f;
            for (int c = lane; c < nchunks; c += 64) acc = dot8(ld_stream(wr + c), xs + 8 * c, acc);
            acc = wave_sum(acc);
            if (lane == 0) {
                if (logits) logits[(size_t)t * rows + r] = acc;
                const unsigned long long k = argmax_key(acc, (uint32_t)r);
                best = k > best ? k : best;
            }
        }
    }
    // one atomic per workgroup: device-scope atomics on one word serialize,
    // one per wavefront (8192 of them) costed a third of the kernel
    __shared__ unsigned long long wbest[kThreads / 64];
    if (lane == 0) wbest[tid >> 6] = best;
    __syncthreads();
    if (key && tid == 0) {
        unsigned long long b = wbest[0];
#pragma unroll
        for (int i = 1; i < kThreads / 64; i++) b = wbest[i] > b ? wbest[i] : b;
        if (b) atomicMax(&key[t], b);
    }
}

// Final RMSNorm of row blockIdx.x into xn (the LM head prologue's
// arithmetic, written out once for the batched head below).
__global__ __launch_bounds__(kThreads) void row_norm_kernel(const float* x, int cols, const float* norm_w, float eps,
                                                            float* xn) {
    __shared__ __align__(16) float red[kRedFloats];
    const int t = blockIdx.x, tid = threadIdx.x;
    const float* xr = x + (size_t)t * cols;
    float* dst = xn + (size_t)t * cols;
    if (cols <= 16 * kThreads) {
        float v[16];
        load_norm_row<16>(SrcF32{xr}, cols, norm_w, eps, v, red);
#pragma unroll
        for (int e = 0; e < 16; e++)
            if (row_elem(tid, e) < cols) dst[row_elem(tid, e)] = v[e];
    } else {
        const float rr = norm_factor_global(SrcF32{xr}, cols, norm_w, eps, red);
        for (int i = tid; i < cols; i += kThreads) dst[i] = norm_w ? (xr[i] * rr) * norm_w[i] : xr[i];
    }
}

// ---------------------------------------------------------------------------
// Opt-in int8 LM head (crates/lb-ternary/src/q8head.rs).
//
// Q8Head::from_bf16 (q8head.rs:18-32), one workgroup per row (grid-strided):
// scale = amax / 127 (1.0 for an all-zero row; NaN ignored by the max),
// q = round_ties_even(w / scale) clamped to [-127, 127] (NaN -> 0), with the
// IEEE f32 division of the reference.
__global__ __launch_bounds__(kThreads) void q8_quantize_kernel(const uint16_t* w, int rows, int cols, int8_t* q,
                                                               float* scale) {
    __shared__ __align__(16) float red[kRedFloats];
    for (int r = blockIdx.x; r < rows; r += gridDim.x) {
        const uint16_t* wr = w + (size_t)r * cols;
        float am = 0.0f;
        for (int i = threadIdx.x; i < cols; i += kThreads) am = fmaxf(am, fabsf(bf16_to_f32(wr[i])));
        am = block_max(am, red);
        const float s = am == 0.0f ? 1.0f : am / 127.0f;
        for (int i = threadIdx.x; i < cols; i += kThreads) {
            const float y = __builtin_rintf(bf16_to_f32(wr[i]) / s);
            const float c = y != y ? 0.0f : fminf(fmaxf(y, -127.0f), 127.0f);
            q[(size_t)r * cols + i] = (int8_t)(int)c;
        }
        if (threadIdx.x == 0) scale[r] = s;
        __syncthreads();  // red is reused by the next row
    }
}

// Q8Head::gemv (q8head.rs:34-57) for token row blockIdx.y with the final
// RMSNorm fused as a prologue (as lmhead_kernel): logit[r] = scale[r] *
// sum_k q[r,k] * xn[k].  One wavefront per row, several rows in flight; lane l
// takes the 8-byte chunks l, l+64, ... with fused multiply-adds in element
// order, then the xor butterfly, then the scale.  The first-max key of the
// row's logits is maxed into key[t] (one atomic per workgroup).
__global__ __launch_bounds__(kThreads) void q8head_kernel(const int8_t* Q, const float* S, int rows, int cols,
                                                          const float* x, const float* norm_w, float eps,
                                                          float* logits, unsigned long long* key) {
    extern __shared__ __align__(16) float xs[];  // cols
    __shared__ __align__(16) float red[kRedFloats];
    const int t = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
    const float* xr = x + (size_t)t * cols;
    auto prologue = [&]() {
        if (cols <= 16 * kThreads) {
            float v[16];
            load_norm_row<16>(SrcF32{xr}, cols, norm_w, eps, v, red);
#pragma unroll
            for (int e = 0; e < 16; e++)
                if (tid < kThreads && row_elem(tid, e) < cols) xs[row_elem(tid, e)] = v[e];
        } else {
            const float rr = norm_factor_global(SrcF32{xr}, cols, norm_w, eps, red);
            for (int i = tid; i < cols; i += kThreads) xs[i] = norm_w ? (xr[i] * rr) * norm_w[i] : xr[i];
        }
        __syncthreads();
    };
    const int nchunks = cols >> 3;
    const int gw = blockIdx.x * 4 + (tid >> 6), nw = gridDim.x * 4;
    unsigned long long best = 0ull;
    auto emit = [&](int r, float acc) {
        acc = gload(S + r) * wave_sum(acc);
        if (lane == 0) {
            if (logits) logits[(size_t)t * rows + r] = acc;
            const unsigned long long k = argmax_key(acc, (uint32_t)r);
            best = k > best ? k : best;
        }
    };
    if (nchunks == 64 * kLmChunks) {
        // Groups of 2 rows r = gw + nw (2 p + j), j = 0, 1, with the next
        // group's loads (weights and the 2 row scales) in flight while a group
        // computes: untracked loads with explicit waits, unconditional (rows
        // past the end load row 0 and are not used); the first group is
        // issued before the prologue.  Same per-row order as the loop below.
        constexpr int G = 2, NL = G * kLmChunks + G;
        const int ng = gw < rows ? (rows - gw + G * nw - 1) / (G * nw) : 0;
        u32x2 A[2][G][kLmChunks];
        float SC[2][G];
        auto issue = [&](int p, u32x2 (&a)[G][kLmChunks], float (&sc)[G]) {
#pragma unroll
            for (int j = 0; j < G; j++) {
                const int r = gw + nw * (G * p + j), rr = r < rows ? r : 0;
                const int8_t* wr = Q + (size_t)rr * cols;
#pragma unroll
                for (int i = 0; i < kLmChunks; i++) a[j][i] = ld_u2_async_nt(wr + 8 * (lane + 64 * i));
                sc[j] = ld_f32_async(S + rr);
            }
        };
        auto land = [&](u32x2 (&a)[G][kLmChunks], float (&sc)[G]) {
            vm_wait<NL>();  // all but the group issued last
#pragma unroll
            for (int j = 0; j < G; j++) {
#pragma unroll
                for (int i = 0; i < kLmChunks; i++) pin(a[j][i]);
                pin(sc[j]);
            }
        };
        auto consume = [&](int p, u32x2 (&a)[G][kLmChunks], float (&sc)[G]) {
            float4 xv[kLmChunks][2];  // this lane's x chunks, read once for the G rows
#pragma unroll
            for (int i = 0; i < kLmChunks; i++) {
                xv[i][0] = *(const float4*)(xs + 8 * (lane + 64 * i));
                xv[i][1] = *(const float4*)(xs + 8 * (lane + 64 * i) + 4);
            }
#pragma unroll
            for (int j = 0; j < G; j++) {
                const int r = gw + nw * (G * p + j);
                float acc = 0.0f;
#pragma unroll
                for (int i = 0; i < kLmChunks; i++) {
                    const float xe[8] = {xv[i][0].x, xv[i][0].y, xv[i][0].z, xv[i][0].w,
                                         xv[i][1].x, xv[i][1].y, xv[i][1].z, xv[i][1].w};
#pragma unroll
                    for (int e = 0; e < 8; e++)
                        acc = __builtin_fmaf(i8_at(e < 4 ? a[j][i].x : a[j][i].y, e & 3), xe[e], acc);
                }
                acc = sc[j] * wave_sum(acc);
                if (lane == 0 && r < rows) {
                    if (logits) gstore(logits + (size_t)t * rows + r, acc);
                    const unsigned long long k = argmax_key(acc, (uint32_t)r);
                    best = k > best ? k : best;
                }
            }
        };
        issue(0, A[0], SC[0]);
        prologue();
        for (int p = 0; p < ng; p += 2) {
            issue(p + 1, A[1], SC[1]);
            land(A[0], SC[0]);
            consume(p, A[0], SC[0]);
            issue(p + 2, A[0], SC[0]);
            land(A[1], SC[1]);
            if (p + 1 < ng) consume(p + 1, A[1], SC[1]);
        }
        vm_wait<0>();
#pragma unroll
        for (int j = 0; j < G; j++) {
#pragma unroll
            for (int i = 0; i < kLmChunks; i++) {
                keep(A[0][j][i]);
                keep(A[1][j][i]);
            }
            keep(SC[0][j]);
            keep(SC[1][j]);
        }
    } else if (nchunks <= 64 * kLmChunks) {
        prologue();
        constexpr int RW = 4;  // rows per wavefront per iteration
        for (int r0 = gw; r0 < rows; r0 += RW * nw) {
            uint2 a[RW][kLmChunks];
#pragma unroll
            for (int j = 0; j < RW; j++) {
                const int r = r0 + j * nw;
                const uint2* wr = (const uint2*)(Q + (size_t)(r < rows ? r : r0) * cols);
#pragma unroll
                for (int i = 0; i < kLmChunks; i++) {
                    const int c = lane + 64 * i;
                    a[j][i] = c < nchunks ? ld_stream8(wr + c) : make_uint2(0, 0);
                }
            }
#pragma unroll
            for (int j = 0; j < RW; j++) {
                const int r = r0 + j * nw;
                float acc = 0.0f;
#pragma unroll
                for (int i = 0; i < kLmChunks; i++) {
                    const int c = lane + 64 * i;
                    if (c < nchunks) acc = dot8_i8(a[j][i], xs + 8 * c, acc);
                }
                if (r < rows) emit(r, acc);
            }
        }
    } else {
        prologue();
        for (int r = gw; r < rows; r += nw) {
            const uint2* wr = (const uint2*)(Q + (size_t)r * cols);
            float acc = 0.0f;
            for (int c = lane; c < nchunks; c += 64) acc = dot8_i8(ld_stream8(wr + c), xs + 8 * c, acc);
            emit(r, acc);
        }
    }
    __shared__ unsigned long long wbest[kThreads / 64];
    if (lane == 0) wbest[tid >> 6] = best;
    __syncthreads();
    if (key && tid == 0) {
        unsigned long long b = wbest[0];
#pragma unroll
        for (int i = 1; i < kThreads / 64; i++) b = wbest[i] > b ? wbest[i] : b;
        if (b) atomicMax(&key[t], b);
    }
}

// LM head for several token rows at once (normalized rows xn [m][cols]):
// each (weight row, token) dot product has lmhead_kernel's order (lane l
// takes chunks l, l+64, ... with fused multiply-adds in element order, then
// the xor tree over the 64 lanes), so the logits and argmax keys are the same
// bits; what changes is reuse: a workgroup keeps TG = 8 token rows in LDS and
// each wavefront holds R = 4 weight rows unpacked in registers for all of
// them (one LDS read of x per 4 rows), and the 32 (token, row) sums of a
// wavefront reduce together by recursive halving.  Workgroup i takes token
// group i % ngroups of row tile i / ngroups, so the groups of one tile run
// together and share its weight rows through the caches.
//
// Q8: the int8 head (q8head.rs): W is int8 [rows][cols] with one f32 scale
// per row (rscale); chunk c is the 8 bytes 8c..8c+7, and each sum is scaled
// by its row's scale, as in q8head_kernel.
template <int R, int NCH, int TG, bool Q8, int NT = kThreads>
__global__ __launch_bounds__(NT) void lmhead_batch_kernel(const void* W, const float* rscale, int rows, int cols,
                                                          const float* xn, int m, int tile_rows, float* logits,
                                                          unsigned long long* key) {
    constexpr int A = R * TG, NW = NT / 64;
    static_assert(A == 32 || A == 64, "32 or 64 accumulators per lane");
    extern __shared__ __align__(16) float xs[];  // [TG][cols]
    const int ngroups = (m + TG - 1) / TG;
    const int grp = blockIdx.x % ngroups, tile = blockIdx.x / ngroups;
    const int t0 = grp * TG, nt = m - t0 < TG ? m - t0 : TG;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    for (int i = tid * 4; i < nt * cols; i += NT * 4)
        *(float4*)(xs + i) = *(const float4*)(xn + (size_t)t0 * cols + i);
    for (int i = nt * cols + tid; i < TG * cols; i += NT) xs[i] = 0.0f;  // unused token rows
    __syncthreads();
    const int nchunks = cols >> 3;
    const int r_begin = tile * tile_rows, r_end = r_begin + tile_rows < rows ? r_begin + tile_rows : rows;
    // this lane's (token, row) after the reduction: accumulator (lane >> 1) & 31
    // (A = 32, lane pairs hold the same sum) or lane (A = 64)
    const int my_a = A == 32 ? ((lane >> 1) & 31) : lane;
    const int my_t = my_a / R, my_r = my_a % R;
    const bool writer = A == 64 || (lane & 1) == 0;
    unsigned long long best = 0ull;  // of token my_t
    for (int rb = r_begin + w * R; rb < r_end; rb += NW * R) {
        // R weight rows of this wavefront, unpacked to f32
        float wf[R][NCH][8];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = rb + r < r_end ? rb + r : rb;
            if constexpr (Q8) {
                const uint2* wr = (const uint2*)((const int8_t*)W + (size_t)row * cols);
#pragma unroll
                for (int i = 0; i < NCH; i++) {
                    const int c = lane + 64 * i;
                    const uint2 v = c < nchunks ? ld_stream8(wr + c) : make_uint2(0, 0);
#pragma unroll
                    for (int e = 0; e < 8; e++) wf[r][i][e] = i8_at(e < 4 ? v.x : v.y, e & 3);
                }
                continue;
            }
            const uint4* wr = (const uint4*)((const uint16_t*)W + (size_t)row * cols);
#pragma unroll
            for (int i = 0; i < NCH; i++) {
                const int c = lane + 64 * i;
                const uint4 v = c < nchunks ? ld_stream(wr + c) : make_uint4(0, 0, 0, 0);
                wf[r][i][0] = bf_lo(v.x);
                wf[r][i][1] = bf_hi(v.x);
                wf[r][i][2] = bf_lo(v.y);
                wf[r][i][3] = bf_hi(v.y);
                wf[r][i][4] = bf_lo(v.z);
                wf[r][i][5] = bf_hi(v.z);
                wf[r][i][6] = bf_lo(v.w);
                wf[r][i][7] = bf_hi(v.w);
            }
        }
        float acc[A];
#pragma unroll
        for (int t = 0; t < TG; t++) {
            const float* xt = xs + t * cols;
#pragma unroll
            for (int r = 0; r < R; r++) acc[t * R + r] = 0.0f;
#pragma unroll
            for (int i = 0; i < NCH; i++) {
                const int c = lane + 64 * i;
                if (c < nchunks) {
                    const float4 x0 = *(const float4*)(xt + 8 * c);
                    const float4 x1 = *(const float4*)(xt + 8 * c + 4);
                    const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                    for (int r = 0; r < R; r++)
#pragma unroll
                        for (int e = 0; e < 8; e++)
                            acc[t * R + r] = __builtin_fmaf(wf[r][i][e], xv[e], acc[t * R + r]);
                }
            }
        }
        float a;
        {
            float h16[16], h8[8], h4[4], h2[2], h1[1];
            if constexpr (A == 64) {
                float h32[32];
                halve<32>(acc, h32);
                halve<16>(h32, h16);
            } else {
                halve<32>(acc, h16);
            }
            halve<A == 64 ? 8 : 16>(h16, h8);
            halve<A == 64 ? 4 : 8>(h8, h4);
            halve<A == 64 ? 2 : 4>(h4, h2);
            halve<A == 64 ? 1 : 2>(h2, h1);
            a = A == 64 ? h1[0] : xor_add<1>(h1[0]);
        }
        const int row = rb + my_r;
        if (Q8) a = gload(rscale + (row < r_end ? row : r_begin)) * a;
        if (writer && my_t < nt && row < r_end) {
            if (logits) logits[(size_t)(t0 + my_t) * rows + row] = a;
            const unsigned long long k = argmax_key(a, (uint32_t)row);
            best = k > best ? k : best;
        }
    }
    // one atomic per (workgroup, token): the lanes' keys meet in the token
    // rows' LDS once every wavefront is done with them (no static LDS: the
    // token rows fill the workgroup's share of the CU's LDS)
    constexpr int KW = A == 64 ? 64 : 32;  // keys per wavefront
    __syncthreads();
    unsigned long long* wbest = (unsigned long long*)xs;  // [NW][KW]
    if (writer) wbest[w * KW + (A == 64 ? lane : (lane >> 1))] = best;
    __syncthreads();
    if (key && tid < nt) {
        unsigned long long b = 0ull;
        for (int i = 0; i < NW * KW; i++)
            if (i % KW / R == tid) b = wbest[i] > b ? wbest[i] : b;
        if (b) atomicMax(&key[t0 + tid], b);
    }
}

// The bf16 head of several tokens with the weight stream kept in flight:
// one wavefront per SIMD (256 threads, 16 token rows in LDS), each taking R
// rows at a time; the raw bf16 chunks of its next R rows load (untracked
// loads, explicit waits) while the current ones compute, and a chunk is
// widened to f32 once for all 16 tokens.  Every (token, row) accumulator
// takes its products in the order of lmhead_batch_kernel (chunk i, then
// element e) and the accumulators reduce by the same recursive halving, so
// the logits are those of lmhead_batch_kernel and of the one-token head bit
// for bit.
template <int R, int NCH, int TG, int NT>
__global__ __launch_bounds__(NT) void lmhead_stream_kernel(const uint16_t* W, int rows, int cols, const float* xn,
                                                           int m, int tile_rows, float* logits,
                                                           unsigned long long* key) {
    constexpr int A = R * TG, NW = NT / 64;
    static_assert(A == 32 || A == 64, "32 or 64 accumulators per lane");
    extern __shared__ __align__(16) float xs[];  // [TG][cols]
    const int ngroups = (m + TG - 1) / TG;
    // the token groups of a row tile are ntiles apart in the grid: with ntiles
    // a multiple of 8 they sit on one XCD (workgroup b on XCD b mod 8) and
    // share its L2's copy of the tile's weights
    const int ntiles = (int)gridDim.x / ngroups;
    const int grp = blockIdx.x / ntiles, tile = blockIdx.x % ntiles;
    const int t0 = grp * TG, nt = m - t0 < TG ? m - t0 : TG;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int nchunks = cols >> 3;
    const int r_begin = tile * tile_rows, r_end = r_begin + tile_rows < rows ? r_begin + tile_rows : rows;
    const int nblk = r_end > r_begin + w * R ? (r_end - r_begin - w * R + NW * R - 1) / (NW * R) : 0;
    // the first block's weights go out before the token rows are staged
    u32x4 B0[R][NCH], B1[R][NCH];
    auto issue = [&](int b, u32x4 (&d)[R][NCH]) {
        const int rb = r_begin + w * R + b * NW * R;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = rb + r < r_end ? rb + r : r_begin;  // past the end: a row of the tile (unused)
            const uint4* wr = (const uint4*)(W + (size_t)row * cols);
#pragma unroll
            for (int i = 0; i < NCH; i++) {
                const int c = lane + 64 * i;
                d[r][i] = ld_u4_async_nt(wr + (c < nchunks ? c : 0));
            }
        }
    };
    // all but the block issued last have landed (loads complete in issue order)
    auto land = [&](u32x4 (&d)[R][NCH]) {
        vm_wait<R * NCH>();
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int i = 0; i < NCH; i++) pin(d[r][i]);
    };
    // this lane's (token, row) after the reduction: accumulator (lane >> 1) & 31
    // (A = 32, lane pairs hold the same sum) or lane (A = 64)
    const int my_a = A == 32 ? ((lane >> 1) & 31) : lane;
    const int my_t = my_a / R, my_r = my_a % R;
    const bool writer = A == 64 || (lane & 1) == 0;
    unsigned long long best = 0ull;  // of token my_t
    auto compute = [&](int b, const u32x4 (&d)[R][NCH]) {
        float acc[A];
#pragma unroll
        for (int q = 0; q < A; q++) acc[q] = 0.0f;
#pragma unroll
        for (int i = 0; i < NCH; i++) {
            const int c = lane + 64 * i;
            if (c < nchunks) {
                float wf[R][8];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const u32x4 v = d[r][i];
                    wf[r][0] = bf_lo(v.x);
                    wf[r][1] = bf_hi(v.x);
                    wf[r][2] = bf_lo(v.y);
                    wf[r][3] = bf_hi(v.y);
                    wf[r][4] = bf_lo(v.z);
                    wf[r][5] = bf_hi(v.z);
                    wf[r][6] = bf_lo(v.w);
                    wf[r][7] = bf_hi(v.w);
                }
#pragma unroll
                for (int t = 0; t < TG; t++) {
                    const float* xt = xs + t * cols;
                    const float4 x0 = *(const float4*)(xt + 8 * c);
                    const float4 x1 = *(const float4*)(xt + 8 * c + 4);
                    const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                    for (int r = 0; r < R; r++)
#pragma unroll
                        for (int e = 0; e < 8; e++)
                            acc[t * R + r] = __builtin_fmaf(wf[r][e], xv[e], acc[t * R + r]);
                }
            }
        }
        float a;
        {
            float h16[16], h8[8], h4[4], h2[2], h1[1];
            if constexpr (A == 64) {
                float h32[32];
                halve<32>(acc, h32);
                halve<16>(h32, h16);
            } else {
                halve<32>(acc, h16);
            }
            halve<A == 64 ? 8 : 16>(h16, h8);
            halve<A == 64 ? 4 : 8>(h8, h4);
            halve<A == 64 ? 2 : 4>(h4, h2);
            halve<A == 64 ? 1 : 2>(h2, h1);
            a = A == 64 ? h1[0] : xor_add<1>(h1[0]);
        }
        const int row = r_begin + w * R + b * NW * R + my_r;
        if (writer && my_t < nt && row < r_end) {
            if (logits) logits[(size_t)(t0 + my_t) * rows + row] = a;
            const unsigned long long k = argmax_key(a, (uint32_t)row);
            best = k > best ? k : best;
        }
    };
    // the first block's weights go out before the token rows are staged
    issue(0, B0);
    for (int i = tid * 4; i < nt * cols; i += NT * 4)
        *(float4*)(xs + i) = *(const float4*)(xn + (size_t)t0 * cols + i);
    for (int i = nt * cols + tid; i < TG * cols; i += NT) xs[i] = 0.0f;  // unused token rows
    __syncthreads();
    // loads, waits and pins are unconditional (no copy of a register still
    // being loaded); blocks past the last are loaded and not used
    for (int b = 0; b < nblk; b += 2) {
        issue(b + 1, B1);
        land(B0);
        compute(b, B0);
        issue(b + 2, B0);
        land(B1);
        if (b + 1 < nblk) compute(b + 1, B1);
    }
    vm_wait<0>();
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int i = 0; i < NCH; i++) {
            keep(B0[r][i]);
            keep(B1[r][i]);
        }
    // one atomic per (workgroup, token): the lanes' keys meet in LDS
    __syncthreads();
    constexpr int KW = A == 64 ? 64 : 32;  // keys per wavefront
    unsigned long long* wbest = (unsigned long long*)xs;  // [NW][KW]
    if (writer) wbest[w * KW + (A == 64 ? lane : (lane >> 1))] = best;
    __syncthreads();
    if (key && tid < nt) {
        unsigned long long bk = 0ull;
        for (int i = 0; i < NW * KW; i++)
            if (i % KW / R == tid) bk = wbest[i] > bk ? wbest[i] : bk;
        if (bk) atomicMax(&key[t0 + tid], bk);
    }
}

__global__ void set_state_kernel(int* state, int pos, int slot) {
    if (threadIdx.x == 0) {
        state[0] = pos;
        state[1] = slot;
    }
}

// Streaming copy: 16-byte granules (grid-stride, nontemporal), then the tail
// bytes.
__global__ __launch_bounds__(kThreads) void copy_kernel(uint4* __restrict__ dst, const uint4* __restrict__ src,
                                                        size_t n16, uint8_t* dtail, const uint8_t* stail,
                                                        int ntail) {
    const size_t stride = (size_t)gridDim.x * kThreads;
    for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n16; i += stride) {
        const u32x4 v = __builtin_nontemporal_load((const u32x4*)(src + i));
        __builtin_nontemporal_store(v, (u32x4*)(dst + i));
    }
    if (blockIdx.x == 0 && (int)threadIdx.x < ntail) dtail[threadIdx.x] = stail[threadIdx.x];
}

// Byte copy for unaligned buffers (grid-stride).
__global__ __launch_bounds__(kThreads) void copy_bytes_kernel(uint8_t* __restrict__ dst,
                                                              const uint8_t* __restrict__ src, size_t n) {
    const size_t stride = (size_t)gridDim.x * kThreads;
    for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

__global__ void fill_u64_kernel(unsigned long long* p, int n, unsigned long long v) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

// ---------------------------------------------------------------------------
// synthetic weights: same generator as oracle/lbt_oracle.c (or_synth_*).
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

__global__ void synth_packed_kernel(uint64_t seed, uint64_t tensor, int rows, int cols, int rb, uint8_t* out) {
    const size_t n = (size_t)rows * rb;
    const uint64_t base = splitmix64(seed ^ (tensor << 40));
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n; idx += (size_t)gridDim.x * blockDim.x) {
        const size_t r = idx / rb, byte = idx % rb;
        const size_t b = byte / kBlockBytes, j = byte % kBlockBytes;
        uint32_t v = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const size_t c = b * kBlock + k * 32 + j;
            int w = 0;
            if (c < (size_t)cols) {
                const uint64_t bucket = ((splitmix64(base + r * (size_t)cols + c) >> 32) * 10u) >> 32;
                w = bucket < 3 ? -1 : (bucket < 7 ? 0 : 1);
            }
            v |= (uint32_t)(w + 1) << (2 * k);
        }
        out[idx] = (uint8_t)v;
    }
}

__global__ void synth_f32_kernel(uint64_t seed, uint64_t tensor, size_t n, float lo, float span, float* out) {
    const uint64_t base = splitmix64(seed ^ (tensor << 40));
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const float u = (float)(splitmix64(base + i) >> 40) * 5.9604644775390625e-8f;
        out[i] = lo + span * u;
    }
}

__global__ void synth_bf16_kernel(uint64_t seed, uint64_t tensor, size_t n, uint16_t* out) {
    const uint64_t base = splitmix64(seed ^ (tensor << 40));
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const float u = (float)(splitmix64(base + i) >> 40) * 5.9604644775390625e-8f;
        out[i] = f32_to_bf16(u * 2.0f - 1.0f);
    }
}

// Synthetic KV rows: positions [0, len) of every (layer, sequence, KV head)
// of a cache laid out [layers * nseq * kvh][cap][hd], bf16 of an
// approximately N(0,1) value: (u1 + u2 + u3 + u4 - 2) * sqrt(3) of four
// uniforms on [0, 1) from one splitmix64 draw per element.
__global__ void synth_kv_kernel(uint64_t seed, size_t rows, int cap, int len, int hd, uint16_t* out) {
    const uint64_t base = splitmix64(seed);
    const size_t per_row = (size_t)len * hd, n = rows * per_row;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const size_t r = i / per_row, rem = i % per_row;
        const uint64_t z = splitmix64(base + i);
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; k++) acc += (float)((z >> (16 * k)) & 0xffffu) * (1.0f / 65536.0f);
        out[r * (size_t)cap * hd + rem] = f32_to_bf16((acc - 2.0f) * 1.7320508075688772f);
    }
}

// p[i] += 1 for i < n (positions of a batch after a step).
__global__ void advance_pos_kernel(int* p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] += 1;
}

// ---------------------------------------------------------------------------
// launchers
int launch_embed(lbt_ctx* ctx, const uint16_t* embed, int hidden, int vocab, const uint32_t* tokens,
                 const unsigned long long* key, uint32_t* tok_out, int m, float* x, int* state) {
    hipLaunchKernelGGL(embed_kernel, dim3(m), dim3(kThreads), 0, ctx->stream, embed, hidden, vocab, tokens,
                       (unsigned long long*)key, tok_out, x, state);
    LBT_HIP(ctx, hipGetLastError());
    return LBT_OK;
}

namespace {

template <int LK>
hipError_t launch_attn_lk(int gh, bool grouped, int force_wide, dim3 grid, size_t lds, hipStream_t st, hipEvent_t e0, hipEvent_t e1,
                          const float* q, int nh, int kvh, const RowPos& rp, const uint16_t* kc, const uint16_t* vc,
                          int cap, float scaling, float* o, float* ml) {
    if (!grouped) {
        hipExtLaunchKernelGGL(attention_kernel<LK>, grid, dim3(kThreads), lds, st, e0, e1, 0, q, nh, kvh, rp, kc, vc,
                              cap, scaling, o, ml);
        return hipGetLastError();
    }
    const bool wide = force_wide < 0 ? (long)grid.x * grid.y >= 4096 : force_wide != 0;
#define LBT_ATTN_GROUP(GH)                                                                                      \
    if (wide)                                                                                                   \
        hipExtLaunchKernelGGL((attention_group_kernel<LK, GH, true>), grid, dim3(kThreads), lds, st, e0, e1, 0, q, \
                              nh, kvh, rp, kc, vc, cap, scaling, o, ml);                                        \
    else                                                                                                        \
        hipExtLaunchKernelGGL((attention_group_kernel<LK, GH, false>), grid, dim3(kThreads), lds, st, e0, e1, 0, q, \
                              nh, kvh, rp, kc, vc, cap, scaling, o, ml);
    switch (gh) {
        case 1: LBT_ATTN_GROUP(1); break;
        case 2: LBT_ATTN_GROUP(2); break;
        default: LBT_ATTN_GROUP(4); break;
    }
#undef LBT_ATTN_GROUP
    return hipGetLastError();
}

}  // namespace

int launch_attention(lbt_ctx* ctx, const float* q, int m, int nh, int kvh, int hd, const RowPos& rp,
                     const uint16_t* kc, const uint16_t* vc, int cap, float scaling, float* o, float* ml,
                     bool grouped) {
    if (kvh <= 0 || nh % kvh) return set_err(ctx, LBT_E_INVALID, "attention: heads must be a multiple of kv heads");
    const int gh = nh / kvh;
    if (gh != 1 && gh != 2 && gh != 4) grouped = false;
    const size_t lds = grouped ? (size_t)gh * attn_group_score_keys(attn_split_keys(rp.vis_max), hd / 8) * sizeof(float)
                               : (size_t)attn_split_keys(rp.vis_max) * sizeof(float);
    if (lds > 64 * 1024) return set_err(ctx, LBT_E_RANGE, "attention: context too long for the LDS score buffer");
    // rows of one sequence at consecutive positions (a prefill) with at
    // least 8 (row, KV head, split) tasks per CU: one wavefront per task
    // where the shape allows (2B, 2048-token prefill: attention 41.5 ->
    // 18.9 ms; at 64 and 128 tokens the workgroup per task stays faster,
    // 0.25 against 0.42 ms and 0.38 against 0.43 ms).  LBT_ATTN_WAVE=1 / 0
    // forces it on / off for grouped attention.
    const int aw = ctx->tune.attn_wave;
    const long wave_tasks = (long)m * kvh * attn_splits(rp.vis_max);
    if (grouped && gh == 4 && hd == 128 &&
        (aw > 0 || (aw < 0 && m > 1 && !rp.tok_pos && !rp.pos_dev && wave_tasks >= 8L * ctx->cus))) {
        const int nsg = attn_splits(rp.vis_max);
        const int scw = (attn_split_keys(rp.vis_max) + 15) / 16 * 16 * 4;
        const size_t wl = (size_t)4 * scw * sizeof(float);
        const long tasks = wave_tasks;
        if (wl <= 64 * 1024 && (tasks + 3) / 4 < (1L << 31)) {
            hipEvent_t e0, e1;
            prof_pair(ctx, &e0, &e1);
            hipExtLaunchKernelGGL((attention_wave_kernel<16, 4>), dim3((unsigned)((tasks + 3) / 4)), dim3(kThreads), wl,
                                  ctx->stream, e0, e1, 0, q, nh, kvh, rp, kc, vc, cap, scaling, o, ml, m, nsg, scw);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return hip_err(ctx, e, "attention_wave_kernel launch");
            prof_commit(ctx, e0, e1, kProfAttn, 2.0 * kvh * (double)rp.vis_max * hd * 2.0 * m);
            return LBT_OK;
        }
    }
    hipEvent_t e0, e1;
    prof_pair(ctx, &e0, &e1);
    // as many splits as the longest visible row has (rows with fewer exit
    // at once; a graph-replayed step is sized for the whole capacity)
    dim3 grid((grouped ? kvh : nh) * attn_splits(rp.vis_max), m);
    hipError_t e;
    switch (hd) {
        case 64:
            e = launch_attn_lk<8>(gh, grouped, ctx->tune.attn_wide, grid, lds, ctx->stream, e0, e1, q, nh, kvh, rp, kc, vc, cap, scaling, o,
                                  ml);
            break;
        case 128:
            e = launch_attn_lk<16>(gh, grouped, ctx->tune.attn_wide, grid, lds, ctx->stream, e0, e1, q, nh, kvh, rp, kc, vc, cap, scaling,
                                   o, ml);
            break;
        case 256:
            e = launch_attn_lk<32>(gh, grouped, ctx->tune.attn_wide, grid, lds, ctx->stream, e0, e1, q, nh, kvh, rp, kc, vc, cap, scaling,
                                   o, ml);
            break;
        default:
            return set_err(ctx, LBT_E_INVALID, "attention: head_dim must be 64, 128 or 256");
    }
    if (e != hipSuccess) return hip_err(ctx, e, "attention_kernel launch");
    const double kv_bytes = 2.0 * kvh * (double)rp.vis_max * hd * 2.0 * m;
    prof_commit(ctx, e0, e1, kProfAttn, kv_bytes);
    return LBT_OK;
}

int launch_attn_combine(lbt_ctx* ctx, const float* o, const float* ml, int m, int nh, int hd, const RowPos& rp,
                        float* out) {
    const int H = nh * hd;
    if (nh <= 0 || nh > kAttnMaxHeads || hd % 4 || H > 8192)
        return set_err(ctx, LBT_E_INVALID, "attention combine: at most 64 heads and 8192 columns");
    hipEvent_t e0, e1;
    prof_pair(ctx, &e0, &e1);
    if (H <= 16 * kThreads)
        hipExtLaunchKernelGGL(attn_combine_kernel<16>, dim3(m), dim3(kThreads), 0, ctx->stream, e0, e1, 0, o, ml, nh,
                              hd, rp, out);
    else
        hipExtLaunchKernelGGL(attn_combine_kernel<32>, dim3(m), dim3(kThreads), 0, ctx->stream, e0, e1, 0, o, ml, nh,
                              hd, rp, out);
    LBT_HIP(ctx, hipGetLastError());
    prof_commit(ctx, e0, e1, kProfAttn, 0.0);
    return LBT_OK;
}

namespace {
// The LM head launch shared by the bf16 head and the int8 head (rscale set).
int launch_head(lbt_ctx* ctx, const void* w, const float* rscale, int rows, int cols, const float* x, int m,
                const float* norm_w, float eps, float* logits, unsigned long long* key, float* xn) {
    const bool q8 = rscale != nullptr;
    const char* what = q8 ? "int8 head" : "bf16 linear";
    if (cols % 8) return set_err(ctx, LBT_E_INVALID, std::string(what) + ": cols must be a multiple of 8");
    if (m <= 0) return LBT_OK;
    constexpr int kTG = 8, kR = 4;
    const double wbytes = (double)rows * cols * (q8 ? 1.0 : 2.0);
    if (m >= 2 && xn && cols <= 64 * kLmChunks * 8) {
        // several rows: normalize once, then the weight-reusing head
        hipLaunchKernelGGL(row_norm_kernel, dim3(m), dim3(kThreads), 0, ctx->stream, x, cols, norm_w, eps, xn);
        LBT_HIP(ctx, hipGetLastError());
        // more than 8 rows: 16-token groups on 512 threads (the whole LDS of a
        // CU; each weight row is then read from L2 half as often), else
        // 8-token groups on 256 threads (two workgroups per CU)
        const bool big = m > 8 && (size_t)16 * cols * sizeof(float) <= 160 * 1024 && !ctx->tune.head_tg8;
        const int tg = big ? 16 : kTG, nt = big ? 512 : kThreads, nw = nt / 64;
        const int ngroups = (m + tg - 1) / tg;
        int tiles = ctx->cus * (big ? 2 : 4) / ngroups;
        if (tiles < 1) tiles = 1;
        int tile_rows = (rows + tiles - 1) / tiles;
        tile_rows = (tile_rows + nw * kR - 1) / (nw * kR) * (nw * kR);
        tiles = (rows + tile_rows - 1) / tile_rows;
        const size_t lds = (size_t)tg * cols * sizeof(float);
        const void* fn = big ? (q8 ? (const void*)lmhead_batch_kernel<kR, kLmChunks, 16, true, 512>
                                   : (const void*)lmhead_batch_kernel<kR, kLmChunks, 16, false, 512>)
                             : (q8 ? (const void*)lmhead_batch_kernel<kR, kLmChunks, kTG, true>
                                   : (const void*)lmhead_batch_kernel<kR, kLmChunks, kTG, false>);
        static bool attr[4] = {false, false, false, false};
        if (!attr[q8 + 2 * big]) {
            (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, big ? 160 * 1024 : 96 * 1024);
            (void)hipGetLastError();
            attr[q8 + 2 * big] = true;
        }
        if (lds > (big ? 160 : 96) * 1024)
            return set_err(ctx, LBT_E_INVALID, std::string(what) + ": token group exceeds LDS");
        hipEvent_t e0, e1;
        prof_pair(ctx, &e0, &e1);
#define LBT_HEAD_LAUNCH(TGv, Q8v, NTv)                                                                               \
    hipExtLaunchKernelGGL((lmhead_batch_kernel<kR, kLmChunks, TGv, Q8v, NTv>), dim3(tiles * ngroups), dim3(NTv), lds, \
                          ctx->stream, e0, e1, 0, w, rscale, rows, cols, xn, m, tile_rows, logits, key)
        if (big) {
            if (q8) {
                LBT_HEAD_LAUNCH(16, true, 512);
            } else if (!ctx->tune.head_batch_classic) {
                // one wavefront per SIMD, weights a block ahead: ~one workgroup per CU
                constexpr int SR = 2, SNT = 512;  // rows per block, threads
                int st = ctx->cus / ngroups;
                if (st < 1) st = 1;
                int str = (rows + st - 1) / st;
                str = (str + (SNT / 64) * SR - 1) / ((SNT / 64) * SR) * ((SNT / 64) * SR);
                st = (rows + str - 1) / str;
                static bool attr2 = false;
                if (!attr2) {
                    (void)hipFuncSetAttribute((const void*)lmhead_stream_kernel<SR, kLmChunks, 16, SNT>,
                                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
                    (void)hipGetLastError();
                    attr2 = true;
                }
                hipExtLaunchKernelGGL((lmhead_stream_kernel<SR, kLmChunks, 16, SNT>), dim3(st * ngroups), dim3(SNT),
                                      lds, ctx->stream, e0, e1, 0, (const uint16_t*)w, rows, cols, xn, m, str, logits,
                                      key);
            } else {
                LBT_HEAD_LAUNCH(16, false, 512);
            }
        } else {
            if (q8) LBT_HEAD_LAUNCH(kTG, true, kThreads);
            else LBT_HEAD_LAUNCH(kTG, false, kThreads);
        }
#undef LBT_HEAD_LAUNCH
        LBT_HIP(ctx, hipGetLastError());
        prof_commit(ctx, e0, e1, kProfHead, wbytes);
        return LBT_OK;
    }
    const size_t lds = (size_t)cols * sizeof(float);
    if (lds > 64 * 1024) return set_err(ctx, LBT_E_INVALID, std::string(what) + ": cols too large");
    int blocks = (rows + 31) / 32;
    if (blocks > (q8 ? 512 : 768)) blocks = q8 ? 512 : 768;
    if (blocks < 1) blocks = 1;
    hipEvent_t e0, e1;
    prof_pair(ctx, &e0, &e1);
    if (q8)
        hipExtLaunchKernelGGL(q8head_kernel, dim3(blocks, m), dim3(kThreads), lds, ctx->stream, e0, e1, 0,
                              (const int8_t*)w, rscale, rows, cols, x, norm_w, eps, logits, key);
    else
        hipExtLaunchKernelGGL(lmhead_kernel, dim3(blocks, m), dim3(kThreads), lds, ctx->stream, e0, e1, 0,
                              (const uint16_t*)w, rows, cols, x, norm_w, eps, logits, key);
    LBT_HIP(ctx, hipGetLastError());
    prof_commit(ctx, e0, e1, kProfHead, wbytes * m);
    return LBT_OK;
}
}  // namespace

// ---------------------------------------------------------------------------
// The tied bf16 head of several rows on the bf16 matrix cores (head kind 2):
// each normalized row x is split into bf16 parts hi = bf16(x) and
// lo = bf16(x - hi) (x - hi is exact in f32; x - hi - lo is below 2^-17 |x|),
// and logits = W.hi + W.lo accumulate in f32 in v_mfma_f32_32x32x16_bf16
// (the bf16 x bf16 products are exact in f32).  The sum order is the matrix
// core's, so these logits match the exact head within tolerance, not bit for
// bit; a one-row head never takes this path.

// xh / xl [mp][cols] (rows past m zero)
__global__ __launch_bounds__(kThreads) void bf16_split_kernel(const float* xn, int m, int cols, uint16_t* xh,
                                                              uint16_t* xl) {
    const int t = blockIdx.x;
    for (int i = threadIdx.x; i < cols; i += kThreads) {
        const float x = t < m ? xn[(size_t)t * cols + i] : 0.0f;
        const uint16_t h = f32_to_bf16(x);
        xh[(size_t)t * cols + i] = h;
        xl[(size_t)t * cols + i] = f32_to_bf16(x - bf16_to_f32(h));
    }
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Workgroup of 4 wavefronts: TT token tiles of 32 x 4 / TT groups of NV
// vocab tiles of 32 rows; a wavefront takes one token tile and NV vocab tiles
// (each activation load feeds NV MFMA pairs).  k is visited in blocks of 64:
// lane l (half h = l >> 5) holds, for the four 16-k steps s of block b, the
// 8 k values 64 b + 32 h + 8 s .. + 7 of its token (A) and vocab row (B) --
// the same k in both operands, so the products are those of the dot -- which
// makes each lane's loads of a block 64 contiguous bytes per row.  D: vocab
// row l & 31 of the tile, tokens 8 (r >> 2) + 4 (l >> 5) + (r & 3).  The
// first-max keys of a token meet in LDS: one atomic per token and workgroup.
template <int TT, int NV>
__global__ __launch_bounds__(kThreads) void lmhead_mfma_kernel(const uint16_t* W, int rows, int cols,
                                                               const uint16_t* xh, const uint16_t* xl, int m,
                                                               float* logits, unsigned long long* key) {
    constexpr int VG = 4 / TT;
    __shared__ unsigned long long kb[4][64];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int tt = w % TT, vg = w / TT;
    const int row0 = (blockIdx.x * VG + vg) * 32 * NV;
    const bool live = row0 < rows;  // wavefront-uniform
    const int l32 = lane & 31, h = lane >> 5;
    if (lane < 32) {
        kb[w][lane] = 0ull;
        kb[w][lane + 32] = 0ull;
    }
    f32x16 acc[NV];
#pragma unroll
    for (int v = 0; v < NV; v++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[v][r] = 0.0f;
    if (live) {
        const uint4* wp[NV];
#pragma unroll
        for (int v = 0; v < NV; v++) {
            const int r = row0 + 32 * v + l32;
            wp[v] = (const uint4*)(W + (size_t)(r < rows ? r : rows - 1) * cols + 32 * h);
        }
        const int tok = tt * 32 + l32;
        const uint4* hp = (const uint4*)(xh + (size_t)tok * cols + 32 * h);
        const uint4* lp = (const uint4*)(xl + (size_t)tok * cols + 32 * h);
        const int nb = cols / 64;
        // untracked loads (inline asm) with explicit waits: the compiler's
        // own tracking of these loop-carried buffers waits for every load in
        // flight, which left no block of loads ahead of the MFMAs.  The
        // compiler does not know these registers are written late: a copy or
        // spill of one between its load and land() would read stale data, so
        // the kernel must stay free of scratch (tests/test_build_checks.py
        // compiles it and checks the resource report) and every buffer stays
        // live until land() has waited for it.
        constexpr int NL = 4 * NV + 8;  // 16-byte loads per lane and block
        u32x4 bw[2][NV][4], ah[2][4], al[2][4];
        auto gl = [](u32x4& d, const uint4* p) {
            asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(d) : "v"(p) : "memory");
        };
        auto load = [&](int b, u32x4 (&bb)[NV][4], u32x4 (&hh)[4], u32x4 (&ll)[4]) {
            const int bc = b < nb ? b : nb - 1;  // past the end: the last block again (same count)
#pragma unroll
            for (int i = 0; i < 4; i++) {
#pragma unroll
                for (int v = 0; v < NV; v++) gl(bb[v][i], wp[v] + 8 * bc + i);
                gl(hh[i], hp + 8 * bc + i);
                gl(ll[i], lp + 8 * bc + i);
            }
        };
        auto land = [&](u32x4 (&bb)[NV][4], u32x4 (&hh)[4], u32x4 (&ll)[4]) {
            __builtin_amdgcn_s_waitcnt((NL & 15) | ((NL >> 4) << 14) | (7 << 4) | (15 << 8));
#pragma unroll
            for (int i = 0; i < 4; i++) {
#pragma unroll
                for (int v = 0; v < NV; v++) asm volatile("" : "+v"(bb[v][i]));
                asm volatile("" : "+v"(hh[i]));
                asm volatile("" : "+v"(ll[i]));
            }
        };
        auto mfma = [&](const u32x4 (&bb)[NV][4], const u32x4 (&hh)[4], const u32x4 (&ll)[4]) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const bf16x8 a0 = __builtin_bit_cast(bf16x8, hh[i]), a1 = __builtin_bit_cast(bf16x8, ll[i]);
#pragma unroll
                for (int v = 0; v < NV; v++) {
                    const bf16x8 bv = __builtin_bit_cast(bf16x8, bb[v][i]);
                    acc[v] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, bv, acc[v], 0, 0, 0);
                    acc[v] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, bv, acc[v], 0, 0, 0);
                }
            }
        };
        load(0, bw[0], ah[0], al[0]);
        for (int b = 0; b < nb; b += 2) {
            load(b + 1, bw[1], ah[1], al[1]);
            land(bw[0], ah[0], al[0]);
            mfma(bw[0], ah[0], al[0]);
            load(b + 2, bw[0], ah[0], al[0]);
            land(bw[1], ah[1], al[1]);
            if (b + 1 < nb) mfma(bw[1], ah[1], al[1]);
        }
        __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
        for (int k = 0; k < 2; k++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
#pragma unroll
                for (int v = 0; v < NV; v++) asm volatile("" ::"v"(bw[k][v][i]));
                asm volatile("" ::"v"(ah[k][i]));
                asm volatile("" ::"v"(al[k][i]));
            }
        // this wavefront's best key per token of its tile (lanes of one half
        // share a token per r), then its logits
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int tl = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            unsigned long long k = 0ull;
#pragma unroll
            for (int v = 0; v < NV; v++) {
                const int row = row0 + 32 * v + l32;
                if (row < rows) {
                    const unsigned long long kv = argmax_key(acc[v][r], (uint32_t)row);
                    k = kv > k ? kv : k;
                }
            }
#pragma unroll
            for (int msk = 16; msk >= 1; msk >>= 1) {
                const unsigned long long o = __shfl_xor(k, msk, 64);
                k = o > k ? o : k;
            }
            if (l32 == 0) kb[w][tl] = k;
        }
        if (logits) {
#pragma unroll
            for (int v = 0; v < NV; v++) {
                const int row = row0 + 32 * v + l32;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int t = tt * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    if (row < rows && t < m) logits[(size_t)t * rows + row] = acc[v][r];
                }
            }
        }
    }
    __syncthreads();
    // token t = 32 tt' + tl: the best of the wavefronts of token tile tt'
    const int t = (int)threadIdx.x;
    if (key && t < m && t < 32 * TT) {
        const int ttt = t / 32, tl = t % 32;
        unsigned long long b = 0ull;
#pragma unroll
        for (int j = 0; j < VG; j++) {
            const unsigned long long kv = kb[j * TT + ttt][tl];
            b = kv > b ? kv : b;
        }
        if (b) atomicMax(&key[t], b);
    }
}

constexpr int kHeadMfmaNV = 2;

int launch_bf16_mfma_head(lbt_ctx* ctx, const uint16_t* w, int rows, int cols, const float* x, int m,
                          const float* norm_w, float eps, float* logits, unsigned long long* key, float* xn,
                          uint16_t* xs, size_t xs_bytes) {
    // heads of up to 32 rows stay on the f32 kernel (faster there), so only
    // the two-token-tile instantiation exists
    if (m < 33 || m > 64 || !xn || cols % 64 || cols > 16 * kThreads)
        return set_err(ctx, LBT_E_INVALID, "bf16 matrix-core head: 33..64 rows, cols a multiple of 64");
    constexpr int tt = 2, mp = 32 * tt;
    if ((size_t)2 * mp * cols * 2 > xs_bytes) return set_err(ctx, LBT_E_INVALID, "bf16 matrix-core head: scratch");
    uint16_t* xh = xs;
    uint16_t* xl = xs + (size_t)mp * cols;
    hipEvent_t e0, e1;
    prof_pair(ctx, &e0, &e1);
    hipLaunchKernelGGL(row_norm_kernel, dim3(m), dim3(kThreads), 0, ctx->stream, x, cols, norm_w, eps, xn);
    hipLaunchKernelGGL(bf16_split_kernel, dim3(mp), dim3(kThreads), 0, ctx->stream, xn, m, cols, xh, xl);
    const int rows_per_wg = 32 * kHeadMfmaNV * (4 / tt);
    const dim3 grid((unsigned)((rows + rows_per_wg - 1) / rows_per_wg));
    hipExtLaunchKernelGGL((lmhead_mfma_kernel<tt, kHeadMfmaNV>), grid, dim3(kThreads), 0, ctx->stream, e0, e1, 0, w,
                          rows, cols, xh, xl, m, logits, key);
    LBT_HIP(ctx, hipGetLastError());
    prof_commit(ctx, e0, e1, kProfHead, (double)rows * cols * 2.0);
    return LBT_OK;
}

int launch_bf16_linear(lbt_ctx* ctx, const uint16_t* w, int rows, int cols, const float* x, int m,
                       const float* norm_w, float eps, float* logits, unsigned long long* key, float* xn) {
    return launch_head(ctx, w, nullptr, rows, cols, x, m, norm_w, eps, logits, key, xn);
}

int launch_q8_linear(lbt_ctx* ctx, const int8_t* q, const float* scale, int rows, int cols, const float* x, int m,
                     const float* norm_w, float eps, float* logits, unsigned long long* key, float* xn) {
    if (!scale) return set_err(ctx, LBT_E_INVALID, "int8 head: missing row scales");
    return launch_head(ctx, q, scale, rows, cols, x, m, norm_w, eps, logits, key, xn);
}

int launch_q8_quantize(lbt_ctx* ctx, const uint16_t* w, int rows, int cols, int8_t* q, float* scale) {
    if (rows <= 0 || cols <= 0) return set_err(ctx, LBT_E_INVALID, "int8 head: empty matrix");
    const int blocks = rows < ctx->cus * 8 ? rows : ctx->cus * 8;
    hipLaunchKernelGGL(q8_quantize_kernel, dim3(blocks), dim3(kThreads), 0, ctx->stream, w, rows, cols, q, scale);
    LBT_HIP(ctx, hipGetLastError());
    return LBT_OK;
}

int launch_copy(lbt_ctx* ctx, void* dst, const void* src, size_t bytes) {
    const bool aligned = (((uintptr_t)dst | (uintptr_t)src) & 15) == 0;
    const size_t cap = (size_t)ctx->cus * 8;
    if (!aligned) {
        size_t blocks = (bytes + kThreads - 1) / kThreads;
        if (blocks > cap) blocks = cap;
        hipLaunchKernelGGL(copy_bytes_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, ctx->stream, (uint8_t*)dst,
                           (const uint8_t*)src, bytes);
        LBT_HIP(ctx, hipGetLastError());
        return LBT_OK;
    }
    const size_t n16 = bytes / 16;
    const size_t done = n16 * 16;
    size_t blocks = (n16 + kThreads - 1) / kThreads;
    if (blocks > cap) blocks = cap;
    if (blocks == 0) blocks = 1;
    hipLaunchKernelGGL(copy_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, ctx->stream, (uint4*)dst,
                       (const uint4*)src, n16, (uint8_t*)dst + done, (const uint8_t*)src + done, (int)(bytes - done));
    LBT_HIP(ctx, hipGetLastError());
    return LBT_OK;
}

int launch_fill_u64(lbt_ctx* ctx, unsigned long long* p, int n, unsigned long long v) {
    hipLaunchKernelGGL(fill_u64_kernel, dim3((n + 255) / 256), dim3(256), 0, ctx->stream, p, n, v);
    LBT_HIP(ctx, hipGetLastError());
    return LBT_OK;
}

int launch_set_state(lbt_ctx* ctx, int* state, int pos, int slot) {
    hipLaunchKernelGGL(set_state_kernel, dim3(1), dim3(64), 0, ctx->stream, state, pos, slot);
    LBT_HIP(ctx, hipGetLastError());
    return LBT_OK;
}

static unsigned grid_for(size_t n) {
    size_t b = (n + 255) / 256;
    if (b > 65536) b = 65536;
    return (unsigned)(b ? b : 1);
}

int launch_synth_packed(lbt_ctx* ctx, uint64_t seed, uint64_t tensor, int rows, int cols, uint8_t* out) {
    const int rb = (int)(padded_cols((size_t)cols) / 4);
    hipLaunchKernelGGL(synth_packed_kernel, dim3(grid_for((size_t)rows * rb)), dim3(256), 0, ctx->stream, seed,
                       tensor, rows, cols, rb, out);
    LBT_HIP(ctx, hipGetLastError());
    return LBT_OK;
}

int launch_synth_f32(lbt_ctx* ctx, uint64_t seed, uint64_t tensor, size_t n, float lo, float span, float* out) {
    hipLaunchKernelGGL(synth_f32_kernel, dim3(grid_for(n)), dim3(256), 0, ctx->stream, seed, tensor, n, lo, span, out);
    LBT_HIP(ctx, hipGetLastError());
    return LBT_OK;
}

int launch_synth_kv(lbt_ctx* ctx, uint64_t seed, size_t rows, int cap, int len, int hd, uint16_t* out) {
    if (len <= 0) return LBT_OK;
    hipLaunchKernelGGL(synth_kv_kernel, dim3(grid_for(rows * (size_t)len * hd)), dim3(256), 0, ctx->stream, seed, rows,
                       cap, len, hd, out);
    LBT_HIP(ctx, hipGetLastError());
    return LBT_OK;
}

int launch_advance_pos(lbt_ctx* ctx, int* p, int n) {
    hipLaunchKernelGGL(advance_pos_kernel, dim3((n + 255) / 256), dim3(256), 0, ctx->stream, p, n);
    LBT_HIP(ctx, hipGetLastError());
    return LBT_OK;
}

int launch_synth_bf16(lbt_ctx* ctx, uint64_t seed, uint64_t tensor, size_t n, uint16_t* out) {
    hipLaunchKernelGGL(synth_bf16_kernel, dim3(grid_for(n)), dim3(256), 0, ctx->stream, seed, tensor, n, out);
    LBT_HIP(ctx, hipGetLastError());
    return LBT_OK;
}

}  // namespace lbt
