// attn_common.h -- GQA attention for one (query row, head) over the bf16 KV
// cache, shared by the standalone attention kernel and the persistent decode
// kernel so both compute the same bits.
#pragma once
#include "lbt_device.h"

namespace lbt {

// GQA attention for query row t (absolute position p = pos0 + t) and head h,
// over keys 0..p of the bf16 cache (the q/k/v GEMV has already rotated q and
// appended the rotated k and v).  model.rs:349-357: scores = q.K^T * scaling,
// softmax = exp(s - max) / sum, out = probs @ V; the causal mask of :316-328
// is the visibility bound.  One workgroup per (head, row).  Float order (the
// oracle mirrors it), with LK = hd/8 lanes per key and 8 dims per lane:
//   score: lane c sums q[8c+e]*k[8c+e] over e = 0..7 by fused multiply-adds,
//          the LK lanes combine with an xor butterfly (m = LK/2 .. 1), then
//          * scaling;
//   sum:   thread t adds exp(s_j - max) over j = t, t+256, ...; block_sum;
//   p_j:   exp(s_j - max) / sum;
//   out:   thread (group g = t/LK, chunk c = t%LK) accumulates
//          p_j * v[j][8c+e] by fused multiply-adds over j = g, g+256/LK, ...;
//          the 64/LK groups of a wave combine by xor over the group index
//          (m = 1, 2, ...), the four waves as (w0 + w1) + (w2 + w3).
template <int LK>
struct AttnShared {
    __align__(16) float qs[LK * 8];
    float red[16];
    __align__(16) float pv[4][LK * 8];
};

// q: this row's q [nh * hd] (already rotated); p: absolute position (keys
// 0..p are visible); out: this row's output [nh * hd].  The first 256 threads
// do the work; every thread of the workgroup must call it (shared barriers).
template <int LK>
__device__ __forceinline__ void attention_head(const float* q, int h, int nh, int kvh, int p, const uint16_t* kc,
                                               const uint16_t* vc, int cap, float scaling, float* out, float* sc,
                                               AttnShared<LK>& sh) {
    constexpr int HD = LK * 8, GW = 64 / LK, NG = kThreads / LK;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const bool act = tid < kThreads;
    const int vis = p + 1, g = h / (nh / kvh);
    if (tid < HD) sh.qs[tid] = q[(size_t)h * HD + tid];
    __syncthreads();
    const uint16_t* K = kc + (size_t)g * cap * HD;
    const uint16_t* V = vc + (size_t)g * cap * HD;
    const int ks = lane / LK, cc = lane % LK;
    float q8[8];
#pragma unroll
    for (int e = 0; e < 8; e++) q8[e] = sh.qs[8 * cc + e];
    float mx = -__builtin_inff();
    if (act) {
        for (int j0 = w * GW; j0 < vis; j0 += 4 * GW) {
            const int j = j0 + ks;
            float a = 0.0f;
            if (j < vis) {
                const uint4 kv = *(const uint4*)(K + (size_t)j * HD + 8 * cc);
                const uint32_t wv[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    a = __builtin_fmaf(q8[2 * e], bf16_to_f32((uint16_t)(wv[e] & 0xffffu)), a);
                    a = __builtin_fmaf(q8[2 * e + 1], bf16_to_f32((uint16_t)(wv[e] >> 16)), a);
                }
            }
            a = xor_sum_down<LK / 2>(a);
            if (j < vis) {
                const float s = a * scaling;
                if (cc == 0) sc[j] = s;
                mx = fmaxf(mx, s);
            }
        }
    }
    mx = block_max(mx, sh.red);  // includes the barrier that publishes sc
    float ps = 0.0f;
    if (act)
        for (int j = tid; j < vis; j += kThreads) {
            const float e = lbt_expf(sc[j] - mx);
            sc[j] = e;
            ps = ps + e;
        }
    const float sum = block_sum(ps, sh.red);
    if (act)
        for (int j = tid; j < vis; j += kThreads) sc[j] = sc[j] / sum;
    __syncthreads();
    const int grp = tid / LK, c = tid % LK;
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; e++) acc[e] = 0.0f;
    if (act)
        for (int j = grp; j < vis; j += NG) {
            const float pj = sc[j];
            const uint4 vv = *(const uint4*)(V + (size_t)j * HD + 8 * c);
            const uint32_t wv[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                acc[2 * e] = __builtin_fmaf(pj, bf16_to_f32((uint16_t)(wv[e] & 0xffffu)), acc[2 * e]);
                acc[2 * e + 1] = __builtin_fmaf(pj, bf16_to_f32((uint16_t)(wv[e] >> 16)), acc[2 * e + 1]);
            }
        }
    if constexpr (GW > 1) {
#pragma unroll
        for (int e = 0; e < 8; e++) acc[e] = xor_sum_up<LK>(acc[e]);
    }
    if (act && lane < LK) {
#pragma unroll
        for (int e = 0; e < 8; e++) sh.pv[w][8 * c + e] = acc[e];
    }
    __syncthreads();
    if (tid < HD) out[(size_t)h * HD + tid] = (sh.pv[0][tid] + sh.pv[1][tid]) + (sh.pv[2][tid] + sh.pv[3][tid]);
    __syncthreads();
}

}  // namespace lbt
