// attn_common.h -- split-key GQA attention over the bf16 KV cache and the
// combine of its splits, shared by the standalone kernels, the decode GEMV's
// o-projection prologue and the persistent decode kernel, so all of them
// compute the same bits.
//
// The reference (crates/lb-model/src/model.rs:349-357) computes, per query
// row and head, scores = q.K^T * scaling over the visible keys 0..p (the
// causal mask of :316-328), softmax = exp(s - max) / sum, out = probs @ V.
// Here the vis = p + 1 keys are cut into
//   ks = max(kAttnMinKeys, ceil(vis / kAttnSplits)) keys per split,
//   ns = ceil(vis / ks) splits, split s holding keys s*ks .. s*ks + cnt - 1,
// one workgroup per (query head, split).  A split writes its max m_s, its
// exponential sum l_s and its unnormalised output o_s = sum_j exp(s_j - m_s) v_j;
// the combine (flash-decoding form of the same softmax) is
//   M = max_s m_s, f_s = exp(m_s - M), L = sum_s l_s f_s, out = (sum_s o_s f_s) / L.
//
// Float order (the oracle, oracle/lbt_oracle.c, mirrors it), LK = hd/8 lanes
// per key, 8 dims per lane, u the key index inside the split:
//   score:  lane c sums q[8c+e]*k[8c+e] over e = 0..7 by fused multiply-adds,
//           the LK lanes combine by an xor butterfly (m = LK/2 .. 1), then
//           * scaling;
//   l_s:    thread t adds exp(s_u - m_s) over u = t, t+256, ...; block_sum;
//   o_s:    thread (group G = t/LK, chunk c = t%LK) accumulates
//           exp(s_u - m_s) * v_u[8c+e] by fused multiply-adds over
//           u = G, G + 256/LK, ...; the 64/LK groups of a wavefront combine
//           by xor over the group index (m = 1, 2, ...), the four wavefronts
//           as (w0 + w1) + (w2 + w3);
//   combine: f_s = exp(m_s - M); L = xor butterfly (m = 8 .. 1) over the 16
//           split slots of l_s * f_s (0 past ns); O = fma(o_s, f_s, O) over
//           s = 0, 1, ...; out = O * (1 / L).
//
// Partials of one query row (nh heads, hidden H = nh*hd):
//   o  [kAttnSplits][H]          o_s of head h at [s][h*hd .. h*hd + hd)
//   ml [kAttnSplits][nh][2]      (m_s, l_s)
#pragma once
#include "lbt_device.h"
#include "lbt_internal.h"

namespace lbt {

template <int LK>
struct AttnShared {
    __align__(16) float qs[LK * 8];
    float rmax[4];
    float rsum[4];
    __align__(16) float pv[4][LK * 8];
};

// Splits of vis visible keys.
__host__ __device__ __forceinline__ int attn_splits(int vis) {
    const int ks = attn_split_keys(vis);
    return (vis + ks - 1) / ks;
}

// Split s of query head h for one query row at absolute position p (keys
// 0..p visible).  q: the row's q [nh * hd] (rotated); K0/V0: the cache rows
// of h's KV head; o/ml: the row's partials (layout above); sc: LDS scores
// [attn_split_keys(cap)].  KU: key passes whose K (and V) loads are in flight
// together.  The first 256 threads do the work; every thread of the
// workgroup must call it (shared barriers).  Splits past the last return at
// once.
//
// PDEV: the position is *pdev + p, read on the device.  The first K/V rows
// are then issued before it arrives, on the guess that the split holds
// kAttnMinKeys keys (every context up to kAttnSplits * kAttnMinKeys keys):
// rows s * kAttnMinKeys + k, clamped to the cache; if the position says
// otherwise the split is redone with the loads it needs (attention_split).
template <int LK>
__device__ __forceinline__ void attention_split(const float* q, int h, int nh, int s, int p, const uint16_t* K0,
                                                const uint16_t* V0, float scaling, float* o, float* ml, float* sc,
                                                AttnShared<LK>& sh);

template <int LK, int KU, bool PDEV = false>
__device__ __forceinline__ void attention_split_ku(const float* q, int h, int nh, int s, int p, const uint16_t* K0,
                                                   const uint16_t* V0, float scaling, float* o, float* ml, float* sc,
                                                   AttnShared<LK>& sh, const int* pdev = nullptr, int cap = 0) {
    constexpr int HD = LK * 8, GW = 64 / LK, NK = kThreads / LK;
    static_assert(!PDEV || KU * NK >= kAttnMinKeys, "one key pass covers a guessed split");
    const int tid = (int)threadIdx.x, w = tid >> 6, lane = tid & 63;
    const bool act = tid < kThreads;
    const int kslot = lane / LK, cc = lane % LK;  // score loop: key of this lane group, chunk
    const int grp = tid / LK, c = tid % LK;       // PV loop: key group, chunk
    // this lane's 8 q values (read directly: the 16 lane groups share the
    // row through the cache, no LDS pass), then the first batches of K and V
    // rows, all in flight together; the K/V loads are unconditional (rows
    // past the split re-read its last row and are masked out below), so the
    // compiler's waits count exactly
    const f32x4 qa = gload((const f32x4*)(q + (size_t)h * HD + 8 * cc));
    const f32x4 qb = gload((const f32x4*)(q + (size_t)h * HD + 8 * cc + 4));
    uint4 kb[KU], vb[KU];
    int vis, ks, ns, j0, cnt;
    auto split_of = [&]() {
        vis = p + 1;
        ks = attn_split_keys(vis);
        ns = (vis + ks - 1) / ks;
        j0 = s * ks;
        cnt = vis - j0 < ks ? vis - j0 : ks;
    };
    if constexpr (PDEV) {
        const int g0 = s * kAttnMinKeys;
#pragma unroll
        for (int u = 0; u < KU; u++) {
            const int k = g0 + u * NK + w * GW + kslot;
            kb[u] = *(const uint4*)(K0 + (size_t)(k < cap ? k : cap - 1) * HD + 8 * cc);
        }
#pragma unroll
        for (int u = 0; u < KU; u++) {
            const int k = g0 + grp + u * NK;
            vb[u] = *(const uint4*)(V0 + (size_t)(k < cap ? k : cap - 1) * HD + 8 * c);
        }
        p += gload(pdev);
        split_of();
        if (s >= ns) return;
        if (ks != kAttnMinKeys) {
            attention_split<LK>(q, h, nh, s, p, K0, V0, scaling, o, ml, sc, sh);
            return;
        }
    } else {
        split_of();
        if (s >= ns) return;
#pragma unroll
        for (int u = 0; u < KU; u++) {
            const int k = u * NK + w * GW + kslot;
            kb[u] = *(const uint4*)(K0 + ((size_t)j0 + (k < cnt ? k : cnt - 1)) * HD + 8 * cc);
        }
#pragma unroll
        for (int u = 0; u < KU; u++) {
            const int k = grp + u * NK;
            vb[u] = *(const uint4*)(V0 + ((size_t)j0 + (k < cnt ? k : cnt - 1)) * HD + 8 * c);
        }
    }
    const uint16_t* K = K0 + (size_t)j0 * HD;
    const uint16_t* V = V0 + (size_t)j0 * HD;
    const float q8[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};

    // ---- scores and the split max
    float mx = -__builtin_inff();
    if (act) {
        for (int b0 = 0;; b0 += KU * NK) {
            if (b0 > 0) {
#pragma unroll
                for (int u = 0; u < KU; u++) {
                    const int k = b0 + u * NK + w * GW + kslot;
                    kb[u] = k < cnt ? *(const uint4*)(K + (size_t)k * HD + 8 * cc) : make_uint4(0, 0, 0, 0);
                }
            }
#pragma unroll
            for (int u = 0; u < KU; u++) {
                const int k = b0 + u * NK + w * GW + kslot;
                const uint32_t wv[4] = {kb[u].x, kb[u].y, kb[u].z, kb[u].w};
                float a = 0.0f;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    a = __builtin_fmaf(q8[2 * e], bf16_to_f32((uint16_t)(wv[e] & 0xffffu)), a);
                    a = __builtin_fmaf(q8[2 * e + 1], bf16_to_f32((uint16_t)(wv[e] >> 16)), a);
                }
                a = xor_sum_down<LK / 2>(a);
                if (k < cnt) {
                    const float sv = a * scaling;
                    if (cc == 0) sc[k] = sv;
                    mx = fmaxf(mx, sv);
                }
            }
            if (b0 + KU * NK >= cnt) break;
        }
    }
    mx = wave_max(mx);
    if (lane == 0 && w < 4) sh.rmax[w] = mx;
    __syncthreads();  // publishes the scores and the wave maxima
    const float m = fmaxf(fmaxf(sh.rmax[0], sh.rmax[1]), fmaxf(sh.rmax[2], sh.rmax[3]));
    float ps = 0.0f;
    if (act)
        for (int u = tid; u < cnt; u += kThreads) {
            const float e = lbt_expf(sc[u] - m);
            sc[u] = e;
            ps = ps + e;
        }
    ps = wave_sum(ps);
    if (lane == 0 && w < 4) sh.rsum[w] = ps;
    __syncthreads();  // publishes the exponentials and the wave sums

    // ---- unnormalised probs @ V
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; e++) acc[e] = 0.0f;
    if (act) {
        for (int b0 = 0;; b0 += KU * NK) {
            if (b0 > 0) {
#pragma unroll
                for (int u = 0; u < KU; u++) {
                    const int k = b0 + grp + u * NK;
                    vb[u] = k < cnt ? *(const uint4*)(V + (size_t)k * HD + 8 * c) : make_uint4(0, 0, 0, 0);
                }
            }
#pragma unroll
            for (int u = 0; u < KU; u++) {
                const int k = b0 + grp + u * NK;
                if (k < cnt) {
                    const float pj = sc[k];
                    const uint32_t wv[4] = {vb[u].x, vb[u].y, vb[u].z, vb[u].w};
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        acc[2 * e] = __builtin_fmaf(pj, bf16_to_f32((uint16_t)(wv[e] & 0xffffu)), acc[2 * e]);
                        acc[2 * e + 1] = __builtin_fmaf(pj, bf16_to_f32((uint16_t)(wv[e] >> 16)), acc[2 * e + 1]);
                    }
                }
            }
            if (b0 + KU * NK >= cnt) break;
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
    // ---- this split's partial
    if (act && tid < HD)
        o[(size_t)s * nh * HD + (size_t)h * HD + tid] =
            (sh.pv[0][tid] + sh.pv[1][tid]) + (sh.pv[2][tid] + sh.pv[3][tid]);
    if (tid == 0) {
        ml[((size_t)s * nh + h) * 2] = m;
        ml[((size_t)s * nh + h) * 2 + 1] = (sh.rsum[0] + sh.rsum[1]) + (sh.rsum[2] + sh.rsum[3]);
    }
}

// attention_split_ku with the load batch sized to the split: four key passes
// for short splits, eight for long ones.
template <int LK>
__device__ __forceinline__ void attention_split(const float* q, int h, int nh, int s, int p, const uint16_t* K0,
                                                const uint16_t* V0, float scaling, float* o, float* ml, float* sc,
                                                AttnShared<LK>& sh) {
    if (attn_split_keys(p + 1) <= 4 * (kThreads / LK))
        attention_split_ku<LK, 4>(q, h, nh, s, p, K0, V0, scaling, o, ml, sc, sh);
    else
        attention_split_ku<LK, 8>(q, h, nh, s, p, K0, V0, scaling, o, ml, sc, sh);
}

// ---------------------------------------------------------------------------
// The same split for the GH query heads h = g*GH .. g*GH + GH-1 that read KV
// head g, in one workgroup: every K/V row is loaded once for all of them.
// Per head the arithmetic and its order are those of attention_split_ku, so
// both produce the same partials.
template <int LK, int GH>
struct AttnGroupShared {
    __align__(16) float qs[GH][LK * 8];
    float rmax[GH][4];
    float rsum[GH][4];
    __align__(16) float pv[4][GH][LK * 8];
};

// K/V rows of a group split are read once per step: nontemporal loads
// (cache-policy bit 1), measured 7% faster than cached ones at 64 sequences x
// 4096 keys.
constexpr int kAttnNT = 2;

// Score rows of a group split are padded to whole key passes of the widest
// pass (KU = 8): the passes run over them without per-key masks (buffer
// loads past the split's keys return zeros, their scores are set to p = 0,
// and fma(0, 0, acc) = acc: acc is never -0, starting at +0 and adding
// products of p >= 0).
__host__ __device__ constexpr int attn_group_pass_keys(int lk) { return 8 * (kThreads / lk); }
__host__ __device__ inline int attn_group_score_keys(int ks, int lk) {
    const int pk = attn_group_pass_keys(lk);
    return (ks + pk - 1) / pk * pk;
}

// Head slot of lane cc after log2(GH) halving steps: each lane holds its q
// values permuted by it (slot j = head j ^ hh), so every halving step adds
// slot j of its own to slot j + half of the partner lane -- the same head --
// with no select.
template <int M, int K>
__device__ __forceinline__ void halve_slots(const float (&v)[K], float (&o)[K / 2]) {
#pragma unroll
    for (int j = 0; j < K / 2; j++) {
        uint32_t a, b;
        xor_pair<M>(__float_as_uint(v[j + K / 2]), a, b);  // b: the partner's slot j + K/2
        o[j] = v[j] + __uint_as_float(b);
    }
}

// q . k of one key for the GH heads of a group: lane cc of the key's LK lanes
// holds its 8 dims of each head (permuted by its head slot, q8[j] = head
// j ^ hh) and the key's 8 bf16 values kv; fused multiply-adds in dim order,
// then the first log2(GH) butterfly steps by recursive halving (lane cc ends
// with head hh = cc / (LK / GH)), the rest as a butterfly.  Returns head hh's
// score (every lane of the key active).
template <int LK, int GH>
__device__ __forceinline__ float attn_group_score(const u32x4& kv, const float (&q8)[GH][8]) {
    const uint32_t wv[4] = {kv.x, kv.y, kv.z, kv.w};
    float a[GH];
#pragma unroll
    for (int h = 0; h < GH; h++) {
        a[h] = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            a[h] = __builtin_fmaf(q8[h][2 * e], bf16_to_f32((uint16_t)(wv[e] & 0xffffu)), a[h]);
            a[h] = __builtin_fmaf(q8[h][2 * e + 1], bf16_to_f32((uint16_t)(wv[e] >> 16)), a[h]);
        }
    }
    if constexpr (GH == 1) {
        return xor_sum_down<LK / 2>(a[0]);
    } else if constexpr (GH == 2) {
        float h1[1];
        halve_slots<LK / 2>(a, h1);
        return xor_sum_down<LK / 4>(h1[0]);
    } else {
        static_assert(GH == 4, "1, 2 or 4 heads per group");
        float h2[2], h1[1];
        halve_slots<LK / 2>(a, h2);
        halve_slots<LK / 4>(h2, h1);
        return xor_sum_down<LK / 8>(h1[0]);
    }
}

// acc[h][e] += p[h] * v[8 cc + e] for the 8 bf16 values of one V row chunk.
template <int GH>
__device__ __forceinline__ void attn_group_pv(const u32x4& vv, const float (&pj)[GH], float (&acc)[GH][8]) {
    const uint32_t wv[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
    for (int h = 0; h < GH; h++) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            acc[h][2 * e] = __builtin_fmaf(pj[h], bf16_to_f32((uint16_t)(wv[e] & 0xffffu)), acc[h][2 * e]);
            acc[h][2 * e + 1] = __builtin_fmaf(pj[h], bf16_to_f32((uint16_t)(wv[e] >> 16)), acc[h][2 * e + 1]);
        }
    }
}

template <int LK, int GH, int KU>
__device__ __forceinline__ void attention_split_group(const float* q, int g, int nh, int s, int p, const uint16_t* K0,
                                                      const uint16_t* V0, float scaling, float* o, float* ml,
                                                      float* sc, AttnGroupShared<LK, GH>& sh) {
    constexpr int HD = LK * 8, GW = 64 / LK, NK = kThreads / LK;
    const int vis = p + 1;
    const int ks = attn_split_keys(vis);
    const int ns = (vis + ks - 1) / ks;
    if (s >= ns) return;
    const int j0 = s * ks, cnt = vis - j0 < ks ? vis - j0 : ks;
    const int tid = (int)threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int kslot = lane / LK, cc = lane % LK;
    const int grp = tid / LK, c = tid % LK;
    constexpr int LPH = LK / GH;  // lanes per head after the halving
    const int hh = cc / LPH;
    // the split's K and V rows as buffers: rows past cnt read as zeros
    const __amdgpu_buffer_rsrc_t kr = buf_rsrc(K0 + (size_t)j0 * HD, (uint32_t)cnt * HD * 2u);
    const __amdgpu_buffer_rsrc_t vr = buf_rsrc(V0 + (size_t)j0 * HD, (uint32_t)cnt * HD * 2u);
    const uint32_t koff = (uint32_t)((w * GW + kslot) * HD + 8 * cc) * 2u;
    const uint32_t voff = (uint32_t)(grp * HD + 8 * c) * 2u;
    constexpr int QPT = (GH * HD + kThreads - 1) / kThreads;
    float qv[QPT];
#pragma unroll
    for (int i = 0; i < QPT; i++) {
        const int idx = tid + i * kThreads;
        qv[i] = idx < GH * HD ? q[(size_t)g * GH * HD + idx] : 0.0f;
    }
    // K and V rows go through two register buffers each: the next key pass's
    // loads are in flight while a pass computes
    u32x4 kb[2][KU], vb[2][KU];
    auto k_load = [&](int b0, u32x4 (&dst)[KU]) {
#pragma unroll
        for (int u = 0; u < KU; u++)
            dst[u] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, koff, (uint32_t)(b0 + u * NK) * HD * 2u, kAttnNT));
    };
    auto v_load = [&](int b0, u32x4 (&dst)[KU]) {
#pragma unroll
        for (int u = 0; u < KU; u++)
            dst[u] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(vr, voff, (uint32_t)(b0 + u * NK) * HD * 2u, kAttnNT));
    };
    constexpr int STEP = KU * NK;
    k_load(0, kb[0]);
    v_load(0, vb[0]);
#pragma unroll
    for (int i = 0; i < QPT; i++) {
        const int idx = tid + i * kThreads;
        if (idx < GH * HD) (&sh.qs[0][0])[idx] = qv[i];
    }
    __syncthreads();
    float q8[GH][8];
#pragma unroll
    for (int j = 0; j < GH; j++)
#pragma unroll
        for (int e = 0; e < 8; e++) q8[j][e] = sh.qs[j ^ hh][8 * cc + e];

    // The GH scores of a key reduce over the key's LK lanes together: the
    // first log2(GH) butterfly steps by recursive halving (lane cc ends with
    // head hh), the rest as a butterfly; the same sums, bit for bit, as a
    // butterfly per head.  A lane keeps the running max of its head.
    float mxo = -__builtin_inff();
    auto k_pass = [&](int b0, const u32x4 (&kbuf)[KU]) {
#pragma unroll
        for (int u = 0; u < KU; u++) {
            const int k = b0 + u * NK + w * GW + kslot;
            const float sv = attn_group_score<LK, GH>(kbuf[u], q8) * scaling;
            const bool kin = k < cnt;
            if (kin && cc % LPH == 0) sc[k * GH + hh] = sv;
            mxo = fmaxf(mxo, kin ? sv : -__builtin_inff());
        }
    };
    for (int b0 = 0;; b0 += 2 * STEP) {
        k_load(b0 + STEP, kb[1]);
        k_pass(b0, kb[0]);
        if (b0 + STEP >= cnt) break;
        k_load(b0 + 2 * STEP, kb[0]);
        k_pass(b0 + STEP, kb[1]);
        if (b0 + 2 * STEP >= cnt) break;
    }
#pragma unroll
    for (int h = 0; h < GH; h++) {
        const float v = wave_max(hh == h ? mxo : -__builtin_inff());
        if (lane == 0) sh.rmax[h][w] = v;
    }
    __syncthreads();
    // exponentials, all GH heads of a key at once; keys past cnt (up to the
    // passes' extent) get p = 0
    {
        float m[GH], ps[GH];
#pragma unroll
        for (int h = 0; h < GH; h++) {
            m[h] = fmaxf(fmaxf(sh.rmax[h][0], sh.rmax[h][1]), fmaxf(sh.rmax[h][2], sh.rmax[h][3]));
            ps[h] = 0.0f;
        }
        const int ext = (cnt + STEP - 1) / STEP * STEP;
        for (int u = tid; u < ext; u += kThreads) {
            float* sp = sc + u * GH;
            float e[GH];
            if (u < cnt) {
#pragma unroll
                for (int h = 0; h < GH; h++) {
                    e[h] = lbt_expf(sp[h] - m[h]);
                    ps[h] = ps[h] + e[h];
                }
            } else {
#pragma unroll
                for (int h = 0; h < GH; h++) e[h] = 0.0f;
            }
#pragma unroll
            for (int h = 0; h < GH; h++) sp[h] = e[h];
        }
#pragma unroll
        for (int h = 0; h < GH; h++) {
            const float t = wave_sum(ps[h]);
            if (lane == 0) sh.rsum[h][w] = t;
        }
    }
    __syncthreads();

    float acc[GH][8];
#pragma unroll
    for (int h = 0; h < GH; h++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[h][e] = 0.0f;
    auto v_pass = [&](int b0, const u32x4 (&vbuf)[KU]) {
#pragma unroll
        for (int u = 0; u < KU; u++) {
            const int k = b0 + grp + u * NK;
            float pj[GH];
            if constexpr (GH == 4) {
                const float4 t = *(const float4*)(sc + k * 4);
                pj[0] = t.x;
                pj[1 % GH] = t.y;
                pj[2 % GH] = t.z;
                pj[3 % GH] = t.w;
            } else {
#pragma unroll
                for (int h = 0; h < GH; h++) pj[h] = sc[k * GH + h];
            }
            attn_group_pv<GH>(vbuf[u], pj, acc);
        }
    };
    for (int b0 = 0;; b0 += 2 * STEP) {
        v_load(b0 + STEP, vb[1]);
        v_pass(b0, vb[0]);
        if (b0 + STEP >= cnt) break;
        v_load(b0 + 2 * STEP, vb[0]);
        v_pass(b0 + STEP, vb[1]);
        if (b0 + 2 * STEP >= cnt) break;
    }
    if constexpr (GW > 1) {
#pragma unroll
        for (int h = 0; h < GH; h++)
#pragma unroll
            for (int e = 0; e < 8; e++) acc[h][e] = xor_sum_up<LK>(acc[h][e]);
    }
    if (lane < LK) {
#pragma unroll
        for (int h = 0; h < GH; h++)
#pragma unroll
            for (int e = 0; e < 8; e++) sh.pv[w][h][8 * c + e] = acc[h][e];
    }
    __syncthreads();
    for (int idx = tid; idx < GH * HD; idx += kThreads) {
        const int h = idx / HD, d = idx % HD;
        o[(size_t)s * nh * HD + (size_t)(g * GH + h) * HD + d] =
            (sh.pv[0][h][d] + sh.pv[1][h][d]) + (sh.pv[2][h][d] + sh.pv[3][h][d]);
    }
    if (tid < GH) {
        const int h = tid;
        ml[((size_t)s * nh + g * GH + h) * 2] =
            fmaxf(fmaxf(sh.rmax[h][0], sh.rmax[h][1]), fmaxf(sh.rmax[h][2], sh.rmax[h][3]));
        ml[((size_t)s * nh + g * GH + h) * 2 + 1] = (sh.rsum[h][0] + sh.rsum[h][1]) + (sh.rsum[h][2] + sh.rsum[h][3]);
    }
}

// ---------------------------------------------------------------------------
// The split of attention_split_group<LK, GH, .> on ONE wavefront, with the
// same partials bit for bit: the four wavefronts of that workgroup become
// four virtual wavefronts of this one, and no barrier is needed, so the
// wavefronts of a workgroup are independent (row, KV head, split) tasks --
// a long prefill runs four times as many of its short split chains at a
// time.  The order, as in the workgroup form:
//   * key k's score by the LK lanes (kslot = k mod 64/LK) of pass k / (64/LK),
//     attn_group_score; virtual wavefront v = (k / (64/LK)) mod 4 of the
//     workgroup form is the one that held key k, so each lane keeps one
//     running max per v and the head max is the max of the four wave maxima;
//   * exponentials of keys u = 64 v + lane, +256, ... summed per virtual
//     thread in that order, each virtual wavefront's sums reduced by
//     wave_sum, l = (l_0 + l_1) + (l_2 + l_3);
//   * PV: key group grp = 4 v + lane / LK (16 groups of LK lanes) accumulates
//     keys grp, grp + 16, ... by attn_group_pv; per virtual wavefront the
//     groups combine by xor_sum_up<LK>, o = (o_0 + o_1) + (o_2 + o_3).
// Keys past cnt read zero (bounded buffer loads) and get p = 0 (fma(0, 0,
// acc) = acc, acc never -0), so the padding differs from the workgroup form
// without changing a bit.  Cached K/V loads (prefill rows re-read them).
// sc: this wavefront's [ceil16(ks)][GH] score / exponential buffer in LDS.
template <int LK, int GH>
__device__ __forceinline__ void attention_split_wave(const float* q, int g, int nh, int s, int p, const uint16_t* K0,
                                                     const uint16_t* V0, float scaling, float* o, float* ml,
                                                     float* sc) {
    static_assert(LK == 16 && GH == 4, "four keys per pass (head_dim 128), four query heads per KV head");
    constexpr int HD = LK * 8, KPP = 64 / LK, LPH = LK / GH, NG = kThreads / LK;
    const int vis = p + 1;
    const int ks = attn_split_keys(vis);
    const int ns = (vis + ks - 1) / ks;
    if (s >= ns) return;
    const int j0 = s * ks, cnt = vis - j0 < ks ? vis - j0 : ks;
    const int lane = (int)threadIdx.x & 63, kslot = lane / LK, cc = lane % LK, hh = cc / LPH;
    const __amdgpu_buffer_rsrc_t kr = buf_rsrc(K0 + (size_t)j0 * HD, (uint32_t)cnt * HD * 2u);
    const __amdgpu_buffer_rsrc_t vr = buf_rsrc(V0 + (size_t)j0 * HD, (uint32_t)cnt * HD * 2u);
    const uint32_t loff = (uint32_t)(kslot * HD + 8 * cc) * 2u;  // this lane's chunk of its key / V row
    float q8[GH][8];
#pragma unroll
    for (int j = 0; j < GH; j++) {
        const float* qj = q + (size_t)(g * GH + (j ^ hh)) * HD + 8 * cc;
        const f32x4 a = *(const f32x4*)qj, b = *(const f32x4*)(qj + 4);
        q8[j][0] = a.x, q8[j][1] = a.y, q8[j][2] = a.z, q8[j][3] = a.w;
        q8[j][4] = b.x, q8[j][5] = b.y, q8[j][6] = b.z, q8[j][7] = b.w;
    }
    // scores: passes of KPP keys, in batches of 4 passes (4 loads in flight)
    constexpr int PB = 4;

    const int npass = (cnt + KPP - 1) / KPP;
    float mxo[4] = {-__builtin_inff(), -__builtin_inff(), -__builtin_inff(), -__builtin_inff()};
#pragma unroll 1
    for (int pb = 0; pb < npass; pb += PB) {
        u32x4 kb[PB];
#pragma unroll
        for (int i = 0; i < PB; i++)
            kb[i] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, loff, (uint32_t)((pb + i) * KPP) * HD * 2u, 0));
#pragma unroll
        for (int i = 0; i < PB; i++) {
            const int k = (pb + i) * KPP + kslot;
            const float sv = attn_group_score<LK, GH>(kb[i], q8) * scaling;
            const bool kin = k < cnt;
            if (kin && cc % LPH == 0) sc[k * GH + hh] = sv;
            // pass pb + i of this wavefront is pass (pb + i) / 4 of virtual wavefront (pb + i) mod 4
            mxo[i & 3] = fmaxf(mxo[i & 3], kin ? sv : -__builtin_inff());
        }
    }
    // the head max over the four virtual wavefronts' running maxima (a max
    // does not depend on the order; only the sign of a zero max could, and
    // exp(s - m) and every later value are the same with either)
    float m[GH];
    {
        const float mx = fmaxf(fmaxf(mxo[0], mxo[1]), fmaxf(mxo[2], mxo[3]));
#pragma unroll
        for (int h = 0; h < GH; h++) m[h] = wave_max(hh == h ? mx : -__builtin_inff());
    }
    asm volatile("" ::: "memory");  // the score stores before the reads below (LDS is in order per wavefront)
    // exponentials; keys cnt .. ext16 - 1 get p = 0
    const int ext = (cnt + NG - 1) / NG * NG;
    float lsum[GH];
    {
        float ls[4][GH];
#pragma unroll
        for (int v = 0; v < 4; v++) {
            float ps[GH];
#pragma unroll
            for (int h = 0; h < GH; h++) ps[h] = 0.0f;
            if (64 * v >= ext) {  // no key: the sums are +0 (uniform branch)
#pragma unroll
                for (int h = 0; h < GH; h++) ls[v][h] = 0.0f;
                continue;
            }
            for (int u = 64 * v + lane; u < ext; u += kThreads) {
                float* sp = sc + u * GH;
                float e[GH];
                if (u < cnt) {
#pragma unroll
                    for (int h = 0; h < GH; h++) {
                        e[h] = lbt_expf(sp[h] - m[h]);
                        ps[h] = ps[h] + e[h];
                    }
                } else {
#pragma unroll
                    for (int h = 0; h < GH; h++) e[h] = 0.0f;
                }
#pragma unroll
                for (int h = 0; h < GH; h++) sp[h] = e[h];
            }
#pragma unroll
            for (int h = 0; h < GH; h++) ls[v][h] = wave_sum(ps[h]);
        }
#pragma unroll
        for (int h = 0; h < GH; h++) lsum[h] = (ls[0][h] + ls[1][h]) + (ls[2][h] + ls[3][h]);
    }
    asm volatile("" ::: "memory");  // the exponential stores before the PV reads
    // PV per virtual wavefront v: this lane's group 4 v + kslot takes keys
    // 16 u + 4 v + kslot, u ascending; the groups then combine as
    // xor_sum_up<LK> does ((g0 + g1) + (g2 + g3): steps 16, then 32), here by
    // recursive halving, which leaves lane (kslot, cc) the sum for head
    // hv = (kslot >> 1) + 2 (kslot & 1), dims 8 cc .. 8 cc + 7
    const int nu = ext / NG;
    auto pv_v = [&](int v, float (&r)[8]) {
        constexpr int VB = 4;
        float acc[GH][8];
#pragma unroll
        for (int h = 0; h < GH; h++)
#pragma unroll
            for (int e = 0; e < 8; e++) acc[h][e] = 0.0f;
#pragma unroll 1
        for (int ub = 0; ub < nu; ub += VB) {
            u32x4 vb[VB];
#pragma unroll
            for (int i = 0; i < VB; i++)
                vb[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                      vr, loff, (uint32_t)((ub + i) * NG + 4 * v) * HD * 2u, 0));
#pragma unroll
            for (int i = 0; i < VB; i++) {
                if (ub + i >= nu) break;
                const int k = (ub + i) * NG + 4 * v + kslot;
                const float4 t = *(const float4*)(sc + k * 4);
                const float pj[GH] = {t.x, t.y, t.z, t.w};
                attn_group_pv<GH>(vb[i], pj, acc);
            }
        }
        float flat[GH * 8], h16[16];
#pragma unroll
        for (int h = 0; h < GH; h++)
#pragma unroll
            for (int e = 0; e < 8; e++) flat[h * 8 + e] = acc[h][e];
        halve<16, GH * 8>(flat, h16);
        halve<32, 16>(h16, r);
    };
    float r[8], o01[8], o23[8];
    pv_v(0, r);
#pragma unroll
    for (int e = 0; e < 8; e++) o01[e] = r[e];
    pv_v(1, r);
#pragma unroll
    for (int e = 0; e < 8; e++) o01[e] = o01[e] + r[e];
    pv_v(2, r);
#pragma unroll
    for (int e = 0; e < 8; e++) o23[e] = r[e];
    pv_v(3, r);
    {
        const int hv = (kslot >> 1) + 2 * (kslot & 1);
        float* od = o + (size_t)s * nh * HD + (size_t)(g * GH + hv) * HD + 8 * cc;
        float fv[8];
#pragma unroll
        for (int e = 0; e < 8; e++) fv[e] = o01[e] + (o23[e] + r[e]);
        *(f32x4*)od = f32x4{fv[0], fv[1], fv[2], fv[3]};
        *(f32x4*)(od + 4) = f32x4{fv[4], fv[5], fv[6], fv[7]};
    }
    if (lane < GH) {
        const int h = lane;
        float mh = m[0], lh = lsum[0];
#pragma unroll
        for (int j = 1; j < GH; j++)
            if (h == j) mh = m[j], lh = lsum[j];
        ml[((size_t)s * nh + g * GH + h) * 2] = mh;
        ml[((size_t)s * nh + g * GH + h) * 2 + 1] = lh;
    }
}

// ---------------------------------------------------------------------------
// Combine of one row's splits, as a row source for the activation prologues.
// Thread t (< NT) produces the row elements of RowRegs (groups of four,
// v[4g + k] = att[4 NT g + 4 t + k]).  attn_row_issue starts the loads (the
// first NSB splits of the outputs, the (m, l) pairs and the norm weights);
// attn_row_finish builds the per-(head, split) factors in LDS and combines.
// The issue does not depend on the split count (a.ns is read by the finish
// only): the first NSB splits and all (m, l) slots are loaded (the partial
// buffers hold kAttnSplits splits), entries past the row's splits unused.
struct AttnRow {
    const float* o;   // [kAttnSplits][H]
    const float* ml;  // [kAttnSplits][nh][2]
    int ns;           // splits of this row
    int nh, hd, H;
};

// (head, split) pairs per thread
template <int NT>
constexpr int attn_pair_slots() {
    return (kAttnMaxHeads * kAttnSplits + NT - 1) / NT;
}

template <int EPT, int NSB, int NT = kThreads>
struct AttnRegs {
    f32x4 ov[EPT / 4][NSB];
    f32x2 mlv[attn_pair_slots<NT>()];
};

// LDS of the combine: f per (head, split) and 1 / L per head.
struct AttnTab {
    float f[kAttnMaxHeads][kAttnSplits];
    float L[kAttnMaxHeads];
};

template <int EPT, int NSB, int NT = kThreads>
__device__ __forceinline__ void attn_row_issue(const AttnRow& a, const float* norm_w, AttnRegs<EPT, NSB, NT>& ar,
                                               RowRegs<EPT>& r) {
    const int tid = (int)threadIdx.x;
    const bool act = tid < NT;
#pragma unroll
    for (int g = 0; g < EPT / 4; g++) {
        const int i0 = 4 * NT * g + 4 * tid;
#pragma unroll
        for (int s = 0; s < NSB; s++)
            ar.ov[g][s] = (act && i0 < a.H) ? gload((const f32x4*)(a.o + (size_t)s * a.H + i0))
                                            : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if (norm_w && act && i0 < a.H) {
            const f32x4 wv = gload((const f32x4*)(norm_w + i0));
            r.nw[4 * g] = wv.x;
            r.nw[4 * g + 1] = wv.y;
            r.nw[4 * g + 2] = wv.z;
            r.nw[4 * g + 3] = wv.w;
        } else {
#pragma unroll
            for (int k = 0; k < 4; k++) r.nw[4 * g + k] = 0.0f;
        }
    }
#pragma unroll
    for (int j = 0; j < attn_pair_slots<NT>(); j++) {
        const int pi = tid + j * NT, h = pi / kAttnSplits, s = pi % kAttnSplits;
        ar.mlv[j] = (act && h < a.nh) ? gload((const f32x2*)(a.ml + ((size_t)s * a.nh + h) * 2))
                                      : f32x2{0.0f, 0.0f};
    }
}

// attn_row_finish in two steps around its barrier: attn_row_tab builds the
// per-(head, split) factors in LDS, attn_row_combine (after a barrier) forms
// the row.  Threads past NT take no part in either (a caller may skip them
// for whole wavefronts).
template <int EPT, int NSB, int NT = kThreads>
__device__ __forceinline__ void attn_row_tab(const AttnRow& a, AttnRegs<EPT, NSB, NT>& ar, AttnTab& tab) {
    const int tid = (int)threadIdx.x;
    const bool act = tid < NT;
    // (head, split) pairs sit in 16 consecutive lanes per head: M, the split
    // factors f_s and L come from lane butterflies, no LDS round trip
    static_assert(kAttnSplits == 16 && NT % kAttnSplits == 0, "16-lane head segments");
#pragma unroll
    for (int j = 0; j < attn_pair_slots<NT>(); j++) {
        const int pi = tid + j * NT, h = pi / kAttnSplits, s = pi % kAttnSplits;
        if (j * NT >= a.nh * kAttnSplits) break;  // uniform
        const bool live = act && h < a.nh && s < a.ns;
        const float m = live ? ar.mlv[j].x : -__builtin_inff();
        float M = xor_max<8>(m);
        M = xor_max<4>(M);
        M = xor_max<2>(M);
        M = xor_max<1>(M);
        const float f = live ? lbt_expf(m - M) : 0.0f;
        const float L = xor_sum_down<8>(live ? ar.mlv[j].y * f : 0.0f);
        if (act && h < a.nh) {
            tab.f[h][s] = f;
            if (s == 0) tab.L[h] = 1.0f / L;
        }
    }
}

template <int EPT, int NSB, int NT = kThreads>
__device__ __forceinline__ void attn_row_combine(const AttnRow& a, AttnRegs<EPT, NSB, NT>& ar, RowRegs<EPT>& r,
                                                 const AttnTab& tab) {
    const int tid = (int)threadIdx.x;
    const bool act = tid < NT;
    const int hs = __builtin_ctz((unsigned)a.hd);  // head_dim is a power of two
    float O[EPT];
#pragma unroll
    for (int e = 0; e < EPT; e++) O[e] = 0.0f;
    auto accumulate = [&](const f32x4 (&ov)[EPT / 4][NSB], int s0) {
#pragma unroll
        for (int g = 0; g < EPT / 4; g++) {
            const int i0 = 4 * NT * g + 4 * tid;
            if (!act || i0 >= a.H) continue;
            const float* fh = tab.f[i0 >> hs];
#pragma unroll
            for (int s = 0; s < NSB; s++) {
                // selects, not branches: splits past ns leave O unchanged
                const bool live = s0 + s < a.ns;
                const float f = fh[(s0 + s) & (kAttnSplits - 1)];
                O[4 * g] = live ? __builtin_fmaf(ov[g][s].x, f, O[4 * g]) : O[4 * g];
                O[4 * g + 1] = live ? __builtin_fmaf(ov[g][s].y, f, O[4 * g + 1]) : O[4 * g + 1];
                O[4 * g + 2] = live ? __builtin_fmaf(ov[g][s].z, f, O[4 * g + 2]) : O[4 * g + 2];
                O[4 * g + 3] = live ? __builtin_fmaf(ov[g][s].w, f, O[4 * g + 3]) : O[4 * g + 3];
            }
        }
    };
    accumulate(ar.ov, 0);  // the splits loaded by attn_row_issue
    for (int s0 = NSB; s0 < a.ns; s0 += NSB) {
        f32x4 ov[EPT / 4][NSB];
#pragma unroll
        for (int g = 0; g < EPT / 4; g++) {
            const int i0 = 4 * NT * g + 4 * tid;
#pragma unroll
            for (int s = 0; s < NSB; s++)
                ov[g][s] = (act && i0 < a.H && s0 + s < a.ns) ? gload((const f32x4*)(a.o + (size_t)(s0 + s) * a.H + i0))
                                                              : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        accumulate(ov, s0);
    }
#pragma unroll
    for (int g = 0; g < EPT / 4; g++) {
        const int i0 = 4 * NT * g + 4 * tid;
        const bool in = act && i0 < a.H;
        const float rl = in ? tab.L[i0 >> hs] : 0.0f;
#pragma unroll
        for (int k = 0; k < 4; k++) r.v[4 * g + k] = O[4 * g + k] * rl;
    }
}

template <int EPT, int NSB, int NT = kThreads>
__device__ __forceinline__ void attn_row_finish(const AttnRow& a, AttnRegs<EPT, NSB, NT>& ar, RowRegs<EPT>& r,
                                                AttnTab& tab) {
    attn_row_tab<EPT, NSB, NT>(a, ar, tab);
    __syncthreads();
    attn_row_combine<EPT, NSB, NT>(a, ar, r, tab);
}

}  // namespace lbt
