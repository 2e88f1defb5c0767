// decode_step.hip -- the 30 decoder layers of one batch-1 decode token in one
// dispatch (BitNet::forward for one token, crates/lb-model/src/model.rs:331-366),
// on a persistent grid of one 256-thread workgroup per compute unit.
//
// Why one dispatch: at batch 1 every matrix is small (1.6-8.8 MB, 0.2-1.1 us
// of HBM time) and the step is a chain of 150 dependent phases.  A kernel
// boundary costs ~2.9 us per phase on this part even for trivial kernels; a
// device-coherent store -> load hop between two workgroups costs ~0.5 us.
//
// How phases hand data over: every activation vector that crosses
// workgroups (x, q/k/v, the attention partials, h) lives in a buffer of
// 64-bit words {epoch << 32 | f32 bits}, written with device-scope stores and
// read with device-scope loads.  A consumer polls exactly the words it needs
// until each carries the epoch of the producing phase: the value and its
// readiness arrive together, so there is no barrier, no flag and no fence.
// Epochs grow by one per phase for the lifetime of the model (state[2] keeps
// the base between dispatches).  A buffer is rewritten only after every
// reader of its previous contents has finished: each phase consumes all of
// the previous phase's outputs (attention: all partials feed every
// o-projection workgroup), so the phase two steps later cannot start before
// the readers are done.
//
// Weights: each workgroup owns a fixed slice of rows of each of the four
// linears of a layer (q/k/v, o, gate/up, down) and keeps the next layer's
// slice in LDS (global_load_lds_dwordx4, issued right after the slice of the
// current layer has been consumed), so HBM is off the critical path; the
// per-phase work is the activation prologue, the dots from LDS and the
// epilogue.
//
// Arithmetic and float order are those of the multi-kernel path: the same
// prologue (quantize_row_regs, canonical RMSNorm order), the same dot
// identity (acc - sum(q)), the same epilogues, the same split attention and
// combine (attn_common.h), so results equal the oracle bit for bit.
//
// Every wait is bounded: after ~0.5 s without progress a workgroup sets the
// error word, every later wait returns at once, the grid drains and the host
// reports LBT_E_DEVICE.
#include "attn_common.h"
#include "ternary_common.h"
#include "decode_step.h"

// Measured slower than the multi-kernel graph step it equals bit for bit, so
// it is built only on request (LBT_WITH_STEP=1 in the build environment).
#if LBT_WITH_STEP

namespace lbt {

constexpr int kST = 256;  // threads per workgroup
typedef unsigned long long u64;

// ---- epoch-tagged words --------------------------------------------------
// (global address space: a flat store would also count on the LDS counter)
__device__ __forceinline__ void ll_put(u64* p, unsigned ep, float v) {
    __hip_atomic_store((LBT_GLOBAL u64*)p, ((u64)ep << 32) | (u64)__float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
// Two words (16-byte aligned) by a device-coherent load; untracked (waited
// for with vm_wait, then pin()).
__device__ __forceinline__ u32x4 ll_ld2(const u64* p) {
    u32x4 v;
    asm volatile("global_load_dwordx4 %0, %1, off sc1" : "=v"(v) : "v"(p) : "memory");
    return v;
}
__device__ __forceinline__ unsigned ld_err(const unsigned* p) {
    return __hip_atomic_load((const LBT_GLOBAL unsigned*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Bounded-wait bookkeeping of one wavefront.
struct Waiter {
    unsigned* err;
    unsigned long long t0;
    int spins;
    __device__ __forceinline__ void start() {
        t0 = wall_clock64();
        spins = 0;
    }
    // true: give up (timeout, or another workgroup reported one)
    __device__ __forceinline__ bool give_up() {
        if ((++spins & 31) != 0) return false;
        if (ld_err(err) != 0u) return true;
        if (wall_clock64() - t0 > 50000000ull) {  // 0.5 s of the 100 MHz clock
            if ((threadIdx.x & 63) == 0)
                __hip_atomic_fetch_or((LBT_GLOBAL unsigned*)err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return true;
        }
        return false;
    }
};

// Uniform values from device memory through the scalar unit: a pointer in
// the constant address space makes the loads scalar (they count on the
// scalar counter, not on the vector-memory counter that the weight loads into
// LDS are tracked by, so reading an argument never waits for those loads).
template <typename T>
__device__ __forceinline__ T kld(const T* p) {
    return *(const __attribute__((address_space(4))) T*)p;
}
__device__ __forceinline__ StepArgs kargs(const StepArgs* p) {
    static_assert(sizeof(StepArgs) % 4 == 0, "dword copy");
    const uint32_t* src = (const uint32_t*)launder(p);
    StepArgs r;
    uint32_t* dst = (uint32_t*)&r;
#pragma unroll
    for (int i = 0; i < (int)(sizeof(StepArgs) / 4); i++) dst[i] = kld(src + i);
    return r;
}

__device__ __forceinline__ uint4 ld_u4(const void* p) {
    const u32x4 v = gload((const u32x4*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ bool ready2(const u32x4& v, unsigned want) { return v.y == want && v.w == want; }

// Row of K words in the prologue's element layout (thread t holds groups
// t, t + 256, ...: RowRegs v[4g + k] = row[4 (256 g + t) + k]), polled until
// every word carries `want`.  K % 4 == 0.  Norm weights load alongside.
template <int EPT>
__device__ __forceinline__ void ll_row(const u64* src, int K, unsigned want, const float* nw, RowRegs<EPT>& r,
                                       Waiter& wt) {
    constexpr int NG = EPT / 4;
    const int tid = (int)threadIdx.x;
#pragma unroll
    for (int g = 0; g < NG; g++) {
        const int i0 = 4 * (kST * g + tid);
        if (i0 < K) {
            const f32x4 w4 = gload((const f32x4*)(nw + i0));
            r.nw[4 * g] = w4.x;
            r.nw[4 * g + 1] = w4.y;
            r.nw[4 * g + 2] = w4.z;
            r.nw[4 * g + 3] = w4.w;
        } else {
#pragma unroll
            for (int k = 0; k < 4; k++) r.nw[4 * g + k] = 0.0f;
        }
    }
    u32x4 v[NG][2];
    wt.start();
    for (;;) {
#pragma unroll
        for (int g = 0; g < NG; g++) {
            const int i0 = 4 * (kST * g + tid);
            const u64* p = src + (i0 < K ? i0 : 0);
            v[g][0] = ll_ld2(p);
            v[g][1] = ll_ld2(p + 2);
        }
        vm_wait<0>();
        bool ok = true;
#pragma unroll
        for (int g = 0; g < NG; g++) {
            pin(v[g][0]);
            pin(v[g][1]);
            const int i0 = 4 * (kST * g + tid);
            if (i0 < K) ok = ok && ready2(v[g][0], want) && ready2(v[g][1], want);
        }
        if (__all(ok) || wt.give_up()) break;
    }
#pragma unroll
    for (int g = 0; g < NG; g++) {
        const bool in = 4 * (kST * g + tid) < K;
        r.v[4 * g] = in ? __uint_as_float(v[g][0].x) : 0.0f;
        r.v[4 * g + 1] = in ? __uint_as_float(v[g][0].z) : 0.0f;
        r.v[4 * g + 2] = in ? __uint_as_float(v[g][1].x) : 0.0f;
        r.v[4 * g + 3] = in ? __uint_as_float(v[g][1].z) : 0.0f;
    }
}

// ---- phase tiling and weights in LDS ------------------------------------
typedef __attribute__((address_space(3))) void lds_void;

// Row table of a phase, built once per dispatch in LDS: entry t*64 + lane is
// (matrix << 30 | row) of the row that lane loads in tile t (lane l: row
// t*R + l/L, R = 64/L), matrix 0 / row 0 for lanes past the slice.
template <int OUT>
__device__ __forceinline__ void build_rowtab(const GemvArgs& g, const StepTile& T, int vr0, uint32_t* tab) {
    const int R = 64 / T.L, ntiles = (T.rpw + R - 1) / R;
    for (int e = (int)threadIdx.x; e < ntiles * 64; e += kST) {
        const int t = e >> 6, lane = e & 63;
        const int lr = t * R + lane / T.L, vr = vr0 + lr;
        const bool valid = lr < T.rpw && vr < g.total_rows;
        int mat = 0, r = 0;
        if (valid) resolve_row<OUT>(g, vr, mat, r);
        tab[e] = ((uint32_t)mat << 30) | (uint32_t)r;
    }
}

// Issues this wavefront's tiles of a phase's row slice into LDS: tile t (wave
// t % 4), chunk round i < cpl: 64 lanes x 16 bytes at off + (t*cpl + i)*1024,
// lane l holding chunk l%L + L*i of its row.  Every lane loads (chunks past
// the row re-read its last one), so every lane counts the same loads.
__device__ __forceinline__ int tile_load(const StepTile T, const uint8_t* w0, const uint8_t* w1, const uint8_t* w2,
                                         int C, const uint32_t* rowtab, int8_t* lds) {
    const int lane = (int)threadIdx.x & 63, w = (int)threadIdx.x >> 6;
    const int L = T.L, R = 64 / L, cpl = T.cpl, j = lane % L;
    const int ntiles = (T.rpw + R - 1) / R;
    const size_t rb = (size_t)C * 16;  // bytes per packed row
    int n = 0;
    for (int t = w; t < ntiles; t += 4) {
        const uint32_t e = rowtab[t * 64 + lane];
        const uint32_t mat = e >> 30;
        const uint8_t* base = mat == 0 ? w0 : (mat == 1 ? w1 : w2);
        const uint4* rowp = (const uint4*)(base + (size_t)(e & 0x3fffffffu) * rb);
        for (int i = 0; i < cpl; i++) {
            const int c = j + L * i;
            __builtin_amdgcn_global_load_lds((const void*)(rowp + (c < C ? c : C - 1)),
                                             (lds_void*)(lds + T.off + (t * cpl + i) * 1024), 16, 0, 0);
        }
        n += cpl;
    }
    return n;  // loads this wavefront issued
}

// One tile of this wavefront's share of a slice (tile w + 4*lt); returns the
// loads issued (0 past the wavefront's tiles).
__device__ __forceinline__ int tile_load_slot(const StepTile T, const uint8_t* w0, const uint8_t* w1,
                                              const uint8_t* w2, int C, const uint32_t* rowtab, int8_t* lds,
                                              int lt) {
    const int lane = (int)threadIdx.x & 63, w = (int)threadIdx.x >> 6;
    const int L = T.L, R = 64 / L, cpl = T.cpl, j = lane % L;
    const int ntiles = (T.rpw + R - 1) / R, t = w + 4 * lt;
    if (t >= ntiles) return 0;
    const uint32_t e = rowtab[t * 64 + lane];
    const uint32_t mat = e >> 30;
    const uint8_t* base = mat == 0 ? w0 : (mat == 1 ? w1 : w2);
    const uint4* rowp = (const uint4*)(base + (size_t)(e & 0x3fffffffu) * (size_t)C * 16);
    for (int i = 0; i < cpl; i++) {
        const int c = j + L * i;
        __builtin_amdgcn_global_load_lds((const void*)(rowp + (c < C ? c : C - 1)),
                                         (lds_void*)(lds + T.off + (t * cpl + i) * 1024), 16, 0, 0);
    }
    return cpl;
}
__device__ __forceinline__ int tile_slots(const StepTile T) {
    const int w = (int)threadIdx.x >> 6, R = 64 / T.L, ntiles = (T.rpw + R - 1) / R;
    return w < ntiles ? (ntiles - w + 3) / 4 : 0;
}

// Waits until at most n vector-memory operations of this wavefront are
// outstanding (they complete in issue order): everything but the last n.
__device__ __forceinline__ void vm_wait_n(int n) {
    switch (n < 0 ? 0 : (n > 24 ? 24 : n)) {
#define VW(k) case k: vm_wait<k>(); break;
        VW(0) VW(1) VW(2) VW(3) VW(4) VW(5) VW(6) VW(7) VW(8) VW(9) VW(10) VW(11) VW(12)
        VW(13) VW(14) VW(15) VW(16) VW(17) VW(18) VW(19) VW(20) VW(21) VW(22) VW(23)
        default: vm_wait<24>(); break;
#undef VW
    }
}

// Integer dots of this wavefront's tiles (weights in LDS) against the
// quantized activation image xq (perm_pos layout); `epi(lr, entry, dot,
// dot of row lr + 1)` runs on the first lane of each row of the slice
// (lr < rows).  A lane's activation chunks (j + L*i, i < CPL) are the same
// for every tile: they are read from LDS once, into registers, so a chunk of
// a tile costs one LDS read (its weights).  CPL = T.cpl, a compile-time
// count so the chunk loop is straight-line code.
template <int CPL, typename Epi>
__device__ __forceinline__ void tile_dots_n(const StepTile T, int C, int rows, const uint32_t* rowtab,
                                            const int8_t* lds, const int8_t* xq, int qsum, Epi epi) {
    const int lane = (int)threadIdx.x & 63, w = (int)threadIdx.x >> 6;
    const int L = T.L, R = 64 / L;
    const int rg = lane / L, j = lane % L;
    const int ntiles = (T.rpw + R - 1) / R;
    if (w >= ntiles) return;
    int4 xa[CPL][4];
    bool cv[CPL];
#pragma unroll
    for (int i = 0; i < CPL; i++) {
        const int c = j + L * i;
        cv[i] = c < C;
        const int cc = cv[i] ? c : C - 1;
#pragma unroll
        for (int kk = 0; kk < 4; kk++) xa[i][kk] = *(const int4*)(xq + ((kk * C + cc) << 4));
    }
    for (int t = w; t < ntiles; t += 4) {
        const uint32_t rte = rowtab[t * 64 + lane];
        uint4 wv[CPL];
#pragma unroll
        for (int i = 0; i < CPL; i++) wv[i] = *(const uint4*)(lds + T.off + (t * CPL + i) * 1024 + lane * 16);
        int accs[4] = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < CPL; i++) {
            // a chunk past the row (ragged last round) holds a copy of the
            // last chunk: its weights count as zero
            const uint32_t d[4] = {cv[i] ? wv[i].x : 0u, cv[i] ? wv[i].y : 0u, cv[i] ? wv[i].z : 0u,
                                   cv[i] ? wv[i].w : 0u};
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                const int4 x4 = xa[i][kk];
                const uint32_t m = 0x03030303u << (2 * kk);
                int& acc = accs[kk];
                if (kk < 3) {
                    acc = __builtin_amdgcn_sdot4((int)(d[0] & m), x4.x, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)(d[1] & m), x4.y, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)(d[2] & m), x4.z, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)(d[3] & m), x4.w, acc, false);
                } else {
                    acc = __builtin_amdgcn_sdot4((int)((d[0] >> 6) & 0x03030303u), x4.x, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)((d[1] >> 6) & 0x03030303u), x4.y, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)((d[2] >> 6) & 0x03030303u), x4.z, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)((d[3] >> 6) & 0x03030303u), x4.w, acc, false);
                }
            }
        }
        // planes 0..2 hold 4^kk times their dot (masked in place), plane 3 was shifted
        int acc = (accs[0] + (accs[1] >> 2)) + ((accs[2] >> 4) + accs[3]);
        // sum over the row's L lanes (integers: any order)
        if (L >= 64) acc = xor_add_i<32>(acc);
        if (L >= 32) acc = xor_add_i<16>(acc);
        if (L >= 16) acc = xor_add_i<8>(acc);
        if (L >= 8) acc = xor_add_i<4>(acc);
        if (L >= 4) acc = xor_add_i<2>(acc);
        if (L >= 2) acc = xor_add_i<1>(acc);
        const int dot = acc - qsum;
        // the next row's dot, L lanes up (its row pair partner: lane ^ L)
        uint32_t a0, d1u;
        if (L == 4) xor_pair<4>((uint32_t)dot, a0, d1u);
        else if (L == 8) xor_pair<8>((uint32_t)dot, a0, d1u);
        else if (L == 16) xor_pair<16>((uint32_t)dot, a0, d1u);
        else xor_pair<32>((uint32_t)dot, a0, d1u);
        const int d1 = (int)((lane & L) ? a0 : d1u);
        const int lr = t * R + rg;
        if (j == 0 && lr < T.rpw && lr < rows) epi(lr, rte, dot, d1);
    }
}

template <typename Epi>
__device__ __forceinline__ void tile_dots(const StepTile T, int C, int rows, const uint32_t* rowtab,
                                          const int8_t* lds, const int8_t* xq, int qsum, Epi epi) {
    static_assert(kStepMaxCpl == 8, "one instance per chunk count");
    switch (T.cpl) {
        case 1: tile_dots_n<1>(T, C, rows, rowtab, lds, xq, qsum, epi); break;
        case 2: tile_dots_n<2>(T, C, rows, rowtab, lds, xq, qsum, epi); break;
        case 3: tile_dots_n<3>(T, C, rows, rowtab, lds, xq, qsum, epi); break;
        case 4: tile_dots_n<4>(T, C, rows, rowtab, lds, xq, qsum, epi); break;
        case 5: tile_dots_n<5>(T, C, rows, rowtab, lds, xq, qsum, epi); break;
        case 6: tile_dots_n<6>(T, C, rows, rowtab, lds, xq, qsum, epi); break;
        case 7: tile_dots_n<7>(T, C, rows, rowtab, lds, xq, qsum, epi); break;
        default: tile_dots_n<8>(T, C, rows, rowtab, lds, xq, qsum, epi); break;
    }
}

// ---- the prologue: RMSNorm + ActQuant into xq, sum(q) -------------------
struct Quant {
    float sa;
    int qs;
};

template <int EPT>
__device__ __forceinline__ Quant prologue(RowRegs<EPT>& r, int cols, const float* nw, float eps, int8_t* xq,
                                          float* red, float* sa_s) {
    const int kp = (cols + 127) / 128 * 128, C = kp / 64;
    quantize_row_regs<EPT, kST, 1, true>(r, cols, kp, nw, eps, xq, [C](int i) { return perm_pos(i, C); }, sa_s,
                                         nullptr, red);
    __syncthreads();
    const int4 qp = *(const int4*)(red + 32);
    Quant q;
    q.qs = (qp.x + qp.y) + (qp.z + qp.w);
    q.sa = *sa_s;
    return q;
}

// ---- attention: one (query head, key split) item ------------------------
template <int LK>
struct StepAttnShared : AttnShared<LK> {
    float fs[kAttnSplits];  // split factors of the combine
    float linv;
};

// attention_split_ku (attn_common.h) with key p, the row appended by this
// step, taken from the q/k/v words instead of the cache (the cache row is
// written by another workgroup in this dispatch and is not coherent here);
// the same arithmetic in the same order.
template <int LK>
__device__ __forceinline__ void attn_item(const StepArgs& a, int l, int h, int s, int ns, int p, unsigned want,
                                          unsigned ep, float* sc, StepAttnShared<LK>& sh, Waiter& wt) {
    const unsigned want2 = ep;  // the partials of the head's other splits
#define ATR(k)                                                                                      \
    if (a.trace && threadIdx.x == 0)                                                                \
        gstore(a.trace + ((size_t)blockIdx.x * a.layers + l) * 32 + (k), (unsigned long long)wall_clock64());
    ATR(22)
    constexpr int HD = LK * 8, GW = 64 / LK, NK = kST / LK, KU = 4;
    const int tid = (int)threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int kslot = lane / LK, cc = lane % LK;
    const int grp = tid / LK, c = tid % LK;
    const int vis = p + 1, ks = attn_split_keys(vis);
    const int j0 = s * ks, cnt = vis - j0 < ks ? vis - j0 : ks;
    const int g = h / (a.nh / a.kvh);
    const size_t kvoff = (size_t)l * a.layer_kv + (size_t)g * a.cap * HD;
    const uint16_t* K = a.kc + kvoff + (size_t)j0 * HD;
    const uint16_t* V = a.vc + kvoff + (size_t)j0 * HD;
    const int knew = p - j0;  // index of the new key in this split (>= cnt: not here)
    // first key passes from the cache (the new row's slot holds stale data and
    // is replaced below)
    uint4 kb[KU], vb[KU];
#pragma unroll
    for (int u = 0; u < KU; u++) {
        const int k = u * NK + w * GW + kslot;
        kb[u] = ld_u4((K + (size_t)(k < cnt ? k : cnt - 1) * HD + 8 * cc));
    }
#pragma unroll
    for (int u = 0; u < KU; u++) {
        const int k = grp + u * NK;
        vb[u] = ld_u4((V + (size_t)(k < cnt ? k : cnt - 1) * HD + 8 * c));
    }
    // q (rotated, f32) and the new key / value rows (bf16 values) of this lane
    const u64* qw = a.llqkv + (size_t)h * HD + 8 * cc;
    const u64* kw = a.llqkv + a.H + (size_t)g * HD + 8 * cc;
    const u64* vw = a.llqkv + a.H + a.KV + (size_t)g * HD + 8 * c;
    u32x4 qv[4], kn[4], vn[4];
    wt.start();
    for (;;) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            qv[i] = ll_ld2(qw + 2 * i);
            kn[i] = ll_ld2(kw + 2 * i);
            vn[i] = ll_ld2(vw + 2 * i);
        }
        vm_wait<0>();
        bool ok = true;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            pin(qv[i]);
            pin(kn[i]);
            pin(vn[i]);
            ok = ok && ready2(qv[i], want) && ready2(kn[i], want) && ready2(vn[i], want);
        }
        if (__all(ok) || wt.give_up()) break;
    }
    ATR(23)
    float q8[8], kf[8], vf[8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        q8[2 * i] = __uint_as_float(qv[i].x);
        q8[2 * i + 1] = __uint_as_float(qv[i].z);
        kf[2 * i] = __uint_as_float(kn[i].x);
        kf[2 * i + 1] = __uint_as_float(kn[i].z);
        vf[2 * i] = __uint_as_float(vn[i].x);
        vf[2 * i + 1] = __uint_as_float(vn[i].z);
    }

    // ---- scores and the split max
    float mx = -__builtin_inff();
    for (int b0 = 0;; b0 += KU * NK) {
        if (b0 > 0) {
#pragma unroll
            for (int u = 0; u < KU; u++) {
                const int k = b0 + u * NK + w * GW + kslot;
                kb[u] = k < cnt ? ld_u4((K + (size_t)k * HD + 8 * cc)) : make_uint4(0, 0, 0, 0);
            }
        }
#pragma unroll
        for (int u = 0; u < KU; u++) {
            const int k = b0 + u * NK + w * GW + kslot;
            const uint32_t wv[4] = {kb[u].x, kb[u].y, kb[u].z, kb[u].w};
            const bool nk = k == knew;
            float a8 = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float k0 = nk ? kf[2 * e] : bf16_to_f32((uint16_t)(wv[e] & 0xffffu));
                const float k1 = nk ? kf[2 * e + 1] : bf16_to_f32((uint16_t)(wv[e] >> 16));
                a8 = __builtin_fmaf(q8[2 * e], k0, a8);
                a8 = __builtin_fmaf(q8[2 * e + 1], k1, a8);
            }
            a8 = xor_sum_down<LK / 2>(a8);
            if (k < cnt) {
                const float sv = a8 * a.scaling;
                if (cc == 0) sc[k] = sv;
                mx = fmaxf(mx, sv);
            }
        }
        if (b0 + KU * NK >= cnt) break;
    }
    mx = wave_max(mx);
    if (lane == 0) sh.rmax[w] = mx;
    __syncthreads();
    const float m = fmaxf(fmaxf(sh.rmax[0], sh.rmax[1]), fmaxf(sh.rmax[2], sh.rmax[3]));
    float ps = 0.0f;
    for (int u = tid; u < cnt; u += kST) {
        const float e = lbt_expf(sc[u] - m);
        sc[u] = e;
        ps = ps + e;
    }
    ps = wave_sum(ps);
    if (lane == 0) sh.rsum[w] = ps;
    __syncthreads();

    // ---- unnormalised probs @ V
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; e++) acc[e] = 0.0f;
    for (int b0 = 0;; b0 += KU * NK) {
        if (b0 > 0) {
#pragma unroll
            for (int u = 0; u < KU; u++) {
                const int k = b0 + grp + u * NK;
                vb[u] = k < cnt ? ld_u4((V + (size_t)k * HD + 8 * c)) : make_uint4(0, 0, 0, 0);
            }
        }
#pragma unroll
        for (int u = 0; u < KU; u++) {
            const int k = b0 + grp + u * NK;
            if (k < cnt) {
                const float pj = sc[k];
                const uint32_t wv[4] = {vb[u].x, vb[u].y, vb[u].z, vb[u].w};
                const bool nk = k == knew;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float v0 = nk ? vf[2 * e] : bf16_to_f32((uint16_t)(wv[e] & 0xffffu));
                    const float v1 = nk ? vf[2 * e + 1] : bf16_to_f32((uint16_t)(wv[e] >> 16));
                    acc[2 * e] = __builtin_fmaf(pj, v0, acc[2 * e]);
                    acc[2 * e + 1] = __builtin_fmaf(pj, v1, acc[2 * e + 1]);
                }
            }
        }
        if (b0 + KU * NK >= cnt) break;
    }
    if constexpr (GW > 1) {
#pragma unroll
        for (int e = 0; e < 8; e++) acc[e] = xor_sum_up<LK>(acc[e]);
    }
    if (lane < LK) {
#pragma unroll
        for (int e = 0; e < 8; e++) sh.pv[w][8 * c + e] = acc[e];
    }
    __syncthreads();
    ATR(24)
    const float o_own = tid < HD ? (sh.pv[0][tid] + sh.pv[1][tid]) + (sh.pv[2][tid] + sh.pv[3][tid]) : 0.0f;
    const float l_own = (sh.rsum[0] + sh.rsum[1]) + (sh.rsum[2] + sh.rsum[3]);
    u64* ml = a.llpart + (size_t)kAttnSplits * a.H;
    if (s + 1 < ns) {
        // a split other than the last: its partial goes to the head's last split
        if (tid < HD) ll_put(a.llpart + (size_t)s * a.H + (size_t)h * HD + tid, ep, o_own);
        if (tid == 0) {
            ll_put(ml + ((size_t)s * a.nh + h) * 2, ep, m);
            ll_put(ml + ((size_t)s * a.nh + h) * 2 + 1, ep, l_own);
        }
        __syncthreads();  // sc / sh are reused by the next item only after its own barriers
        return;
    }
    // The head's last split combines all of them (attn_row_finish,
    // attn_common.h: the same factors, the same accumulation order) and
    // publishes the head's attention output.
    float ov[kAttnSplits];
    float mv = -__builtin_inff(), lv = 0.0f;
    const int slot = lane & (kAttnSplits - 1);
    wt.start();
    for (;;) {
        bool ok = true;
        if (tid < HD)
#pragma unroll
            for (int q = 0; q < kAttnSplits - 1; q++) {
                if (q >= ns - 1) break;
                const u64 v = __hip_atomic_load((const LBT_GLOBAL u64*)(a.llpart + (size_t)q * a.H + (size_t)h * HD + tid),
                                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ok = ok && (unsigned)(v >> 32) == want2;
                ov[q] = __uint_as_float((uint32_t)v);
            }
        if (w == 0 && slot < ns - 1) {
            const u64 vm = __hip_atomic_load((const LBT_GLOBAL u64*)(ml + ((size_t)slot * a.nh + h) * 2),
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const u64 vl = __hip_atomic_load((const LBT_GLOBAL u64*)(ml + ((size_t)slot * a.nh + h) * 2 + 1),
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ok = ok && (unsigned)(vm >> 32) == want2 && (unsigned)(vl >> 32) == want2;
            mv = __uint_as_float((uint32_t)vm);
            lv = __uint_as_float((uint32_t)vl);
        }
        if (__all(ok) || wt.give_up()) break;
    }
    ATR(25)
    if (w == 0) {
        const bool live = slot < ns;
        const float mm = slot == ns - 1 ? m : (live ? mv : -__builtin_inff());
        const float ll = slot == ns - 1 ? l_own : lv;
        float M = xor_max<8>(mm);
        M = xor_max<4>(M);
        M = xor_max<2>(M);
        M = xor_max<1>(M);
        const float f = live ? lbt_expf(mm - M) : 0.0f;
        const float Ls = xor_sum_down<8>(live ? ll * f : 0.0f);
        if (lane < kAttnSplits) sh.fs[lane] = f;
        if (lane == 0) sh.linv = 1.0f / Ls;
    }
    __syncthreads();
    if (tid < HD) {
        float O = 0.0f;
#pragma unroll
        for (int q = 0; q < kAttnSplits; q++) {
            if (q >= ns) break;
            O = __builtin_fmaf(q == ns - 1 ? o_own : ov[q], sh.fs[q], O);
        }
        ll_put(a.llatt + (size_t)h * HD + tid, ep, O * sh.linv);
    }
    ATR(26)
#undef ATR
    __syncthreads();  // sc / sh are reused by the next item only after its own barriers
}

// ---- the step ------------------------------------------------------------
// Kernel arguments live in device memory and are re-read through a laundered
// pointer in each phase (scalar loads), so the compiler keeps no uniform value
// alive across the layer loop (which would exhaust the scalar registers).
// Matrix k of layer l and norm k of layer l: the model keeps every layer's
// matrices (and norm gains) at one stride from the previous layer's.
#define WP(l, k) (a.w0[k] + (size_t)(l) * a.wstride)
#define NP(l, k) (a.n0[k] + (size_t)(l) * a.nstride)

template <int LK, int EH, int EI>
__global__ __launch_bounds__(kST) void decode_step_kernel(const StepArgs* __restrict__ pa) {
    extern __shared__ __align__(16) int8_t dyn[];  // weight slices, row tables, xq image, scores
    __shared__ __align__(16) float red[kRedFloats];
    __shared__ float sa_s;
    __shared__ StepAttnShared<LK> ash;
    __shared__ float xown[kStepMaxRows];
    __shared__ f32x2 rope[kStepMaxRows];  // (cos, sin) of this workgroup's q/k row pairs at position p
    float* wsc = (float*)(dyn + kld(&launder(pa)->ws_off));  // per-tensor weight scales [layers * 7]
    const int G = (int)gridDim.x, b = (int)blockIdx.x, tid = (int)threadIdx.x;

    int p, slot, layers;
    unsigned base;
    uint32_t tok;
    bool hq, ho, hg;
    {
        const StepArgs a = kargs(pa);
        p = kld(a.state) + 1;
        slot = kld(a.state + 1);
        base = (unsigned)kld(a.state + 2);
        const unsigned long long key = kld(a.key);
        tok = 0xffffffffu - (uint32_t)(key & 0xffffffffull);
        if (tok >= (uint32_t)a.vocab) tok = 0;
        layers = a.layers;
        const int H = a.H, I = a.I, KV = a.KV, hd = a.hd;
        const int vq0 = b * a.t[0].rpw, vo0 = b * a.t[1].rpw, vg0 = b * a.t[2].rpw, vd0 = b * a.t[3].rpw;
        // A workgroup takes part in a phase only if it owns rows of it (then it
        // reads the phase's whole input): every reader of a buffer is then an
        // ancestor of the buffer's next writer.
        hq = vq0 < H + 2 * KV;
        ho = vo0 < H;
        hg = vg0 < 2 * I;
        GemvArgs g{};
        g.rows[0] = H;
        g.rows[1] = KV;
        g.rows[2] = KV;
        g.total_rows = H + 2 * KV;
        g.hd = hd;
        build_rowtab<kOutQKV>(g, a.t[0], vq0, (uint32_t*)(dyn + a.rt_off[0]));
        g.rows[0] = H;
        g.total_rows = H;
        build_rowtab<kOutF32Add>(g, a.t[1], vo0, (uint32_t*)(dyn + a.rt_off[1]));
        build_rowtab<kOutF32Add>(g, a.t[3], vd0, (uint32_t*)(dyn + a.rt_off[3]));
        g.rows[0] = I;
        g.rows[1] = I;
        g.total_rows = 2 * I;
        build_rowtab<kOutRelu2>(g, a.t[2], vg0, (uint32_t*)(dyn + a.rt_off[2]));
        // RoPE factors of the q/k row pairs (v pairs unused)
        g.rows[0] = H;
        g.rows[1] = KV;
        g.total_rows = H + 2 * KV;
        const int h2 = hd >> 1;
        for (int q = tid; 2 * q < a.t[0].rpw; q += kST) {
            const int vr = vq0 + 2 * q;
            f32x2 cs{1.0f, 0.0f};
            if (vr < H + 2 * KV) {
                int mat, r0;
                resolve_row<kOutQKV>(g, vr, mat, r0);
                if (mat < 2) {
                    const int d = r0 & (hd - 1);
                    cs = f32x2{gload(a.cos_t + (size_t)p * h2 + d), gload(a.sin_t + (size_t)p * h2 + d)};
                }
            }
            rope[q] = cs;
        }
        for (int i = tid; i < a.layers * 7; i += kST) wsc[i] = gload(a.wscale + i);
        // the residual rows of this workgroup (its o / down rows) start as the embedding
        const uint16_t* erow = a.embed + (size_t)tok * H;
        if (ho)
            for (int r = tid; r < a.t[1].rpw; r += kST) xown[r] = vo0 + r < H ? bf16_to_f32(gload(erow + vo0 + r)) : 0.0f;
        __syncthreads();  // row tables
    }
    Waiter wt{nullptr, 0ull, 0};
    // Weight slices of the next layer, loaded into LDS a tile at a time at
    // each phase's start (a few tiles per phase, so the HBM stream stays
    // spread over the layer instead of bursting while other workgroups poll):
    // pend[P] = the layer slice P is being loaded for (-1: none), cur[P] = its
    // next tile of this wavefront, last[P] = the load count nl after its last
    // tile (the loads issued since may still be in flight when P is used).
    int pend[4] = {-1, -1, -1, -1}, cur[4] = {0, 0, 0, 0}, last[4] = {0, 0, 0, 0};
    int nl = 0;
    auto load_tile = [&](const StepArgs& a, int P, int ly, int lt) -> int {
        const uint32_t* rt = (const uint32_t*)(dyn + a.rt_off[P]);
        switch (P) {
            case 0: return tile_load_slot(a.t[0], WP(ly, 0), WP(ly, 1), WP(ly, 2), a.CH, rt, dyn, lt);
            case 1: return tile_load_slot(a.t[1], WP(ly, 3), WP(ly, 3), WP(ly, 3), a.CH, rt, dyn, lt);
            case 2: return tile_load_slot(a.t[2], WP(ly, 4), WP(ly, 5), WP(ly, 5), a.CH, rt, dyn, lt);
            default: return tile_load_slot(a.t[3], WP(ly, 6), WP(ly, 6), WP(ly, 6), a.CI, rt, dyn, lt);
        }
    };
    // up to `quota` tiles of the pending slices
    auto feed = [&](int quota) {
        if ((pend[0] & pend[1] & pend[2] & pend[3]) == -1) return;  // uniform
        const StepArgs a = kargs(pa);
#pragma unroll
        for (int P = 0; P < 4; P++) {
            if (pend[P] >= 0) {
                const int ns_ = tile_slots(a.t[P]);
                while (quota > 0 && cur[P] < ns_) {
                    nl += load_tile(a, P, pend[P], cur[P]);
                    cur[P]++;
                    quota--;
                }
                if (cur[P] >= ns_) {
                    pend[P] = -1;
                    last[P] = nl;
                }
            }
        }
    };
    // Before the dots of slice P: its loads issued (now if still pending)
    // and landed; loads issued after it may stay in flight.
    auto slice_ready = [&](int P) {
        if (pend[P] >= 0) {
            const StepArgs a = kargs(pa);
            const int ns_ = tile_slots(a.t[P]);
            while (cur[P] < ns_) {
                nl += load_tile(a, P, pend[P], cur[P]);
                cur[P]++;
            }
            pend[P] = -1;
            last[P] = nl;
            vm_wait<0>();
        } else {
            vm_wait_n(nl - last[P]);
        }
    };
    auto enqueue = [&](int P, int ly) {
        pend[P] = ly;
        cur[P] = 0;
    };
    // layer 0's slices (those of phases this workgroup takes part in)
    if (hq) enqueue(0, 0);
    if (ho) enqueue(1, 0);
    if (hg) enqueue(2, 0);
    if (ho) enqueue(3, 0);
    feed(64);
#define STEP_TR(k)                                                                        \
    if (tid == 0) {                                                                       \
        unsigned long long* tr_ = kld(&launder(pa)->trace);                               \
        if (tr_) gstore(tr_ + ((size_t)b * layers + l) * 32 + (k), (unsigned long long)wall_clock64()); \
    }

    for (int l = 0; l < layers; l++) {
        const unsigned e0 = base + 5u * (unsigned)l;
        STEP_TR(0)
        // ---- q/k/v on input_layernorm(x), RoPE, K/V append (model.rs:331-340)
        if (hq) {
            const StepArgs a = kargs(pa);
            wt.err = a.err;
            const int H = a.H, KV = a.KV, hd = a.hd, h2 = hd >> 1, hs = __builtin_ctz((unsigned)hd);
            const float* nw = NP(l, 0);
            RowRegs<EH> r;
            if (l == 0) row_load<EH, kST>(SrcBf16{a.embed + (size_t)tok * H}, H, nw, r);
            else ll_row<EH>(a.llx, H, e0, nw, r, wt);
            STEP_TR(1)
            const Quant qa = prologue<EH>(r, H, nw, a.eps, dyn + a.xq_off, red, &sa_s);
            STEP_TR(2)
            slice_ready(0);
            STEP_TR(3)
            const float sw0 = wsc[l * 7], sw1 = wsc[l * 7 + 1], sw2 = wsc[l * 7 + 2];
            uint16_t* kcl = a.kc + (size_t)l * a.layer_kv;
            uint16_t* vcl = a.vc + (size_t)l * a.layer_kv;
            u64* q_out = a.llqkv;
            const int cap = a.cap;
            const unsigned ep = e0 + 1u;
            const uint32_t* rt = (const uint32_t*)(dyn + a.rt_off[0]);
            tile_dots(a.t[0], a.CH, H + 2 * KV - b * a.t[0].rpw, rt, dyn, dyn + a.xq_off, qa.qs,
                      [&](int lr, uint32_t e, int d0, int d1) {
                          if (lr & 1) return;  // pairs (2p, 2p + 1): the even row stores both
                          const int mat = (int)(e >> 30), r0 = (int)(e & 0x3fffffffu);
                          const float swm = mat == 0 ? sw0 : (mat == 1 ? sw1 : sw2);
                          const float inv = 1.0f / (qa.sa * swm);
                          const float y0 = (float)d0 * inv, y1 = (float)d1 * inv;
                          const int gh = r0 >> hs, d = r0 & (hd - 1);
                          if (mat == 2) {  // v rows r0, r0 + 1
                              uint16_t* dst = vcl + ((size_t)gh * cap + p) * hd + d;
                              const uint16_t b0 = f32_to_bf16(y0), b1 = f32_to_bf16(y1);
                              gstore(dst, b0);
                              gstore(dst + 1, b1);
                              ll_put(q_out + H + KV + r0, ep, bf16_to_f32(b0));
                              ll_put(q_out + H + KV + r0 + 1, ep, bf16_to_f32(b1));
                              return;
                          }
                          const f32x2 cs = rope[lr >> 1];
                          const float z0 = y0 * cs.x + (-y1) * cs.y;
                          const float z1 = y1 * cs.x + y0 * cs.y;
                          if (mat == 0) {
                              ll_put(q_out + r0, ep, z0);
                              ll_put(q_out + r0 + h2, ep, z1);
                          } else {
                              uint16_t* dst = kcl + ((size_t)gh * cap + p) * hd + d;
                              const uint16_t b0 = f32_to_bf16(z0), b1 = f32_to_bf16(z1);
                              gstore(dst, b0);
                              gstore(dst + h2, b1);
                              ll_put(q_out + H + r0, ep, bf16_to_f32(b0));
                              ll_put(q_out + H + r0 + h2, ep, bf16_to_f32(b1));
                          }
                      });
            STEP_TR(4)
            if (l + 1 < layers) {
                enqueue(0, l + 1);
                feed(64);
            }
        }
        STEP_TR(5)
        // ---- attention over keys 0..p (model.rs:341-357)
        {
            const StepArgs a = kargs(pa);
            wt.err = a.err;
            const int ns = attn_splits(p + 1);
            for (int it = b; it < a.nh * ns; it += G)
                attn_item<LK>(a, l, it / ns, it % ns, ns, p, e0 + 1u, e0 + 2u, (float*)(dyn + a.sc_off), ash, wt);
            STEP_TR(6)
        }
        // ---- o_proj(attn_sub_norm(attn)), x += o (model.rs:358-359)
        if (ho) {
            const StepArgs a = kargs(pa);
            wt.err = a.err;
            const int H = a.H;
            const float* nw = NP(l, 2);
            RowRegs<EH> r;
            ll_row<EH>(a.llatt, H, e0 + 2u, nw, r, wt);
            STEP_TR(7)
            const Quant qa = prologue<EH>(r, H, nw, a.eps, dyn + a.xq_off, red, &sa_s);
            STEP_TR(8)
            slice_ready(1);
            STEP_TR(9)
            const float inv = 1.0f / (qa.sa * wsc[l * 7 + 3]);
            const int vo0 = b * a.t[1].rpw;
            u64* xo = a.llx + vo0;
            const unsigned ep = e0 + 3u;
            const uint32_t* rt = (const uint32_t*)(dyn + a.rt_off[1]);
            tile_dots(a.t[1], a.CH, H - vo0, rt, dyn, dyn + a.xq_off, qa.qs, [&](int lr, uint32_t, int d0, int) {
                const float xv = xown[lr] + (float)d0 * inv;
                xown[lr] = xv;
                ll_put(xo + lr, ep, xv);
            });
            STEP_TR(10)
            if (l + 1 < layers) {
                enqueue(1, l + 1);
                feed(64);
            }
        }
        STEP_TR(11)
        // ---- gate/up on post_attention_layernorm(x), relu(g)^2 * u (model.rs:361-363)
        if (hg) {
            const StepArgs a = kargs(pa);
            wt.err = a.err;
            const int H = a.H, I = a.I;
            const float* nw = NP(l, 1);
            RowRegs<EH> r;
            ll_row<EH>(a.llx, H, e0 + 3u, nw, r, wt);
            STEP_TR(12)
            const Quant qa = prologue<EH>(r, H, nw, a.eps, dyn + a.xq_off, red, &sa_s);
            STEP_TR(13)
            slice_ready(2);
            STEP_TR(14)
            const float ig = 1.0f / (qa.sa * wsc[l * 7 + 4]), iu = 1.0f / (qa.sa * wsc[l * 7 + 5]);
            const int vg0 = b * a.t[2].rpw;
            u64* hout = a.llh + (vg0 >> 1);
            const unsigned ep = e0 + 4u;
            const uint32_t* rt = (const uint32_t*)(dyn + a.rt_off[2]);
            tile_dots(a.t[2], a.CH, 2 * I - vg0, rt, dyn, dyn + a.xq_off, qa.qs,
                      [&](int lr, uint32_t, int d0, int d1) {
                          if (lr & 1) return;
                          const float y0 = (float)d0 * ig;
                          const float u = (float)d1 * iu;
                          const float rl = y0 > 0.0f ? y0 : 0.0f;
                          ll_put(hout + (lr >> 1), ep, (rl * rl) * u);
                      });
            STEP_TR(15)
            if (l + 1 < layers) {
                enqueue(2, l + 1);
                feed(64);
            }
        }
        STEP_TR(16)
        // ---- down on ffn_sub_norm(h), x += down (model.rs:364-365)
        if (ho) {
            const StepArgs a = kargs(pa);
            wt.err = a.err;
            const int H = a.H, I = a.I;
            const float* nw = NP(l, 3);
            RowRegs<EI> r;
            ll_row<EI>(a.llh, I, e0 + 4u, nw, r, wt);
            STEP_TR(17)
            const Quant qa = prologue<EI>(r, I, nw, a.eps, dyn + a.xq_off, red, &sa_s);
            STEP_TR(18)
            slice_ready(3);
            STEP_TR(19)
            const float inv = 1.0f / (qa.sa * wsc[l * 7 + 6]);
            const int vo0 = b * a.t[1].rpw;
            const bool last = l + 1 == layers;
            u64* xo = a.llx + vo0;
            float* xf = a.xout + vo0;
            const unsigned ep = e0 + 5u;
            const uint32_t* rt = (const uint32_t*)(dyn + a.rt_off[3]);
            tile_dots(a.t[3], a.CI, H - vo0, rt, dyn, dyn + a.xq_off, qa.qs, [&](int lr, uint32_t, int d0, int) {
                const float xv = xown[lr] + (float)d0 * inv;
                xown[lr] = xv;
                if (last) gstore(xf + lr, xv);  // the LM head's input, next dispatch
                else ll_put(xo + lr, ep, xv);
            });
            STEP_TR(20)
            if (!last) {
                enqueue(3, l + 1);
                feed(64);
            }
        }
        STEP_TR(21)
    }
#undef STEP_TR
    // Every workgroup read the state and the key before its first phase, and
    // workgroup 0 gets here only after every workgroup's last gate/up output,
    // so it may advance them for the next step.  The LM head runs next.
    if (b == 0 && tid == 0) {
        const StepArgs a = kargs(pa);
        gstore(a.tok_out + slot, tok);
        gstore(a.state, p);
        gstore(a.state + 1, slot + 1);
        gstore(a.state + 2, (int)(base + 5u * (unsigned)layers));
        gstore(a.key, 0ull);
    }
}

// ---- host side -------------------------------------------------------------
namespace {

// Tiling of one phase: rows per workgroup rpw; L lanes per row chosen to
// minimise the chunks per lane of the busiest wavefront (paired outputs keep
// L <= 32 so a row pair shares a wavefront).
StepTile make_tile(int total, int G, int C, bool paired, int& off) {
    StepTile t{};
    int rpw = (total + G - 1) / G;
    rpw = (rpw + 1) & ~1;
    t.rpw = rpw;
    // cost of the busiest wavefront in VALU instructions: per tile, cpl chunks
    // of ~36 (unpack + 16 dot4), the row reduction and the epilogue
    int best = 1 << 30;
    t.L = 64;
    t.cpl = (C + 63) / 64;
    for (int L = 4; L <= (paired ? 32 : 64); L *= 2) {
        const int R = 64 / L, ntiles = (rpw + R - 1) / R, cpl = (C + L - 1) / L;
        if (cpl > kStepMaxCpl) continue;
        const int lg = L == 4 ? 2 : L == 8 ? 3 : L == 16 ? 4 : L == 32 ? 5 : 6;
        const int cost = ((ntiles + 3) / 4) * (36 * cpl + 6 * lg + 20);
        if (cost < best) {
            best = cost;
            t.L = L;
            t.cpl = cpl;
        }
    }
    const int R = 64 / t.L, ntiles = (rpw + R - 1) / R;
    t.off = off;
    off += ntiles * t.cpl * 1024;
    return t;
}

template <int LK, int EH, int EI>
const void* step_fn() {
    return (const void*)decode_step_kernel<LK, EH, EI>;
}

struct StepFn {
    const void* fn;
    int eh, ei;
};

StepFn pick_fn(int hd, int kpH, int kpI) {
    const int eh = (kpH + 4 * kST - 1) / (4 * kST) * 4, ei = (kpI + 4 * kST - 1) / (4 * kST) * 4;
    if (hd == 128 && eh <= 12 && ei <= 28) return {step_fn<16, 12, 28>(), 12, 28};
    if (eh > 16 || ei > 32) return {nullptr, 0, 0};
    switch (hd) {
        case 64: return {step_fn<8, 16, 32>(), 16, 32};
        case 128: return {step_fn<16, 16, 32>(), 16, 32};
        case 256: return {step_fn<32, 16, 32>(), 16, 32};
        default: return {nullptr, 0, 0};
    }
}

size_t dyn_limit(const void* fn) {
    hipFuncAttributes at{};
    if (hipFuncGetAttributes(&at, fn) != hipSuccess || at.sharedSizeBytes >= 160 * 1024) {
        (void)hipGetLastError();
        return 0;
    }
    return 160 * 1024 - at.sharedSizeBytes;
}

}  // namespace

int step_plan(const lbt_config& c, int cap, int G, StepPlan& pl, const char** why) {
    const int H = c.hidden_size, I = c.intermediate_size;
    const int hd = H / c.num_attention_heads, KV = c.num_key_value_heads * hd;
    if (hd != 64 && hd != 128 && hd != 256) return *why = "head_dim", 0;
    if ((hd & (hd - 1)) != 0) return *why = "head_dim", 0;
    if (c.num_attention_heads > kAttnMaxHeads) return *why = "heads", 0;
    if (H % 4 || I % 4) return *why = "hidden/intermediate not a multiple of 4", 0;
    const int kpH = (H + 127) / 128 * 128, kpI = (I + 127) / 128 * 128;
    const StepFn f = pick_fn(hd, kpH, kpI);
    if (!f.fn) return *why = "hidden/intermediate too large", 0;
    int off = 0;
    pl.t[0] = make_tile(H + 2 * KV, G, kpH / 64, true, off);
    pl.t[1] = make_tile(H, G, kpH / 64, false, off);
    pl.t[2] = make_tile(2 * I, G, kpH / 64, true, off);
    pl.t[3] = make_tile(H, G, kpI / 64, false, off);
    for (int i = 0; i < 4; i++)
        if (pl.t[i].cpl > kStepMaxCpl) return *why = "row chunks per lane", 0;
    if (pl.t[1].rpw != pl.t[3].rpw || pl.t[1].rpw > kStepMaxRows || pl.t[0].rpw > 2 * kStepMaxRows)
        return *why = "rows per workgroup", 0;
    for (int i = 0; i < 4; i++) {
        const int R = 64 / pl.t[i].L;
        pl.rt_off[i] = off;
        off += (pl.t[i].rpw + R - 1) / R * 64 * 4;
    }
    pl.xq_off = off;
    off += (kpI > kpH ? kpI : kpH);
    off = (off + 15) & ~15;
    pl.sc_off = off;
    off += attn_split_keys(cap) * 4;
    pl.ws_off = off;
    off += c.num_hidden_layers * 7 * 4;
    pl.lds = (size_t)off;
    pl.fn = f.fn;
    const size_t lim = dyn_limit(f.fn);
    if (pl.lds > lim) return *why = "LDS", 0;
    if (hipFuncSetAttribute(f.fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)pl.lds) != hipSuccess) {
        (void)hipGetLastError();
        return *why = "LDS attribute", 0;
    }
    return 1;
}

void step_fill(const StepPlan& pl, const lbt_config& c, StepArgs& a) {
    for (int i = 0; i < 4; i++) {
        a.t[i] = pl.t[i];
        a.rt_off[i] = pl.rt_off[i];
    }
    a.xq_off = pl.xq_off;
    a.sc_off = pl.sc_off;
    a.ws_off = pl.ws_off;
    a.CH = (int)(padded_cols((size_t)c.hidden_size) / 64);
    a.CI = (int)(padded_cols((size_t)c.intermediate_size) / 64);
}

int launch_decode_step(lbt_ctx* ctx, const StepPlan& pl, const StepArgs* dargs, hipStream_t s) {
    void* args[] = {&dargs};
    hipEvent_t e0, e1;
    prof_pair(ctx, &e0, &e1);
    if (e0) (void)hipEventRecord(e0, s);
    const hipError_t e = hipLaunchCooperativeKernel(pl.fn, dim3(pl.G), dim3(kST), args, pl.lds, s);
    if (e1) (void)hipEventRecord(e1, s);
    if (e != hipSuccess) return hip_err(ctx, e, "decode step launch");
    prof_commit(ctx, e0, e1, kProfStep, pl.bytes);
    return LBT_OK;
}

}  // namespace lbt

#else

namespace lbt {
int step_plan(const lbt_config&, int, int, StepPlan&, const char** why) {
    if (why) *why = "the one-dispatch step is not in this build (LBT_WITH_STEP=1)";
    return 0;
}
void step_fill(const StepPlan&, const lbt_config&, StepArgs&) {}
int launch_decode_step(lbt_ctx* ctx, const StepPlan&, const StepArgs*, hipStream_t) {
    return set_err(ctx, LBT_E_INVALID, "the one-dispatch step is not in this build (LBT_WITH_STEP=1)");
}
}  // namespace lbt

#endif

