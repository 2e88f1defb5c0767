// decode_persistent.hip -- one dispatch per decode token for the 30 decoder
// layers of BitNet b1.58 (batch 1), on a persistent grid of G workgroups of
// 1024 threads (cooperative launch: all resident).
//
// Why: every dispatch on this system costs >= 3.3 us even when empty, and a
// decode step of separate kernels needs five per layer.  Here the layer's
// five dependent phases (q/k/v GEMV + RoPE + KV append, attention, o GEMV +
// residual, gate/up GEMV + relu^2*up, down GEMV + residual; model.rs:331-366)
// are separated by a flag barrier instead (one flag per workgroup, relayed by
// workgroup 0; no read-modify-write atomics, which serialise at ~40 ns each).
// Each workgroup owns a fixed slice of rows of every matrix, so the weights of
// the next phase are loaded into registers between "arrive" and "wait": HBM
// latency overlaps the barrier.  Every barrier spin is bounded; a timeout sets
// an error word, the kernel still drains and the host reports LBT_E_DEVICE.
//
// Arithmetic is the decode GEMV's and the attention kernel's (shared code in
// ternary_common.h and attn_common.h; reductions use the first 256 threads in
// the same order), so results equal the multi-kernel path bit for bit.
#include "attn_common.h"
#include "ternary_common.h"

#include <map>
#include <mutex>

namespace lbt {

constexpr int kPT = 512;       // threads per persistent workgroup (256 VGPRs per lane)
constexpr int kWaves = kPT / 64;
constexpr unsigned kSpinLimit = 1u << 20;  // ~1 s of polling
constexpr size_t kCuLds = 160 * 1024;  // LDS per CU (gfx950)
constexpr size_t kTraceStride = 16, kTraceHalf = 4096;  // dynamic LDS budget per workgroup (160 KB per CU)

struct PersistArgs {
    const uint8_t* const* w;   // [layers * 7] packed matrices
    const float* wscale;       // [layers * 7]
    const float* const* norm;  // [layers * 4]: input, post_attn, attn_sub, ffn_sub
    const uint16_t* embed;
    const float* cos_t;
    const float* sin_t;
    uint16_t* kc;
    uint16_t* vc;
    int cap;
    size_t layer_kv;  // elements per layer of the K (or V) cache
    int layers, H, I, nh, kvh, hd, vocab;
    float eps, scaling;
    int* state;  // [0] position - 1, [1] output slot, [2] barrier epoch
    unsigned long long* key;
    uint32_t* tok_out;
    float* x;
    float* q;
    float* att;
    float* ao;   // attention split outputs [kAttnSplits][H]
    float* aml;  // attention split (max, sum) [kAttnSplits][nh][2]
    float* h;
    unsigned* flags;  // [G * 16]
    unsigned* go;
    unsigned* err;
    int rpw[4];  // virtual rows per workgroup: q/k/v, o, gate/up, down
    int wbytes;  // LDS bytes of the weight-tile region
    unsigned long long* trace;  // optional: per-phase timestamps of workgroups 0 and G-1
};

__device__ __forceinline__ unsigned ld_flag(const unsigned* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// All of this workgroup's global writes so far become visible, then its flag
// announces `epoch`.
__device__ __forceinline__ void grid_arrive(const PersistArgs& a, unsigned epoch) {
    __syncthreads();
    if (threadIdx.x == 0) {
        __threadfence();
        __hip_atomic_store(&a.flags[blockIdx.x * 16], epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Workgroup 0 waits for every flag to reach `epoch` and then publishes it in
// `go`; the others wait for `go`.  Spins are bounded, and once any wait has
// timed out (error word set) no later wait spins, so the grid always drains.
__device__ __forceinline__ bool spin_abort(const PersistArgs& a, unsigned spins) {
    if (spins > kSpinLimit) return true;
    return (spins & 1023u) == 1023u && ld_flag(a.err) != 0u;
}

__device__ __forceinline__ void grid_wait(const PersistArgs& a, unsigned epoch) {
    const int G = gridDim.x;
    if (blockIdx.x == 0) {
        if (threadIdx.x < 64) {
            unsigned spins = 0;
            bool ok = ld_flag(a.err) == 0u;
            while (ok) {
                bool mine = true;
                for (int b = threadIdx.x; b < G; b += 64) mine &= ld_flag(&a.flags[b * 16]) >= epoch;
                if (__all(mine)) break;
                if (spin_abort(a, ++spins)) ok = false;
            }
            if (threadIdx.x == 0) {
                if (!ok) atomicAdd(a.err, 1u);
                __threadfence();
                __hip_atomic_store(a.go, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    } else if (threadIdx.x == 0) {
        unsigned spins = 0;
        if (ld_flag(a.err) == 0u) {
            while (ld_flag(a.go) < epoch) {
                if (spin_abort(a, ++spins)) {
                    atomicAdd(a.err, 1u);
                    break;
                }
            }
        }
    }
    if (threadIdx.x == 0) __threadfence();
    __syncthreads();
}

typedef __attribute__((address_space(3))) void lds_void;

// Row tiling of one phase inside the workgroup: R = 64/L rows per tile, tile t
// goes to wave t % 16; lane j of a row takes chunks j, j+L, ..., cpl of them.
// The wave streams its tiles straight into its own LDS slots with
// global_load_lds_dwordx4 (16 bytes per lane, no registers): tile t, chunk
// round i lives at wlds + (t * cpl + i) * 1024, lane l at + 16 l.
template <int L, int OUT>
__device__ __forceinline__ void phase_load(const GemvArgs& g, int vr0, int nrows, int cpl, int8_t* wlds) {
    constexpr int R = 64 / L;
    const int tid = fresh_tid();
    const int w = tid >> 6, lane = tid & 63, rg = lane / L, j = lane % L;
    const int ntiles = (nrows + R - 1) / R;
    for (int t = w; t < ntiles; t += kWaves) {
        const int lr = t * R + rg, vr = vr0 + lr;
        const bool valid = lr < nrows && vr < g.total_rows;
        int mat, r;
        resolve_row<OUT>(g, valid ? vr : 0, mat, r);
        const uint4* rowp = (const uint4*)(sel3(g.w, mat) + (size_t)r * (size_t)(g.kp >> 2));
        for (int i = 0; i < cpl; i++) {
            const int c = j + L * i;
            if (valid && c < g.C)
                __builtin_amdgcn_global_load_lds((const void*)(rowp + c), (lds_void*)(wlds + (t * cpl + i) * 1024),
                                                 16, 0, 0);
        }
    }
}

template <int L, int OUT>
__device__ __forceinline__ void phase_compute(const GemvArgs& g, int vr0, int nrows, int cpl, const int8_t* wlds,
                                              const int8_t* xq, float sa, int qs,
                                              unsigned long long* trace = nullptr) {
    constexpr int R = 64 / L;
    const int tid = fresh_tid();
    const int w = tid >> 6, lane = tid & 63, rg = lane / L, j = lane % L;
    const int C = g.C, ntiles = (nrows + R - 1) / R;
    __builtin_amdgcn_s_waitcnt(0);  // this wave's weight tiles have landed in LDS
    if (trace && threadIdx.x == 0) *trace = wall_clock64();
    for (int t = w; t < ntiles; t += kWaves) {
        int acc = 0;
        for (int i = 0; i < cpl; i++) {
            const int c = j + L * i;
            if (c < C) {
                const uint4 wv = *(const uint4*)(wlds + (t * cpl + i) * 1024 + lane * 16);
#pragma unroll
                for (int kk = 0; kk < 4; kk++) {
                    const int4 xv = *(const int4*)(xq + ((kk * C + c) << 4));
                    const int sh = 2 * kk;
                    acc = __builtin_amdgcn_sdot4((int)((wv.x >> sh) & 0x03030303u), xv.x, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)((wv.y >> sh) & 0x03030303u), xv.y, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)((wv.z >> sh) & 0x03030303u), xv.z, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)((wv.w >> sh) & 0x03030303u), xv.w, acc, false);
                }
            }
        }
        acc = xor_sum_down_i<L / 2>(acc);
        const int dot = acc - qs;
        const int lr = t * R + rg, vr = vr0 + lr;
        const bool ok = lr < nrows && vr < g.total_rows;
        if (OUT == kOutRelu2 || OUT == kOutQKV) {
            const int dp = __shfl_xor(dot, L);
            if (ok && j == 0 && (rg & 1) == 0) store_pair<OUT>(g, 0, vr, dot, dp, sa);
        } else if (ok && j == 0) {
            store_single<OUT>(g, 0, vr, dot, sa);
        }
    }
}

// Quantize the phase input (first 256 threads, the GEMV prologue's order) into
// the permuted LDS image.
template <typename Src>
__device__ __forceinline__ void phase_prologue(Src x, int cols, const float* norm_w, float eps, int8_t* xq,
                                               float* sa, int* qs, float* red) {
    const int kp = (int)((cols + 127) / 128 * 128), C = kp / 64;
    auto pos = [C](int i) { return perm_pos(i, C); };
    if (cols <= 16 * kThreads) quantize_row_block<16>(x, cols, kp, norm_w, eps, xq, pos, sa, qs, red);
    else quantize_row_block<32>(x, cols, kp, norm_w, eps, xq, pos, sa, qs, red);
    __syncthreads();
}

// The o-projection input: the combine of the attention splits, then the
// prologue's norm and quantization.
__device__ __forceinline__ void phase_prologue_attn(const AttnRow& row, const float* norm_w, float eps, int8_t* xq,
                                                    float* sa, int* qs, float* red, AttnTab& tab) {
    const int kp = (row.H + 127) / 128 * 128, C = kp / 64;
    auto pos = [C](int i) { return perm_pos(i, C); };
    if (kp <= 16 * kThreads) {
        RowRegs<16> r;
        AttnRegs<16, 4> ar;
        attn_row_issue(row, norm_w, ar, r);
        attn_row_finish(row, ar, r, tab);
        quantize_row_regs(r, row.H, kp, norm_w, eps, xq, pos, sa, qs, red);
    } else {
        RowRegs<32> r;
        AttnRegs<32, 2> ar;
        attn_row_issue(row, norm_w, ar, r);
        attn_row_finish(row, ar, r, tab);
        quantize_row_regs(r, row.H, kp, norm_w, eps, xq, pos, sa, qs, red);
    }
    __syncthreads();
}

__device__ __forceinline__ GemvArgs make_args(const PersistArgs& a, int layer, int first, int n, int cols) {
    GemvArgs g{};
    for (int i = 0; i < 3; i++) {
        const int wi = layer * 7 + first + (i < n ? i : 0);
        g.w[i] = a.w[wi];
        g.sw[i] = a.wscale[wi];
    }
    g.cols = cols;
    g.kp = (cols + 127) / 128 * 128;
    g.C = g.kp / 64;
    g.m = 1;
    g.eps = a.eps;
    return g;
}

template <int LK>
__global__ __launch_bounds__(kPT) void decode_persistent_kernel(PersistArgs a) {
    extern __shared__ __align__(16) int8_t dyn[];  // [weight tiles: wbytes][activation image / scores]
    __shared__ __align__(16) float red[kRedFloats];
    __shared__ float sa_s;
    __shared__ int qs_s;
    __shared__ AttnShared<LK> ash;
    __shared__ AttnTab atab;
    const int G = gridDim.x, b = blockIdx.x;
    const int H = a.H, I = a.I, hd = a.hd, KV = a.kvh * hd;
    const int p = a.state[0] + 1;
    const int slot = a.state[1];
    unsigned epoch = (unsigned)a.state[2];
    uint32_t tok = 0xffffffffu - (uint32_t)(a.key[0] & 0xffffffffull);
    if (tok >= (uint32_t)a.vocab) tok = 0;
    const uint16_t* erow = a.embed + (size_t)tok * H;

    // row slices of this workgroup (virtual rows, even for the paired modes)
    const int vq0 = b * a.rpw[0], vo0 = b * a.rpw[1], vg0 = b * a.rpw[2], vd0 = b * a.rpw[3];
    const int nq = a.rpw[0], no = a.rpw[1], ng = a.rpw[2], nd = a.rpw[3];
    const int kpH = (H + 127) / 128 * 128, kpI = (I + 127) / 128 * 128;
    const int Lq = kpH <= 4096 ? 8 : 16, Ld = kpI <= 4096 ? 8 : 16;  // chunk lanes for K = H, K = I
    const int cplH = (kpH / 64 + Lq - 1) / Lq, cplI = (kpI / 64 + Ld - 1) / Ld;
    int8_t* wl = dyn;
    int8_t* act = dyn + a.wbytes;

    auto gq = [&](int l) {
        GemvArgs g = make_args(a, l, 0, 3, H);
        g.rows[0] = H;
        g.rows[1] = KV;
        g.rows[2] = KV;
        g.total_rows = H + 2 * KV;
        g.hd = hd;
        g.pos0 = p;
        g.cap = a.cap;
        g.cos_t = a.cos_t;
        g.sin_t = a.sin_t;
        g.kc = a.kc + (size_t)l * a.layer_kv;
        g.vc = a.vc + (size_t)l * a.layer_kv;
        g.out[0] = a.q;
        return g;
    };
    auto go_ = [&](int l) {
        GemvArgs g = make_args(a, l, 3, 1, H);
        g.rows[0] = H;
        g.total_rows = H;
        g.out[0] = a.x;
        return g;
    };
    auto gg = [&](int l) {
        GemvArgs g = make_args(a, l, 4, 2, H);
        g.rows[0] = I;
        g.rows[1] = I;
        g.total_rows = 2 * I;
        g.out[0] = a.h;
        return g;
    };
    auto gd = [&](int l) {
        GemvArgs g = make_args(a, l, 6, 1, I);
        g.rows[0] = H;
        g.total_rows = H;
        g.out[0] = a.x;
        return g;
    };
    auto load_for = [&](int phase, int l) {
        if (phase == 0) {
            if (Lq == 8) phase_load<8, kOutQKV>(gq(l), vq0, nq, cplH, wl);
            else phase_load<16, kOutQKV>(gq(l), vq0, nq, cplH, wl);
        } else if (phase == 1) {
            if (Lq == 8) phase_load<8, kOutF32Add>(go_(l), vo0, no, cplH, wl);
            else phase_load<16, kOutF32Add>(go_(l), vo0, no, cplH, wl);
        } else if (phase == 2) {
            if (Lq == 8) phase_load<8, kOutRelu2>(gg(l), vg0, ng, cplH, wl);
            else phase_load<16, kOutRelu2>(gg(l), vg0, ng, cplH, wl);
        } else {
            if (Ld == 8) phase_load<8, kOutF32Add>(gd(l), vd0, nd, cplI, wl);
            else phase_load<16, kOutF32Add>(gd(l), vd0, nd, cplI, wl);
        }
    };

    load_for(0, 0);
    // residual stream of this workgroup's o/down rows starts as the embedding
    for (int r = threadIdx.x; r < no; r += kPT)
        if (vo0 + r < H) a.x[vo0 + r] = bf16_to_f32(erow[vo0 + r]);

#define LBT_TR(k)                                                                          \
    if (a.trace && threadIdx.x == 0 && (b == 0 || b == G - 1))                             \
        a.trace[(b ? kTraceHalf : 0) + (size_t)l * kTraceStride + (k)] = wall_clock64();
    for (int l = 0; l < a.layers; l++) {
        const float* const* nw = a.norm + (size_t)l * 4;
        LBT_TR(0)
        // ---- q/k/v + RoPE + KV append
        if (l == 0) phase_prologue(SrcBf16{erow}, H, nw[0], a.eps, act, &sa_s, &qs_s, red);
        else phase_prologue(SrcF32{a.x}, H, nw[0], a.eps, act, &sa_s, &qs_s, red);
        LBT_TR(1)
        if (Lq == 8) phase_compute<8, kOutQKV>(gq(l), vq0, nq, cplH, wl, act, sa_s, qs_s);
        else phase_compute<16, kOutQKV>(gq(l), vq0, nq, cplH, wl, act, sa_s, qs_s);
        LBT_TR(2)
        grid_arrive(a, ++epoch);
        load_for(1, l);
        LBT_TR(3)
        grid_wait(a, epoch);
        LBT_TR(4)
        // ---- attention: (query head, key split) items b, b + G, ... on the first 256 threads
        for (int it = b; it < a.nh * kAttnSplits; it += G) {
            const int hq = it / kAttnSplits, g = hq / (a.nh / a.kvh);
            const size_t kvoff = (size_t)l * a.layer_kv + (size_t)g * a.cap * hd;
            attention_split_ku<LK, 4>(a.q, hq, a.nh, it % kAttnSplits, p, a.kc + kvoff, a.vc + kvoff, a.scaling, a.ao,
                                      a.aml, (float*)act, ash);
        }
        LBT_TR(5)
        grid_arrive(a, ++epoch);
        grid_wait(a, epoch);
        LBT_TR(6)
        // ---- o_proj(attn_sub_norm(attn)), x += y
        phase_prologue_attn(AttnRow{a.ao, a.aml, attn_splits(p + 1), a.nh, hd, H}, nw[2], a.eps, act, &sa_s,
                            &qs_s, red, atab);
        LBT_TR(7)
        if (Lq == 8) phase_compute<8, kOutF32Add>(go_(l), vo0, no, cplH, wl, act, sa_s, qs_s);
        else phase_compute<16, kOutF32Add>(go_(l), vo0, no, cplH, wl, act, sa_s, qs_s);
        LBT_TR(8)
        grid_arrive(a, ++epoch);
        load_for(2, l);
        grid_wait(a, epoch);
        LBT_TR(9)
        // ---- gate/up on post_attention_norm(x), relu(g)^2 * u
        phase_prologue(SrcF32{a.x}, H, nw[1], a.eps, act, &sa_s, &qs_s, red);
        LBT_TR(10)
        unsigned long long* tr_gu =
            (a.trace && (b == 0 || b == G - 1)) ? a.trace + (b ? kTraceHalf : 0) + 2048 + l * 4 : nullptr;
        if (Lq == 8) phase_compute<8, kOutRelu2>(gg(l), vg0, ng, cplH, wl, act, sa_s, qs_s, tr_gu);
        else phase_compute<16, kOutRelu2>(gg(l), vg0, ng, cplH, wl, act, sa_s, qs_s, tr_gu);
        LBT_TR(11)
        grid_arrive(a, ++epoch);
        load_for(3, l);
        grid_wait(a, epoch);
        LBT_TR(12)
        // ---- down on ffn_sub_norm(h), x += y
        phase_prologue(SrcF32{a.h}, I, nw[3], a.eps, act, &sa_s, &qs_s, red);
        LBT_TR(13)
        unsigned long long* tr_dn =
            (a.trace && (b == 0 || b == G - 1)) ? a.trace + (b ? kTraceHalf : 0) + 2048 + l * 4 + 1 : nullptr;
        if (Ld == 8) phase_compute<8, kOutF32Add>(gd(l), vd0, nd, cplI, wl, act, sa_s, qs_s, tr_dn);
        else phase_compute<16, kOutF32Add>(gd(l), vd0, nd, cplI, wl, act, sa_s, qs_s, tr_dn);
        LBT_TR(14)
        if (l + 1 < a.layers) {
            grid_arrive(a, ++epoch);
            load_for(0, l + 1);
            grid_wait(a, epoch);
        }
        LBT_TR(15)
    }
#undef LBT_TR
    // The LM head runs as the next dispatch.  Every workgroup read the state
    // and the key before the first barrier, so workgroup 0 may update them.
    if (b == 0 && threadIdx.x == 0) {
        a.tok_out[slot] = tok;
        a.state[0] = p;
        a.state[1] = slot + 1;
        a.state[2] = (int)epoch;
        a.key[0] = 0ull;
    }
}

// Weight-tile LDS bytes and activation/score bytes of a configuration.
static void persistent_lds(const lbt_config& c, int cap, const int* rpw, size_t* wbytes, size_t* abytes) {
    const int kpH = (c.hidden_size + 127) / 128 * 128, kpI = (c.intermediate_size + 127) / 128 * 128;
    const int Ks[4] = {kpH, kpH, kpH, kpI};
    size_t w = 0;
    for (int i = 0; i < 4; i++) {
        const int L = Ks[i] <= 4096 ? 8 : 16, R = 64 / L;
        const int cpl = (Ks[i] / 64 + L - 1) / L;
        const size_t tiles = (size_t)((rpw[i] + R - 1) / R);
        if (tiles * cpl * 1024 > w) w = tiles * cpl * 1024;
    }
    *wbytes = w;
    const size_t sc = (size_t)attn_split_keys(cap) * 4;
    *abytes = (size_t)(kpI > kpH ? kpI : kpH) > sc ? (size_t)(kpI > kpH ? kpI : kpH) : sc;
}

namespace {

const void* persistent_fn(int hd) {
    switch (hd) {
        case 64: return (const void*)decode_persistent_kernel<8>;
        case 128: return (const void*)decode_persistent_kernel<16>;
        case 256: return (const void*)decode_persistent_kernel<32>;
        default: return nullptr;
    }
}

// Dynamic LDS available to an instantiation: the CU's LDS less its static
// shared memory (the attention scratch grows with the head shape).
size_t persistent_dyn_limit(const void* fn) {
    static std::mutex mu;
    static std::map<const void*, size_t> lim;
    std::lock_guard<std::mutex> lk(mu);
    auto it = lim.find(fn);
    if (it != lim.end()) return it->second;
    hipFuncAttributes at{};
    size_t v = 0;
    if (hipFuncGetAttributes(&at, fn) == hipSuccess && at.sharedSizeBytes < kCuLds) v = kCuLds - at.sharedSizeBytes;
    (void)hipGetLastError();
    if (v && hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)v) != hipSuccess) v = 0;
    (void)hipGetLastError();
    lim[fn] = v;
    return v;
}

}  // namespace

int persistent_supported(const lbt_config& c, int cap, int G, int* rpw, const char** why) {
    const int hd = c.hidden_size / c.num_attention_heads;
    const int H = c.hidden_size, I = c.intermediate_size, KV = c.num_key_value_heads * hd;
    if (hd != 64 && hd != 128 && hd != 256) return *why = "head_dim", 0;
    if (c.num_attention_heads > kAttnMaxHeads) return *why = "heads", 0;
    const int kpH = (H + 127) / 128 * 128, kpI = (I + 127) / 128 * 128;
    if (kpH > 8192 || kpI > 8192) return *why = "hidden/intermediate > 8192", 0;
    const int tot[4] = {H + 2 * KV, H, 2 * I, H};
    for (int i = 0; i < 4; i++) {
        int r = (tot[i] + G - 1) / G;
        rpw[i] = (r + 1) & ~1;  // pairs never straddle workgroups
    }
    size_t wb, ab;
    persistent_lds(c, cap, rpw, &wb, &ab);
    const void* fn = persistent_fn(hd);
    if (!fn) return *why = "head shape", 0;
    if (wb + ab > persistent_dyn_limit(fn)) return *why = "LDS", 0;
    return 1;
}


int launch_decode_persistent(lbt_ctx* ctx, const PersistHost& h, int G, hipStream_t s) {
    PersistArgs a{};
    a.w = h.w;
    a.wscale = h.wscale;
    a.norm = h.norm;
    a.embed = h.embed;
    a.cos_t = h.cos_t;
    a.sin_t = h.sin_t;
    a.kc = h.kc;
    a.vc = h.vc;
    a.cap = h.cap;
    a.layer_kv = h.layer_kv;
    a.layers = h.cfg.num_hidden_layers;
    a.H = h.cfg.hidden_size;
    a.I = h.cfg.intermediate_size;
    a.nh = h.cfg.num_attention_heads;
    a.kvh = h.cfg.num_key_value_heads;
    a.hd = a.H / a.nh;
    a.vocab = h.cfg.vocab_size;
    a.eps = (float)h.cfg.rms_norm_eps;
    a.scaling = h.scaling;
    a.state = h.state;
    a.key = h.key;
    a.tok_out = h.tok_out;
    a.x = h.x;
    a.q = h.q;
    a.att = h.att;
    a.ao = h.ao;
    a.aml = h.aml;
    a.h = h.h;
    a.flags = h.flags;
    a.go = h.go;
    a.err = h.err;
    for (int i = 0; i < 4; i++) a.rpw[i] = h.rpw[i];
    size_t wb, ab;
    persistent_lds(h.cfg, h.cap, h.rpw, &wb, &ab);
    a.wbytes = (int)wb;
    a.trace = h.trace;
    const size_t lds = wb + ab;
    void* args[] = {&a};
    const void* fn = persistent_fn(a.hd);
    if (!fn) return set_err(ctx, LBT_E_INVALID, "persistent decode: unsupported head shape");
    if (lds > persistent_dyn_limit(fn)) return set_err(ctx, LBT_E_INVALID, "persistent decode: LDS budget");
    hipEvent_t e0, e1;
    prof_pair(ctx, &e0, &e1);
    if (e0) (void)hipEventRecord(e0, s);
    const hipError_t e = hipLaunchCooperativeKernel(fn, dim3(G), dim3(kPT), args, lds, s);
    if (e1) (void)hipEventRecord(e1, s);
    if (e != hipSuccess) return hip_err(ctx, e, "persistent decode launch");
    prof_commit(ctx, e0, e1, kProfOther, 0.0);
    return LBT_OK;
}

}  // namespace lbt
