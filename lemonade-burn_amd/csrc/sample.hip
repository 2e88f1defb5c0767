// sample.hip -- token sampling on the device: Sampler::sample
// (crates/lb-model/src/sample.rs:45-82) for rows of logits, so that only
// token ids leave the GPU (the reference ships every 128256-float logit row
// to the host and sorts it there, lb-server/src/main.rs:141-160).
//
// Three launches per call: the row max and the candidate pass over chunks of
// 2048 logits (sample_max_kernel, sample_cand_kernel, one 256-thread
// workgroup per chunk), then one workgroup of 1024 threads per row for the
// selects and the draw (sample_kernel).  The reference's steps, in its
// order: temperature <= 0 is the argmax (sample.rs:17-25); otherwise the
// logits are ordered by descending total_cmp (ties: ascending index -- the
// reference's unstable sort leaves their order open), truncated to top_k,
// p = exp((l - max) / t), cut to the shortest prefix whose cumulative
// probability reaches top_p, and one xorshift64 draw r = (state >> 40) / 2^24
// (sample.rs:36-43) picks the first element whose cumulative probability
// exceeds r.  The probabilities are summed as exact integers,
// w = floor(p * 2^45) (p <= 1, so 2^17 of them stay below 2^62):
//   c >= top_p  <=>  sum(w) >= ceil(top_p * W),
//   r < c       <=>  sum(w) >= floor(draw * W_keep / 2^24) + 1,
// so no float sum depends on an order and no sort is needed: each "first
// element in sorted order whose prefix reaches T" is a radix select over the
// keys (~total order << index bits | index) with weight histograms: three
// rounds over the value, then the index bits only where values tie.
// Elements with w = 0 can never be chosen, so only elements with w > 0 (a
// prefix of the sorted order) are kept as candidates -- in LDS when
// they fit, else in a global scratch of 16 bytes per logit.  A NaN among the
// top-k p (a NaN logit in the set, max = +inf, all -inf, a NaN temperature)
// makes every comparison of the reference false: it returns the last element
// of the set, and so does this kernel.
#include "lbt_device.h"
#include "lbt_internal.h"

namespace lbt {

namespace {

constexpr int kST = 1024;  // threads
constexpr int kBins = 2048;  // histogram bins: digits of up to 11 bits
constexpr int kLdsCand = 4096;  // candidates kept in LDS
constexpr unsigned long long kNone = ~0ull;
// The candidate pass runs in chunks of a row, one 256-thread workgroup each
constexpr int kChunk = 2048, kCT = 256;

struct Cand {
    unsigned long long s, w;
};

struct SampleShared {
    Cand cand[kLdsCand];
    unsigned long long hist[kBins];
    unsigned long long minkey[kBins];  // smallest key per bin (last value round)
    unsigned bcnt[kBins];              // elements per bin (last value round)
    unsigned long long red[kST / 64];
    unsigned long long red2[kST / 64];
    unsigned long long sel_below, sel_through;
    unsigned sel_bin;
    unsigned long long sel_min;
    unsigned sel_cnt;
    unsigned cnt;
    float fred[kST / 64];
    unsigned ired[kST / 64];
};

// Per-chunk results of the candidate pass: the largest total-order key of
// the chunk (sample_max_kernel), then its candidates' weight sum, the
// smallest key of a NaN p and the largest key (sample_cand_kernel).
struct ChunkSum {
    unsigned long long w, nan_s, smax;
    unsigned cmax, pad;
};

// Ascending key of the IEEE total order (total_cmp) of x's bits.
__device__ __forceinline__ unsigned total_asc(float x) {
    const unsigned b = __float_as_uint(x);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Sorted-order key of element i: ascending keys = descending logits, then
// ascending index (ib index bits, so keys stay below 2^(32 + ib)).
__device__ __forceinline__ unsigned long long sample_key(float x, unsigned i, int ib) {
    return ((unsigned long long)(~total_asc(x)) << ib) | i;
}

__device__ __forceinline__ unsigned long long wave_sum(unsigned long long v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
    return v;
}
__device__ __forceinline__ unsigned long long wave_min(unsigned long long v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        const unsigned long long o = __shfl_xor(v, d, 64);
        v = o < v ? o : v;
    }
    return v;
}
__device__ __forceinline__ unsigned long long wave_max(unsigned long long v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        const unsigned long long o = __shfl_xor(v, d, 64);
        v = o > v ? o : v;
    }
    return v;
}

// Block reductions (every thread gets the result); kind 0 sum, 1 min, 2 max.
template <int KIND>
__device__ unsigned long long block_red(unsigned long long v, unsigned long long* buf) {
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    v = KIND == 0 ? wave_sum(v) : KIND == 1 ? wave_min(v) : wave_max(v);
    __syncthreads();
    if (lane == 0) buf[w] = v;
    __syncthreads();
    unsigned long long r = buf[0];
    for (int i = 1; i < kST / 64; i++) {
        const unsigned long long o = buf[i];
        r = KIND == 0 ? r + o : KIND == 1 ? (o < r ? o : r) : (o > r ? o : r);
    }
    return r;
}

// ceil(top_p * W) for top_p < 1 (0 for top_p <= 0), exactly: top_p = M 2^-sh
// with M < 2^24, M * W < 2^86 held as two 64-bit words.
__device__ unsigned long long top_p_target(float top_p, unsigned long long W) {
    if (!(top_p > 0.0f)) return 0;
    const unsigned b = __float_as_uint(top_p);
    const int be = (int)((b >> 23) & 0xff);
    const unsigned long long M = be ? ((b & 0x7fffffu) | 0x800000u) : (b & 0x7fffffu);
    const int sh = be ? 150 - be : 149;  // top_p = M 2^-sh
    if (sh >= 128) return 1;
    const unsigned long long lo = M * W, hi = __umul64hi(M, W);
    unsigned long long q, rem;
    if (sh >= 64) {
        q = sh == 64 ? hi : hi >> (sh - 64);
        rem = lo | (sh == 64 ? 0ull : (hi & ((1ull << (sh - 64)) - 1)));
    } else {
        q = (lo >> sh) | (hi << (64 - sh));
        rem = lo & ((1ull << sh) - 1);
    }
    return q + (rem ? 1 : 0);
}

// The smallest key s* among candidates with s <= lim whose cumulative weight
// (w with MASS, else 1 each) through s* reaches `target` (which must not
// exceed their total); `through` = that cumulative weight.  All threads call.
// Source of (key, weight) pairs: the candidate list, or every logit of the
// row with weight 1.
// Sources of (key, weight) pairs, visited by all threads of the workgroup:
// the candidate list or every logit of the row with weight 1.
struct CandSrc {
    const Cand* c;
    unsigned n;
    template <class F>
    __device__ void for_each(F f) const {
        for (unsigned i = threadIdx.x; i < n; i += kST) f(c[i].s, c[i].w);
    }
};
struct LogitSrc {
    const float* lg;
    int ib;
    unsigned n;
    template <class F>
    __device__ void for_each(F f) const {
        for (unsigned i = threadIdx.x; i < n; i += kST) f(sample_key(lg[i], i, ib), 1ull);
    }
};

// One round of the select: the histogram of digit (s >> shift) & (2^bits - 1)
// over the elements with s <= lim whose bits above shift + bits equal
// `prefix`, then the first bin (ascending) whose cumulative weight from
// `below` reaches `target`.  LAST also counts the elements of each bin and
// keeps its smallest key.
template <bool MASS, bool LAST, class Src>
__device__ void select_round(const Src& c, unsigned long long lim, unsigned long long target, int shift, int bits,
                             unsigned long long prefix, unsigned long long below, SampleShared& sh) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int nb = 1 << bits;
    for (int b = tid; b < nb; b += kST) {
        sh.hist[b] = 0;
        if (LAST) {
            sh.bcnt[b] = 0;
            sh.minkey[b] = kNone;
        }
    }
    __syncthreads();
    c.for_each([&](unsigned long long s, unsigned long long w) {
        if (s <= lim && (s >> (shift + bits)) == prefix) {
            const unsigned bin = (unsigned)(s >> shift) & (unsigned)(nb - 1);
            atomicAdd(&sh.hist[bin], MASS ? w : 1ull);
            if (LAST) {
                atomicAdd(&sh.bcnt[bin], 1u);
                atomicMin(&sh.minkey[bin], s);
            }
        }
    });
    __syncthreads();
    if (tid < 64) {
        // PL bins per lane; bins past nb (rounds of fewer than 64 bins) are
        // empty, whatever an earlier round left there
        const int PL = nb >= 64 ? nb / 64 : 1;
        auto hbin = [&](int b) { return b < nb ? sh.hist[b] : 0ull; };
        unsigned long long sum = 0;
        for (int j = 0; j < PL; j++) sum += hbin(PL * lane + j);
        unsigned long long inc = sum;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const unsigned long long v = __shfl_up(inc, d, 64);
            if (lane >= d) inc += v;
        }
        unsigned long long run = below + inc - sum, bel = 0, thr = 0;
        unsigned found = kBins;
        for (int j = 0; j < PL; j++) {
            const unsigned long long h = hbin(PL * lane + j);
            if (h && found == kBins && run + h >= target) {
                found = PL * lane + j;
                bel = run;
                thr = run + h;
            }
            run += h;
        }
        const unsigned long long fmin = wave_min((unsigned long long)found);
        if (found == fmin && found < kBins) {
            sh.sel_bin = found;
            sh.sel_below = bel;
            sh.sel_through = thr;
            if (LAST) {
                sh.sel_cnt = sh.bcnt[found];
                sh.sel_min = sh.minkey[found];
            }
        }
    }
    __syncthreads();
}

// The smallest key s* among candidates with s <= lim whose cumulative weight
// (w with MASS, else 1 each) through s* reaches `target` (which must not
// exceed their total); `through` = that cumulative weight.  All threads call.
// Keys are (value key << ib) | index: three rounds over the 32-bit value key
// (11, 11 and 10 bits); when the selected value is held by one element (no
// tie) that element is s*, else rounds over the ib index bits among the
// elements of that value follow.  The same s* as a radix select over the
// whole key, in fewer passes.
template <bool MASS, class Src>
__device__ unsigned long long radix_select(const Src& c, unsigned long long lim, unsigned long long target, int ib,
                                           SampleShared& sh, unsigned long long& through) {
    unsigned long long prefix = 0, below = 0;
    select_round<MASS, false>(c, lim, target, ib + 21, 11, prefix, below, sh);
    prefix = sh.sel_bin;
    below = sh.sel_below;
    select_round<MASS, false>(c, lim, target, ib + 10, 11, prefix, below, sh);
    prefix = (prefix << 11) | sh.sel_bin;
    below = sh.sel_below;
    select_round<MASS, true>(c, lim, target, ib, 10, prefix, below, sh);
    prefix = (prefix << 10) | sh.sel_bin;
    below = sh.sel_below;
    through = sh.sel_through;
    if (sh.sel_cnt == 1) return sh.sel_min;
    // a tie of values: the index bits, high digits first (11 bits at most)
    for (int done = 0; done < ib;) {
        const int bits = ib - done < 11 ? ib - done : 11;
        const int shift = ib - done - bits;
        select_round<MASS, false>(c, lim, target, shift, bits, prefix, below, sh);
        prefix = (prefix << bits) | sh.sel_bin;
        below = sh.sel_below;
        through = sh.sel_through;
        done += bits;
    }
    return prefix;
}

struct SampleArgs {
    const float* logits;
    long ld;  // floats between rows
    int V;
    float temperature, top_p;
    unsigned long long top_k;  // 0: no truncation
    const lbt_sample_params* rowp;  // [rows] per-row parameters in device memory (null: the ones above)
    unsigned long long* states;  // [rows] xorshift states, advanced by one draw when temperature > 0
    uint32_t* out_tok;            // [rows] (nullable)
    unsigned long long* out_key;  // [rows] argmax-key words the next embedding reads (nullable)
    Cand* scratch;                // [rows][V] candidates, chunk g's at [row][g * kChunk ..)
    ChunkSum* sums;               // [rows][G]
    unsigned* ncand;              // [rows] candidates of the row (zeroed by sample_max_kernel)
    int G;                        // chunks of a row
};

__device__ __forceinline__ float row_temperature(const SampleArgs& a, int row) {
    return a.rowp ? gload(&a.rowp[row].temperature) : a.temperature;
}

// Largest total-order key of chunk blockIdx.x of row blockIdx.y.
__global__ __launch_bounds__(kCT) void sample_max_kernel(SampleArgs a) {
    __shared__ unsigned red[kCT / 64];
    const int g = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    if (row_temperature(a, row) <= 0.0f) return;  // argmax rows (a NaN temperature samples, as in sample_kernel)
    if (g == 0 && tid == 0) a.ncand[row] = 0u;
    const float* lg = a.logits + (size_t)row * a.ld;
    const int c0 = g * kChunk, c1 = c0 + kChunk < a.V ? c0 + kChunk : a.V;
    unsigned mk = 0;
    for (int i = c0 + tid; i < c1; i += kCT) {
        const unsigned k = total_asc(lg[i]);
        mk = k > mk ? k : mk;
    }
    mk = (unsigned)wave_max((unsigned long long)mk);
    if ((tid & 63) == 0) red[tid >> 6] = mk;
    __syncthreads();
    if (tid == 0) {
        unsigned m = red[0];
        for (int w = 1; w < kCT / 64; w++) m = red[w] > m ? red[w] : m;
        a.sums[(size_t)row * a.G + g].cmax = m;
    }
}

// The candidates (w > 0) of chunk blockIdx.x of row blockIdx.y, compacted in
// LDS and appended to the row's list in one range (one atomic per
// workgroup: the list's order varies, the set does not), and the chunk's
// sums; the row max from the chunk maxima.  The same keys and weights,
// element by element, as a single pass over the row: the selects, which
// depend on the set only, pick the same element.
__global__ __launch_bounds__(kCT) void sample_cand_kernel(SampleArgs a) {
    __shared__ unsigned long long red[3][kCT / 64];
    __shared__ unsigned ured[kCT / 64];
    __shared__ unsigned cnt, base;
    __shared__ Cand lc[kChunk];
    const int g = blockIdx.x, row = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const float t = row_temperature(a, row);
    if (t <= 0.0f) return;
    const float* lg = a.logits + (size_t)row * a.ld;
    ChunkSum* sums = a.sums + (size_t)row * a.G;
    unsigned mk = 0;
    for (int j = tid; j < a.G; j += kCT) {
        const unsigned k = gload(&sums[j].cmax);
        mk = k > mk ? k : mk;
    }
    mk = (unsigned)wave_max((unsigned long long)mk);
    if (lane == 0) ured[wv] = mk;
    if (tid == 0) cnt = 0;
    __syncthreads();
    mk = ured[0];
    for (int w = 1; w < kCT / 64; w++) mk = ured[w] > mk ? ured[w] : mk;
    const float mx = __uint_as_float((mk & 0x80000000u) ? (mk & 0x7fffffffu) : ~mk);
    const int V = a.V;
    int ib = 1;
    while (ib < 32 && (1u << ib) < (unsigned)V) ib++;
    const int c0 = g * kChunk, c1 = c0 + kChunk < V ? c0 + kChunk : V;
    unsigned long long wsum = 0, nan_s = kNone, smax = 0;
    for (int i0 = c0; i0 < c1; i0 += kCT) {
        const int i = i0 + tid;
        bool keep = false;
        unsigned long long s = 0, w = 0;
        if (i < c1) {
            const float l = lg[i];
            s = sample_key(l, (unsigned)i, ib);
            smax = s > smax ? s : smax;
            const float p = lbt_expf((l - mx) / t);
            if (p != p) {
                nan_s = s < nan_s ? s : nan_s;
            } else {
                w = (unsigned long long)(p * 0x1p45f);
                keep = w != 0;
                wsum += w;
            }
        }
        const unsigned long long m = __ballot(keep);
        if (m) {
            unsigned base = 0;
            if (lane == 0) base = atomicAdd(&cnt, (unsigned)__popcll(m));
            base = __shfl(base, 0, 64);
            if (keep) lc[base + (unsigned)__popcll(m & ((1ull << lane) - 1))] = Cand{s, w};
        }
    }
    wsum = wave_sum(wsum);
    nan_s = wave_min(nan_s);
    smax = wave_max(smax);
    if (lane == 0) {
        red[0][wv] = wsum;
        red[1][wv] = nan_s;
        red[2][wv] = smax;
    }
    __syncthreads();
    if (tid == 0) {
        unsigned long long W = 0, ns = kNone, sm = 0;
        for (int w = 0; w < kCT / 64; w++) {
            W += red[0][w];
            ns = red[1][w] < ns ? red[1][w] : ns;
            sm = red[2][w] > sm ? red[2][w] : sm;
        }
        sums[g].w = W;
        sums[g].nan_s = ns;
        sums[g].smax = sm;
        base = cnt ? atomicAdd(&a.ncand[row], cnt) : 0u;
    }
    __syncthreads();
    Cand* gc = a.scratch + (size_t)row * V + base;
    for (unsigned i = tid; i < cnt; i += kCT) gc[i] = lc[i];
}

// The top-k cut, the NaN rule, the top-p cut and the draw over the row's n
// candidates (source c), from their total weight Wall, the smallest key of a
// NaN p and the largest key; returns the token.  All threads call.
template <class Src>
__device__ unsigned sample_pick(const SampleArgs& a, const Src& c, const float* lg, int V, int ib, unsigned n,
                                unsigned long long Wall, unsigned long long nan_s, unsigned long long smax,
                                unsigned long long u, SampleShared& sh) {
    const unsigned long long imask = (1ull << ib) - 1;
    const unsigned long long kk = (a.top_k > 0 && a.top_k < (unsigned long long)V) ? a.top_k : (unsigned long long)V;
    unsigned long long lim = kNone, W = Wall, thr;
    if (kk < n) {
        lim = radix_select<false>(c, kNone, kk, ib, sh, thr);
        unsigned long long part = 0;
        c.for_each([&](unsigned long long s, unsigned long long w) {
            if (s <= lim) part += w;
        });
        W = block_red<0>(part, sh.red);
    }
    bool bad = false;
    unsigned long long last = smax;  // last element of the top-k set
    if (nan_s != kNone) {
        if (kk < (unsigned long long)V) {
            if (kk < n) {
                last = lim;
            } else {
                // the k-th element lies beyond the candidates: select over all logits
                last = radix_select<false>(LogitSrc{lg, ib, (unsigned)V}, kNone, kk, ib, sh, thr);
            }
        }
        bad = nan_s <= last;
    }
    if (bad) return (unsigned)(last & imask);
    unsigned long long keep_lim = lim, WK = W;
    if (a.top_p < 1.0f) keep_lim = radix_select<true>(c, lim, top_p_target(a.top_p, W), ib, sh, WK);
    const unsigned long long Td = ((u * (WK & 0xffffffull)) >> 24) + u * (WK >> 24) + 1;
    const unsigned long long sd = radix_select<true>(c, keep_lim, Td, ib, sh, thr);
    return (unsigned)(sd & imask);
}

__global__ __launch_bounds__(kST) void sample_kernel(SampleArgs a) {
    __shared__ SampleShared sh;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int row = blockIdx.x, V = a.V;
    const float* lg = a.logits + (size_t)row * a.ld;
    if (a.rowp) {
        a.temperature = gload(&a.rowp[row].temperature);
        a.top_p = gload(&a.rowp[row].top_p);
        a.top_k = (unsigned long long)gload(&a.rowp[row].top_k);
    }
    const float t = a.temperature;
    unsigned out = 0;
    if (t <= 0.0f) {
        // argmax (sample.rs:17-25): the first index of the largest value under
        // float comparison; a NaN never wins, and a NaN at index 0 stays
        float bv = 0.0f;
        int bi = V;
        for (int i = tid; i < V; i += kST) {
            const float v = lg[i];
            if (v == v && (bi == V || v > bv)) {
                bv = v;
                bi = i;
            }
        }
        for (int d = 32; d >= 1; d >>= 1) {
            const float ov = __shfl_xor(bv, d, 64);
            const int oi = __shfl_xor(bi, d, 64);
            if (oi != V && (bi == V || ov > bv || (ov == bv && oi < bi))) {
                bv = ov;
                bi = oi;
            }
        }
        if (lane == 0) {
            sh.fred[wv] = bv;
            sh.ired[wv] = (unsigned)bi;
        }
        __syncthreads();
        if (tid == 0) {
            for (int w = 0; w < kST / 64; w++) {
                const float ov = sh.fred[w];
                const int oi = (int)sh.ired[w];
                if (oi != V && (bi == V || ov > bv || (ov == bv && oi < bi))) {
                    bv = ov;
                    bi = oi;
                }
            }
            const float l0 = lg[0];
            out = (l0 != l0 || bi == V) ? 0u : (unsigned)bi;
            if (a.out_tok) a.out_tok[row] = out;
            if (a.out_key) a.out_key[row] = 0xffffffffull - out;
        }
        return;
    }

    // the candidate pass ran in chunks (sample_max_kernel, sample_cand_kernel):
    // their counts, total weight, NaN and largest keys
    int ib = 1;
    while (ib < 32 && (1u << ib) < (unsigned)V) ib++;
    const int G = a.G;
    const ChunkSum* sums = a.sums + (size_t)row * G;
    unsigned long long wsum = 0, nan_s = kNone, smax = 0;
    for (int g = tid; g < G; g += kST) {
        wsum += gload(&sums[g].w);
        const unsigned long long ns = gload(&sums[g].nan_s), sm = gload(&sums[g].smax);
        nan_s = ns < nan_s ? ns : nan_s;
        smax = sm > smax ? sm : smax;
    }
    const unsigned long long Wall = block_red<0>(wsum, sh.red);
    nan_s = block_red<1>(nan_s, sh.red2);
    smax = block_red<2>(smax, sh.red);
    const unsigned n = gload(&a.ncand[row]);
    const Cand* gc = a.scratch + (size_t)row * V;
    // few candidates: copied into LDS
    if (n <= (unsigned)kLdsCand) {
        for (unsigned i = tid; i < n; i += kST) sh.cand[i] = gc[i];
        __syncthreads();
    }
    const CandSrc c{n <= (unsigned)kLdsCand ? sh.cand : gc, n};
    // one draw per call (sample.rs:36-43, 71)
    unsigned long long st = a.states[row];
    st ^= st << 13;
    st ^= st >> 7;
    st ^= st << 17;
    const unsigned long long u = st >> 40;
    __syncthreads();
    if (tid == 0) a.states[row] = st;

    out = sample_pick(a, c, lg, V, ib, n, Wall, nan_s, smax, u, sh);
    if (tid == 0) {
        if (a.out_tok) a.out_tok[row] = out;
        if (a.out_key) a.out_key[row] = 0xffffffffull - out;
    }
}

}  // namespace

namespace {
size_t cand_bytes(int rows, int vocab) { return ((size_t)rows * (size_t)vocab * sizeof(Cand) + 255) & ~(size_t)255; }
int chunks_of(int vocab) { return (vocab + kChunk - 1) / kChunk; }

size_t sums_bytes(int rows, int vocab) {
    return ((size_t)rows * (size_t)chunks_of(vocab) * sizeof(ChunkSum) + 255) & ~(size_t)255;
}
}  // namespace

int sample_scratch_bytes(int rows, int vocab, size_t* bytes) {
    *bytes = cand_bytes(rows, vocab) + sums_bytes(rows, vocab) + (size_t)rows * 4;
    return LBT_OK;
}

int launch_sample(lbt_ctx* ctx, const float* logits, long ld, int rows, int vocab, const lbt_sample_params& p,
                  unsigned long long* states, uint32_t* out_tok, unsigned long long* out_key, void* scratch,
                  const lbt_sample_params* rowp) {
    if (rows <= 0) return LBT_OK;
    if (vocab <= 0 || ld < vocab || !logits || !states || !scratch)
        return set_err(ctx, LBT_E_INVALID, "sample: bad arguments");
    SampleArgs a;
    a.logits = logits;
    a.ld = ld;
    a.V = vocab;
    a.temperature = p.temperature;
    a.top_p = p.top_p;
    a.top_k = (unsigned long long)p.top_k;
    a.rowp = rowp;
    a.states = states;
    a.out_tok = out_tok;
    a.out_key = out_key;
    a.scratch = (Cand*)scratch;
    a.G = chunks_of(vocab);
    a.sums = (ChunkSum*)((char*)scratch + cand_bytes(rows, vocab));
    a.ncand = (unsigned*)((char*)scratch + cand_bytes(rows, vocab) + sums_bytes(rows, vocab));
    // the candidate pass over chunks of the row, then one workgroup per row
    hipLaunchKernelGGL(sample_max_kernel, dim3(a.G, rows), dim3(kCT), 0, ctx->stream, a);
    hipLaunchKernelGGL(sample_cand_kernel, dim3(a.G, rows), dim3(kCT), 0, ctx->stream, a);
    hipLaunchKernelGGL(sample_kernel, dim3(rows), dim3(kST), 0, ctx->stream, a);
    LBT_HIP(ctx, hipGetLastError());
    return LBT_OK;
}

}  // namespace lbt
