// lbt_internal.h -- host-side internals shared by the C ABI, the model loop
// and the kernel launchers.
#pragma once
#include <functional>
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "../../include/lbt.h"

// Path selection read once from the environment when a context is created
// (lbt_ctx_create); measurements and tests choose a path per context.
struct LbtTuning {
    bool no_graph = false;    // LBT_NO_GRAPH: decode steps as separate launches, no captured graph
    bool no_mfma = false;     // LBT_NO_MFMA: several-token products on the VALU GEMV
    int mfma_min = 2;         // LBT_MFMA_MIN: fewest tokens for the MFMA GEMMs
    int gemm_mode = 0;        // LBT_GEMM_MODE: 0 auto, 4 / 5 = 64 / 128 tiles, 6 = few-token kernel, 7 / 8 = 128 x 256 / 64 x 320 tiles
    int small_max = 32;       // LBT_GEMM_SMALL_MAX: the few-token kernel serves up to this many tokens
    long small_tiles = 100;   // LBT_GEMM_SMALL_TILES: ... and up to 64 tokens below this many 64x64 tiles
    int small_ms = 1;         // LBT_GEMM_SMALL_MS: cap of its token tiles (16 * ms)
    int small_ns = 0;         // LBT_GEMM_SMALL_NS: 1 / 2 forces its row tile (0 auto)
    bool small_pf = true;     // LBT_GEMM_SMALL_PF=0: no epilogue prefetch
    int attn_wave = -1;       // LBT_ATTN_WAVE=1/0: one wavefront per (row, KV head, split) on/off (-1: prefill rows)
    int attn_wide = -1;       // LBT_ATTN_WIDE=1/0: eight-pass K/V pipeline of the grouped attention on/off (-1: by grid size)
    bool head_tg8 = false;           // LBT_HEAD_TG8: 8-token groups in the batched LM head
    bool head_batch_classic = false;  // LBT_HEAD_BATCH_CLASSIC: batched bf16 head on lmhead_batch_kernel (16-token groups)
    int gemv_pw = 4;          // LBT_GEMV_PW=16: single-token GEMV prologue (f32 rows) on all 16 wavefronts (default 4)
    int gemv_pwo = 16;        // LBT_GEMV_PWO=4: ... of the o projection (attention-combine rows) on four (default 16)
    bool quant_wide = false;  // LBT_QUANT_WIDE: row quantizer on 1024 threads (quantize_wide_kernel) instead of 4 wavefronts
    int gemm_ksplit = 0;      // LBT_GEMM_KSPLIT: k ranges of the pipelined GEMM's small grids (0 auto, 1 off)
};

struct lbt_ctx {
    int device = 0;
    LbtTuning tune;
    int cus = 256;  // compute units of the device
    hipStream_t stream = nullptr;
    std::string err;
    // grow-only device workspace for the host-pointer entry points
    void* ws = nullptr;
    size_t ws_bytes = 0;
    // profiling
    bool prof = false;
    struct Pending {
        int cls;
        double bytes;
        hipEvent_t a, b;
    };
    std::vector<Pending> pending;
    std::vector<hipEvent_t> free_events;
    lbt_prof acc{};
    // grow-only device scratch of the prefill GEMM (quantized activations)
    void* qws = nullptr;
    size_t qws_bytes = 0;
    // split-k scratch of the prefill GEMM, allocated once: tile counters
    // (zero between launches), then the partial tiles
    void* kws = nullptr;
    // grow-only scratch of lbt_sample_dev
    void* sws = nullptr;
    size_t sws_bytes = 0;
    // this device's static scratch of the allocation-free entry point
    void* noalloc = nullptr;
    size_t noalloc_bytes = 0;
};

struct lbt_weight {
    lbt_ctx* ctx = nullptr;
    uint8_t* d = nullptr;  // device bytes, rows * kp / 4
    size_t rows = 0, cols = 0, kp = 0;
    float scale = 1.0f;
    bool owns = true;
};

struct lbt_bf16 {
    lbt_ctx* ctx = nullptr;
    uint16_t* d = nullptr;
    size_t rows = 0, cols = 0;
    bool owns = true;
};

struct lbt_q8head {
    lbt_ctx* ctx = nullptr;
    int8_t* q = nullptr;
    float* scale = nullptr;
    size_t rows = 0, cols = 0;
};

namespace lbt {
// The switches of LbtTuning from the environment.
LbtTuning read_tuning();

// Error helpers: every entry point converts failures into a status code.
int set_err(lbt_ctx* ctx, int code, const std::string& msg);
int hip_err(lbt_ctx* ctx, hipError_t e, const char* what);
#define LBT_HIP(ctx, call)                                        \
    do {                                                          \
        hipError_t e_ = (call);                                   \
        if (e_ != hipSuccess) return ::lbt::hip_err(ctx, e_, #call); \
    } while (0)

// Grow-only device workspace.
int ws_reserve(lbt_ctx* ctx, size_t bytes, void** out);

// Profiling brackets around one launch (no-ops unless ctx->prof).
enum ProfClass { kProfGemv = 0, kProfGemm = 1, kProfHead = 2, kProfAttn = 3, kProfOther = 4 };
// prof_pair hands out a start/stop event pair (null when profiling is off)
// for hipExtLaunchKernelGGL, which timestamps the dispatch itself, so the
// measured time is the kernel's execution (as rocprofv3 reports it).
void prof_pair(lbt_ctx* ctx, hipEvent_t* a, hipEvent_t* b);
void prof_commit(lbt_ctx* ctx, hipEvent_t a, hipEvent_t b, int cls, double bytes);

// ---- ternary GEMV / GEMM ------------------------------------------------
// kInAttn: one token whose input row is the combine of the attention splits
// (o-projection of a decode step, attn_common.h), with the norm of kInF32.
enum InMode { kInPreQ = 0, kInF32 = 1, kInAttn = 2 };
enum OutMode { kOutI32 = 0, kOutF32 = 1, kOutF32Add = 2, kOutRelu2 = 3, kOutQKV = 4 };

struct TernaryOp {
    int nmat = 1;
    const uint8_t* w[3] = {nullptr, nullptr, nullptr};
    int rows[3] = {0, 0, 0};
    float sw[3] = {1.f, 1.f, 1.f};
    int cols = 0;
    int m = 0;
    // kInPreQ
    const int8_t* q = nullptr;
    const float* qscale = nullptr;
    const int32_t* qsum = nullptr;
    // kInF32
    const float* x = nullptr;
    const float* norm_w = nullptr;  // nullable: plain ActQuant
    float eps = 0.f;
    // kInAttn (m == 1): split partials of the row, position from pos0 / pos_dev
    const float* att_o = nullptr;
    const float* att_ml = nullptr;
    int att_nh = 0;
    int in_mode = kInPreQ;
    int out_mode = kOutF32;
    void* out[3] = {nullptr, nullptr, nullptr};
    // kOutQKV: out[0] gets rotated q (f32); rotated k and v go to the bf16
    // cache at positions pos0 + token ([kv_heads][cap][hd] of this layer)
    int hd = 0, pos0 = 0, cap = 0;
    const int* pos_dev = nullptr;  // device position (graph replay) instead of pos0
    // batch of sequences: token t is sequence t at position tok_pos[t], its
    // cache rows seq_stride elements after sequence t-1's (replaces pos0/pos_dev)
    const int* tok_pos = nullptr;
    size_t seq_stride = 0;
    const float* cos_t = nullptr;
    const float* sin_t = nullptr;
    uint16_t* kc = nullptr;
    uint16_t* vc = nullptr;
    // caller-provided device scratch for the quantized activations of the
    // several-row paths (null: the context's grow-only buffer)
    void* scratch = nullptr;
    size_t scratch_bytes = 0;
};
// Dispatches the single-token decode GEMV (m = 1) or the int8-MFMA GEMMs
// (m >= kMfmaMinTokens; the VALU few-token GEMV tgemv_kernel stays behind
// LBT_NO_MFMA / LBT_MFMA_MIN, measured 1.2-2x slower at 2..12 tokens).
constexpr int kMfmaMinTokens = 2;
// the few-token MFMA GEMM (16-row tiles) serves up to this many tokens
constexpr int kSmallMaxTokens = 32;
int launch_ternary(lbt_ctx* ctx, const TernaryOp& op);
int launch_ternary_gemv(lbt_ctx* ctx, const TernaryOp& op);
// Single-token GEMV with one 1024-thread workgroup per compute unit (f32 or
// attention-combine input); returns 1 (nothing launched) for shapes it does
// not take.
int launch_ternary_gemv_cu(lbt_ctx* ctx, const TernaryOp& op);
int launch_ternary_mfma(lbt_ctx* ctx, const TernaryOp& op);

// Standalone (rms)norm + quantize of m rows into global q [m, kp], scale, sum.
// RMSNorm + ActQuant of m rows on one 256-thread workgroup each (rows up to
// 256 * 28 padded columns, 16-byte aligned, k % 4 == 0).
int launch_quantize_pw(lbt_ctx* ctx, const float* x, const float* norm_w, float eps, int m, int k, int kp,
                       int8_t* q, float* scale, int32_t* sum);
int launch_quantize(lbt_ctx* ctx, const float* x, const float* norm_w, float eps, int m, int k, int8_t* q,
                    float* scale, int32_t* sum);

// ---- bf16 linear / LM head ------------------------------------------------
// logits[t*rows + r] = sum_k xn[t,k] * W[r,k] with xn = rmsnorm(x) if norm_w.
// If key != nullptr, the first-max key of row t is atomically maxed into key[t].
int launch_bf16_linear(lbt_ctx* ctx, const uint16_t* w, int rows, int cols, const float* x, int m,
                       const float* norm_w, float eps, float* logits, unsigned long long* key, float* xn = nullptr);
// The same head for 2..64 rows on the bf16 matrix cores (head kind 2 uses it
// for 33..64 rows):
// xn = rmsnorm(x) split into bf16 hi + lo parts in xs (2 * 32 * ceil(m/32)
// * cols bf16), f32 accumulation in the matrix core's order (logits within
// tolerance of launch_bf16_linear's, the same first-max key contract).
int launch_bf16_mfma_head(lbt_ctx* ctx, const uint16_t* w, int rows, int cols, const float* x, int m,
                          const float* norm_w, float eps, float* logits, unsigned long long* key, float* xn,
                          uint16_t* xs, size_t xs_bytes);
// The opt-in int8 head (q8head.rs): logits[t*rows + r] = scale[r] *
// sum_k xn[t,k] * q[r,k]; same norm, key and xn contract as above.
int launch_q8_linear(lbt_ctx* ctx, const int8_t* q, const float* scale, int rows, int cols, const float* x, int m,
                     const float* norm_w, float eps, float* logits, unsigned long long* key, float* xn = nullptr);
// Q8Head::from_bf16 (q8head.rs:18-32) of a device bf16 [rows][cols] matrix.
int launch_q8_quantize(lbt_ctx* ctx, const uint16_t* w, int rows, int cols, int8_t* q, float* scale);

// ---- model pieces --------------------------------------------------------
// state (nullable, device): {position, output slot}; when set, the kernel
// advances the position by one and writes the token to tok_out[slot++].
// Sampler::sample on `rows` rows of logits (sample.hip); the token of row r
// goes to out_tok[r] and/or, as an argmax-key word the next embedding reads,
// to out_key[r]; scratch: sample_scratch_bytes.
int launch_sample(lbt_ctx* ctx, const float* logits, long ld, int rows, int vocab, const lbt_sample_params& p,
                  unsigned long long* states, uint32_t* out_tok, unsigned long long* out_key, void* scratch,
                  const lbt_sample_params* rowp = nullptr);
int sample_scratch_bytes(int rows, int vocab, size_t* bytes);
int launch_embed(lbt_ctx* ctx, const uint16_t* embed, int hidden, int vocab, const uint32_t* tokens,
                 const unsigned long long* key, uint32_t* tok_out, int m, float* x, int* state = nullptr);
// Split-key attention (attn_common.h): keys per split for vis visible keys,
// at most kAttnSplits splits per (row, query head).
constexpr int kAttnSplits = 16;
constexpr int kAttnMinKeys = 64;
// the largest row count, column count or token count the entry points take
// (sizes reach the kernels as int; products of two stay within 64 bits)
constexpr size_t kMaxDim = (size_t)1 << 30;
constexpr int kAttnMaxHeads = 64;  // heads of the split combine
__host__ __device__ __forceinline__ int attn_split_keys(int vis) {
    const int ks = (vis + kAttnSplits - 1) / kAttnSplits;
    return ks < kAttnMinKeys ? kAttnMinKeys : ks;
}

// Positions of the rows of a forward pass: one sequence (row t at pos0 + t,
// or *pos_dev + t in a graph-replayed step) or a batch of sequences (row t is
// sequence t at position tok_pos[t]; its cache rows start seq_stride
// elements after sequence t-1's).  vis_max bounds every row's visible keys.
struct RowPos {
    int pos0 = 0;
    const int* pos_dev = nullptr;
    const int* tok_pos = nullptr;
    size_t seq_stride = 0;
    int vis_max = 0;
};
__host__ __device__ __forceinline__ int row_position(const RowPos& r, int t) {
    return r.tok_pos ? r.tok_pos[t] : (r.pos_dev ? *r.pos_dev : r.pos0) + t;
}
__host__ __device__ __forceinline__ size_t row_cache_offset(const RowPos& r, int t) {
    return r.tok_pos ? (size_t)t * r.seq_stride : 0;
}

// Attention splits of m query rows: partials o [m][kAttnSplits][nh*hd],
// ml [m][kAttnSplits][nh][2].  grouped: one workgroup per KV head and split
// takes all its query heads (K/V read once; long contexts), else one per query
// head and split (more workgroups; short contexts).  Both give the same bits.
int launch_attention(lbt_ctx* ctx, const float* q, int m, int nh, int kvh, int hd, const RowPos& rp,
                     const uint16_t* kc, const uint16_t* vc, int cap, float scaling, float* o, float* ml,
                     bool grouped = false);
// Combine of the splits into out [m][nh*hd].
int launch_attn_combine(lbt_ctx* ctx, const float* o, const float* ml, int m, int nh, int hd, const RowPos& rp,
                        float* out);
// Combine of the splits, RMSNorm (norm_w) and ActQuant per row, into q [m][kp]
// (0 past nh*hd), s_a and sum(q): the attention-combine input of a GEMM in
// one kernel (the values combine + quantize would give).
int launch_attn_quantize(lbt_ctx* ctx, const float* o, const float* ml, int m, int nh, int hd, const RowPos& rp,
                         const float* norm_w, float eps, int kp, int8_t* q, float* scale, int32_t* sum);
// The context a model was created on.
lbt_ctx* model_ctx(const lbt_model* m);
// Grow-only per-context device scratch for quantized activations.
int qws_reserve(lbt_ctx* ctx, size_t bytes, void** out);
// Scratch of `bytes` for op's quantized activations: op.scratch when set
// (an error when it is smaller), else the context's buffer (qws_reserve).
int act_scratch(lbt_ctx* ctx, const TernaryOp& op, size_t bytes, void** out);
// Device address of this device's static no-alloc scratch (noalloc.hip),
// looked up once per device; called by lbt_ctx_create with the device current.
int noalloc_scratch_init(int device, void** out, size_t* bytes);
// Runs `launch` (stream `s`) in this device's order of no-alloc calls
// (noalloc.hip): one at a time on the host, each after the previous call's
// kernels on the device.
int noalloc_ordered(int device, hipStream_t s, const std::function<int()>& launch);
int launch_fill_u64(lbt_ctx* ctx, unsigned long long* p, int n, unsigned long long v);
// Streaming device copy (16-byte granules, byte tail).
int launch_copy(lbt_ctx* ctx, void* dst, const void* src, size_t bytes);
int launch_set_state(lbt_ctx* ctx, int* state, int pos, int slot);

// Synthetic weights (same generator as oracle/lbt_oracle.c or_synth_*).
int launch_synth_packed(lbt_ctx* ctx, uint64_t seed, uint64_t tensor, int rows, int cols, uint8_t* out);
int launch_synth_f32(lbt_ctx* ctx, uint64_t seed, uint64_t tensor, size_t n, float lo, float span,
                     float* out);
int launch_synth_bf16(lbt_ctx* ctx, uint64_t seed, uint64_t tensor, size_t n, uint16_t* out);
// Synthetic KV rows (approximately N(0,1), bf16) at positions [0, len) of
// `rows` (layer, sequence, KV head) rows of `cap` positions each.
int launch_synth_kv(lbt_ctx* ctx, uint64_t seed, size_t rows, int cap, int len, int hd, uint16_t* out);
// p[i] += 1 for i < n.
int launch_advance_pos(lbt_ctx* ctx, int* p, int n);

inline size_t padded_cols(size_t cols) { return (cols + 127) / 128 * 128; }

}  // namespace lbt
