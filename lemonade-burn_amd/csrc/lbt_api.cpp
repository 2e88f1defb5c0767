// lbt_api.cpp -- the C ABI (include/lbt.h): context, errors, profiling,
// weights and the per-op entry points.  Host-pointer entry points stage
// through a grow-only device workspace; `_dev` ones enqueue on the stream.
#include <hip/hip_runtime.h>
#include <string.h>

#include <string>
#include <vector>

#include "lbt_internal.h"

namespace lbt {

LbtTuning read_tuning() {
    LbtTuning t;
    auto num = [](const char* k, long d) {
        const char* v = getenv(k);
        return v && *v ? atol(v) : d;
    };
    t.no_graph = getenv("LBT_NO_GRAPH") != nullptr;
    t.no_mfma = getenv("LBT_NO_MFMA") != nullptr;
    t.mfma_min = (int)num("LBT_MFMA_MIN", kMfmaMinTokens);
    if (t.mfma_min < 2) t.mfma_min = 2;
    t.gemm_mode = (int)num("LBT_GEMM_MODE", 0);
    if (t.gemm_mode < 4 || t.gemm_mode > 8) t.gemm_mode = 0;
    t.small_max = (int)num("LBT_GEMM_SMALL_MAX", kSmallMaxTokens);
    t.small_tiles = num("LBT_GEMM_SMALL_TILES", 100);
    t.small_ms = (int)num("LBT_GEMM_SMALL_MS", 1);
    if (t.small_ms < 1) t.small_ms = 1;
    t.small_ns = (int)num("LBT_GEMM_SMALL_NS", 0);
    t.small_pf = num("LBT_GEMM_SMALL_PF", 1) != 0;
    {
        const char* v = getenv("LBT_ATTN_WAVE");
        t.attn_wave = v ? (atoi(v) != 0 ? 1 : 0) : -1;
    }
    {
        const char* v = getenv("LBT_ATTN_WIDE");
        t.attn_wide = v ? (atoi(v) != 0 ? 1 : 0) : -1;
    }
    t.head_tg8 = getenv("LBT_HEAD_TG8") != nullptr;
    t.head_batch_classic = getenv("LBT_HEAD_BATCH_CLASSIC") != nullptr;
    t.gemv_pw = num("LBT_GEMV_PW", 4) == 16 ? 16 : 4;
    t.gemv_pwo = num("LBT_GEMV_PWO", 16) == 4 ? 4 : 16;
    t.gemm_ksplit = (int)num("LBT_GEMM_KSPLIT", 0);
    t.quant_wide = getenv("LBT_QUANT_WIDE") != nullptr;
    if (t.gemm_ksplit < 0 || t.gemm_ksplit > 16) t.gemm_ksplit = 0;
    return t;
}


int set_err(lbt_ctx* ctx, int code, const std::string& msg) {
    if (ctx) ctx->err = msg;
    return code;
}

int hip_err(lbt_ctx* ctx, hipError_t e, const char* what) {
    std::string m = std::string(what) + ": " + hipGetErrorString(e);
    return set_err(ctx, e == hipErrorOutOfMemory ? LBT_E_NOMEM : LBT_E_DEVICE, m);
}

int ws_reserve(lbt_ctx* ctx, size_t bytes, void** out) {
    if (bytes > ctx->ws_bytes) {
        if (ctx->ws) {
            hipStreamSynchronize(ctx->stream);
            hipFree(ctx->ws);
            ctx->ws = nullptr;
            ctx->ws_bytes = 0;
        }
        size_t nb = bytes < (1u << 20) ? (1u << 20) : bytes;
        LBT_HIP(ctx, hipMalloc(&ctx->ws, nb));
        ctx->ws_bytes = nb;
    }
    *out = ctx->ws;
    return LBT_OK;
}

static hipEvent_t take_event(lbt_ctx* ctx) {
    hipEvent_t e = nullptr;
    if (!ctx->free_events.empty()) {
        e = ctx->free_events.back();
        ctx->free_events.pop_back();
    } else if (hipEventCreate(&e) != hipSuccess) {
        e = nullptr;
    }
    return e;
}

void prof_pair(lbt_ctx* ctx, hipEvent_t* a, hipEvent_t* b) {
    *a = *b = nullptr;
    if (!ctx->prof) return;
    *a = take_event(ctx);
    *b = take_event(ctx);
    if (!*a || !*b) {
        if (*a) ctx->free_events.push_back(*a);
        if (*b) ctx->free_events.push_back(*b);
        *a = *b = nullptr;
    }
}

void prof_commit(lbt_ctx* ctx, hipEvent_t a, hipEvent_t b, int cls, double bytes) {
    if (!ctx->prof || !a || !b) return;
    ctx->pending.push_back({cls, bytes, a, b});
}

}  // namespace lbt

using namespace lbt;

namespace {

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// Carves consecutive 256-byte aligned regions out of the workspace.
struct Carve {
    std::vector<size_t> sizes;
    size_t add(size_t b) {
        size_t off = 0;
        for (size_t s : sizes) off += align256(s);
        sizes.push_back(b);
        return off;
    }
    size_t total() const {
        size_t t = 0;
        for (size_t s : sizes) t += align256(s);
        return t;
    }
};

int check_ws(lbt_ctx* ctx, const lbt_weight* const* ws, size_t n, size_t cols_expected, bool check_cols) {
    if (!ws || n < 1 || n > 3) return set_err(ctx, LBT_E_INVALID, "expected 1 to 3 matrices");
    for (size_t i = 0; i < n; i++) {
        if (!ws[i]) return set_err(ctx, LBT_E_INVALID, "null weight");
        if (ws[i]->cols != ws[0]->cols) return set_err(ctx, LBT_E_INVALID, "matrices differ in cols");
    }
    if (check_cols && ws[0]->cols != cols_expected) return set_err(ctx, LBT_E_INVALID, "inner dimension mismatch");
    return LBT_OK;
}

TernaryOp make_op(const lbt_weight* const* ws, size_t n, size_t m) {
    TernaryOp op;
    op.nmat = (int)n;
    for (size_t i = 0; i < n; i++) {
        op.w[i] = ws[i]->d;
        op.rows[i] = (int)ws[i]->rows;
        op.sw[i] = ws[i]->scale;
    }
    op.cols = (int)ws[0]->cols;
    op.m = (int)m;
    return op;
}

}  // namespace

extern "C" {

const char* lbt_version(void) { return "lbt-hip 0.3 gfx950"; }


int lbt_ctx_create(int device, lbt_ctx** out) {
    if (!out) return LBT_E_INVALID;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return LBT_E_DEVICE;
    if (device < 0 || device >= n) return LBT_E_INVALID;
    if (hipSetDevice(device) != hipSuccess) return LBT_E_DEVICE;
    lbt_ctx* c = new lbt_ctx();
    c->device = device;
    c->tune = read_tuning();
    if (noalloc_scratch_init(device, &c->noalloc, &c->noalloc_bytes) != LBT_OK) {
        delete c;
        return LBT_E_DEVICE;
    }
    if (hipDeviceGetAttribute(&c->cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || c->cus <= 0)
        c->cus = 256;
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return LBT_E_DEVICE;
    }
    *out = c;
    return LBT_OK;
}

void lbt_ctx_destroy(lbt_ctx* ctx) {
    if (!ctx) return;
    hipSetDevice(ctx->device);
    hipStreamSynchronize(ctx->stream);
    for (auto& p : ctx->pending) {
        hipEventDestroy(p.a);
        hipEventDestroy(p.b);
    }
    for (auto e : ctx->free_events) hipEventDestroy(e);
    if (ctx->ws) hipFree(ctx->ws);
    if (ctx->qws) hipFree(ctx->qws);
    if (ctx->kws) hipFree(ctx->kws);
    if (ctx->sws) hipFree(ctx->sws);
    hipStreamDestroy(ctx->stream);
    delete ctx;
}

const char* lbt_last_error(const lbt_ctx* ctx) { return ctx ? ctx->err.c_str() : "null context"; }

int lbt_ctx_synchronize(lbt_ctx* ctx) {
    if (!ctx) return LBT_E_INVALID;
    LBT_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return LBT_OK;
}

void* lbt_ctx_stream(lbt_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

int lbt_dev_alloc(lbt_ctx* ctx, size_t bytes, void** out) {
    if (!ctx || !out) return LBT_E_INVALID;
    LBT_HIP(ctx, hipMalloc(out, bytes ? bytes : 1));
    return LBT_OK;
}

int lbt_dev_free(lbt_ctx* ctx, void* p) {
    if (!ctx) return LBT_E_INVALID;
    if (p) {
        LBT_HIP(ctx, hipStreamSynchronize(ctx->stream));
        LBT_HIP(ctx, hipFree(p));
    }
    return LBT_OK;
}

int lbt_memcpy_h2d(lbt_ctx* ctx, void* dst, const void* src, size_t bytes) {
    if (!ctx) return LBT_E_INVALID;
    LBT_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    LBT_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return LBT_OK;
}

int lbt_memcpy_d2h(lbt_ctx* ctx, void* dst, const void* src, size_t bytes) {
    if (!ctx) return LBT_E_INVALID;
    LBT_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    LBT_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return LBT_OK;
}

int lbt_memcpy_d2d(lbt_ctx* ctx, void* dst, const void* src, size_t bytes) {
    if (!ctx || (bytes && (!dst || !src))) return set_err(ctx, LBT_E_INVALID, "memcpy_d2d: bad arguments");
    if (!bytes) return LBT_OK;
    return lbt::launch_copy(ctx, dst, src, bytes);
}

// ---- weights ---------------------------------------------------------------
static int weight_new(lbt_ctx* ctx, const uint8_t* src, bool src_dev, size_t rows, size_t cols, float scale,
                      lbt_weight** out) {
    if (!ctx || !out || !src || rows == 0 || cols == 0) return set_err(ctx, LBT_E_INVALID, "weight: bad arguments");
    if (rows > kMaxDim || cols > kMaxDim) return set_err(ctx, LBT_E_INVALID, "weight: dimension above 2^30");
    *out = nullptr;
    lbt_weight* w = new lbt_weight();
    w->ctx = ctx;
    w->rows = rows;
    w->cols = cols;
    w->kp = padded_cols(cols);
    w->scale = scale;
    const size_t bytes = rows * w->kp / 4;
    hipError_t e = hipMalloc(&w->d, bytes);
    if (e != hipSuccess) {
        delete w;
        return hip_err(ctx, e, "hipMalloc(weight)");
    }
    e = hipMemcpyAsync(w->d, src, bytes, src_dev ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        hipFree(w->d);
        delete w;
        return hip_err(ctx, e, "upload weight");
    }
    *out = w;
    return LBT_OK;
}

int lbt_weight_upload(lbt_ctx* ctx, const uint8_t* packed, size_t rows, size_t cols, float scale, lbt_weight** out) {
    return weight_new(ctx, packed, false, rows, cols, scale, out);
}

int lbt_weight_upload_dev(lbt_ctx* ctx, const uint8_t* packed_dev, size_t rows, size_t cols, float scale,
                          lbt_weight** out) {
    return weight_new(ctx, packed_dev, true, rows, cols, scale, out);
}

void lbt_weight_free(lbt_weight* w) {
    if (!w) return;
    if (w->owns && w->d) {
        hipStreamSynchronize(w->ctx->stream);
        hipFree(w->d);
    }
    delete w;
}

size_t lbt_weight_rows(const lbt_weight* w) { return w ? w->rows : 0; }
size_t lbt_weight_cols(const lbt_weight* w) { return w ? w->cols : 0; }
const uint8_t* lbt_weight_device_ptr(const lbt_weight* w) { return w ? w->d : nullptr; }

// ---- quantization ------------------------------------------------------------
int lbt_quantize_acts_dev(lbt_ctx* ctx, const float* x, size_t m, size_t k, int8_t* q, float* scale, int32_t* sum) {
    if (!ctx || k == 0) return set_err(ctx, LBT_E_INVALID, "quantize: bad arguments");
    if (m > kMaxDim || k > kMaxDim) return set_err(ctx, LBT_E_INVALID, "quantize: dimension above 2^30");
    return launch_quantize(ctx, x, nullptr, 0.0f, (int)m, (int)k, q, scale, sum);
}

int lbt_rmsnorm_quantize_dev(lbt_ctx* ctx, const float* x, const float* norm_w, float eps, size_t m, size_t k,
                             int8_t* q, float* scale, int32_t* sum) {
    if (!ctx || k == 0 || !norm_w) return set_err(ctx, LBT_E_INVALID, "rmsnorm_quantize: bad arguments");
    if (m > kMaxDim || k > kMaxDim) return set_err(ctx, LBT_E_INVALID, "rmsnorm_quantize: dimension above 2^30");
    return launch_quantize(ctx, x, norm_w, eps, (int)m, (int)k, q, scale, sum);
}

int lbt_quantize_acts(lbt_ctx* ctx, const float* x, size_t m, size_t k, int8_t* q, float* scale, int32_t* sum) {
    if (!ctx || k == 0) return set_err(ctx, LBT_E_INVALID, "quantize: bad arguments");
    if (m > kMaxDim || k > kMaxDim) return set_err(ctx, LBT_E_INVALID, "quantize: dimension above 2^30");
    if (m == 0) return LBT_OK;
    if (m > kMaxDim) return set_err(ctx, LBT_E_INVALID, "row count above 2^30");
    const size_t kp = padded_cols(k);
    Carve cv;
    size_t ox = cv.add(m * k * 4), oq = cv.add(m * kp), os = cv.add(m * 4), ou = cv.add(m * 4);
    void* ws;
    int rc = ws_reserve(ctx, cv.total(), &ws);
    if (rc) return rc;
    char* b = (char*)ws;
    LBT_HIP(ctx, hipMemcpyAsync(b + ox, x, m * k * 4, hipMemcpyHostToDevice, ctx->stream));
    rc = launch_quantize(ctx, (const float*)(b + ox), nullptr, 0.0f, (int)m, (int)k, (int8_t*)(b + oq),
                         (float*)(b + os), (int32_t*)(b + ou));
    if (rc) return rc;
    LBT_HIP(ctx, hipMemcpyAsync(q, b + oq, m * kp, hipMemcpyDeviceToHost, ctx->stream));
    LBT_HIP(ctx, hipMemcpyAsync(scale, b + os, m * 4, hipMemcpyDeviceToHost, ctx->stream));
    LBT_HIP(ctx, hipMemcpyAsync(sum, b + ou, m * 4, hipMemcpyDeviceToHost, ctx->stream));
    LBT_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return LBT_OK;
}

// ---- ternary GEMM ------------------------------------------------------------
int lbt_gemm_i32_dev(lbt_ctx* ctx, const lbt_weight* w, const int8_t* q, const int32_t* sum, size_t m, int32_t* out) {
    if (!ctx || !w) return set_err(ctx, LBT_E_INVALID, "gemm_i32: bad arguments");
    if (m == 0) return LBT_OK;
    if (m > kMaxDim) return set_err(ctx, LBT_E_INVALID, "row count above 2^30");
    TernaryOp op = make_op(&w, 1, m);
    op.in_mode = kInPreQ;
    op.out_mode = kOutI32;
    op.q = q;
    op.qsum = sum;
    op.out[0] = out;
    return launch_ternary(ctx, op);
}

int lbt_gemm_i32(lbt_ctx* ctx, const lbt_weight* w, const int8_t* q, const int32_t* sum, size_t m, int32_t* out) {
    if (!ctx || !w) return set_err(ctx, LBT_E_INVALID, "gemm_i32: bad arguments");
    if (m == 0) return LBT_OK;
    if (m > kMaxDim) return set_err(ctx, LBT_E_INVALID, "row count above 2^30");
    Carve cv;
    size_t oq = cv.add(m * w->kp), os = cv.add(m * 4), oo = cv.add(m * w->rows * 4);
    void* ws;
    int rc = ws_reserve(ctx, cv.total(), &ws);
    if (rc) return rc;
    char* b = (char*)ws;
    LBT_HIP(ctx, hipMemcpyAsync(b + oq, q, m * w->kp, hipMemcpyHostToDevice, ctx->stream));
    LBT_HIP(ctx, hipMemcpyAsync(b + os, sum, m * 4, hipMemcpyHostToDevice, ctx->stream));
    rc = lbt_gemm_i32_dev(ctx, w, (const int8_t*)(b + oq), (const int32_t*)(b + os), m, (int32_t*)(b + oo));
    if (rc) return rc;
    LBT_HIP(ctx, hipMemcpyAsync(out, b + oo, m * w->rows * 4, hipMemcpyDeviceToHost, ctx->stream));
    LBT_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return LBT_OK;
}

int lbt_gemm_multi_dev(lbt_ctx* ctx, const lbt_weight* const* ws, size_t n, const int8_t* q, const float* scale,
                       const int32_t* sum, size_t m, float* const* outs) {
    int rc = check_ws(ctx, ws, n, 0, false);
    if (rc) return rc;
    if (m == 0) return LBT_OK;
    if (m > kMaxDim) return set_err(ctx, LBT_E_INVALID, "row count above 2^30");
    TernaryOp op = make_op(ws, n, m);
    op.in_mode = kInPreQ;
    op.out_mode = kOutF32;
    op.q = q;
    op.qscale = scale;
    op.qsum = sum;
    for (size_t i = 0; i < n; i++) op.out[i] = outs[i];
    return launch_ternary(ctx, op);
}

int lbt_gemm_multi(lbt_ctx* ctx, const lbt_weight* const* ws, size_t n, const int8_t* q, const float* scale,
                   const int32_t* sum, size_t m, float* const* outs) {
    int rc = check_ws(ctx, ws, n, 0, false);
    if (rc) return rc;
    if (m == 0) return LBT_OK;
    if (m > kMaxDim) return set_err(ctx, LBT_E_INVALID, "row count above 2^30");
    const size_t kp = ws[0]->kp;
    Carve cv;
    size_t oq = cv.add(m * kp), osc = cv.add(m * 4), osu = cv.add(m * 4);
    size_t oo[3];
    for (size_t i = 0; i < n; i++) oo[i] = cv.add(m * ws[i]->rows * 4);
    void* wsp;
    rc = ws_reserve(ctx, cv.total(), &wsp);
    if (rc) return rc;
    char* b = (char*)wsp;
    LBT_HIP(ctx, hipMemcpyAsync(b + oq, q, m * kp, hipMemcpyHostToDevice, ctx->stream));
    LBT_HIP(ctx, hipMemcpyAsync(b + osc, scale, m * 4, hipMemcpyHostToDevice, ctx->stream));
    LBT_HIP(ctx, hipMemcpyAsync(b + osu, sum, m * 4, hipMemcpyHostToDevice, ctx->stream));
    float* douts[3];
    for (size_t i = 0; i < n; i++) douts[i] = (float*)(b + oo[i]);
    rc = lbt_gemm_multi_dev(ctx, ws, n, (const int8_t*)(b + oq), (const float*)(b + osc), (const int32_t*)(b + osu),
                            m, douts);
    if (rc) return rc;
    for (size_t i = 0; i < n; i++)
        LBT_HIP(ctx, hipMemcpyAsync(outs[i], douts[i], m * ws[i]->rows * 4, hipMemcpyDeviceToHost, ctx->stream));
    LBT_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return LBT_OK;
}

int lbt_ternary_linear_dev(lbt_ctx* ctx, const lbt_weight* const* ws, size_t n, const float* x, size_t m, size_t cols,
                           float* const* outs) {
    int rc = check_ws(ctx, ws, n, cols, true);
    if (rc) return rc;
    if (m == 0) return LBT_OK;
    if (m > kMaxDim) return set_err(ctx, LBT_E_INVALID, "row count above 2^30");
    TernaryOp op = make_op(ws, n, m);
    op.in_mode = kInF32;
    op.out_mode = kOutF32;
    op.x = x;
    for (size_t i = 0; i < n; i++) op.out[i] = outs[i];
    return launch_ternary(ctx, op);
}

int lbt_sample_dev(lbt_ctx* ctx, const float* logits, size_t rows, size_t vocab, const lbt_sample_params* p,
                   uint64_t* states, uint32_t* out) {
    if (!ctx) return LBT_E_INVALID;
    if (!p || !logits || !states || !out || vocab == 0 || vocab > 0x7fffffff || rows > 0x7fffffff)
        return set_err(ctx, LBT_E_INVALID, "lbt_sample: bad arguments");
    if (rows == 0) return LBT_OK;
    size_t need;
    sample_scratch_bytes((int)rows, (int)vocab, &need);
    if (need > ctx->sws_bytes) {
        if (ctx->sws) {
            hipStreamSynchronize(ctx->stream);
            hipFree(ctx->sws);
            ctx->sws = nullptr;
            ctx->sws_bytes = 0;
        }
        LBT_HIP(ctx, hipMalloc(&ctx->sws, need));
        ctx->sws_bytes = need;
    }
    return launch_sample(ctx, logits, (long)vocab, (int)rows, (int)vocab, *p, (unsigned long long*)states, out,
                         nullptr, ctx->sws);
}

int lbt_sample(lbt_ctx* ctx, const float* logits, size_t rows, size_t vocab, const lbt_sample_params* p,
               uint64_t* states, uint32_t* out) {
    if (!ctx) return LBT_E_INVALID;
    if (!p || !logits || !states || !out || vocab == 0) return set_err(ctx, LBT_E_INVALID, "lbt_sample: bad arguments");
    if (rows == 0) return LBT_OK;
    Carve cv;
    const size_t ol = cv.add(rows * vocab * 4), os = cv.add(rows * 8), oo = cv.add(rows * 4);
    void* wsp;
    int rc = ws_reserve(ctx, cv.total(), &wsp);
    if (rc) return rc;
    char* b = (char*)wsp;
    LBT_HIP(ctx, hipMemcpyAsync(b + ol, logits, rows * vocab * 4, hipMemcpyHostToDevice, ctx->stream));
    LBT_HIP(ctx, hipMemcpyAsync(b + os, states, rows * 8, hipMemcpyHostToDevice, ctx->stream));
    rc = lbt_sample_dev(ctx, (const float*)(b + ol), rows, vocab, p, (uint64_t*)(b + os), (uint32_t*)(b + oo));
    if (rc) return rc;
    LBT_HIP(ctx, hipMemcpyAsync(states, b + os, rows * 8, hipMemcpyDeviceToHost, ctx->stream));
    LBT_HIP(ctx, hipMemcpyAsync(out, b + oo, rows * 4, hipMemcpyDeviceToHost, ctx->stream));
    LBT_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return LBT_OK;
}

int lbt_ternary_linear_dev_noalloc(lbt_ctx* ctx, const lbt_weight* const* ws, size_t n, const float* x, size_t m,
                                   size_t cols, float* const* outs) {
    if (!ctx) return LBT_E_INVALID;
    int rc = check_ws(ctx, ws, n, cols, true);
    if (rc) return rc;
    if (m == 0) return LBT_OK;
    if (m > kMaxDim) return set_err(ctx, LBT_E_INVALID, "row count above 2^30");
    const size_t kp = ws[0]->kp;
    const size_t need = ((m * kp + 255) & ~(size_t)255) + m * 8;
    if (need > ctx->noalloc_bytes) {
        const size_t max_m = (ctx->noalloc_bytes - 255) / (kp + 8);
        return set_err(ctx, LBT_E_INVALID,
                       "lbt_ternary_linear_dev_noalloc: " + std::to_string(m) + " rows of " + std::to_string(kp) +
                           " packed columns need " + std::to_string(need) + " bytes of scratch, over the static " +
                           std::to_string(ctx->noalloc_bytes) + " (about " + std::to_string(max_m) +
                           " rows of this width fit)");
    }
    if (ctx->prof)
        return set_err(ctx, LBT_E_INVALID, "lbt_ternary_linear_dev_noalloc: profiling is on (it creates events)");
    TernaryOp op = make_op(ws, n, m);
    op.in_mode = kInF32;
    op.out_mode = kOutF32;
    op.x = x;
    op.scratch = ctx->noalloc;
    op.scratch_bytes = ctx->noalloc_bytes;
    for (size_t i = 0; i < n; i++) op.out[i] = outs[i];
    // the device's scratch is shared by every context: calls are ordered
    const int rc2 = noalloc_ordered(ctx->device, ctx->stream, [&] { return launch_ternary(ctx, op); });
    if (rc2 == LBT_E_DEVICE && ctx->err.empty()) return set_err(ctx, rc2, "lbt_ternary_linear_dev_noalloc: ordering");
    return rc2;
}

int lbt_ternary_linear(lbt_ctx* ctx, const lbt_weight* const* ws, size_t n, const float* x, size_t m, size_t cols,
                       float* const* outs) {
    int rc = check_ws(ctx, ws, n, cols, true);
    if (rc) return rc;
    if (m == 0) return LBT_OK;
    if (m > kMaxDim) return set_err(ctx, LBT_E_INVALID, "row count above 2^30");
    Carve cv;
    size_t ox = cv.add(m * cols * 4);
    size_t oo[3];
    for (size_t i = 0; i < n; i++) oo[i] = cv.add(m * ws[i]->rows * 4);
    void* wsp;
    rc = ws_reserve(ctx, cv.total(), &wsp);
    if (rc) return rc;
    char* b = (char*)wsp;
    LBT_HIP(ctx, hipMemcpyAsync(b + ox, x, m * cols * 4, hipMemcpyHostToDevice, ctx->stream));
    float* douts[3];
    for (size_t i = 0; i < n; i++) douts[i] = (float*)(b + oo[i]);
    rc = lbt_ternary_linear_dev(ctx, ws, n, (const float*)(b + ox), m, cols, douts);
    if (rc) return rc;
    for (size_t i = 0; i < n; i++)
        LBT_HIP(ctx, hipMemcpyAsync(outs[i], douts[i], m * ws[i]->rows * 4, hipMemcpyDeviceToHost, ctx->stream));
    LBT_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return LBT_OK;
}

// ---- bf16 ----------------------------------------------------------------------
int lbt_bf16_upload(lbt_ctx* ctx, const uint16_t* w, size_t rows, size_t cols, lbt_bf16** out) {
    if (!ctx || !w || !out || rows == 0 || cols == 0 || cols % 8)
        return set_err(ctx, LBT_E_INVALID, "bf16_upload: bad arguments (cols must be a multiple of 8)");
    if (rows > kMaxDim || cols > kMaxDim) return set_err(ctx, LBT_E_INVALID, "bf16_upload: dimension above 2^30");
    *out = nullptr;
    lbt_bf16* b = new lbt_bf16();
    b->ctx = ctx;
    b->rows = rows;
    b->cols = cols;
    hipError_t e = hipMalloc(&b->d, rows * cols * 2);
    if (e == hipSuccess) e = hipMemcpy(b->d, w, rows * cols * 2, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        if (b->d) hipFree(b->d);
        delete b;
        return hip_err(ctx, e, "bf16 upload");
    }
    *out = b;
    return LBT_OK;
}

void lbt_bf16_free(lbt_bf16* w) {
    if (!w) return;
    if (w->owns && w->d) {
        hipStreamSynchronize(w->ctx->stream);
        hipFree(w->d);
    }
    delete w;
}

int lbt_bf16_linear_dev(lbt_ctx* ctx, const lbt_bf16* w, const float* x, size_t m, float* out) {
    if (!ctx || !w) return set_err(ctx, LBT_E_INVALID, "bf16_linear: bad arguments");
    return launch_bf16_linear(ctx, w->d, (int)w->rows, (int)w->cols, x, (int)m, nullptr, 0.0f, out, nullptr);
}

int lbt_bf16_linear(lbt_ctx* ctx, const lbt_bf16* w, const float* x, size_t m, float* out) {
    if (!ctx || !w) return set_err(ctx, LBT_E_INVALID, "bf16_linear: bad arguments");
    if (m == 0) return LBT_OK;
    if (m > kMaxDim) return set_err(ctx, LBT_E_INVALID, "row count above 2^30");
    Carve cv;
    size_t ox = cv.add(m * w->cols * 4), oo = cv.add(m * w->rows * 4);
    void* wsp;
    int rc = ws_reserve(ctx, cv.total(), &wsp);
    if (rc) return rc;
    char* b = (char*)wsp;
    LBT_HIP(ctx, hipMemcpyAsync(b + ox, x, m * w->cols * 4, hipMemcpyHostToDevice, ctx->stream));
    rc = lbt_bf16_linear_dev(ctx, w, (const float*)(b + ox), m, (float*)(b + oo));
    if (rc) return rc;
    LBT_HIP(ctx, hipMemcpyAsync(out, b + oo, m * w->rows * 4, hipMemcpyDeviceToHost, ctx->stream));
    LBT_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return LBT_OK;
}

// ---- int8 LM head ----------------------------------------------------------------
int lbt_q8head_from_bf16(lbt_ctx* ctx, const lbt_bf16* w, lbt_q8head** out) {
    if (!ctx || !w || !out) return set_err(ctx, LBT_E_INVALID, "q8head_from_bf16: bad arguments");
    *out = nullptr;
    if (w->rows > (size_t)INT32_MAX || w->cols > (size_t)INT32_MAX)
        return set_err(ctx, LBT_E_INVALID, "q8head_from_bf16: matrix too large");
    lbt_q8head* h = new lbt_q8head();
    h->ctx = ctx;
    h->rows = w->rows;
    h->cols = w->cols;
    hipError_t e = hipMalloc(&h->q, w->rows * w->cols);
    if (e == hipSuccess) e = hipMalloc(&h->scale, w->rows * 4);
    if (e != hipSuccess) {
        lbt_q8head_free(h);
        return hip_err(ctx, e, "q8head alloc");
    }
    int rc = launch_q8_quantize(ctx, w->d, (int)w->rows, (int)w->cols, h->q, h->scale);
    if (!rc && (e = hipStreamSynchronize(ctx->stream)) != hipSuccess) rc = hip_err(ctx, e, "q8head quantize");
    if (rc) {
        lbt_q8head_free(h);
        return rc;
    }
    *out = h;
    return LBT_OK;
}

void lbt_q8head_free(lbt_q8head* h) {
    if (!h) return;
    hipStreamSynchronize(h->ctx->stream);
    if (h->q) hipFree(h->q);
    if (h->scale) hipFree(h->scale);
    delete h;
}

int lbt_q8head_read(lbt_ctx* ctx, const lbt_q8head* h, int8_t* q, float* scale) {
    if (!ctx || !h) return set_err(ctx, LBT_E_INVALID, "q8head_read: bad arguments");
    if (q) LBT_HIP(ctx, hipMemcpyAsync(q, h->q, h->rows * h->cols, hipMemcpyDeviceToHost, ctx->stream));
    if (scale) LBT_HIP(ctx, hipMemcpyAsync(scale, h->scale, h->rows * 4, hipMemcpyDeviceToHost, ctx->stream));
    LBT_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return LBT_OK;
}

int lbt_q8head_linear_dev(lbt_ctx* ctx, const lbt_q8head* h, const float* x, size_t m, float* out) {
    if (!ctx || !h) return set_err(ctx, LBT_E_INVALID, "q8head_linear: bad arguments");
    return launch_q8_linear(ctx, h->q, h->scale, (int)h->rows, (int)h->cols, x, (int)m, nullptr, 0.0f, out, nullptr);
}

int lbt_q8head_linear(lbt_ctx* ctx, const lbt_q8head* h, const float* x, size_t m, float* out) {
    if (!ctx || !h) return set_err(ctx, LBT_E_INVALID, "q8head_linear: bad arguments");
    if (m == 0) return LBT_OK;
    if (m > kMaxDim) return set_err(ctx, LBT_E_INVALID, "row count above 2^30");
    Carve cv;
    size_t ox = cv.add(m * h->cols * 4), oo = cv.add(m * h->rows * 4);
    void* wsp;
    int rc = ws_reserve(ctx, cv.total(), &wsp);
    if (rc) return rc;
    char* b = (char*)wsp;
    LBT_HIP(ctx, hipMemcpyAsync(b + ox, x, m * h->cols * 4, hipMemcpyHostToDevice, ctx->stream));
    rc = lbt_q8head_linear_dev(ctx, h, (const float*)(b + ox), m, (float*)(b + oo));
    if (rc) return rc;
    LBT_HIP(ctx, hipMemcpyAsync(out, b + oo, m * h->rows * 4, hipMemcpyDeviceToHost, ctx->stream));
    LBT_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return LBT_OK;
}

// ---- profiling -------------------------------------------------------------------
int lbt_prof_enable(lbt_ctx* ctx, int on) {
    if (!ctx) return LBT_E_INVALID;
    ctx->prof = on != 0;
    return LBT_OK;
}

int lbt_prof_read(lbt_ctx* ctx, lbt_prof* out, int reset) {
    if (!ctx || !out) return LBT_E_INVALID;
    LBT_HIP(ctx, hipStreamSynchronize(ctx->stream));
    for (auto& p : ctx->pending) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) {
            ctx->acc.ms[p.cls] += ms;
            ctx->acc.bytes[p.cls] += p.bytes;
            ctx->acc.launches[p.cls] += 1;
        }
        ctx->free_events.push_back(p.a);
        ctx->free_events.push_back(p.b);
    }
    ctx->pending.clear();
    *out = ctx->acc;
    if (reset) ctx->acc = lbt_prof{};
    return LBT_OK;
}

}  // extern "C"
