// lbt_model.cpp -- BitNet b1.58 2B4T token loop on the device.
//
// Host-side mirror of crates/lb-model/src/model.rs: BitNet::load (:149-232),
// new_cache (:234), ensure_cap (:238-265), forward (:305-374).  Every op of a
// step runs on the device; the host only enqueues kernels.  Per layer:
//   qkv   : ternary GEMV, prologue RMSNorm(input_norm)+ActQuant (3 matrices)
//   rope  : RoPE on k + bf16 append of K and V
//   attn  : GQA attention over the bf16 cache (q rotated in-kernel)
//   o     : ternary GEMV, prologue RMSNorm(attn_sub_norm)+ActQuant, x += y
//   gu    : ternary GEMV over interleaved gate/up rows, prologue
//           RMSNorm(post_attention_norm)+ActQuant, epilogue relu(g)^2 * u
//   down  : ternary GEMV, prologue RMSNorm(ffn_sub_norm)+ActQuant, x += y
// then the bf16 LM head with fused final RMSNorm and device argmax.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "lbt_internal.h"

using namespace lbt;

// ---------------------------------------------------------------------------
// minimal JSON reader (config.json and the safetensors header)
namespace {

struct JVal {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    double num = 0.0;
    std::string str;
    std::vector<JVal> arr;
    std::vector<std::pair<std::string, JVal>> obj;
    const JVal* get(const std::string& k) const {
        for (auto& kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
};

struct JParser {
    const char* p;
    const char* e;
    bool ok = true;
    void ws() {
        while (p < e && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) p++;
    }
    bool lit(const char* s) {
        size_t n = strlen(s);
        if ((size_t)(e - p) >= n && !memcmp(p, s, n)) {
            p += n;
            return true;
        }
        return false;
    }
    std::string str() {
        std::string out;
        if (p >= e || *p != '"') {
            ok = false;
            return out;
        }
        p++;
        while (p < e && *p != '"') {
            if (*p == '\\' && p + 1 < e) {
                p++;
                char c = *p;
                if (c == 'n') out += '\n';
                else if (c == 't') out += '\t';
                else if (c == 'u') {
                    // keep escapes verbatim (not needed for the keys we read)
                    out += "\\u";
                } else out += c;
                p++;
            } else {
                out += *p++;
            }
        }
        if (p >= e) ok = false;
        else p++;
        return out;
    }
    JVal val(int depth = 0) {
        JVal v;
        if (depth > 64) {
            ok = false;
            return v;
        }
        ws();
        if (p >= e) {
            ok = false;
            return v;
        }
        if (*p == '{') {
            p++;
            v.kind = JVal::Obj;
            ws();
            if (p < e && *p == '}') {
                p++;
                return v;
            }
            while (ok) {
                ws();
                std::string k = str();
                ws();
                if (p >= e || *p != ':') {
                    ok = false;
                    break;
                }
                p++;
                JVal c = val(depth + 1);
                v.obj.emplace_back(k, std::move(c));
                ws();
                if (p < e && *p == ',') {
                    p++;
                    continue;
                }
                if (p < e && *p == '}') {
                    p++;
                    break;
                }
                ok = false;
            }
        } else if (*p == '[') {
            p++;
            v.kind = JVal::Arr;
            ws();
            if (p < e && *p == ']') {
                p++;
                return v;
            }
            while (ok) {
                v.arr.push_back(val(depth + 1));
                ws();
                if (p < e && *p == ',') {
                    p++;
                    continue;
                }
                if (p < e && *p == ']') {
                    p++;
                    break;
                }
                ok = false;
            }
        } else if (*p == '"') {
            v.kind = JVal::Str;
            v.str = str();
        } else if (lit("true")) {
            v.kind = JVal::Bool;
            v.b = true;
        } else if (lit("false")) {
            v.kind = JVal::Bool;
        } else if (lit("null")) {
            v.kind = JVal::Null;
        } else {
            char* end = nullptr;
            std::string tmp(p, (size_t)std::min<ptrdiff_t>(e - p, 64));
            v.num = strtod(tmp.c_str(), &end);
            if (end == tmp.c_str()) {
                ok = false;
                return v;
            }
            v.kind = JVal::Num;
            p += end - tmp.c_str();
        }
        return v;
    }
};

bool parse_json(const char* s, size_t n, JVal& out) {
    JParser jp{s, s + n};
    out = jp.val();
    return jp.ok;
}

struct MappedFile {
    void* base = MAP_FAILED;
    size_t size = 0;
    ~MappedFile() {
        if (base != MAP_FAILED) munmap(base, size);
    }
    bool open(const std::string& path) {
        int fd = ::open(path.c_str(), O_RDONLY);
        if (fd < 0) return false;
        struct stat st;
        if (fstat(fd, &st) != 0 || st.st_size <= 0) {
            ::close(fd);
            return false;
        }
        size = (size_t)st.st_size;
        base = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
        ::close(fd);
        return base != MAP_FAILED;
    }
};

struct StTensor {
    std::string dtype;
    std::vector<size_t> shape;
    const uint8_t* data = nullptr;
    size_t bytes = 0;
};

}  // namespace

// ---------------------------------------------------------------------------
struct lbt_model {
    lbt_ctx* ctx = nullptr;
    lbt_config cfg{};
    int hd = 0;
    uint8_t* wbuf = nullptr;  // all packed linears
    std::vector<lbt_weight> lin;  // layers * 7, views into wbuf
    float* fbuf = nullptr;        // norms (layers * 4) + final norm
    std::vector<const float*> norm;
    const float* final_norm = nullptr;
    uint16_t* embed = nullptr;
    // opt-in int8 head (q8head.rs), quantized from embed when selected
    int head_kind = 0;
    int8_t* q8 = nullptr;
    float* q8s = nullptr;
    uint16_t* hx = nullptr;  // head kind 2: bf16 hi / lo parts of up to 64 normalized rows
    size_t hx_bytes = 0;
    float* cos_t = nullptr;
    float* sin_t = nullptr;
    float scaling = 0.0f;
    // workspace sized for `mcap` tokens
    int mcap = 0;
    float *x = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *att = nullptr, *h = nullptr, *logits = nullptr;
    uint32_t* toks = nullptr;
    uint32_t* tok_out = nullptr;
    int tok_out_cap = 0;
    unsigned long long* key = nullptr;
    float* ao = nullptr;   // attention split outputs [mcap][splits][hidden]
    float* aml = nullptr;  // attention split (max, sum) [mcap][splits][heads][2]
    int last_n = 0;
    // graph of one decode step (embed from the argmax key .. LM head), valid
    // for the cache buffers and workspace it was captured with
    int* state = nullptr;  // device {position - 1, output slot, barrier epoch, spare}
    // Captured steps are kept per key (buffers, head kind, sampling
    // parameters) for as long as the buffers they name live: a head switch or
    // a sampling step captures its own graph beside the others instead of
    // destroying and re-capturing one.
    static constexpr int kStepKey = 11;
    static constexpr int kStepGraphs = 8;
    struct StepGraph {
        const void* key[kStepKey];
        hipGraphExec_t exec;
    };
    std::vector<StepGraph> steps;
    // device sampler (sample.hip) of the sampling decode loop: the sampler
    // state and the candidate scratch of one row
    unsigned long long* sstate = nullptr;
    void* sscratch = nullptr;
};

namespace lbt {
lbt_ctx* model_ctx(const lbt_model* m) { return m ? m->ctx : nullptr; }
}  // namespace lbt

namespace {
// Final RMSNorm + the model's LM head (model.rs:368-373): the tied bf16 head,
// or the int8 head when selected.
int model_head(lbt_model* m, const float* x, int rows, float eps, float* logits, unsigned long long* key,
               float* xn) {
    const lbt_config& c = m->cfg;
    if (m->head_kind == 1)
        return launch_q8_linear(m->ctx, m->q8, m->q8s, c.vocab_size, c.hidden_size, x, rows, m->final_norm, eps,
                                logits, key, xn);
    // kind 2 from 33 rows (two token tiles per workgroup): below that the
    // f32 head is faster (B = 16: 267 us against 380)
    if (m->head_kind == 2 && rows > 32 && rows <= 64 && xn)
        return launch_bf16_mfma_head(m->ctx, m->embed, c.vocab_size, c.hidden_size, x, rows, m->final_norm, eps,
                                     logits, key, xn, m->hx, m->hx_bytes);
    return launch_bf16_linear(m->ctx, m->embed, c.vocab_size, c.hidden_size, x, rows, m->final_norm, eps, logits,
                              key, xn);
}
}  // namespace

struct lbt_cache {
    lbt_model* m = nullptr;
    uint16_t* k = nullptr;  // [layers][kvh][cap][hd]
    uint16_t* v = nullptr;
    int len = 0;
    int cap = 0;
};

// nseq sequences with fixed-capacity caches [layers][nseq][kvh][cap][hd].
struct lbt_batch {
    lbt_model* m = nullptr;
    int nseq = 0;
    int cap = 0;
    uint16_t* k = nullptr;
    uint16_t* v = nullptr;
    std::vector<int> len;
    int* pos = nullptr;        // device positions of the current step [nseq]
    uint32_t* tok_out = nullptr;
    size_t tok_out_cap = 0;
    // device sampler of the batch: per-sequence parameters and states, and
    // the candidate scratch of nseq rows (allocated on first use)
    lbt_sample_params* sp = nullptr;
    unsigned long long* sst = nullptr;
    void* sscratch = nullptr;
    size_t seq_stride() const;
    size_t layer_stride() const { return (size_t)nseq * seq_stride(); }
};

namespace {

void lin_shape(const lbt_config& c, int which, int& rows, int& cols) {
    const int hd = c.hidden_size / c.num_attention_heads;
    const int kv = c.num_key_value_heads * hd;
    rows = (which == 1 || which == 2) ? kv : ((which == 4 || which == 5) ? c.intermediate_size : c.hidden_size);
    cols = which == 6 ? c.intermediate_size : c.hidden_size;
}

int validate_config(lbt_ctx* ctx, const lbt_config& c) {
    if (c.hidden_size <= 0 || c.intermediate_size <= 0 || c.num_attention_heads <= 0 || c.num_key_value_heads <= 0 ||
        c.num_hidden_layers <= 0 || c.vocab_size <= 0 || c.max_position_embeddings <= 0)
        return set_err(ctx, LBT_E_INVALID, "config: non-positive dimension");
    for (int32_t d : {c.hidden_size, c.intermediate_size, c.num_attention_heads, c.num_key_value_heads,
                      c.num_hidden_layers, c.vocab_size, c.max_position_embeddings})
        if ((size_t)d > kMaxDim) return set_err(ctx, LBT_E_INVALID, "config: dimension above 2^30");
    if (c.hidden_size % c.num_attention_heads || c.num_attention_heads % c.num_key_value_heads)
        return set_err(ctx, LBT_E_INVALID, "config: heads do not divide");
    const int hd = c.hidden_size / c.num_attention_heads;
    if (hd % 8 || hd > 256) return set_err(ctx, LBT_E_INVALID, "config: head_dim must be a multiple of 8, <= 256");
    if (c.hidden_size % 8) return set_err(ctx, LBT_E_INVALID, "config: hidden_size must be a multiple of 8");
    return LBT_OK;
}

// Device buffers and RoPE tables shared by load and synthetic creation.
int model_alloc(lbt_model* m) {
    lbt_ctx* ctx = m->ctx;
    const lbt_config& c = m->cfg;
    m->hd = c.hidden_size / c.num_attention_heads;
    size_t wbytes = 0;
    std::vector<size_t> off;
    for (int l = 0; l < c.num_hidden_layers; l++)
        for (int w = 0; w < 7; w++) {
            int rows, cols;
            lin_shape(c, w, rows, cols);
            off.push_back(wbytes);
            wbytes += ((size_t)rows * padded_cols((size_t)cols) / 4 + 255) & ~(size_t)255;
        }
    LBT_HIP(ctx, hipMalloc(&m->wbuf, wbytes));
    m->lin.resize(off.size());
    for (int l = 0; l < c.num_hidden_layers; l++)
        for (int w = 0; w < 7; w++) {
            int rows, cols;
            lin_shape(c, w, rows, cols);
            lbt_weight& lw = m->lin[l * 7 + w];
            lw.ctx = ctx;
            lw.d = m->wbuf + off[l * 7 + w];
            lw.rows = (size_t)rows;
            lw.cols = (size_t)cols;
            lw.kp = padded_cols((size_t)cols);
            lw.owns = false;
        }
    size_t nf = 0;
    std::vector<size_t> foff;
    for (int l = 0; l < c.num_hidden_layers; l++)
        for (int k = 0; k < 4; k++) {
            foff.push_back(nf);
            nf += (size_t)(k == 3 ? c.intermediate_size : c.hidden_size);
        }
    foff.push_back(nf);
    nf += (size_t)c.hidden_size;
    LBT_HIP(ctx, hipMalloc(&m->fbuf, nf * sizeof(float)));
    for (size_t i = 0; i + 1 < foff.size(); i++) m->norm.push_back(m->fbuf + foff[i]);
    m->final_norm = m->fbuf + foff.back();
    LBT_HIP(ctx, hipMalloc(&m->embed, (size_t)c.vocab_size * c.hidden_size * 2));

    // RoPE tables as model.rs:213-230 builds them: inv in f64 rounded to f32,
    // angle = pos (f32) * inv (f32), sin/cos in f64 rounded to f32.  Only the
    // first half is stored: dims i and i + hd/2 share an entry.
    const int h2 = m->hd / 2;
    const size_t tn = (size_t)c.max_position_embeddings * h2;
    std::vector<float> ct(tn), st(tn), inv(h2);
    for (int i = 0; i < h2; i++) inv[i] = (float)(1.0 / pow(c.rope_theta, (double)(2 * i) / (double)m->hd));
    for (int p = 0; p < c.max_position_embeddings; p++)
        for (int i = 0; i < h2; i++) {
            const float f = (float)p * inv[i];
            ct[(size_t)p * h2 + i] = (float)cos((double)f);
            st[(size_t)p * h2 + i] = (float)sin((double)f);
        }
    LBT_HIP(ctx, hipMalloc(&m->cos_t, tn * sizeof(float)));
    LBT_HIP(ctx, hipMalloc(&m->sin_t, tn * sizeof(float)));
    LBT_HIP(ctx, hipMemcpy(m->cos_t, ct.data(), tn * sizeof(float), hipMemcpyHostToDevice));
    LBT_HIP(ctx, hipMemcpy(m->sin_t, st.data(), tn * sizeof(float), hipMemcpyHostToDevice));
    m->scaling = powf((float)m->hd, -0.5f);  // (hd as f32).powf(-0.5), model.rs:314
    return LBT_OK;
}

// A captured decode-step graph holds the addresses of the workspace, the
// token slots and one cache: every graph is destroyed (after the stream has
// drained) before any of them is freed, so no live graph ever refers to
// freed memory.  Switching the head or the sampling parameters frees nothing
// and destroys nothing.
void drop_step_graph(lbt_model* m) {
    if (m->steps.empty()) return;
    hipStreamSynchronize(m->ctx->stream);
    for (auto& g : m->steps) hipGraphExecDestroy(g.exec);
    m->steps.clear();
}

int grow_tok_out(lbt_model* m, int need) {
    if (need <= m->tok_out_cap) return LBT_OK;
    drop_step_graph(m);
    hipStreamSynchronize(m->ctx->stream);
    if (m->tok_out) hipFree(m->tok_out);
    m->tok_out = nullptr;
    m->tok_out_cap = 0;
    LBT_HIP(m->ctx, hipMalloc(&m->tok_out, (size_t)need * 4));
    m->tok_out_cap = need;
    return LBT_OK;
}

int ensure_ws(lbt_model* m, int n) {
    if (n <= m->mcap) return LBT_OK;
    lbt_ctx* ctx = m->ctx;
    drop_step_graph(m);
    hipStreamSynchronize(ctx->stream);
    float** bufs[] = {&m->x, &m->q, &m->k, &m->v, &m->att, &m->h, &m->logits};
    for (auto b : bufs)
        if (*b) {
            hipFree(*b);
            *b = nullptr;
        }
    if (m->toks) hipFree(m->toks);
    if (m->key) hipFree(m->key);
    if (m->ao) hipFree(m->ao);
    if (m->aml) hipFree(m->aml);
    const lbt_config& c = m->cfg;
    const size_t H = (size_t)c.hidden_size, I = (size_t)c.intermediate_size;
    const size_t KV = (size_t)c.num_key_value_heads * m->hd;
    LBT_HIP(ctx, hipMalloc(&m->x, n * H * 4));
    LBT_HIP(ctx, hipMalloc(&m->q, n * H * 4));
    LBT_HIP(ctx, hipMalloc(&m->k, n * KV * 4));
    LBT_HIP(ctx, hipMalloc(&m->v, n * KV * 4));
    LBT_HIP(ctx, hipMalloc(&m->att, n * H * 4));
    LBT_HIP(ctx, hipMalloc(&m->h, n * I * 4));
    LBT_HIP(ctx, hipMalloc(&m->logits, (size_t)n * c.vocab_size * 4));
    LBT_HIP(ctx, hipMalloc(&m->toks, n * 4));
    LBT_HIP(ctx, hipMalloc(&m->key, n * 8));
    LBT_HIP(ctx, hipMalloc(&m->ao, n * kAttnSplits * H * 4));
    LBT_HIP(ctx, hipMalloc(&m->aml, n * kAttnSplits * (size_t)c.num_attention_heads * 2 * 4));
    m->mcap = n;
    return LBT_OK;
}

// ensure_cap (model.rs:238-265): next power of two, at least 256, at most
// max_position_embeddings (or the need); old contents are kept.
int ensure_cap(lbt_cache* cc, int need) {
    if (need <= cc->cap) return LBT_OK;
    lbt_model* m = cc->m;
    lbt_ctx* ctx = m->ctx;
    const lbt_config& c = m->cfg;
    if (need > c.max_position_embeddings)
        return set_err(ctx, LBT_E_RANGE, "context length " + std::to_string(c.max_position_embeddings) + " exceeded");
    int cap = 256;
    while (cap < need && cap < (1 << 30)) cap <<= 1;
    if (cap < need) cap = need;
    if (cap > c.max_position_embeddings) cap = c.max_position_embeddings;
    const size_t kvh = (size_t)c.num_key_value_heads, hd = (size_t)m->hd, L = (size_t)c.num_hidden_layers;
    uint16_t *nk = nullptr, *nv = nullptr;
    LBT_HIP(ctx, hipMalloc(&nk, L * kvh * cap * hd * 2));
    LBT_HIP(ctx, hipMalloc(&nv, L * kvh * cap * hd * 2));
    if (cc->k && cc->len > 0) {
        // per (layer, head): copy the first len rows
        LBT_HIP(ctx, hipMemcpy2DAsync(nk, (size_t)cap * hd * 2, cc->k, (size_t)cc->cap * hd * 2, (size_t)cc->len * hd * 2,
                                      L * kvh, hipMemcpyDeviceToDevice, ctx->stream));
        LBT_HIP(ctx, hipMemcpy2DAsync(nv, (size_t)cap * hd * 2, cc->v, (size_t)cc->cap * hd * 2, (size_t)cc->len * hd * 2,
                                      L * kvh, hipMemcpyDeviceToDevice, ctx->stream));
    }
    LBT_HIP(ctx, hipStreamSynchronize(ctx->stream));
    drop_step_graph(m);
    if (cc->k) hipFree(cc->k);
    if (cc->v) hipFree(cc->v);
    cc->k = nk;
    cc->v = nv;
    cc->cap = cap;
    return LBT_OK;
}

// Room in the cache for `a` + `b` more positions (sizes as the caller gave
// them, checked before any narrowing): the context-length error past
// max_position_embeddings, else ensure_cap.
int ensure_room(lbt_cache* cc, size_t a, size_t b = 0) {
    const lbt_config& c = cc->m->cfg;
    const size_t room = (size_t)c.max_position_embeddings - (size_t)cc->len;
    if (a > room || b > room - a)
        return set_err(cc->m->ctx, LBT_E_RANGE,
                       "context length " + std::to_string(c.max_position_embeddings) + " exceeded");
    return ensure_cap(cc, cc->len + (int)(a + b));
}

// KV cache rows of a forward pass: layer l of sequence 0 starts at
// k + l * layer_stride; cap positions per (sequence, KV head).
struct KvView {
    uint16_t* k;
    uint16_t* v;
    size_t layer_stride;
    int cap;
};

// One forward over n rows placed by `rp` (tokens from `toks_dev`, or from the
// previous step's argmax keys when null).  Leaves the argmax key of each
// returned row in m->key and logits (if `all_logits` or `want_logits`);
// without all_logits only the last row goes through the LM head, unless
// every row is its own sequence (rp.tok_pos), when all rows do.  `grouped`
// picks the KV-head-grouped attention (long contexts).
int forward_rows(lbt_model* m, const KvView& kv, const RowPos& rp, const uint32_t* toks_dev, int n, bool all_logits,
                 bool want_logits, uint32_t* tok_out_dev, int* state, bool grouped) {
    lbt_ctx* ctx = m->ctx;
    const lbt_config& c = m->cfg;
    const int H = c.hidden_size, I = c.intermediate_size, nh = c.num_attention_heads, kvh = c.num_key_value_heads;
    const int hd = m->hd;
    const float eps = (float)c.rms_norm_eps;
    // with `state`, positions come from the device (state[0]) so that the step
    // can be captured once and replayed
    int rc = launch_embed(ctx, m->embed, H, c.vocab_size, toks_dev, m->key, tok_out_dev, n, m->x, state);
    if (rc) return rc;
    const size_t layer_kv = kv.layer_stride;
    for (int l = 0; l < c.num_hidden_layers; l++) {
        const lbt_weight* W = &m->lin[l * 7];
        TernaryOp op;
        op.cols = H;
        op.m = n;
        op.in_mode = kInF32;
        op.eps = eps;
        // q/k/v (forward3, model.rs:68-74 / :333)
        op.nmat = 3;
        for (int i = 0; i < 3; i++) {
            op.w[i] = W[i].d;
            op.rows[i] = (int)W[i].rows;
            op.sw[i] = W[i].scale;
        }
        op.x = m->x;
        op.norm_w = m->norm[l * 4 + 0];
        op.out_mode = kOutQKV;
        op.out[0] = m->q;
        uint16_t* Kl = kv.k + (size_t)l * layer_kv;
        uint16_t* Vl = kv.v + (size_t)l * layer_kv;
        op.hd = hd;
        op.pos0 = rp.pos0;
        op.pos_dev = rp.pos_dev;
        op.tok_pos = rp.tok_pos;
        op.seq_stride = rp.seq_stride;
        op.cap = kv.cap;
        op.cos_t = m->cos_t;
        op.sin_t = m->sin_t;
        op.kc = Kl;
        op.vc = Vl;
        if ((rc = launch_ternary(ctx, op))) return rc;
        if ((rc = launch_attention(ctx, m->q, n, nh, kvh, hd, rp, Kl, Vl, kv.cap, m->scaling, m->ao, m->aml,
                                   grouped)))
            return rc;
        // the o projection takes the splits: one token of one sequence combines
        // them in the GEMV prologue, several rows in one combine + quantize kernel
        const bool fused = nh <= kAttnMaxHeads && H <= 4096;
        if (!fused && (rc = launch_attn_combine(ctx, m->ao, m->aml, n, nh, hd, rp, m->att))) return rc;
        // o_proj on attn_sub_norm(attn), residual (model.rs:358-359)
        TernaryOp o;
        o.nmat = 1;
        o.w[0] = W[3].d;
        o.rows[0] = (int)W[3].rows;
        o.sw[0] = W[3].scale;
        o.cols = H;
        o.m = n;
        o.in_mode = fused ? kInAttn : kInF32;
        o.x = m->att;
        o.att_o = m->ao;
        o.att_ml = m->aml;
        o.att_nh = nh;
        o.hd = hd;
        o.pos0 = rp.pos0;
        o.pos_dev = rp.pos_dev;
        o.tok_pos = fused ? rp.tok_pos : nullptr;
        o.norm_w = m->norm[l * 4 + 2];
        o.eps = eps;
        o.out_mode = kOutF32Add;
        o.out[0] = m->x;
        if ((rc = launch_ternary(ctx, o))) return rc;
        // gate/up on post_attention_norm(x), relu(g)^2 * u (model.rs:361-363)
        TernaryOp gu;
        gu.nmat = 2;
        for (int i = 0; i < 2; i++) {
            gu.w[i] = W[4 + i].d;
            gu.rows[i] = (int)W[4 + i].rows;
            gu.sw[i] = W[4 + i].scale;
        }
        gu.cols = H;
        gu.m = n;
        gu.in_mode = kInF32;
        gu.x = m->x;
        gu.norm_w = m->norm[l * 4 + 1];
        gu.eps = eps;
        gu.out_mode = kOutRelu2;
        gu.out[0] = m->h;
        if ((rc = launch_ternary(ctx, gu))) return rc;
        // down on ffn_sub_norm(h), residual (model.rs:364-365)
        TernaryOp dn;
        dn.nmat = 1;
        dn.w[0] = W[6].d;
        dn.rows[0] = (int)W[6].rows;
        dn.sw[0] = W[6].scale;
        dn.cols = I;
        dn.m = n;
        dn.in_mode = kInF32;
        dn.x = m->h;
        dn.norm_w = m->norm[l * 4 + 3];
        dn.eps = eps;
        dn.out_mode = kOutF32Add;
        dn.out[0] = m->x;
        if ((rc = launch_ternary(ctx, dn))) return rc;
    }
    m->last_n = n;
    // final norm + tied LM head (model.rs:368-373) + argmax
    const int first = (all_logits || rp.tok_pos) ? 0 : n - 1;
    const int rows_out = n - first;
    return model_head(m, m->x + (size_t)first * H, rows_out, eps, (all_logits || want_logits) ? m->logits : nullptr,
                      (all_logits && !rp.tok_pos) ? nullptr : m->key, m->att);
}

// One forward of n tokens of one sequence at positions cache.len.. (or, with
// `state`, at the device position of a graph-replayed step).
int forward_dev(lbt_model* m, lbt_cache* cc, const uint32_t* toks_dev, int n, bool all_logits, bool want_logits,
                uint32_t* tok_out_dev, int* state = nullptr) {
    const lbt_config& c = m->cfg;
    KvView kv{cc->k, cc->v, (size_t)c.num_key_value_heads * cc->cap * m->hd, cc->cap};
    RowPos rp;
    rp.pos0 = cc->len;
    rp.pos_dev = state;
    rp.vis_max = state ? cc->cap : cc->len + n;
    // several rows (prefill): the KV-head-grouped attention, every K/V row
    // loaded once for the query heads that share it
    const int rc = forward_rows(m, kv, rp, toks_dev, n, all_logits, want_logits, tok_out_dev, state, n > 1);
    if (!rc) cc->len += n;
    return rc;
}

int ensure_state(lbt_model* m) {
    if (m->state) return LBT_OK;
    lbt_ctx* ctx = m->ctx;
    LBT_HIP(ctx, hipMalloc(&m->state, 4 * sizeof(int)));
    LBT_HIP(ctx, hipMemsetAsync(m->state, 0, 4 * sizeof(int), ctx->stream));
    return LBT_OK;
}

int ensure_sampler(lbt_model* m) {
    if (m->sstate) return LBT_OK;
    lbt_ctx* ctx = m->ctx;
    size_t bytes;
    sample_scratch_bytes(1, m->cfg.vocab_size, &bytes);
    void *scr = nullptr, *st = nullptr;
    hipError_t e = hipMalloc(&scr, bytes);
    if (e == hipSuccess) e = hipMalloc(&st, 8);
    if (e != hipSuccess) {  // all or nothing: a later call allocates afresh
        if (scr) hipFree(scr);
        return hip_err(ctx, e, "sampler scratch");
    }
    m->sscratch = scr;
    m->sstate = (unsigned long long*)st;
    return LBT_OK;
}

// The token after the last LM head: the sampler's pick written as the
// argmax-key word the next embedding reads (sp null: the head's argmax stays).
int sample_key(lbt_model* m, const lbt_sample_params* sp) {
    if (!sp) return LBT_OK;
    return launch_sample(m->ctx, m->logits, m->cfg.vocab_size, 1, m->cfg.vocab_size, *sp, m->sstate, nullptr, m->key,
                         m->sscratch);
}

// Runs n decode steps, each fed with the previous step's argmax (the key);
// the token consumed by step s goes to m->tok_out[slot0 + s].  Outside
// profiling one captured step is replayed as a HIP graph (positions and
// output slots advance on the device); the graph is re-captured when the
// cache or workspace buffers change.
// With `sp`, each step's LM head also writes its logits and the sampler
// (state m->sstate) replaces the argmax in the key.
int decode_steps(lbt_model* m, lbt_cache* c, int n, int slot0, const lbt_sample_params* sp = nullptr) {
    lbt_ctx* ctx = m->ctx;
    if (n <= 0) return LBT_OK;
    int rc;
    if (ctx->prof || ctx->tune.no_graph) {
        for (int s = 0; s < n; s++) {
            if ((rc = forward_dev(m, c, nullptr, 1, false, sp != nullptr, m->tok_out + slot0 + s))) return rc;
            if ((rc = sample_key(m, sp))) return rc;
        }
        return LBT_OK;
    }
    if ((rc = ensure_state(m))) return rc;
    // what the captured step depends on: buffers, head, sampler and its parameters
    uint32_t tb = 0, pb = 0;
    if (sp) {
        memcpy(&tb, &sp->temperature, 4);
        memcpy(&pb, &sp->top_p, 4);
    }
    const void* key[lbt_model::kStepKey] = {c->k,
                                            c->v,
                                            (const void*)(intptr_t)c->cap,
                                            m->tok_out,
                                            m->x,
                                            m->key,
                                            (const void*)(intptr_t)m->head_kind,
                                            (const void*)(intptr_t)(sp ? 1 : 0),
                                            (const void*)(uintptr_t)tb,
                                            (const void*)(uintptr_t)pb,
                                            (const void*)(uintptr_t)(sp ? sp->top_k : 0)};
    hipGraphExec_t exec = nullptr;
    for (auto& sg : m->steps)
        if (memcmp(key, sg.key, sizeof(key)) == 0) exec = sg.exec;
    if (!exec) {
        if ((int)m->steps.size() >= lbt_model::kStepGraphs) drop_step_graph(m);
        hipGraph_t g = nullptr;
        LBT_HIP(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
        const int len = c->len;
        rc = forward_dev(m, c, nullptr, 1, false, sp != nullptr, m->tok_out, m->state);
        if (!rc) rc = sample_key(m, sp);
        c->len = len;
        hipError_t e = hipStreamEndCapture(ctx->stream, &g);
        if (rc) {
            if (g) hipGraphDestroy(g);
            return rc;
        }
        if (e != hipSuccess) return hip_err(ctx, e, "capture decode step");
        e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
        hipGraphDestroy(g);
        if (e != hipSuccess) return hip_err(ctx, e, "instantiate decode step");
        lbt_model::StepGraph sg;
        memcpy(sg.key, key, sizeof(key));
        sg.exec = exec;
        m->steps.push_back(sg);
    }
    if ((rc = launch_set_state(ctx, m->state, c->len - 1, slot0))) return rc;
    for (int s = 0; s < n; s++) LBT_HIP(ctx, hipGraphLaunch(exec, ctx->stream));
    c->len += n;
    m->last_n = 1;
    return LBT_OK;
}

int read_config(lbt_ctx* ctx, const std::string& dir, lbt_config& c) {
    std::string path = dir + "/config.json";
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) return set_err(ctx, LBT_E_IO, "cannot open " + path);
    std::string s;
    char buf[4096];
    size_t n;
    while ((n = fread(buf, 1, sizeof(buf), f)) > 0) s.append(buf, n);
    fclose(f);
    JVal j;
    if (!parse_json(s.data(), s.size(), j) || j.kind != JVal::Obj) return set_err(ctx, LBT_E_IO, "bad json: " + path);
    auto num = [&](const char* k, double& out) -> bool {
        const JVal* v = j.get(k);
        if (!v || v->kind != JVal::Num) return false;
        out = v->num;
        return true;
    };
    double d;
    const char* keys[] = {"hidden_size", "intermediate_size", "num_attention_heads", "num_key_value_heads",
                          "num_hidden_layers", "vocab_size", "max_position_embeddings"};
    int32_t* dst[] = {&c.hidden_size, &c.intermediate_size, &c.num_attention_heads, &c.num_key_value_heads,
                      &c.num_hidden_layers, &c.vocab_size, &c.max_position_embeddings};
    // dimensions: whole numbers that an int32 holds (the range check of
    // each dimension follows in validate_config)
    for (int i = 0; i < 7; i++) {
        if (!num(keys[i], d)) return set_err(ctx, LBT_E_IO, std::string("config.json: missing ") + keys[i]);
        if (!(d >= -2147483648.0 && d <= 2147483647.0) || d != (double)(int64_t)d)
            return set_err(ctx, LBT_E_INVALID, std::string("config.json: ") + keys[i] + " is not a whole number");
        *dst[i] = (int32_t)d;
    }
    if (!num("rms_norm_eps", c.rms_norm_eps)) return set_err(ctx, LBT_E_IO, "config.json: missing rms_norm_eps");
    if (!num("rope_theta", c.rope_theta)) return set_err(ctx, LBT_E_IO, "config.json: missing rope_theta");
    c.bos_token_id = num("bos_token_id", d) && d >= 0.0 && d <= 4294967295.0 ? (uint32_t)d : 0u;
    const JVal* act = j.get("hidden_act");
    const JVal* tied = j.get("tie_word_embeddings");
    // model.rs:151-153
    if (!act || act->kind != JVal::Str || act->str != "relu2" || !tied || tied->kind != JVal::Bool || !tied->b)
        return set_err(ctx, LBT_E_INVALID, "unsupported config: needs hidden_act=relu2 and tie_word_embeddings=true");
    return LBT_OK;
}

}  // namespace

extern "C" {

int lbt_model_create_synthetic(lbt_ctx* ctx, const lbt_config* cfg, uint64_t seed, lbt_model** out) {
    if (!ctx || !cfg || !out) return set_err(ctx, LBT_E_INVALID, "create_synthetic: bad arguments");
    *out = nullptr;
    int rc = validate_config(ctx, *cfg);
    if (rc) return rc;
    std::unique_ptr<lbt_model> m(new lbt_model());
    m->ctx = ctx;
    m->cfg = *cfg;
    if ((rc = model_alloc(m.get()))) {
        lbt_model_free(m.release());
        return rc;
    }
    const lbt_config& c = m->cfg;
    const uint64_t T_EMBED = 1, T_FINAL = 2;
    for (int l = 0; l < c.num_hidden_layers; l++) {
        for (int w = 0; w < 7; w++) {
            lbt_weight& lw = m->lin[l * 7 + w];
            lw.scale = (float)sqrt(0.6 * (double)lw.cols);
            if ((rc = launch_synth_packed(ctx, seed, 16u + (uint64_t)l * 16u + w, (int)lw.rows, (int)lw.cols,
                                          lw.d))) {
                lbt_model_free(m.release());
                return rc;
            }
        }
        for (int k = 0; k < 4; k++) {
            const size_t n = (size_t)(k == 3 ? c.intermediate_size : c.hidden_size);
            if ((rc = launch_synth_f32(ctx, seed, 16u + (uint64_t)l * 16u + 7 + k, n, 0.5f, 1.0f,
                                       (float*)m->norm[l * 4 + k]))) {
                lbt_model_free(m.release());
                return rc;
            }
        }
    }
    if ((rc = launch_synth_f32(ctx, seed, T_FINAL, (size_t)c.hidden_size, 0.5f, 1.0f, (float*)m->final_norm)) ||
        (rc = launch_synth_bf16(ctx, seed, T_EMBED, (size_t)c.vocab_size * c.hidden_size, m->embed))) {
        lbt_model_free(m.release());
        return rc;
    }
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        lbt_model_free(m.release());
        return hip_err(ctx, e, "synthetic model");
    }
    *out = m.release();
    return LBT_OK;
}

int lbt_model_load(lbt_ctx* ctx, const char* dir, lbt_model** out) {
    if (!ctx || !dir || !out) return set_err(ctx, LBT_E_INVALID, "model_load: bad arguments");
    *out = nullptr;
    lbt_config c{};
    int rc = read_config(ctx, dir, c);
    if (rc) return rc;
    if ((rc = validate_config(ctx, c))) return rc;
    MappedFile mf;
    std::string path = std::string(dir) + "/model.lbt.safetensors";
    if (!mf.open(path)) return set_err(ctx, LBT_E_IO, "cannot open " + path);
    const uint8_t* base = (const uint8_t*)mf.base;
    if (mf.size < 8) return set_err(ctx, LBT_E_IO, "truncated safetensors file");
    uint64_t hlen = 0;
    memcpy(&hlen, base, 8);
    if (hlen > mf.size - 8) return set_err(ctx, LBT_E_IO, "bad safetensors header length");
    JVal hdr;
    if (!parse_json((const char*)base + 8, (size_t)hlen, hdr) || hdr.kind != JVal::Obj)
        return set_err(ctx, LBT_E_IO, "bad safetensors header");
    const uint8_t* data0 = base + 8 + hlen;
    const size_t data_size = mf.size - 8 - hlen;
    // format check (model.rs:158-161, lb-convert/src/lib.rs:14)
    const JVal* meta = hdr.get("__metadata__");
    const JVal* fmt = meta ? meta->get("format") : nullptr;
    if (!fmt || fmt->kind != JVal::Str || fmt->str != "lemonade-burn-ternary")
        return set_err(ctx, LBT_E_IO, path + " is not a lemonade-burn ternary file");
    // a JSON number that is a whole byte count or dimension (no sign, no
    // fraction, below 2^53: what a double holds exactly)
    auto as_size = [](const JVal& v, size_t& o) {
        if (v.kind != JVal::Num || !(v.num >= 0.0) || v.num >= 9007199254740992.0 || v.num != (double)(uint64_t)v.num)
            return false;
        o = (size_t)v.num;
        return true;
    };
    std::map<std::string, StTensor> tensors;
    for (auto& kv : hdr.obj) {
        if (kv.first == "__metadata__") continue;
        const JVal& t = kv.second;
        const JVal* dt = t.get("dtype");
        const JVal* sh = t.get("shape");
        const JVal* of = t.get("data_offsets");
        if (!dt || !sh || !of || of->arr.size() != 2) return set_err(ctx, LBT_E_IO, "bad tensor entry " + kv.first);
        StTensor st;
        st.dtype = dt->str;
        for (auto& d : sh->arr) {
            size_t n = 0;
            if (!as_size(d, n)) return set_err(ctx, LBT_E_IO, "bad shape for " + kv.first);
            st.shape.push_back(n);
        }
        size_t b = 0, e = 0;
        if (!as_size(of->arr[0], b) || !as_size(of->arr[1], e) || b > e || e > data_size)
            return set_err(ctx, LBT_E_IO, "bad offsets for " + kv.first);
        st.data = data0 + b;
        st.bytes = e - b;
        tensors[kv.first] = st;
    }
    std::unique_ptr<lbt_model> m(new lbt_model());
    m->ctx = ctx;
    m->cfg = c;
    if ((rc = model_alloc(m.get()))) {
        lbt_model_free(m.release());
        return rc;
    }
    auto fail = [&](int code, const std::string& msg) {
        lbt_model_free(m.release());
        return set_err(ctx, code, msg);
    };
    static const char* lin_names[7] = {"self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                                       "mlp.gate_proj",    "mlp.up_proj",      "mlp.down_proj"};
    static const char* norm_names[4] = {"input_layernorm.weight", "post_attention_layernorm.weight",
                                        "self_attn.attn_sub_norm.weight", "mlp.ffn_sub_norm.weight"};
    for (int l = 0; l < c.num_hidden_layers; l++) {
        const std::string p = "model.layers." + std::to_string(l) + ".";
        for (int w = 0; w < 7; w++) {
            lbt_weight& lw = m->lin[l * 7 + w];
            auto qi = tensors.find(p + lin_names[w] + ".qweight");
            auto si = tensors.find(p + lin_names[w] + ".wscale");
            if (qi == tensors.end() || si == tensors.end())
                return fail(LBT_E_IO, "missing " + p + lin_names[w]);
            const StTensor& qt = qi->second;
            const size_t rb = lw.kp / 4;
            if (qt.dtype != "U8" || qt.shape.size() != 2 || qt.shape[0] != lw.rows || qt.shape[1] != rb ||
                qt.bytes != lw.rows * rb)
                return fail(LBT_E_IO, "unexpected qweight shape for " + p + lin_names[w]);
            if (si->second.dtype != "F32" || si->second.bytes < 4) return fail(LBT_E_IO, "bad wscale " + p + lin_names[w]);
            memcpy(&lw.scale, si->second.data, 4);
            hipError_t e = hipMemcpy(lw.d, qt.data, qt.bytes, hipMemcpyHostToDevice);
            if (e != hipSuccess) {
                int r = hip_err(ctx, e, "upload qweight");
                lbt_model_free(m.release());
                return r;
            }
        }
        for (int k = 0; k < 4; k++) {
            auto ni = tensors.find(p + norm_names[k]);
            const size_t n = (size_t)(k == 3 ? c.intermediate_size : c.hidden_size);
            if (ni == tensors.end() || ni->second.dtype != "F32" || ni->second.bytes != n * 4)
                return fail(LBT_E_IO, "missing or bad " + p + norm_names[k]);
            if (hipMemcpy((void*)m->norm[l * 4 + k], ni->second.data, n * 4, hipMemcpyHostToDevice) != hipSuccess)
                return fail(LBT_E_DEVICE, "upload norm");
        }
    }
    auto fi = tensors.find("model.norm.weight");
    if (fi == tensors.end() || fi->second.dtype != "F32" || fi->second.bytes != (size_t)c.hidden_size * 4)
        return fail(LBT_E_IO, "missing or bad model.norm.weight");
    if (hipMemcpy((void*)m->final_norm, fi->second.data, fi->second.bytes, hipMemcpyHostToDevice) != hipSuccess)
        return fail(LBT_E_DEVICE, "upload final norm");
    auto ei = tensors.find("model.embed_tokens.weight");
    // model.rs:203-206
    if (ei == tensors.end() || ei->second.dtype != "BF16" || ei->second.shape.size() != 2 ||
        ei->second.shape[0] != (size_t)c.vocab_size || ei->second.shape[1] != (size_t)c.hidden_size ||
        ei->second.bytes != (size_t)c.vocab_size * (size_t)c.hidden_size * 2)
        return fail(LBT_E_IO, "embed_tokens: unexpected dtype/shape/size");
    if (hipMemcpy(m->embed, ei->second.data, ei->second.bytes, hipMemcpyHostToDevice) != hipSuccess)
        return fail(LBT_E_DEVICE, "upload embedding");
    *out = m.release();
    return LBT_OK;
}

void lbt_model_free(lbt_model* m) {
    if (!m) return;
    hipStreamSynchronize(m->ctx->stream);
    drop_step_graph(m);
    if (m->sstate) hipFree(m->sstate);
    if (m->sscratch) hipFree(m->sscratch);
    void* bufs[] = {m->wbuf, m->fbuf, m->embed, m->cos_t, m->sin_t, m->x,   m->q,       m->k,
                    m->v,    m->att,  m->h,     m->logits, m->toks, m->key, m->tok_out, m->state,
                    m->ao,   m->aml,  m->q8,    m->q8s,     m->hx};
    for (void* b : bufs)
        if (b) hipFree(b);
    delete m;
}

int lbt_model_get_config(const lbt_model* m, lbt_config* out) {
    if (!m || !out) return LBT_E_INVALID;
    *out = m->cfg;
    return LBT_OK;
}

const lbt_weight* lbt_model_linear(const lbt_model* m, int layer, int which) {
    if (!m || layer < 0 || layer >= m->cfg.num_hidden_layers || which < 0 || which > 6) return nullptr;
    return &m->lin[layer * 7 + which];
}

int lbt_cache_new(lbt_model* m, lbt_cache** out) {
    if (!m || !out) return LBT_E_INVALID;
    lbt_cache* c = new lbt_cache();
    c->m = m;
    *out = c;
    return LBT_OK;
}

void lbt_cache_free(lbt_cache* c) {
    if (!c) return;
    hipStreamSynchronize(c->m->ctx->stream);
    drop_step_graph(c->m);
    if (c->k) hipFree(c->k);
    if (c->v) hipFree(c->v);
    delete c;
}

int lbt_cache_len(const lbt_cache* c) { return c ? c->len : -1; }

int lbt_cache_read(lbt_cache* c, int layer, int is_v, uint16_t* out) {
    if (!c || !out) return LBT_E_INVALID;
    lbt_model* m = c->m;
    lbt_ctx* ctx = m->ctx;
    if (layer < 0 || layer >= m->cfg.num_hidden_layers) return set_err(ctx, LBT_E_INVALID, "cache_read: bad layer");
    if (c->len == 0) return LBT_OK;
    const size_t kvh = (size_t)m->cfg.num_key_value_heads, hd = (size_t)m->hd;
    const uint16_t* src = (is_v ? c->v : c->k) + (size_t)layer * kvh * c->cap * hd;
    LBT_HIP(ctx, hipMemcpy2DAsync(out, (size_t)c->len * hd * 2, src, (size_t)c->cap * hd * 2, (size_t)c->len * hd * 2,
                                  kvh, hipMemcpyDeviceToHost, ctx->stream));
    LBT_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return LBT_OK;
}

static int upload_tokens(lbt_model* m, const uint32_t* tokens, size_t n) {
    lbt_ctx* ctx = m->ctx;
    for (size_t i = 0; i < n; i++)
        if (tokens[i] >= (uint32_t)m->cfg.vocab_size) return set_err(ctx, LBT_E_INVALID, "token id out of range");
    LBT_HIP(ctx, hipMemcpyAsync(m->toks, tokens, n * 4, hipMemcpyHostToDevice, ctx->stream));
    return LBT_OK;
}

int lbt_model_forward(lbt_model* m, const uint32_t* tokens, size_t n, lbt_cache* c, int all_logits, float* logits) {
    if (!m || !c || !tokens || n == 0) return set_err(m ? m->ctx : nullptr, LBT_E_INVALID, "forward: bad arguments");
    lbt_ctx* ctx = m->ctx;
    int rc;
    if ((rc = ensure_room(c, n))) return rc;
    if ((rc = ensure_ws(m, (int)n))) return rc;
    if ((rc = upload_tokens(m, tokens, n))) return rc;
    if ((rc = forward_dev(m, c, m->toks, (int)n, all_logits != 0, true, nullptr))) return rc;
    const size_t rows = all_logits ? n : 1;
    if (logits)
        LBT_HIP(ctx, hipMemcpyAsync(logits, m->logits, rows * (size_t)m->cfg.vocab_size * 4, hipMemcpyDeviceToHost,
                                    ctx->stream));
    LBT_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return LBT_OK;
}

int lbt_model_forward_argmax(lbt_model* m, const uint32_t* tokens, size_t n, lbt_cache* c, uint32_t* next) {
    if (!m || !c || !tokens || n == 0 || !next) return set_err(m ? m->ctx : nullptr, LBT_E_INVALID, "bad arguments");
    lbt_ctx* ctx = m->ctx;
    int rc;
    if ((rc = ensure_room(c, n))) return rc;
    if ((rc = ensure_ws(m, (int)n))) return rc;
    if ((rc = upload_tokens(m, tokens, n))) return rc;
    if ((rc = forward_dev(m, c, m->toks, (int)n, false, false, nullptr))) return rc;
    unsigned long long key = 0;
    LBT_HIP(ctx, hipMemcpyAsync(&key, m->key, 8, hipMemcpyDeviceToHost, ctx->stream));
    LBT_HIP(ctx, hipStreamSynchronize(ctx->stream));
    *next = 0xffffffffu - (uint32_t)(key & 0xffffffffull);
    return LBT_OK;
}

int lbt_model_generate_greedy(lbt_model* m, const uint32_t* prompt, size_t n, size_t steps, lbt_cache* c,
                              uint32_t* out_tokens, float* ms_prefill, float* ms_decode) {
    if (!m || !c || !prompt || n == 0 || !out_tokens) return set_err(m ? m->ctx : nullptr, LBT_E_INVALID, "bad arguments");
    lbt_ctx* ctx = m->ctx;
    int rc;
    if ((rc = ensure_room(c, n, steps))) return rc;
    if ((rc = ensure_ws(m, (int)n))) return rc;
    if ((rc = grow_tok_out(m, (int)steps + 1))) return rc;
    if ((rc = upload_tokens(m, prompt, n))) return rc;
    hipEvent_t e0, e1, e2;
    LBT_HIP(ctx, hipEventCreate(&e0));
    LBT_HIP(ctx, hipEventCreate(&e1));
    LBT_HIP(ctx, hipEventCreate(&e2));
    LBT_HIP(ctx, hipEventRecord(e0, ctx->stream));
    rc = forward_dev(m, c, m->toks, (int)n, false, false, nullptr);
    if (!rc) {
        hipEventRecord(e1, ctx->stream);
        rc = decode_steps(m, c, (int)steps, 0);
        // the last argmax
        if (!rc) rc = launch_embed(ctx, m->embed, 0, m->cfg.vocab_size, nullptr, m->key, m->tok_out + steps, 1, m->x);
        hipEventRecord(e2, ctx->stream);
    }
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (!rc && e != hipSuccess) rc = hip_err(ctx, e, "generate");
    if (!rc) {
        float a = 0, b = 0;
        hipEventElapsedTime(&a, e0, e1);
        hipEventElapsedTime(&b, e1, e2);
        if (ms_prefill) *ms_prefill = a;
        if (ms_decode) *ms_decode = b;
        e = hipMemcpy(out_tokens, m->tok_out, (steps + 1) * 4, hipMemcpyDeviceToHost);
        if (e != hipSuccess) rc = hip_err(ctx, e, "read tokens");
    }
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    hipEventDestroy(e2);
    return rc;
}

int lbt_model_decode_greedy(lbt_model* m, lbt_cache* c, uint32_t first, size_t steps, uint32_t* out_tokens,
                            float* ms_decode) {
    if (!m || !c || !out_tokens || steps == 0) return set_err(m ? m->ctx : nullptr, LBT_E_INVALID, "bad arguments");
    lbt_ctx* ctx = m->ctx;
    if (first >= (uint32_t)m->cfg.vocab_size) return set_err(ctx, LBT_E_INVALID, "token id out of range");
    int rc;
    if ((rc = ensure_room(c, steps))) return rc;
    if ((rc = ensure_ws(m, 1))) return rc;
    if ((rc = grow_tok_out(m, (int)steps + 1))) return rc;
    LBT_HIP(ctx, hipMemcpyAsync(m->toks, &first, 4, hipMemcpyHostToDevice, ctx->stream));
    hipEvent_t e0, e1;
    LBT_HIP(ctx, hipEventCreate(&e0));
    LBT_HIP(ctx, hipEventCreate(&e1));
    hipEventRecord(e0, ctx->stream);
    rc = forward_dev(m, c, m->toks, 1, false, false, nullptr);
    if (!rc) rc = decode_steps(m, c, (int)steps - 1, 0);
    if (!rc) rc = launch_embed(ctx, m->embed, 0, m->cfg.vocab_size, nullptr, m->key, m->tok_out + steps - 1, 1, m->x);
    hipEventRecord(e1, ctx->stream);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (!rc && e != hipSuccess) rc = hip_err(ctx, e, "decode");
    if (!rc) {
        float a = 0;
        hipEventElapsedTime(&a, e0, e1);
        if (ms_decode) *ms_decode = a;
        e = hipMemcpy(out_tokens, m->tok_out, steps * 4, hipMemcpyDeviceToHost);
        if (e != hipSuccess) rc = hip_err(ctx, e, "read tokens");
    }
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    return rc;
}

int lbt_model_forward_sample(lbt_model* m, const uint32_t* tokens, size_t n, lbt_cache* c,
                             const lbt_sample_params* p, uint64_t* state, uint32_t* next) {
    if (!m || !c || !tokens || n == 0 || !next || !p || !state)
        return set_err(m ? m->ctx : nullptr, LBT_E_INVALID, "bad arguments");
    lbt_ctx* ctx = m->ctx;
    int rc;
    if ((rc = ensure_room(c, n))) return rc;
    if ((rc = ensure_ws(m, (int)n))) return rc;
    if ((rc = ensure_sampler(m))) return rc;
    if ((rc = upload_tokens(m, tokens, n))) return rc;
    LBT_HIP(ctx, hipMemcpyAsync(m->sstate, state, 8, hipMemcpyHostToDevice, ctx->stream));
    if ((rc = forward_dev(m, c, m->toks, (int)n, false, true, nullptr))) return rc;
    if ((rc = sample_key(m, p))) return rc;
    unsigned long long key = 0;
    LBT_HIP(ctx, hipMemcpyAsync(&key, m->key, 8, hipMemcpyDeviceToHost, ctx->stream));
    LBT_HIP(ctx, hipMemcpyAsync(state, m->sstate, 8, hipMemcpyDeviceToHost, ctx->stream));
    LBT_HIP(ctx, hipStreamSynchronize(ctx->stream));
    *next = 0xffffffffu - (uint32_t)(key & 0xffffffffull);
    return LBT_OK;
}

int lbt_model_decode_sample(lbt_model* m, lbt_cache* c, uint32_t first, size_t steps, const lbt_sample_params* p,
                            uint64_t* state, uint32_t* out_tokens, float* ms_decode) {
    if (!m || !c || !out_tokens || steps == 0 || !p || !state)
        return set_err(m ? m->ctx : nullptr, LBT_E_INVALID, "bad arguments");
    lbt_ctx* ctx = m->ctx;
    if (first >= (uint32_t)m->cfg.vocab_size) return set_err(ctx, LBT_E_INVALID, "token id out of range");
    int rc;
    if ((rc = ensure_room(c, steps))) return rc;
    if ((rc = ensure_ws(m, 1))) return rc;
    if ((rc = grow_tok_out(m, (int)steps + 1))) return rc;
    if ((rc = ensure_sampler(m))) return rc;
    LBT_HIP(ctx, hipMemcpyAsync(m->toks, &first, 4, hipMemcpyHostToDevice, ctx->stream));
    LBT_HIP(ctx, hipMemcpyAsync(m->sstate, state, 8, hipMemcpyHostToDevice, ctx->stream));
    hipEvent_t e0, e1;
    LBT_HIP(ctx, hipEventCreate(&e0));
    LBT_HIP(ctx, hipEventCreate(&e1));
    hipEventRecord(e0, ctx->stream);
    rc = forward_dev(m, c, m->toks, 1, false, true, nullptr);
    if (!rc) rc = sample_key(m, p);
    if (!rc) rc = decode_steps(m, c, (int)steps - 1, 0, p);
    if (!rc) rc = launch_embed(ctx, m->embed, 0, m->cfg.vocab_size, nullptr, m->key, m->tok_out + steps - 1, 1, m->x);
    hipEventRecord(e1, ctx->stream);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (!rc && e != hipSuccess) rc = hip_err(ctx, e, "decode");
    if (!rc) {
        float a = 0;
        hipEventElapsedTime(&a, e0, e1);
        if (ms_decode) *ms_decode = a;
        e = hipMemcpy(out_tokens, m->tok_out, steps * 4, hipMemcpyDeviceToHost);
        if (e == hipSuccess) e = hipMemcpy(state, m->sstate, 8, hipMemcpyDeviceToHost);
        if (e != hipSuccess) rc = hip_err(ctx, e, "read tokens");
    }
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    return rc;
}

int lbt_model_set_head(lbt_model* m, int kind) {
    if (!m) return LBT_E_INVALID;
    lbt_ctx* ctx = m->ctx;
    if (kind < 0 || kind > 2)
        return set_err(ctx, LBT_E_INVALID, "set_head: kind must be 0 (bf16), 1 (int8) or 2 (bf16 matrix cores)");
    const lbt_config& c = m->cfg;
    if (kind == 2 && !m->hx) {
        if (c.hidden_size % 64) return set_err(ctx, LBT_E_INVALID, "set_head: kind 2 needs hidden_size % 64 == 0");
        const size_t bytes = (size_t)2 * 64 * c.hidden_size * 2;
        void* p = nullptr;
        hipError_t e = hipMalloc(&p, bytes);
        if (e != hipSuccess) return hip_err(ctx, e, "bf16 matrix-core head scratch");
        m->hx = (uint16_t*)p;
        m->hx_bytes = bytes;
    }
    if (kind == 1 && !m->q8) {
        const size_t n = (size_t)c.vocab_size * c.hidden_size;
        int8_t* q = nullptr;
        float* qs = nullptr;
        hipError_t e = hipMalloc(&q, n);
        if (e == hipSuccess) e = hipMalloc(&qs, (size_t)c.vocab_size * 4);
        int rc = e == hipSuccess ? launch_q8_quantize(ctx, m->embed, c.vocab_size, c.hidden_size, q, qs)
                                 : hip_err(ctx, e, "int8 head allocation");
        if (!rc && (e = hipStreamSynchronize(ctx->stream)) != hipSuccess) rc = hip_err(ctx, e, "int8 head quantize");
        if (rc) {  // the model keeps its bf16 head
            if (q) hipFree(q);
            if (qs) hipFree(qs);
            return rc;
        }
        m->q8 = q;
        m->q8s = qs;
    }
    m->head_kind = kind;  // the step graphs are keyed by it
    return LBT_OK;
}

int lbt_model_read_hidden(lbt_model* m, float* out, size_t n) {
    if (!m || !out) return LBT_E_INVALID;
    lbt_ctx* ctx = m->ctx;
    if (n > (size_t)m->last_n) return set_err(ctx, LBT_E_INVALID, "read_hidden: more rows than the last forward");
    LBT_HIP(ctx, hipMemcpyAsync(out, m->x, n * (size_t)m->cfg.hidden_size * 4, hipMemcpyDeviceToHost, ctx->stream));
    LBT_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return LBT_OK;
}

// ---- batched decode --------------------------------------------------------
size_t lbt_batch::seq_stride() const { return (size_t)m->cfg.num_key_value_heads * cap * m->hd; }

namespace {

// KV view and row positions of one step of every sequence of the batch,
// with b->pos holding the positions.
int batch_step(lbt_batch* b, const uint32_t* toks_dev, bool want_logits, uint32_t* tok_out_dev) {
    lbt_model* m = b->m;
    KvView kv{b->k, b->v, b->layer_stride(), b->cap};
    RowPos rp;
    rp.tok_pos = b->pos;
    rp.seq_stride = b->seq_stride();
    int vmax = 0;
    for (int l : b->len) vmax = l + 1 > vmax ? l + 1 : vmax;
    rp.vis_max = vmax;
    return forward_rows(m, kv, rp, toks_dev, b->nseq, want_logits, want_logits, tok_out_dev, nullptr, true);
}

int batch_upload_pos(lbt_batch* b) {
    lbt_ctx* ctx = b->m->ctx;
    LBT_HIP(ctx, hipMemcpyAsync(b->pos, b->len.data(), (size_t)b->nseq * 4, hipMemcpyHostToDevice, ctx->stream));
    return LBT_OK;
}

}  // namespace

int lbt_batch_new(lbt_model* m, int nseq, int cap, lbt_batch** out) {
    if (!m || !out || nseq <= 0 || cap <= 0) return set_err(m ? m->ctx : nullptr, LBT_E_INVALID, "bad arguments");
    lbt_ctx* ctx = m->ctx;
    *out = nullptr;
    if (cap > m->cfg.max_position_embeddings)
        return set_err(ctx, LBT_E_RANGE, "batch: capacity above max_position_embeddings");
    lbt_batch* b = new lbt_batch();
    b->m = m;
    b->nseq = nseq;
    b->cap = cap;
    b->len.assign(nseq, 0);
    const size_t bytes = (size_t)m->cfg.num_hidden_layers * b->layer_stride() * 2;
    hipError_t e = hipMalloc(&b->k, bytes);
    if (e == hipSuccess) e = hipMalloc(&b->v, bytes);
    if (e == hipSuccess) e = hipMalloc(&b->pos, (size_t)nseq * 4);
    if (e != hipSuccess) {
        lbt_batch_free(b);
        return set_err(ctx, LBT_E_NOMEM, "batch: cache allocation failed");
    }
    *out = b;
    return LBT_OK;
}

void lbt_batch_free(lbt_batch* b) {
    if (!b) return;
    hipStreamSynchronize(b->m->ctx->stream);
    void* bufs[] = {b->k, b->v, b->pos, b->tok_out, b->sp, b->sst, b->sscratch};
    for (void* p : bufs)
        if (p) hipFree(p);
    delete b;
}

int lbt_batch_reset(lbt_batch* b, int seq) {
    if (!b || seq < 0 || seq >= b->nseq) return set_err(b ? b->m->ctx : nullptr, LBT_E_INVALID, "bad arguments");
    b->len[seq] = 0;
    return LBT_OK;
}

int lbt_batch_len(const lbt_batch* b, int seq) {
    if (!b || seq < 0 || seq >= b->nseq) return -1;
    return b->len[seq];
}

int lbt_batch_prefill(lbt_batch* b, int seq, const uint32_t* tokens, size_t n, uint32_t* next) {
    if (!b || !tokens || n == 0 || seq < 0 || seq >= b->nseq)
        return set_err(b ? b->m->ctx : nullptr, LBT_E_INVALID, "bad arguments");
    lbt_model* m = b->m;
    lbt_ctx* ctx = m->ctx;
    if (n > (size_t)(b->cap - b->len[seq])) return set_err(ctx, LBT_E_RANGE, "batch: sequence capacity exceeded");
    int rc;
    if ((rc = ensure_ws(m, (int)n))) return rc;
    if ((rc = upload_tokens(m, tokens, n))) return rc;
    const size_t off = (size_t)seq * b->seq_stride();
    KvView kv{b->k + off, b->v + off, b->layer_stride(), b->cap};
    RowPos rp;
    rp.pos0 = b->len[seq];
    rp.vis_max = b->len[seq] + (int)n;
    if ((rc = forward_rows(m, kv, rp, m->toks, (int)n, false, false, nullptr, nullptr, (int)n > 1))) return rc;
    b->len[seq] += (int)n;
    unsigned long long key = 0;
    LBT_HIP(ctx, hipMemcpyAsync(&key, m->key, 8, hipMemcpyDeviceToHost, ctx->stream));
    LBT_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (next) *next = 0xffffffffu - (uint32_t)(key & 0xffffffffull);
    return LBT_OK;
}

namespace {
int batch_sampler(lbt_batch* b) {
    if (b->sp) return LBT_OK;
    lbt_ctx* ctx = b->m->ctx;
    size_t bytes;
    sample_scratch_bytes(b->nseq, b->m->cfg.vocab_size, &bytes);
    void *scr = nullptr, *st = nullptr, *sp = nullptr;
    hipError_t e = hipMalloc(&scr, bytes);
    if (e == hipSuccess) e = hipMalloc(&st, (size_t)b->nseq * 8);
    if (e == hipSuccess) e = hipMalloc(&sp, (size_t)b->nseq * sizeof(lbt_sample_params));
    if (e != hipSuccess) {  // all or nothing: a later call allocates afresh
        if (scr) hipFree(scr);
        if (st) hipFree(st);
        return hip_err(ctx, e, "batch sampler scratch");
    }
    b->sscratch = scr;
    b->sst = (unsigned long long*)st;
    b->sp = (lbt_sample_params*)sp;
    return LBT_OK;
}
}  // namespace

int lbt_batch_prefill_sample(lbt_batch* b, int seq, const uint32_t* tokens, size_t n, const lbt_sample_params* p,
                             uint64_t* state, uint32_t* next) {
    if (!b || !tokens || n == 0 || seq < 0 || seq >= b->nseq || !p || !state)
        return set_err(b ? b->m->ctx : nullptr, LBT_E_INVALID, "bad arguments");
    lbt_model* m = b->m;
    lbt_ctx* ctx = m->ctx;
    if (n > (size_t)(b->cap - b->len[seq])) return set_err(ctx, LBT_E_RANGE, "batch: sequence capacity exceeded");
    int rc;
    if ((rc = ensure_ws(m, (int)n))) return rc;
    if ((rc = batch_sampler(b))) return rc;
    if ((rc = upload_tokens(m, tokens, n))) return rc;
    LBT_HIP(ctx, hipMemcpyAsync(b->sst + seq, state, 8, hipMemcpyHostToDevice, ctx->stream));
    const size_t off = (size_t)seq * b->seq_stride();
    KvView kv{b->k + off, b->v + off, b->layer_stride(), b->cap};
    RowPos rp;
    rp.pos0 = b->len[seq];
    rp.vis_max = b->len[seq] + (int)n;
    if ((rc = forward_rows(m, kv, rp, m->toks, (int)n, false, true, nullptr, nullptr, (int)n > 1))) return rc;
    b->len[seq] += (int)n;
    if ((rc = launch_sample(ctx, m->logits, m->cfg.vocab_size, 1, m->cfg.vocab_size, *p, b->sst + seq, nullptr, m->key,
                            b->sscratch)))
        return rc;
    unsigned long long key = 0;
    LBT_HIP(ctx, hipMemcpyAsync(&key, m->key, 8, hipMemcpyDeviceToHost, ctx->stream));
    LBT_HIP(ctx, hipMemcpyAsync(state, b->sst + seq, 8, hipMemcpyDeviceToHost, ctx->stream));
    LBT_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (next) *next = 0xffffffffu - (uint32_t)(key & 0xffffffffull);
    return LBT_OK;
}

int lbt_batch_forward_sample(lbt_batch* b, const uint32_t* tokens, const lbt_sample_params* params, uint64_t* states,
                             uint32_t* next) {
    if (!b || !tokens || !params || !states || !next)
        return set_err(b ? b->m->ctx : nullptr, LBT_E_INVALID, "bad arguments");
    lbt_model* m = b->m;
    lbt_ctx* ctx = m->ctx;
    for (int s = 0; s < b->nseq; s++) {
        if (b->len[s] + 1 > b->cap) return set_err(ctx, LBT_E_RANGE, "batch: sequence capacity exceeded");
        if (tokens[s] >= (uint32_t)m->cfg.vocab_size) return set_err(ctx, LBT_E_INVALID, "token id out of range");
    }
    int rc;
    if ((rc = ensure_ws(m, b->nseq))) return rc;
    if ((rc = batch_sampler(b))) return rc;
    if ((rc = upload_tokens(m, tokens, (size_t)b->nseq))) return rc;
    LBT_HIP(ctx, hipMemcpyAsync(b->sp, params, (size_t)b->nseq * sizeof(lbt_sample_params), hipMemcpyHostToDevice,
                                ctx->stream));
    LBT_HIP(ctx, hipMemcpyAsync(b->sst, states, (size_t)b->nseq * 8, hipMemcpyHostToDevice, ctx->stream));
    if ((rc = batch_upload_pos(b))) return rc;
    if ((rc = batch_step(b, m->toks, true, nullptr))) return rc;
    for (int s = 0; s < b->nseq; s++) b->len[s] += 1;
    if ((rc = launch_sample(ctx, m->logits, m->cfg.vocab_size, b->nseq, m->cfg.vocab_size, params[0], b->sst,
                            nullptr, m->key, b->sscratch, b->sp)))
        return rc;
    std::vector<unsigned long long> keys((size_t)b->nseq);
    LBT_HIP(ctx, hipMemcpyAsync(keys.data(), m->key, keys.size() * 8, hipMemcpyDeviceToHost, ctx->stream));
    LBT_HIP(ctx, hipMemcpyAsync(states, b->sst, (size_t)b->nseq * 8, hipMemcpyDeviceToHost, ctx->stream));
    LBT_HIP(ctx, hipStreamSynchronize(ctx->stream));
    for (int s = 0; s < b->nseq; s++) next[s] = 0xffffffffu - (uint32_t)(keys[s] & 0xffffffffull);
    return LBT_OK;
}

int lbt_batch_fill_synthetic(lbt_batch* b, int len, uint64_t seed) {
    if (!b || len < 0) return set_err(b ? b->m->ctx : nullptr, LBT_E_INVALID, "bad arguments");
    lbt_model* m = b->m;
    lbt_ctx* ctx = m->ctx;
    if (len > b->cap) return set_err(ctx, LBT_E_RANGE, "batch: fill beyond capacity");
    const size_t rows = (size_t)m->cfg.num_hidden_layers * b->nseq * m->cfg.num_key_value_heads;
    int rc;
    if ((rc = launch_synth_kv(ctx, seed * 2 + 1, rows, b->cap, len, m->hd, b->k))) return rc;
    if ((rc = launch_synth_kv(ctx, seed * 2 + 2, rows, b->cap, len, m->hd, b->v))) return rc;
    LBT_HIP(ctx, hipStreamSynchronize(ctx->stream));
    b->len.assign(b->nseq, len);
    return LBT_OK;
}

int lbt_batch_forward(lbt_batch* b, const uint32_t* tokens, float* logits, uint32_t* next) {
    if (!b || !tokens) return set_err(b ? b->m->ctx : nullptr, LBT_E_INVALID, "bad arguments");
    lbt_model* m = b->m;
    lbt_ctx* ctx = m->ctx;
    for (int s = 0; s < b->nseq; s++) {
        if (b->len[s] + 1 > b->cap) return set_err(ctx, LBT_E_RANGE, "batch: sequence capacity exceeded");
        if (tokens[s] >= (uint32_t)m->cfg.vocab_size) return set_err(ctx, LBT_E_INVALID, "token id out of range");
    }
    int rc;
    if ((rc = ensure_ws(m, b->nseq))) return rc;
    if ((rc = upload_tokens(m, tokens, (size_t)b->nseq))) return rc;
    if ((rc = batch_upload_pos(b))) return rc;
    if ((rc = batch_step(b, m->toks, logits != nullptr, nullptr))) return rc;
    for (int s = 0; s < b->nseq; s++) b->len[s] += 1;
    std::vector<unsigned long long> keys((size_t)b->nseq);
    LBT_HIP(ctx, hipMemcpyAsync(keys.data(), m->key, keys.size() * 8, hipMemcpyDeviceToHost, ctx->stream));
    if (logits)
        LBT_HIP(ctx, hipMemcpyAsync(logits, m->logits, (size_t)b->nseq * m->cfg.vocab_size * 4, hipMemcpyDeviceToHost,
                                    ctx->stream));
    LBT_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (next)
        for (int s = 0; s < b->nseq; s++) next[s] = 0xffffffffu - (uint32_t)(keys[s] & 0xffffffffull);
    return LBT_OK;
}

int lbt_batch_decode_greedy(lbt_batch* b, const uint32_t* first, size_t steps, uint32_t* out_tokens,
                            float* ms_decode) {
    if (!b || !first || !out_tokens || steps == 0)
        return set_err(b ? b->m->ctx : nullptr, LBT_E_INVALID, "bad arguments");
    lbt_model* m = b->m;
    lbt_ctx* ctx = m->ctx;
    const int n = b->nseq;
    for (int s = 0; s < n; s++) {
        if (b->len[s] + (int)steps > b->cap) return set_err(ctx, LBT_E_RANGE, "batch: sequence capacity exceeded");
        if (first[s] >= (uint32_t)m->cfg.vocab_size) return set_err(ctx, LBT_E_INVALID, "token id out of range");
    }
    int rc;
    if ((rc = ensure_ws(m, n))) return rc;
    if (steps * n > b->tok_out_cap) {
        if (b->tok_out) hipFree(b->tok_out);
        b->tok_out = nullptr;
        LBT_HIP(ctx, hipMalloc(&b->tok_out, steps * n * 4));
        b->tok_out_cap = steps * n;
    }
    if ((rc = upload_tokens(m, first, (size_t)n))) return rc;
    if ((rc = batch_upload_pos(b))) return rc;
    hipEvent_t e0, e1;
    LBT_HIP(ctx, hipEventCreate(&e0));
    LBT_HIP(ctx, hipEventCreate(&e1));
    hipEventRecord(e0, ctx->stream);
    // step i consumes the previous step's argmax keys; its embed records them
    // as step i-1's tokens; positions advance on the device
    const std::vector<int> len0 = b->len;
    for (size_t i = 0; i < steps && !rc; i++) {
        rc = batch_step(b, i == 0 ? m->toks : nullptr, false, i == 0 ? nullptr : b->tok_out + (i - 1) * n);
        if (!rc) rc = launch_advance_pos(ctx, b->pos, n);
        for (int s = 0; s < n; s++) b->len[s] += 1;  // vis_max of the next step
    }
    if (!rc) rc = launch_embed(ctx, m->embed, 0, m->cfg.vocab_size, nullptr, m->key, b->tok_out + (steps - 1) * n, n, m->x);
    hipEventRecord(e1, ctx->stream);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (!rc && e != hipSuccess) rc = hip_err(ctx, e, "batch decode");
    if (rc) {
        b->len = len0;
    } else {
        float a = 0;
        hipEventElapsedTime(&a, e0, e1);
        if (ms_decode) *ms_decode = a;
        e = hipMemcpy(out_tokens, b->tok_out, steps * n * 4, hipMemcpyDeviceToHost);
        if (e != hipSuccess) rc = hip_err(ctx, e, "read tokens");
    }
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    return rc;
}

}  // extern "C"
