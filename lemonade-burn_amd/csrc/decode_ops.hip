// decode_ops.hip -- the non-GEMM pieces of the BitNet b1.58 step on gfx950:
// token embedding, RoPE + bf16 KV append, GQA attention over the bf16 cache,
// the tied bf16 LM head with fused final RMSNorm and device argmax, and the
// synthetic-weight generator.
//
// Reference: crates/lb-model/src/model.rs (embed :274-282, rope :284-301,
// KV cache :340-347, GQA attention :349-357, final norm + head :368-373),
// crates/lb-ternary/src/bf16.rs (bf16_gemv :14-25), sample.rs:17-25 (argmax).
// Float order follows lbt_device.h; the oracle mirrors it.
#include "lbt_device.h"
#include "lbt_internal.h"

namespace lbt {

// ---------------------------------------------------------------------------
// embedding (model.rs:274-282).  Token ids come from `tokens`, or, when it is
// null, from the argmax key of the previous step (device-side feedback).  The
// key is cleared for the next LM head.
__global__ __launch_bounds__(kThreads) void embed_kernel(const uint16_t* embed, int hidden, int vocab,
                                                         const uint32_t* tokens, unsigned long long* key,
                                                         uint32_t* tok_out, float* x) {
    __shared__ uint32_t tok_s;
    const int t = blockIdx.x;
    if (threadIdx.x == 0) {
        uint32_t tok = tokens ? tokens[t] : 0xffffffffu - (uint32_t)(key[t] & 0xffffffffull);
        // a key that was never written (no finite logit) must not index past the table
        if (tok >= (uint32_t)vocab) tok = 0;
        tok_s = tok;
        if (tok_out) tok_out[t] = tok;
    }
    __syncthreads();
    if (threadIdx.x == 0 && key) key[t] = 0ull;
    const uint16_t* row = embed + (size_t)tok_s * hidden;
    float* dst = x + (size_t)t * hidden;
    for (int i = threadIdx.x; i < hidden; i += kThreads) dst[i] = bf16_to_f32(row[i]);
}

// ---------------------------------------------------------------------------
// RoPE on the new keys and bf16 append of K and V at positions pos0.. .
// apply_rope (model.rs:295-301): out = x*cos + rot*sin, rot = cat(-x2, x1).
__global__ void rope_append_kernel(const float* k, const float* v, int kvh, int hd, int pos0, const float* cos_t,
                                   const float* sin_t, uint16_t* kc, uint16_t* vc, int cap) {
    const int t = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
    const int h2 = hd >> 1, p = pos0 + t, i = d % h2;
    const float* kr = k + ((size_t)t * kvh + h) * hd;
    const float rot = d < h2 ? -kr[d + h2] : kr[d - h2];
    const float y = kr[d] * cos_t[(size_t)p * h2 + i] + rot * sin_t[(size_t)p * h2 + i];
    const size_t o = ((size_t)h * cap + p) * hd + d;
    kc[o] = f32_to_bf16(y);
    vc[o] = f32_to_bf16(v[((size_t)t * kvh + h) * hd + d]);
}

// ---------------------------------------------------------------------------
// GQA attention for query row t (absolute position pos0 + t) and head h:
// q is rotated here, scores = q.K^T * scaling over the visible keys 0..p,
// softmax (exp(s - max) / sum), then probs @ V (model.rs:349-357; the causal
// mask of :316-328 is the visibility bound).  One workgroup per (head, row).
__global__ __launch_bounds__(kThreads) void attention_kernel(const float* q, int nh, int kvh, int hd, int pos0,
                                                             const float* cos_t, const float* sin_t,
                                                             const uint16_t* kc, const uint16_t* vc, int cap,
                                                             float scaling, float* out) {
    extern __shared__ float sc[];  // [p + 1]
    __shared__ float qr[256];
    __shared__ float red[kThreads];
    const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
    const int H = nh * hd, h2 = hd >> 1, p = pos0 + t, vis = p + 1, g = h / (nh / kvh);
    const float* qh = q + (size_t)t * H + (size_t)h * hd;
    if (tid < hd) {
        const int i = tid % h2;
        const float rot = tid < h2 ? -qh[tid + h2] : qh[tid - h2];
        qr[tid] = qh[tid] * cos_t[(size_t)p * h2 + i] + rot * sin_t[(size_t)p * h2 + i];
    }
    __syncthreads();
    const uint16_t* K = kc + (size_t)g * cap * hd;
    const uint16_t* V = vc + (size_t)g * cap * hd;
    float mx = -__builtin_inff();
    for (int j = tid; j < vis; j += kThreads) {
        const uint16_t* kr = K + (size_t)j * hd;
        float a = 0.0f;
        for (int d = 0; d < hd; d += 8) {
            const uint4 kv = *(const uint4*)(kr + d);
            const uint32_t wv[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                a = __builtin_fmaf(qr[d + 2 * e], bf16_to_f32((uint16_t)(wv[e] & 0xffffu)), a);
                a = __builtin_fmaf(qr[d + 2 * e + 1], bf16_to_f32((uint16_t)(wv[e] >> 16)), a);
            }
        }
        const float s = a * scaling;
        sc[j] = s;
        mx = fmaxf(mx, s);
    }
    mx = block_max(mx, red);
    float ps = 0.0f;
    for (int j = tid; j < vis; j += kThreads) {
        const float e = lbt_expf(sc[j] - mx);
        sc[j] = e;
        ps = ps + e;
    }
    const float sum = block_tree256(ps, red);
    for (int j = tid; j < vis; j += kThreads) sc[j] = sc[j] / sum;
    __syncthreads();
    if (tid < hd) {
        float a = 0.0f;
        for (int j = 0; j < vis; j++) a = __builtin_fmaf(sc[j], bf16_to_f32(V[(size_t)j * hd + tid]), a);
        out[(size_t)t * H + (size_t)h * hd + tid] = a;
    }
}

// ---------------------------------------------------------------------------
// bf16 GEMV / tied LM head (bf16.rs:14-25, model.rs:369-373) with the final
// RMSNorm fused as a prologue.  One wavefront per output row; lane l takes
// the 16-byte chunks l, l+64, ... (8 bf16 each), fused multiply-adds in
// element order, then an xor butterfly.  The first-max key of each row t is
// atomically maxed into key[t] (argmax, sample.rs:17-25).
__device__ __forceinline__ float norm_factor_lm(const float* xr, int cols, const float* norm_w, float eps,
                                                float* red) {
    if (!norm_w) return 1.0f;
    float p = 0.0f;
    for (int i = threadIdx.x; i < cols; i += kThreads) p = __builtin_fmaf(xr[i], xr[i], p);
    float ss = block_tree256(p, red);
    float mean = ss / (float)cols;
    return 1.0f / __builtin_sqrtf(mean + eps);
}

__device__ __forceinline__ float bf_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }

__global__ __launch_bounds__(kThreads) void lmhead_kernel(const uint16_t* W, int rows, int cols, const float* x,
                                                          const float* norm_w, float eps, float* logits,
                                                          unsigned long long* key) {
    extern __shared__ __align__(16) float xs[];  // cols
    __shared__ float red[kThreads];
    const int t = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
    const float* xr = x + (size_t)t * cols;
    const float rr = norm_factor_lm(xr, cols, norm_w, eps, red);
    for (int i = tid; i < cols; i += kThreads) xs[i] = norm_w ? (xr[i] * rr) * norm_w[i] : xr[i];
    __syncthreads();
    const int nchunks = cols >> 3;
    const int gw = blockIdx.x * 4 + (tid >> 6), nw = gridDim.x * 4;
    unsigned long long best = 0ull;
    for (int r = gw; r < rows; r += nw) {
        const uint4* wr = (const uint4*)(W + (size_t)r * cols);
        float acc = 0.0f;
        for (int c = lane; c < nchunks; c += 64) {
            const uint4 wv = wr[c];
            const float4 x0 = *(const float4*)(xs + 8 * c);
            const float4 x1 = *(const float4*)(xs + 8 * c + 4);
            acc = __builtin_fmaf(bf_lo(wv.x), x0.x, acc);
            acc = __builtin_fmaf(bf_hi(wv.x), x0.y, acc);
            acc = __builtin_fmaf(bf_lo(wv.y), x0.z, acc);
            acc = __builtin_fmaf(bf_hi(wv.y), x0.w, acc);
            acc = __builtin_fmaf(bf_lo(wv.z), x1.x, acc);
            acc = __builtin_fmaf(bf_hi(wv.z), x1.y, acc);
            acc = __builtin_fmaf(bf_lo(wv.w), x1.z, acc);
            acc = __builtin_fmaf(bf_hi(wv.w), x1.w, acc);
        }
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) acc = acc + __shfl_xor(acc, m);
        if (lane == 0) {
            if (logits) logits[(size_t)t * rows + r] = acc;
            const unsigned long long k = argmax_key(acc, (uint32_t)r);
            best = k > best ? k : best;
        }
    }
    if (key && lane == 0 && best) atomicMax(&key[t], best);
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

// ---------------------------------------------------------------------------
// launchers
int launch_embed(lbt_ctx* ctx, const uint16_t* embed, int hidden, int vocab, const uint32_t* tokens,
                 const unsigned long long* key, uint32_t* tok_out, int m, float* x) {
    hipLaunchKernelGGL(embed_kernel, dim3(m), dim3(kThreads), 0, ctx->stream, embed, hidden, vocab, tokens,
                       (unsigned long long*)key, tok_out, x);
    LBT_HIP(ctx, hipGetLastError());
    return LBT_OK;
}

int launch_rope_append(lbt_ctx* ctx, const float* k, const float* v, int m, int kvh, int hd, int pos0,
                       const float* cos_t, const float* sin_t, uint16_t* kc, uint16_t* vc, int cap) {
    hipLaunchKernelGGL(rope_append_kernel, dim3(m, kvh), dim3(hd), 0, ctx->stream, k, v, kvh, hd, pos0, cos_t,
                       sin_t, kc, vc, cap);
    LBT_HIP(ctx, hipGetLastError());
    return LBT_OK;
}

int launch_attention(lbt_ctx* ctx, const float* q, int m, int nh, int kvh, int hd, int pos0, const float* cos_t,
                     const float* sin_t, const uint16_t* kc, const uint16_t* vc, int cap, float scaling,
                     float* out) {
    if (hd > 256 || hd % 8) return set_err(ctx, LBT_E_INVALID, "attention: head_dim must be <= 256, multiple of 8");
    const size_t lds = (size_t)(pos0 + m) * sizeof(float);
    if (lds > 64 * 1024) return set_err(ctx, LBT_E_RANGE, "attention: context too long for the LDS score buffer");
    hipEvent_t ev = nullptr;
    prof_begin(ctx, &ev);
    hipLaunchKernelGGL(attention_kernel, dim3(nh, m), dim3(kThreads), lds, ctx->stream, q, nh, kvh, hd, pos0, cos_t,
                       sin_t, kc, vc, cap, scaling, out);
    LBT_HIP(ctx, hipGetLastError());
    const double kv_bytes = 2.0 * kvh * (double)(pos0 + m) * hd * 2.0;
    prof_end(ctx, ev, kProfAttn, kv_bytes);
    return LBT_OK;
}

int launch_bf16_linear(lbt_ctx* ctx, const uint16_t* w, int rows, int cols, const float* x, int m,
                       const float* norm_w, float eps, float* logits, unsigned long long* key) {
    if (cols % 8) return set_err(ctx, LBT_E_INVALID, "bf16 linear: cols must be a multiple of 8");
    if (m <= 0) return LBT_OK;
    const size_t lds = (size_t)cols * sizeof(float);
    if (lds > 64 * 1024) return set_err(ctx, LBT_E_INVALID, "bf16 linear: cols too large");
    int blocks = (rows + 31) / 32;
    if (blocks > 2048) blocks = 2048;
    if (blocks < 1) blocks = 1;
    hipEvent_t ev = nullptr;
    prof_begin(ctx, &ev);
    hipLaunchKernelGGL(lmhead_kernel, dim3(blocks, m), dim3(kThreads), lds, ctx->stream, w, rows, cols, x, norm_w,
                       eps, logits, key);
    LBT_HIP(ctx, hipGetLastError());
    prof_end(ctx, ev, kProfHead, (double)rows * cols * 2.0 * m);
    return LBT_OK;
}

int launch_fill_u64(lbt_ctx* ctx, unsigned long long* p, int n, unsigned long long v) {
    hipLaunchKernelGGL(fill_u64_kernel, dim3((n + 255) / 256), dim3(256), 0, ctx->stream, p, n, v);
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

int launch_synth_bf16(lbt_ctx* ctx, uint64_t seed, uint64_t tensor, size_t n, uint16_t* out) {
    hipLaunchKernelGGL(synth_bf16_kernel, dim3(grid_for(n)), dim3(256), 0, ctx->stream, seed, tensor, n, out);
    LBT_HIP(ctx, hipGetLastError());
    return LBT_OK;
}

}  // namespace lbt
