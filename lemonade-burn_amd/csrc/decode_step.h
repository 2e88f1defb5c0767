// decode_step.h -- host/device interface of the one-dispatch decode step
// (decode_step.hip): all decoder layers of one batch-1 token on a persistent
// grid of one workgroup per compute unit.
#pragma once
#include "lbt_internal.h"

namespace lbt {

constexpr int kStepMaxRows = 64;  // o / down rows per workgroup (kept in LDS for the residual)
constexpr int kStepMaxCpl = 8;


// Row slice of one linear per workgroup: rpw virtual rows, L lanes per row,
// cpl 16-byte chunks per lane, the slice's LDS bytes start at `off`.
struct StepTile {
    int rpw, L, cpl, off;
};

struct StepArgs {
    const uint8_t* w0[7];      // layer 0's packed matrices (q, k, v, o, gate, up, down)
    size_t wstride;            // bytes from one layer's matrices to the next's
    const float* n0[4];        // layer 0's norm gains: input, post_attention, attn_sub, ffn_sub
    size_t nstride;            // floats from one layer's norm gains to the next's
    const float* wscale;       // device [layers * 7] per-tensor weight scales
    const uint16_t* embed;
    const float* cos_t;
    const float* sin_t;
    uint16_t* kc;
    uint16_t* vc;
    int cap;
    size_t layer_kv;  // cache elements per layer (K or V)
    int layers, H, I, nh, kvh, hd, KV, vocab;
    float eps, scaling;
    int* state;  // [0] position - 1, [1] output slot, [2] epoch base
    unsigned long long* key;  // argmax key of the previous token (reset here for the next head)
    uint32_t* tok_out;
    float* xout;  // final hidden state (input of the LM head dispatch)
    // epoch-tagged activation words {epoch << 32 | f32}
    unsigned long long* llx;    // [H]
    unsigned long long* llqkv;  // [H + 2 KV]: rotated q, k (bf16 values), v (bf16 values)
    unsigned long long* llpart; // [kAttnSplits][H] split outputs, then [kAttnSplits][nh][2] (max, sum)
    unsigned long long* llatt;  // [H] attention output (the splits combined)
    unsigned long long* llh;    // [I]
    unsigned* err;
    StepTile t[4];  // q/k/v, o, gate/up, down
    int rt_off[4];  // LDS bytes of each phase's row table
    int xq_off, sc_off, ws_off;
    int CH, CI;     // 16-byte chunks of a packed row of K = H, K = I
    // optional phase timestamps of every workgroup ([G][layers][32] ticks of
    // the 100 MHz clock), for measurements only
    unsigned long long* trace;
};

struct StepPlan {
    int G = 0;
    StepTile t[4];
    int rt_off[4] = {0, 0, 0, 0};
    int xq_off = 0, sc_off = 0, ws_off = 0;
    size_t lds = 0;
    const void* fn = nullptr;
    double bytes = 0.0;  // algorithmic bytes per dispatch (packed weights)
};

// Fills the plan for G workgroups; 0 with a reason when the shape is not
// supported (the multi-kernel step then serves it).
int step_plan(const lbt_config& c, int cap, int G, StepPlan& pl, const char** why);
// Fills the plan's fields of `a` (tiles, LDS offsets).
void step_fill(const StepPlan& pl, const lbt_config& c, StepArgs& a);
// `dargs`: the arguments in device memory (written by the caller, stream-ordered).
int launch_decode_step(lbt_ctx* ctx, const StepPlan& pl, const StepArgs* dargs, hipStream_t s);

// words of each epoch-tagged buffer
inline size_t step_words_x(const lbt_config& c) { return (size_t)c.hidden_size; }

}  // namespace lbt
