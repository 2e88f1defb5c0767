//! Raw bindings of include/lbt.h (the C ABI of liblbt_hip), one declaration
//! per entry point, in the header's order.  Every function returns 0 or a
//! negative LBT_E_* status; `lbt_last_error` holds the message.
#![allow(non_camel_case_types)]

use std::os::raw::{c_char, c_int, c_void};

pub const LBT_OK: c_int = 0;
pub const LBT_E_INVALID: c_int = -1;
pub const LBT_E_DEVICE: c_int = -2;
pub const LBT_E_NOMEM: c_int = -3;
pub const LBT_E_IO: c_int = -4;
pub const LBT_E_RANGE: c_int = -5;

#[repr(C)]
pub struct LbtCtx {
    _p: [u8; 0],
}
#[repr(C)]
pub struct LbtWeight {
    _p: [u8; 0],
}
#[repr(C)]
pub struct LbtBf16 {
    _p: [u8; 0],
}
#[repr(C)]
pub struct LbtModel {
    _p: [u8; 0],
}
#[repr(C)]
pub struct LbtCache {
    _p: [u8; 0],
}
#[repr(C)]
pub struct LbtQ8Head {
    _p: [u8; 0],
}
#[repr(C)]
pub struct LbtBatch {
    _p: [u8; 0],
}
#[repr(C)]
pub struct LbtSched {
    _p: [u8; 0],
}

/// SamplingParams (lb-model/src/sample.rs:3-15) without the seed.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct LbtSampleParams {
    pub temperature: f32,
    pub top_p: f32,
    pub top_k: usize,
}

/// Config (lb-model/src/model.rs:22-42).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct LbtConfig {
    pub hidden_size: i32,
    pub intermediate_size: i32,
    pub num_attention_heads: i32,
    pub num_key_value_heads: i32,
    pub num_hidden_layers: i32,
    pub vocab_size: i32,
    pub max_position_embeddings: i32,
    pub bos_token_id: u32,
    pub rms_norm_eps: f64,
    pub rope_theta: f64,
}

/// Per-class device time of the kernels launched while profiling is on
/// (0 decode GEMV, 1 GEMM, 2 LM head, 3 attention, 4 other).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct LbtProf {
    pub ms: [f64; 6],
    pub bytes: [f64; 6],
    pub launches: [u64; 6],
}

#[link(name = "lbt_hip")]
extern "C" {
    // ---- context and device memory
    pub fn lbt_ctx_create(device: c_int, out: *mut *mut LbtCtx) -> c_int;
    pub fn lbt_ctx_destroy(ctx: *mut LbtCtx);
    pub fn lbt_last_error(ctx: *const LbtCtx) -> *const c_char;
    pub fn lbt_ctx_synchronize(ctx: *mut LbtCtx) -> c_int;
    pub fn lbt_ctx_stream(ctx: *mut LbtCtx) -> *mut c_void;
    pub fn lbt_dev_alloc(ctx: *mut LbtCtx, bytes: usize, out: *mut *mut c_void) -> c_int;
    pub fn lbt_dev_free(ctx: *mut LbtCtx, p: *mut c_void) -> c_int;
    pub fn lbt_memcpy_h2d(ctx: *mut LbtCtx, dst: *mut c_void, src: *const c_void, bytes: usize) -> c_int;
    pub fn lbt_memcpy_d2h(ctx: *mut LbtCtx, dst: *mut c_void, src: *const c_void, bytes: usize) -> c_int;
    pub fn lbt_memcpy_d2d(ctx: *mut LbtCtx, dst: *mut c_void, src: *const c_void, bytes: usize) -> c_int;
    pub fn lbt_version() -> *const c_char;

    // ---- packed ternary weights (pack.rs)
    pub fn lbt_weight_upload(
        ctx: *mut LbtCtx,
        packed: *const u8,
        rows: usize,
        cols: usize,
        scale: f32,
        out: *mut *mut LbtWeight,
    ) -> c_int;
    pub fn lbt_weight_upload_dev(
        ctx: *mut LbtCtx,
        packed_dev: *const u8,
        rows: usize,
        cols: usize,
        scale: f32,
        out: *mut *mut LbtWeight,
    ) -> c_int;
    pub fn lbt_weight_free(w: *mut LbtWeight);
    pub fn lbt_weight_rows(w: *const LbtWeight) -> usize;
    pub fn lbt_weight_cols(w: *const LbtWeight) -> usize;
    pub fn lbt_weight_device_ptr(w: *const LbtWeight) -> *const u8;

    // ---- ActQuant (quant.rs)
    pub fn lbt_quantize_acts(
        ctx: *mut LbtCtx,
        x: *const f32,
        m: usize,
        k: usize,
        q: *mut i8,
        scale: *mut f32,
        sum: *mut i32,
    ) -> c_int;
    pub fn lbt_quantize_acts_dev(
        ctx: *mut LbtCtx,
        x: *const f32,
        m: usize,
        k: usize,
        q: *mut i8,
        scale: *mut f32,
        sum: *mut i32,
    ) -> c_int;
    pub fn lbt_rmsnorm_quantize_dev(
        ctx: *mut LbtCtx,
        x: *const f32,
        norm_w: *const f32,
        eps: f32,
        m: usize,
        k: usize,
        q: *mut i8,
        scale: *mut f32,
        sum: *mut i32,
    ) -> c_int;

    // ---- ternary GEMV / GEMM (gemm.rs)
    pub fn lbt_gemm_i32(
        ctx: *mut LbtCtx,
        w: *const LbtWeight,
        q: *const i8,
        sum: *const i32,
        m: usize,
        out: *mut i32,
    ) -> c_int;
    pub fn lbt_gemm_i32_dev(
        ctx: *mut LbtCtx,
        w: *const LbtWeight,
        q: *const i8,
        sum: *const i32,
        m: usize,
        out: *mut i32,
    ) -> c_int;
    pub fn lbt_gemm_multi(
        ctx: *mut LbtCtx,
        ws: *const *const LbtWeight,
        n: usize,
        q: *const i8,
        scale: *const f32,
        sum: *const i32,
        m: usize,
        outs: *const *mut f32,
    ) -> c_int;
    pub fn lbt_gemm_multi_dev(
        ctx: *mut LbtCtx,
        ws: *const *const LbtWeight,
        n: usize,
        q: *const i8,
        scale: *const f32,
        sum: *const i32,
        m: usize,
        outs: *const *mut f32,
    ) -> c_int;
    pub fn lbt_ternary_linear(
        ctx: *mut LbtCtx,
        ws: *const *const LbtWeight,
        n: usize,
        x: *const f32,
        m: usize,
        cols: usize,
        outs: *const *mut f32,
    ) -> c_int;
    pub fn lbt_ternary_linear_dev(
        ctx: *mut LbtCtx,
        ws: *const *const LbtWeight,
        n: usize,
        x: *const f32,
        m: usize,
        cols: usize,
        outs: *const *mut f32,
    ) -> c_int;
    pub fn lbt_ternary_linear_dev_noalloc(
        ctx: *mut LbtCtx,
        ws: *const *const LbtWeight,
        n: usize,
        x: *const f32,
        m: usize,
        cols: usize,
        outs: *const *mut f32,
    ) -> c_int;

    // ---- bf16 linear (bf16.rs) and the int8 head (q8head.rs)
    pub fn lbt_bf16_upload(ctx: *mut LbtCtx, w: *const u16, rows: usize, cols: usize, out: *mut *mut LbtBf16)
        -> c_int;
    pub fn lbt_bf16_free(w: *mut LbtBf16);
    pub fn lbt_bf16_linear(ctx: *mut LbtCtx, w: *const LbtBf16, x: *const f32, m: usize, out: *mut f32) -> c_int;
    pub fn lbt_bf16_linear_dev(ctx: *mut LbtCtx, w: *const LbtBf16, x: *const f32, m: usize, out: *mut f32)
        -> c_int;
    pub fn lbt_q8head_from_bf16(ctx: *mut LbtCtx, w: *const LbtBf16, out: *mut *mut LbtQ8Head) -> c_int;
    pub fn lbt_q8head_free(h: *mut LbtQ8Head);
    pub fn lbt_q8head_read(ctx: *mut LbtCtx, h: *const LbtQ8Head, q: *mut i8, scale: *mut f32) -> c_int;
    pub fn lbt_q8head_linear(ctx: *mut LbtCtx, h: *const LbtQ8Head, x: *const f32, m: usize, out: *mut f32)
        -> c_int;
    pub fn lbt_q8head_linear_dev(ctx: *mut LbtCtx, h: *const LbtQ8Head, x: *const f32, m: usize, out: *mut f32)
        -> c_int;

    // ---- sampling (sample.rs)
    pub fn lbt_sample(
        ctx: *mut LbtCtx,
        logits: *const f32,
        rows: usize,
        vocab: usize,
        p: *const LbtSampleParams,
        states: *mut u64,
        out: *mut u32,
    ) -> c_int;
    pub fn lbt_sample_dev(
        ctx: *mut LbtCtx,
        logits: *const f32,
        rows: usize,
        vocab: usize,
        p: *const LbtSampleParams,
        states: *mut u64,
        out: *mut u32,
    ) -> c_int;

    // ---- the BitNet model (model.rs)
    pub fn lbt_model_load(ctx: *mut LbtCtx, dir: *const c_char, out: *mut *mut LbtModel) -> c_int;
    pub fn lbt_model_create_synthetic(
        ctx: *mut LbtCtx,
        cfg: *const LbtConfig,
        seed: u64,
        out: *mut *mut LbtModel,
    ) -> c_int;
    pub fn lbt_model_free(m: *mut LbtModel);
    pub fn lbt_model_get_config(m: *const LbtModel, out: *mut LbtConfig) -> c_int;
    pub fn lbt_model_linear(m: *const LbtModel, layer: c_int, which: c_int) -> *const LbtWeight;
    pub fn lbt_cache_new(m: *mut LbtModel, out: *mut *mut LbtCache) -> c_int;
    pub fn lbt_cache_free(c: *mut LbtCache);
    pub fn lbt_cache_len(c: *const LbtCache) -> c_int;
    pub fn lbt_cache_read(c: *mut LbtCache, layer: c_int, is_v: c_int, out: *mut u16) -> c_int;
    pub fn lbt_model_forward(
        m: *mut LbtModel,
        tokens: *const u32,
        n: usize,
        c: *mut LbtCache,
        all_logits: c_int,
        logits: *mut f32,
    ) -> c_int;
    pub fn lbt_model_forward_argmax(m: *mut LbtModel, tokens: *const u32, n: usize, c: *mut LbtCache, next: *mut u32)
        -> c_int;
    pub fn lbt_model_generate_greedy(
        m: *mut LbtModel,
        prompt: *const u32,
        n: usize,
        steps: usize,
        c: *mut LbtCache,
        out_tokens: *mut u32,
        ms_prefill: *mut f32,
        ms_decode: *mut f32,
    ) -> c_int;
    pub fn lbt_model_decode_greedy(
        m: *mut LbtModel,
        c: *mut LbtCache,
        first: u32,
        steps: usize,
        out_tokens: *mut u32,
        ms_decode: *mut f32,
    ) -> c_int;
    pub fn lbt_model_forward_sample(
        m: *mut LbtModel,
        tokens: *const u32,
        n: usize,
        c: *mut LbtCache,
        p: *const LbtSampleParams,
        state: *mut u64,
        next: *mut u32,
    ) -> c_int;
    pub fn lbt_model_decode_sample(
        m: *mut LbtModel,
        c: *mut LbtCache,
        first: u32,
        steps: usize,
        p: *const LbtSampleParams,
        state: *mut u64,
        out_tokens: *mut u32,
        ms_decode: *mut f32,
    ) -> c_int;
    pub fn lbt_model_set_head(m: *mut LbtModel, kind: c_int) -> c_int;
    pub fn lbt_model_read_hidden(m: *mut LbtModel, out: *mut f32, n: usize) -> c_int;

    // ---- batched decode and the continuous-batching scheduler
    pub fn lbt_batch_new(m: *mut LbtModel, nseq: c_int, cap: c_int, out: *mut *mut LbtBatch) -> c_int;
    pub fn lbt_batch_free(b: *mut LbtBatch);
    pub fn lbt_batch_len(b: *const LbtBatch, seq: c_int) -> c_int;
    pub fn lbt_batch_prefill(b: *mut LbtBatch, seq: c_int, tokens: *const u32, n: usize, next: *mut u32) -> c_int;
    pub fn lbt_batch_fill_synthetic(b: *mut LbtBatch, len: c_int, seed: u64) -> c_int;
    pub fn lbt_batch_forward(b: *mut LbtBatch, tokens: *const u32, logits: *mut f32, next: *mut u32) -> c_int;
    pub fn lbt_batch_prefill_sample(
        b: *mut LbtBatch,
        seq: c_int,
        tokens: *const u32,
        n: usize,
        p: *const LbtSampleParams,
        state: *mut u64,
        next: *mut u32,
    ) -> c_int;
    pub fn lbt_batch_forward_sample(
        b: *mut LbtBatch,
        tokens: *const u32,
        params: *const LbtSampleParams,
        states: *mut u64,
        next: *mut u32,
    ) -> c_int;
    pub fn lbt_batch_decode_greedy(
        b: *mut LbtBatch,
        first: *const u32,
        steps: usize,
        out_tokens: *mut u32,
        ms_decode: *mut f32,
    ) -> c_int;
    pub fn lbt_batch_reset(b: *mut LbtBatch, seq: c_int) -> c_int;
    pub fn lbt_sched_new(m: *mut LbtModel, slots: c_int, cap: c_int, out: *mut *mut LbtSched) -> c_int;
    pub fn lbt_sched_free(s: *mut LbtSched);
    pub fn lbt_sched_submit(
        s: *mut LbtSched,
        prompt: *const u32,
        n: usize,
        max_new: usize,
        stop: u32,
        id: *mut u64,
    ) -> c_int;
    pub fn lbt_sched_submit_sample(
        s: *mut LbtSched,
        prompt: *const u32,
        n: usize,
        max_new: usize,
        stop: u32,
        p: *const LbtSampleParams,
        seed: u64,
        id: *mut u64,
    ) -> c_int;
    pub fn lbt_sched_step(s: *mut LbtSched, pending: *mut c_int) -> c_int;
    pub fn lbt_sched_result(
        s: *mut LbtSched,
        id: u64,
        tokens: *mut u32,
        cap: usize,
        n: *mut usize,
        done: *mut c_int,
    ) -> c_int;
    pub fn lbt_sched_release(s: *mut LbtSched, id: u64) -> c_int;

    // ---- profiling
    pub fn lbt_prof_enable(ctx: *mut LbtCtx, on: c_int) -> c_int;
    pub fn lbt_prof_read(ctx: *mut LbtCtx, out: *mut LbtProf, reset: c_int) -> c_int;
}
