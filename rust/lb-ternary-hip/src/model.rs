//! `BitNet` (lb-model/src/model.rs:124-374) with every layer, the KV cache,
//! the LM head and the token choice on the MI355X.

use std::ffi::CString;
use std::marker::PhantomData;
use std::os::raw::c_int;
use std::path::Path;

use crate::{ffi, Ctx, Result};

/// SamplingParams (lb-model/src/sample.rs:3-15).
#[derive(Debug, Clone)]
pub struct SamplingParams {
    pub temperature: f32,
    pub top_p: f32,
    pub top_k: usize,
    pub seed: u64,
}

impl Default for SamplingParams {
    fn default() -> Self {
        Self { temperature: 0.0, top_p: 1.0, top_k: 0, seed: 0x5eed }
    }
}

impl SamplingParams {
    pub(crate) fn ffi(&self) -> ffi::LbtSampleParams {
        ffi::LbtSampleParams { temperature: self.temperature, top_p: self.top_p, top_k: self.top_k }
    }
}

/// Sampler (sample.rs:28-43): the parameters and the xorshift64 state
/// (seed.max(1) at the start of a job); the draws happen on the device.
pub struct Sampler {
    pub p: SamplingParams,
    pub state: u64,
}

impl Sampler {
    pub fn new(p: SamplingParams) -> Self {
        let state = p.seed.max(1);
        Self { p, state }
    }
}

/// A loaded model and its device context.
pub struct HipBitNet {
    ctx: Ctx,
    raw: *mut ffi::LbtModel,
    pub cfg: ffi::LbtConfig,
}

unsafe impl Send for HipBitNet {}

/// KvCache (model.rs:140-146) in device memory; grows like ensure_cap.  It
/// borrows its model, which must outlive it.
pub struct HipCache<'m> {
    raw: *mut ffi::LbtCache,
    _m: PhantomData<&'m HipBitNet>,
}

impl HipCache<'_> {
    pub fn len(&self) -> usize {
        unsafe { ffi::lbt_cache_len(self.raw) as usize }
    }
    pub fn is_empty(&self) -> bool {
        self.len() == 0
    }
}

impl Drop for HipCache<'_> {
    fn drop(&mut self) {
        unsafe { ffi::lbt_cache_free(self.raw) }
    }
}

impl HipBitNet {
    /// BitNet::load (model.rs:149-232): DIR/config.json and the lb-convert
    /// file DIR/model.lbt.safetensors, read unchanged.
    pub fn load(dir: &Path, device: i32) -> Result<Self> {
        let ctx = Ctx::new(device)?;
        let cdir = CString::new(dir.to_string_lossy().as_bytes()).map_err(|e| e.to_string())?;
        let mut raw = std::ptr::null_mut();
        ctx.check(unsafe { ffi::lbt_model_load(ctx.raw(), cdir.as_ptr(), &mut raw) })?;
        let mut cfg = ffi::LbtConfig::default();
        ctx.check(unsafe { ffi::lbt_model_get_config(raw, &mut cfg) })?;
        Ok(Self { ctx, raw, cfg })
    }

    pub fn ctx(&self) -> &Ctx {
        &self.ctx
    }

    /// BitNet::new_cache (model.rs:234-236).
    pub fn new_cache(&self) -> Result<HipCache<'_>> {
        let mut raw = std::ptr::null_mut();
        self.ctx.check(unsafe { ffi::lbt_cache_new(self.raw, &mut raw) })?;
        Ok(HipCache { raw, _m: PhantomData })
    }

    /// BitNet::forward (model.rs:305-374): logits `[all_logits ? n : 1, vocab]`
    /// row-major (the reference returns them as a Tensor<2>).
    pub fn forward(&self, tokens: &[u32], cache: &mut HipCache<'_>, all_logits: bool) -> Result<Vec<f32>> {
        let rows = if all_logits { tokens.len() } else { 1 };
        let mut out = vec![0.0f32; rows * self.cfg.vocab_size as usize];
        self.ctx.check(unsafe {
            ffi::lbt_model_forward(self.raw, tokens.as_ptr(), tokens.len(), cache.raw, all_logits as c_int,
                                   out.as_mut_ptr())
        })?;
        Ok(out)
    }

    /// forward + argmax (sample.rs:17-25) on the device; only the id returns.
    pub fn forward_argmax(&self, tokens: &[u32], cache: &mut HipCache<'_>) -> Result<u32> {
        let mut next = 0u32;
        self.ctx.check(unsafe {
            ffi::lbt_model_forward_argmax(self.raw, tokens.as_ptr(), tokens.len(), cache.raw, &mut next)
        })?;
        Ok(next)
    }

    /// `steps` greedy tokens after `first` (the server's decode loop,
    /// main.rs:141-160, at temperature 0), each fed back on the device.
    pub fn decode_greedy(&self, cache: &mut HipCache<'_>, first: u32, steps: usize) -> Result<Vec<u32>> {
        let mut out = vec![0u32; steps];
        self.ctx.check(unsafe {
            ffi::lbt_model_decode_greedy(self.raw, cache.raw, first, steps, out.as_mut_ptr(), std::ptr::null_mut())
        })?;
        Ok(out)
    }

    /// The prompt, then the first token drawn by `sampler` (main.rs:102-109).
    pub fn forward_sample(&self, tokens: &[u32], cache: &mut HipCache<'_>, sampler: &mut Sampler) -> Result<u32> {
        let p = sampler.p.ffi();
        let mut next = 0u32;
        self.ctx.check(unsafe {
            ffi::lbt_model_forward_sample(self.raw, tokens.as_ptr(), tokens.len(), cache.raw, &p, &mut sampler.state,
                                          &mut next)
        })?;
        Ok(next)
    }

    /// `steps` sampled tokens after `first` (main.rs:141-160), on the device.
    pub fn decode_sample(&self, cache: &mut HipCache<'_>, first: u32, steps: usize, sampler: &mut Sampler)
        -> Result<Vec<u32>> {
        let p = sampler.p.ffi();
        let mut out = vec![0u32; steps];
        self.ctx.check(unsafe {
            ffi::lbt_model_decode_sample(self.raw, cache.raw, first, steps, &p, &mut sampler.state, out.as_mut_ptr(),
                                         std::ptr::null_mut())
        })?;
        Ok(out)
    }

    /// 0: the exact bf16 tied head; 1: the opt-in int8 head (q8head.rs).
    pub fn set_head(&self, kind: i32) -> Result<()> {
        self.ctx.check(unsafe { ffi::lbt_model_set_head(self.raw, kind as c_int) })
    }
}

impl Drop for HipBitNet {
    fn drop(&mut self) {
        unsafe { ffi::lbt_model_free(self.raw) }
    }
}
