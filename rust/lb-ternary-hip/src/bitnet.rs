//! `lb_model::BitNet` with the reference's own signatures (feature `burn`),
//! so lb-server and lb-run switch by changing one `use` line:
//!
//! * `BitNet::load(dir: &Path, device: &Device) -> anyhow::Result<BitNet>`
//!   (lb-model/src/model.rs:149); `device` is the Burn device the logits are
//!   returned on, the GPU is the process's HIP device `LBT_DEVICE` (default 0);
//! * `BitNet::new_cache(&self) -> KvCache` (model.rs:234): a cache with no
//!   capacity yet, allocated on first use like `ensure_cap`;
//! * `BitNet::forward(&self, tokens: &[u32], cache: &mut KvCache,
//!   all_logits: bool) -> Tensor<2>` (model.rs:305): logits `[m, vocab]`
//!   (all_logits) or `[1, vocab]`; a failure panics, as the reference's
//!   asserts do (context length exceeded included).
//!
//! `KvCache` keeps `len` and `cap` readable like the reference's fields.

use std::path::Path;
use std::sync::Arc;

use burn::tensor::{Device, Tensor, TensorData};

use crate::{ffi, Ctx};

struct Inner {
    ctx: Ctx,
    raw: *mut ffi::LbtModel,
}

unsafe impl Send for Inner {}
unsafe impl Sync for Inner {}

impl Drop for Inner {
    fn drop(&mut self) {
        unsafe { ffi::lbt_model_free(self.raw) }
    }
}

/// BitNet (model.rs:124-139): the model in device memory.
pub struct BitNet {
    inner: Arc<Inner>,
    device: Device,
    pub cfg: ffi::LbtConfig,
}

/// KvCache (model.rs:140-146): the per-layer K/V rows in device memory.
pub struct KvCache {
    inner: Arc<Inner>,
    raw: *mut ffi::LbtCache,
    pub len: usize,
    pub cap: usize,
}

unsafe impl Send for KvCache {}

impl Drop for KvCache {
    fn drop(&mut self) {
        if !self.raw.is_null() {
            unsafe { ffi::lbt_cache_free(self.raw) }
        }
    }
}

impl BitNet {
    pub fn load(dir: &Path, device: &Device) -> anyhow::Result<Self> {
        let gpu = std::env::var("LBT_DEVICE").ok().and_then(|v| v.parse().ok()).unwrap_or(0);
        let ctx = Ctx::new(gpu).map_err(anyhow::Error::msg)?;
        let cdir = std::ffi::CString::new(dir.to_string_lossy().as_bytes())?;
        let mut raw = std::ptr::null_mut();
        ctx.check(unsafe { ffi::lbt_model_load(ctx.raw(), cdir.as_ptr(), &mut raw) }).map_err(anyhow::Error::msg)?;
        let mut cfg = ffi::LbtConfig::default();
        ctx.check(unsafe { ffi::lbt_model_get_config(raw, &mut cfg) }).map_err(anyhow::Error::msg)?;
        Ok(Self { inner: Arc::new(Inner { ctx, raw }), device: device.clone(), cfg })
    }

    pub fn new_cache(&self) -> KvCache {
        KvCache { inner: self.inner.clone(), raw: std::ptr::null_mut(), len: 0, cap: 0 }
    }

    pub fn forward(&self, tokens: &[u32], cache: &mut KvCache, all_logits: bool) -> Tensor<2> {
        let ctx = &self.inner.ctx;
        assert!(Arc::ptr_eq(&self.inner, &cache.inner), "cache of another model");
        if cache.raw.is_null() {
            let mut raw = std::ptr::null_mut();
            ctx.check(unsafe { ffi::lbt_cache_new(self.inner.raw, &mut raw) }).expect("KV cache");
            cache.raw = raw;
        }
        let vocab = self.cfg.vocab_size as usize;
        let rows = if all_logits { tokens.len() } else { 1 };
        let mut out = vec![0.0f32; rows * vocab];
        ctx.check(unsafe {
            ffi::lbt_model_forward(self.inner.raw, tokens.as_ptr(), tokens.len(), cache.raw, all_logits as i32,
                                   out.as_mut_ptr())
        })
        .unwrap_or_else(|e| panic!("{e}"));
        cache.len = unsafe { ffi::lbt_cache_len(cache.raw) } as usize;
        cache.cap = cache.cap.max(cache.len.next_power_of_two().max(256).min(self.cfg.max_position_embeddings as usize));
        Tensor::from_data(TensorData::new(out, [rows, vocab]), &self.device)
    }
}
