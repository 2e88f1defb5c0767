//! lb-ternary-hip: lemonade-burn's W1.58A8 kernels and BitNet b1.58 token
//! loop on an AMD MI355X, through liblbt_hip's C ABI (`ffi`).
//!
//! The safe layer keeps lb-ternary's types and entry points:
//! * [`Ctx::upload`] takes a [`TernaryView`] (the LB2 bytes of pack.rs,
//!   unchanged) and keeps the matrix in device memory;
//! * [`Ctx::quantize_acts`] fills a [`QuantActs`] exactly as
//!   `lb_ternary::quantize_acts` does (quant.rs:37-75);
//! * [`ternary_gemm_i32`], [`ternary_gemm`] and [`ternary_gemm_multi`] have the
//!   signatures of gemm.rs:95-195 with a device matrix in place of the view and
//!   no `Kernel` (the device picks its kernel by token count);
//! * [`TernaryOps`] is the slice-level form of `TernaryBackend`
//!   (lb-model/src/ops.rs:20-77): quantize inside the op, one fused product for
//!   the 1-3 matrices sharing an input, the bf16 linear of the tied head;
//! * [`model::HipBitNet`] is `BitNet::{load, new_cache, forward}`
//!   (model.rs:149-374) with the whole token loop on the device, plus the
//!   device-side greedy and sampling loops of the server (main.rs:102-160);
//! * with the `burn` feature, [`bitnet::BitNet`] / [`bitnet::KvCache`] carry
//!   the reference's exact signatures (`load(&Path, &Device)`,
//!   `new_cache() -> KvCache`, `forward(..) -> Tensor<2>`), so lb-server and
//!   lb-run switch by one `use` line.
//!
//! Errors are `Err(String)` with the library's message (the reference's CPU
//! kernels assert; its CubeCL crate returned `Result<_, String>`).

#[cfg(feature = "burn")]
pub mod bitnet;
pub mod ffi;
pub mod model;

use std::ffi::CStr;
use std::os::raw::c_int;

pub use lb_ternary::{QuantActs, TernaryView};
pub use model::{HipBitNet, HipCache, Sampler, SamplingParams};

pub type Result<T> = std::result::Result<T, String>;

/// One device context: a HIP stream on one GPU and the library's workspaces.
/// Used from one thread at a time (one per model worker, as the server's
/// worker loop runs, lb-server/src/main.rs:92-100).
pub struct Ctx {
    raw: *mut ffi::LbtCtx,
}

unsafe impl Send for Ctx {}

impl Ctx {
    pub fn new(device: i32) -> Result<Ctx> {
        let mut raw = std::ptr::null_mut();
        let rc = unsafe { ffi::lbt_ctx_create(device as c_int, &mut raw) };
        if rc != ffi::LBT_OK {
            return Err(format!("lbt_ctx_create({device}) failed with status {rc}"));
        }
        Ok(Ctx { raw })
    }

    pub fn raw(&self) -> *mut ffi::LbtCtx {
        self.raw
    }

    /// Status code -> Result with the library's last message.
    pub fn check(&self, rc: c_int) -> Result<()> {
        if rc == ffi::LBT_OK {
            return Ok(());
        }
        let msg = unsafe { CStr::from_ptr(ffi::lbt_last_error(self.raw)) };
        Err(format!("lbt status {rc}: {}", msg.to_string_lossy()))
    }

    pub fn synchronize(&self) -> Result<()> {
        self.check(unsafe { ffi::lbt_ctx_synchronize(self.raw) })
    }

    /// `PackedTernary::view()` bytes to the device, once (at model load).
    pub fn upload(&self, w: TernaryView<'_>) -> Result<HipTernary<'_>> {
        let mut raw = std::ptr::null_mut();
        self.check(unsafe { ffi::lbt_weight_upload(self.raw, w.data.as_ptr(), w.rows, w.cols, w.scale, &mut raw) })?;
        Ok(HipTernary { ctx: self, raw, rows: w.rows, cols: w.cols, scale: w.scale })
    }

    /// `quantize_acts` (quant.rs:37-75) on the device: the same q, scale, sum.
    pub fn quantize_acts(&self, x: &[f32], m: usize, k: usize) -> Result<QuantActs> {
        assert_eq!(x.len(), m * k);
        let kp = lb_ternary::pack::padded_cols(k);
        let mut out = QuantActs { m, k, kp, q: vec![0; m * kp], scale: vec![0.0; m], sum: vec![0; m] };
        self.check(unsafe {
            ffi::lbt_quantize_acts(self.raw, x.as_ptr(), m, k, out.q.as_mut_ptr(), out.scale.as_mut_ptr(),
                                   out.sum.as_mut_ptr())
        })?;
        Ok(out)
    }

    /// The tied bf16 LM head matrix (`[rows, cols]` bf16 bits) to the device.
    pub fn upload_bf16(&self, w: &[u16], rows: usize, cols: usize) -> Result<HipBf16<'_>> {
        assert_eq!(w.len(), rows * cols);
        let mut raw = std::ptr::null_mut();
        self.check(unsafe { ffi::lbt_bf16_upload(self.raw, w.as_ptr(), rows, cols, &mut raw) })?;
        Ok(HipBf16 { ctx: self, raw, rows, cols })
    }

    /// `Sampler::sample` (sample.rs:45-82) for rows of host logits, on the
    /// device; `states` are the samplers' states (one per row), advanced.
    pub fn sample(&self, logits: &[f32], vocab: usize, p: &SamplingParams, states: &mut [u64]) -> Result<Vec<u32>> {
        let rows = states.len();
        assert_eq!(logits.len(), rows * vocab);
        let mut out = vec![0u32; rows];
        let fp = p.ffi();
        self.check(unsafe {
            ffi::lbt_sample(self.raw, logits.as_ptr(), rows, vocab, &fp, states.as_mut_ptr(), out.as_mut_ptr())
        })?;
        Ok(out)
    }
}

impl Drop for Ctx {
    fn drop(&mut self) {
        unsafe { ffi::lbt_ctx_destroy(self.raw) }
    }
}

/// A packed ternary matrix in device memory (the device twin of
/// `PackedTernary`, pack.rs:60-80).
pub struct HipTernary<'c> {
    ctx: &'c Ctx,
    raw: *mut ffi::LbtWeight,
    pub rows: usize,
    pub cols: usize,
    pub scale: f32,
}

impl HipTernary<'_> {
    pub fn raw(&self) -> *const ffi::LbtWeight {
        self.raw
    }
}

impl Drop for HipTernary<'_> {
    fn drop(&mut self) {
        unsafe { ffi::lbt_weight_free(self.raw) }
    }
}

/// A bf16 matrix in device memory (the tied LM head, bf16.rs).
pub struct HipBf16<'c> {
    ctx: &'c Ctx,
    raw: *mut ffi::LbtBf16,
    pub rows: usize,
    pub cols: usize,
}

impl Drop for HipBf16<'_> {
    fn drop(&mut self) {
        unsafe { ffi::lbt_bf16_free(self.raw) }
    }
}

/// `ternary_gemm_i32` (gemm.rs:95-114): `out[t * rows + r]` = the exact dot of
/// row r with token t.
pub fn ternary_gemm_i32(w: &HipTernary<'_>, x: &QuantActs) -> Result<Vec<i32>> {
    assert_eq!(x.k, w.cols, "inner dimension mismatch");
    let mut out = vec![0i32; x.m * w.rows];
    w.ctx.check(unsafe {
        ffi::lbt_gemm_i32(w.ctx.raw, w.raw, x.q.as_ptr(), x.sum.as_ptr(), x.m, out.as_mut_ptr())
    })?;
    Ok(out)
}

/// `ternary_gemm` (gemm.rs:117-119): f32 out = dot * (1 / (s_a * s_w)).
pub fn ternary_gemm(w: &HipTernary<'_>, x: &QuantActs, out: &mut [f32]) -> Result<()> {
    ternary_gemm_multi(&[w], x, &mut [out])
}

/// `ternary_gemm_multi` (gemm.rs:128-195): 1-3 matrices sharing the
/// activations, in one device dispatch; each output equals the single call's.
pub fn ternary_gemm_multi(ws: &[&HipTernary<'_>], x: &QuantActs, outs: &mut [&mut [f32]]) -> Result<()> {
    assert!(!ws.is_empty() && ws.len() <= 3 && ws.len() == outs.len());
    let ctx = ws[0].ctx;
    for (w, o) in ws.iter().zip(outs.iter()) {
        assert_eq!(w.cols, x.k, "inner dimension mismatch");
        assert_eq!(o.len(), x.m * w.rows);
    }
    let raws: Vec<*const ffi::LbtWeight> = ws.iter().map(|w| w.raw as *const _).collect();
    let ptrs: Vec<*mut f32> = outs.iter_mut().map(|o| o.as_mut_ptr()).collect();
    ctx.check(unsafe {
        ffi::lbt_gemm_multi(ctx.raw, raws.as_ptr(), ws.len(), x.q.as_ptr(), x.scale.as_ptr(), x.sum.as_ptr(), x.m,
                            ptrs.as_ptr())
    })
}

/// The slice-level form of `TernaryBackend` (lb-model/src/ops.rs:20-77) on
/// the device: `x` is `[m, cols]` f32, quantized inside the op (ActQuant);
/// the 2- and 3-matrix forms quantize once and run one fused product whose
/// outputs equal the single-matrix op's bit for bit (ops.rs:301-329).
pub trait TernaryOps {
    fn ternary_linear(&self, x: &[f32], m: usize, w: &HipTernary<'_>) -> Result<Vec<f32>>;
    fn ternary_linear2(&self, x: &[f32], m: usize, w: [&HipTernary<'_>; 2]) -> Result<[Vec<f32>; 2]>;
    fn ternary_linear3(&self, x: &[f32], m: usize, w: [&HipTernary<'_>; 3]) -> Result<[Vec<f32>; 3]>;
    /// `bf16_linear` (ops.rs:75-76, :199-218): `x[m, k] @ W^T`, f32 accumulation.
    fn bf16_linear(&self, x: &[f32], m: usize, w: &HipBf16<'_>) -> Result<Vec<f32>>;
}

impl Ctx {
    fn linear_n(&self, x: &[f32], m: usize, ws: &[&HipTernary<'_>]) -> Result<Vec<Vec<f32>>> {
        let cols = ws[0].cols;
        assert_eq!(x.len(), m * cols);
        let mut outs: Vec<Vec<f32>> = ws.iter().map(|w| vec![0.0f32; m * w.rows]).collect();
        let raws: Vec<*const ffi::LbtWeight> = ws.iter().map(|w| w.raw as *const _).collect();
        let ptrs: Vec<*mut f32> = outs.iter_mut().map(|o| o.as_mut_ptr()).collect();
        self.check(unsafe {
            ffi::lbt_ternary_linear(self.raw, raws.as_ptr(), ws.len(), x.as_ptr(), m, cols, ptrs.as_ptr())
        })?;
        Ok(outs)
    }
}

impl TernaryOps for Ctx {
    fn ternary_linear(&self, x: &[f32], m: usize, w: &HipTernary<'_>) -> Result<Vec<f32>> {
        Ok(self.linear_n(x, m, &[w])?.remove(0))
    }
    fn ternary_linear2(&self, x: &[f32], m: usize, w: [&HipTernary<'_>; 2]) -> Result<[Vec<f32>; 2]> {
        let mut o = self.linear_n(x, m, &w)?;
        let b = o.pop().unwrap();
        let a = o.pop().unwrap();
        Ok([a, b])
    }
    fn ternary_linear3(&self, x: &[f32], m: usize, w: [&HipTernary<'_>; 3]) -> Result<[Vec<f32>; 3]> {
        let mut o = self.linear_n(x, m, &w)?;
        let c = o.pop().unwrap();
        let b = o.pop().unwrap();
        let a = o.pop().unwrap();
        Ok([a, b, c])
    }
    fn bf16_linear(&self, x: &[f32], m: usize, w: &HipBf16<'_>) -> Result<Vec<f32>> {
        assert_eq!(x.len(), m * w.cols);
        let mut out = vec![0.0f32; m * w.rows];
        self.check(unsafe { ffi::lbt_bf16_linear(self.raw, w.raw, x.as_ptr(), m, out.as_mut_ptr()) })?;
        Ok(out)
    }
}
