"""ctypes binding of liblbt_hip.so (include/lbt.h) for Python callers.

This is the Python mirror of the reference's `lb-ternary` / `lb-model`
entry points (quantize_acts, ternary_gemm_i32, ternary_gemm_multi,
ternary_linear{,2,3}, bf16_linear, BitNet::load/new_cache/forward) over the
C ABI.  It loads the in-tree HIP library and raises if it is missing: there is
no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "liblbt_hip.so"

LBT_OK = 0
ERRORS = {-1: "LBT_E_INVALID", -2: "LBT_E_DEVICE", -3: "LBT_E_NOMEM", -4: "LBT_E_IO", -5: "LBT_E_RANGE"}

# Every exported entry point and its (restype, argtypes); test_abi checks that
# this list equals the declarations of include/lbt.h.
vp = C.c_void_p
sz = C.c_size_t
i32 = C.c_int
f32 = C.c_float
u64 = C.c_uint64


class LbtSampleParams(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("top_k", C.c_size_t)]


class LbtConfig(C.Structure):
    _fields_ = [
        ("hidden_size", C.c_int32),
        ("intermediate_size", C.c_int32),
        ("num_attention_heads", C.c_int32),
        ("num_key_value_heads", C.c_int32),
        ("num_hidden_layers", C.c_int32),
        ("vocab_size", C.c_int32),
        ("max_position_embeddings", C.c_int32),
        ("bos_token_id", C.c_uint32),
        ("rms_norm_eps", C.c_double),
        ("rope_theta", C.c_double),
    ]


class LbtProf(C.Structure):
    _fields_ = [("ms", C.c_double * 6), ("bytes", C.c_double * 6), ("launches", C.c_uint64 * 6)]


SIGNATURES = {
    "lbt_ctx_create": (i32, [i32, C.POINTER(vp)]),
    "lbt_ctx_destroy": (None, [vp]),
    "lbt_last_error": (C.c_char_p, [vp]),
    "lbt_ctx_synchronize": (i32, [vp]),
    "lbt_ctx_stream": (vp, [vp]),
    "lbt_dev_alloc": (i32, [vp, sz, C.POINTER(vp)]),
    "lbt_dev_free": (i32, [vp, vp]),
    "lbt_memcpy_h2d": (i32, [vp, vp, vp, sz]),
    "lbt_memcpy_d2h": (i32, [vp, vp, vp, sz]),
    "lbt_memcpy_d2d": (i32, [vp, vp, vp, sz]),
    "lbt_version": (C.c_char_p, []),
    "lbt_weight_upload": (i32, [vp, vp, sz, sz, f32, C.POINTER(vp)]),
    "lbt_weight_upload_dev": (i32, [vp, vp, sz, sz, f32, C.POINTER(vp)]),
    "lbt_weight_free": (None, [vp]),
    "lbt_weight_rows": (sz, [vp]),
    "lbt_weight_cols": (sz, [vp]),
    "lbt_weight_device_ptr": (vp, [vp]),
    "lbt_quantize_acts": (i32, [vp, vp, sz, sz, vp, vp, vp]),
    "lbt_quantize_acts_dev": (i32, [vp, vp, sz, sz, vp, vp, vp]),
    "lbt_rmsnorm_quantize_dev": (i32, [vp, vp, vp, f32, sz, sz, vp, vp, vp]),
    "lbt_gemm_i32": (i32, [vp, vp, vp, vp, sz, vp]),
    "lbt_gemm_i32_dev": (i32, [vp, vp, vp, vp, sz, vp]),
    "lbt_gemm_multi": (i32, [vp, vp, sz, vp, vp, vp, sz, vp]),
    "lbt_gemm_multi_dev": (i32, [vp, vp, sz, vp, vp, vp, sz, vp]),
    "lbt_ternary_linear": (i32, [vp, vp, sz, vp, sz, sz, vp]),
    "lbt_ternary_linear_dev": (i32, [vp, vp, sz, vp, sz, sz, vp]),
    "lbt_ternary_linear_dev_noalloc": (i32, [vp, vp, sz, vp, sz, sz, vp]),
    "lbt_bf16_upload": (i32, [vp, vp, sz, sz, C.POINTER(vp)]),
    "lbt_bf16_free": (None, [vp]),
    "lbt_bf16_linear": (i32, [vp, vp, vp, sz, vp]),
    "lbt_bf16_linear_dev": (i32, [vp, vp, vp, sz, vp]),
    "lbt_q8head_from_bf16": (i32, [vp, vp, C.POINTER(vp)]),
    "lbt_q8head_free": (None, [vp]),
    "lbt_q8head_read": (i32, [vp, vp, vp, vp]),
    "lbt_q8head_linear": (i32, [vp, vp, vp, sz, vp]),
    "lbt_q8head_linear_dev": (i32, [vp, vp, vp, sz, vp]),
    "lbt_model_load": (i32, [vp, C.c_char_p, C.POINTER(vp)]),
    "lbt_model_create_synthetic": (i32, [vp, C.POINTER(LbtConfig), u64, C.POINTER(vp)]),
    "lbt_model_free": (None, [vp]),
    "lbt_model_get_config": (i32, [vp, C.POINTER(LbtConfig)]),
    "lbt_model_linear": (vp, [vp, i32, i32]),
    "lbt_cache_new": (i32, [vp, C.POINTER(vp)]),
    "lbt_cache_free": (None, [vp]),
    "lbt_cache_len": (i32, [vp]),
    "lbt_cache_read": (i32, [vp, i32, i32, vp]),
    "lbt_model_forward": (i32, [vp, vp, sz, vp, i32, vp]),
    "lbt_model_forward_argmax": (i32, [vp, vp, sz, vp, vp]),
    "lbt_model_generate_greedy": (i32, [vp, vp, sz, sz, vp, vp, vp, vp]),
    "lbt_model_decode_greedy": (i32, [vp, vp, C.c_uint32, sz, vp, vp]),
    "lbt_model_forward_sample": (i32, [vp, vp, sz, vp, vp, vp, vp]),
    "lbt_model_decode_sample": (i32, [vp, vp, C.c_uint32, sz, vp, vp, vp, vp]),
    "lbt_sample": (i32, [vp, vp, sz, sz, vp, vp, vp]),
    "lbt_sample_dev": (i32, [vp, vp, sz, sz, vp, vp, vp]),
    "lbt_model_read_hidden": (i32, [vp, vp, sz]),
    "lbt_model_set_head": (i32, [vp, i32]),
    "lbt_batch_new": (i32, [vp, i32, i32, C.POINTER(vp)]),
    "lbt_batch_free": (None, [vp]),
    "lbt_batch_len": (i32, [vp, i32]),
    "lbt_batch_prefill": (i32, [vp, i32, vp, sz, vp]),
    "lbt_batch_fill_synthetic": (i32, [vp, i32, C.c_uint64]),
    "lbt_batch_forward": (i32, [vp, vp, vp, vp]),
    "lbt_batch_prefill_sample": (i32, [vp, i32, vp, sz, vp, vp, vp]),
    "lbt_batch_forward_sample": (i32, [vp, vp, vp, vp, vp]),
    "lbt_batch_decode_greedy": (i32, [vp, vp, sz, vp, vp]),
    "lbt_batch_reset": (i32, [vp, i32]),
    "lbt_sched_new": (i32, [vp, i32, i32, C.POINTER(vp)]),
    "lbt_sched_free": (None, [vp]),
    "lbt_sched_submit": (i32, [vp, vp, sz, sz, C.c_uint32, C.POINTER(C.c_uint64)]),
    "lbt_sched_submit_sample": (i32, [vp, vp, sz, sz, C.c_uint32, vp, C.c_uint64, C.POINTER(C.c_uint64)]),
    "lbt_sched_step": (i32, [vp, C.POINTER(i32)]),
    "lbt_sched_result": (i32, [vp, C.c_uint64, vp, sz, C.POINTER(sz), C.POINTER(i32)]),
    "lbt_sched_release": (i32, [vp, C.c_uint64]),
    "lbt_prof_enable": (i32, [vp, i32]),
    "lbt_prof_read": (i32, [vp, C.POINTER(LbtProf), i32]),
}

_lib = None


def load_library(path: str | os.PathLike | None = None) -> C.CDLL:
    """Loads the HIP library; raises FileNotFoundError if it was not built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else Path(os.environ.get("LBT_LIB", LIB_PATH))
    if not p.exists():
        raise FileNotFoundError(f"{p} is missing: build it with __graft_entry__.build() (no CPU fallback exists)")
    lib = C.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


class LbtError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{ERRORS.get(code, code)}: {msg}")
        self.code = code


def _ptr(a: np.ndarray) -> C.c_void_p:
    assert a.flags["C_CONTIGUOUS"], "arrays passed to the C ABI must be contiguous"
    return C.c_void_p(a.ctypes.data)


def padded_cols(cols: int) -> int:
    return (cols + 127) // 128 * 128


class Ctx:
    """One device context (stream + workspace); lbt_ctx_create/destroy."""

    def __init__(self, device: int = 0):
        self.lib = load_library()
        h = C.c_void_p()
        rc = self.lib.lbt_ctx_create(device, C.byref(h))
        if rc != LBT_OK:
            raise LbtError(rc, f"lbt_ctx_create({device}) failed")
        self.h = h

    def check(self, rc: int):
        if rc != LBT_OK:
            raise LbtError(rc, self.lib.lbt_last_error(self.h).decode())

    def close(self):
        if self.h:
            self.lib.lbt_ctx_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def sync(self):
        self.check(self.lib.lbt_ctx_synchronize(self.h))

    # ---- weights -----------------------------------------------------------
    def upload(self, packed: np.ndarray, rows: int, cols: int, scale: float) -> "Weight":
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        h = C.c_void_p()
        self.check(self.lib.lbt_weight_upload(self.h, _ptr(packed), rows, cols, C.c_float(scale), C.byref(h)))
        return Weight(self, h, rows, cols, scale)

    # ---- ops ------------------------------------------------------------------
    def quantize_acts(self, x: np.ndarray):
        x = np.ascontiguousarray(x, dtype=np.float32)
        m, k = x.shape
        kp = padded_cols(k)
        q = np.zeros((m, kp), np.int8)
        s = np.zeros(m, np.float32)
        su = np.zeros(m, np.int32)
        self.check(self.lib.lbt_quantize_acts(self.h, _ptr(x), m, k, _ptr(q), _ptr(s), _ptr(su)))
        return q, s, su

    def gemm_i32(self, w: "Weight", q: np.ndarray, qsum: np.ndarray) -> np.ndarray:
        q = np.ascontiguousarray(q, dtype=np.int8)
        qsum = np.ascontiguousarray(qsum, dtype=np.int32)
        m = q.shape[0]
        out = np.zeros((m, w.rows), np.int32)
        self.check(self.lib.lbt_gemm_i32(self.h, w.h, _ptr(q), _ptr(qsum), m, _ptr(out)))
        return out

    def gemm_multi(self, ws: list["Weight"], q, scale, qsum) -> list[np.ndarray]:
        q = np.ascontiguousarray(q, dtype=np.int8)
        scale = np.ascontiguousarray(scale, dtype=np.float32)
        qsum = np.ascontiguousarray(qsum, dtype=np.int32)
        m = q.shape[0]
        outs = [np.zeros((m, w.rows), np.float32) for w in ws]
        wa = (C.c_void_p * len(ws))(*[w.h for w in ws])
        oa = (C.c_void_p * len(ws))(*[o.ctypes.data for o in outs])
        self.check(self.lib.lbt_gemm_multi(self.h, wa, len(ws), _ptr(q), _ptr(scale), _ptr(qsum), m, oa))
        return outs

    def sample(self, logits: np.ndarray, temperature: float, top_p: float, top_k: int, states: np.ndarray) -> np.ndarray:
        """Sampler::sample on the device for each row of `logits`; `states`
        (uint64 per row) is updated in place."""
        lg = np.ascontiguousarray(logits, dtype=np.float32)
        if lg.ndim == 1:
            lg = lg[None]
        assert states.dtype == np.uint64 and states.flags.c_contiguous and states.size == lg.shape[0]
        out = np.zeros(lg.shape[0], np.uint32)
        p = LbtSampleParams(temperature, top_p, top_k)
        self.check(self.lib.lbt_sample(self.h, _ptr(lg), lg.shape[0], lg.shape[1], C.byref(p), _ptr(states), _ptr(out)))
        return out

    def ternary_linear(self, ws: list["Weight"], x: np.ndarray) -> list[np.ndarray]:
        x = np.ascontiguousarray(x, dtype=np.float32)
        m, cols = x.shape
        outs = [np.zeros((m, w.rows), np.float32) for w in ws]
        wa = (C.c_void_p * len(ws))(*[w.h for w in ws])
        oa = (C.c_void_p * len(ws))(*[o.ctypes.data for o in outs])
        self.check(self.lib.lbt_ternary_linear(self.h, wa, len(ws), _ptr(x), m, cols, oa))
        return outs

    def bf16_upload(self, w: np.ndarray) -> "Bf16Weight":
        w = np.ascontiguousarray(w, dtype=np.uint16)
        rows, cols = w.shape
        h = C.c_void_p()
        self.check(self.lib.lbt_bf16_upload(self.h, _ptr(w), rows, cols, C.byref(h)))
        return Bf16Weight(self, h, rows, cols)

    def bf16_linear(self, w: "Bf16Weight", x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        m = x.shape[0]
        out = np.zeros((m, w.rows), np.float32)
        self.check(self.lib.lbt_bf16_linear(self.h, w.h, _ptr(x), m, _ptr(out)))
        return out

    def q8head_from_bf16(self, w: "Bf16Weight") -> "Q8Head":
        h = C.c_void_p()
        self.check(self.lib.lbt_q8head_from_bf16(self.h, w.h, C.byref(h)))
        return Q8Head(self, h, w.rows, w.cols)

    def q8head_linear(self, h: "Q8Head", x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        m = x.shape[0]
        out = np.zeros((m, h.rows), np.float32)
        self.check(self.lib.lbt_q8head_linear(self.h, h.h, _ptr(x), m, _ptr(out)))
        return out

    # ---- profiling ---------------------------------------------------------------
    def prof_enable(self, on: bool):
        self.check(self.lib.lbt_prof_enable(self.h, 1 if on else 0))

    def prof_read(self, reset: bool = True) -> dict:
        p = LbtProf()
        self.check(self.lib.lbt_prof_read(self.h, C.byref(p), 1 if reset else 0))
        names = ["gemv", "gemm", "head", "attn", "other", "step"]
        return {n: {"ms": p.ms[i], "bytes": p.bytes[i], "launches": int(p.launches[i])} for i, n in enumerate(names)}


class Weight:
    def __init__(self, ctx: Ctx, h, rows, cols, scale):
        self.ctx, self.h, self.rows, self.cols, self.scale = ctx, h, rows, cols, scale

    def free(self):
        if self.h:
            self.ctx.lib.lbt_weight_free(self.h)
            self.h = None

    def __del__(self):
        try:
            if self.ctx.h:
                self.free()
        except Exception:
            pass


class Bf16Weight:
    def __init__(self, ctx: Ctx, h, rows, cols):
        self.ctx, self.h, self.rows, self.cols = ctx, h, rows, cols

    def free(self):
        if self.h:
            self.ctx.lib.lbt_bf16_free(self.h)
            self.h = None

    def __del__(self):
        try:
            if self.ctx.h:
                self.free()
        except Exception:
            pass


class Q8Head:
    """Q8Head (q8head.rs:9-15) on the device."""

    def __init__(self, ctx: Ctx, h, rows, cols):
        self.ctx, self.h, self.rows, self.cols = ctx, h, rows, cols

    def read(self):
        q = np.zeros((self.rows, self.cols), np.int8)
        s = np.zeros(self.rows, np.float32)
        self.ctx.check(self.ctx.lib.lbt_q8head_read(self.ctx.h, self.h, _ptr(q), _ptr(s)))
        return q, s

    def free(self):
        if self.h:
            self.ctx.lib.lbt_q8head_free(self.h)
            self.h = None

    def __del__(self):
        try:
            if self.ctx.h:
                self.free()
        except Exception:
            pass


def make_config(hidden=2560, intermediate=6912, heads=20, kv_heads=5, layers=30, vocab=128256, max_pos=4096,
                eps=1e-5, theta=500000.0, bos=128000) -> LbtConfig:
    """BitNet b1.58 2B4T shape by default."""
    return LbtConfig(hidden, intermediate, heads, kv_heads, layers, vocab, max_pos, bos, eps, theta)


class Model:
    """BitNet::load / synthetic creation + new_cache + forward over the C ABI."""

    def __init__(self, ctx: Ctx, handle):
        self.ctx, self.h = ctx, handle
        self.cfg = LbtConfig()
        ctx.check(ctx.lib.lbt_model_get_config(handle, C.byref(self.cfg)))

    @classmethod
    def synthetic(cls, ctx: Ctx, cfg: LbtConfig, seed: int) -> "Model":
        h = C.c_void_p()
        ctx.check(ctx.lib.lbt_model_create_synthetic(ctx.h, C.byref(cfg), C.c_uint64(seed), C.byref(h)))
        return cls(ctx, h)

    @classmethod
    def load(cls, ctx: Ctx, path: str) -> "Model":
        h = C.c_void_p()
        ctx.check(ctx.lib.lbt_model_load(ctx.h, str(path).encode(), C.byref(h)))
        return cls(ctx, h)

    def free(self):
        if self.h:
            self.ctx.lib.lbt_model_free(self.h)
            self.h = None

    def new_cache(self) -> "Cache":
        h = C.c_void_p()
        self.ctx.check(self.ctx.lib.lbt_cache_new(self.h, C.byref(h)))
        return Cache(self, h)

    def set_head(self, kind: int):
        """0 = the exact tied bf16 head, 1 = the opt-in int8 head (q8head.rs), 2 = the
        bf16 head on the matrix cores for heads of 33..64 rows (within tolerance)."""
        self.ctx.check(self.ctx.lib.lbt_model_set_head(self.h, kind))

    def forward(self, tokens, cache: "Cache", all_logits: bool = False) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        rows = len(t) if all_logits else 1
        out = np.zeros((rows, self.cfg.vocab_size), np.float32)
        self.ctx.check(self.ctx.lib.lbt_model_forward(self.h, _ptr(t), len(t), cache.h, 1 if all_logits else 0,
                                                      _ptr(out)))
        return out

    def forward_sample(self, tokens, cache: "Cache", params: "LbtSampleParams", state: C.c_uint64) -> int:
        """Prompt forward, then one device sample (state updated in place)."""
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        nxt = C.c_uint32()
        self.ctx.check(self.ctx.lib.lbt_model_forward_sample(self.h, _ptr(t), len(t), cache.h, C.byref(params),
                                                             C.byref(state), C.byref(nxt)))
        return int(nxt.value)

    def decode_sample(self, cache: "Cache", first: int, steps: int, params: "LbtSampleParams", state: C.c_uint64):
        out = np.zeros(steps, np.uint32)
        md = C.c_float()
        self.ctx.check(self.ctx.lib.lbt_model_decode_sample(self.h, cache.h, C.c_uint32(first), steps, C.byref(params),
                                                            C.byref(state), _ptr(out), C.byref(md)))
        return out, md.value

    def forward_argmax(self, tokens, cache: "Cache") -> int:
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        nxt = C.c_uint32()
        self.ctx.check(self.ctx.lib.lbt_model_forward_argmax(self.h, _ptr(t), len(t), cache.h, C.byref(nxt)))
        return int(nxt.value)

    def generate_greedy(self, prompt, steps: int, cache: "Cache"):
        t = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.zeros(steps + 1, np.uint32)
        mp, md = C.c_float(), C.c_float()
        self.ctx.check(self.ctx.lib.lbt_model_generate_greedy(self.h, _ptr(t), len(t), steps, cache.h, _ptr(out),
                                                              C.byref(mp), C.byref(md)))
        return out, float(mp.value), float(md.value)

    def decode_greedy(self, cache: "Cache", first: int, steps: int):
        out = np.zeros(steps, np.uint32)
        md = C.c_float()
        self.ctx.check(self.ctx.lib.lbt_model_decode_greedy(self.h, cache.h, C.c_uint32(first), steps, _ptr(out),
                                                            C.byref(md)))
        return out, float(md.value)

    def read_hidden(self, n: int) -> np.ndarray:
        out = np.zeros((n, self.cfg.hidden_size), np.float32)
        self.ctx.check(self.ctx.lib.lbt_model_read_hidden(self.h, _ptr(out), n))
        return out

    def linear(self, layer: int, which: int) -> int:
        return self.ctx.lib.lbt_model_linear(self.h, layer, which)

    def new_sched(self, slots: int, cap: int) -> "Sched":
        h = C.c_void_p()
        self.ctx.check(self.ctx.lib.lbt_sched_new(self.h, slots, cap, C.byref(h)))
        return Sched(self, h)

    def new_batch(self, nseq: int, cap: int) -> "Batch":
        h = C.c_void_p()
        self.ctx.check(self.ctx.lib.lbt_batch_new(self.h, nseq, cap, C.byref(h)))
        return Batch(self, h, nseq)


class Cache:
    def __init__(self, model: Model, h):
        self.model, self.h = model, h

    def __len__(self):
        return self.model.ctx.lib.lbt_cache_len(self.h)

    def read(self, layer: int, is_v: bool) -> np.ndarray:
        c = self.model.cfg
        hd = c.hidden_size // c.num_attention_heads
        out = np.zeros((c.num_key_value_heads, len(self), hd), np.uint16)
        self.model.ctx.check(self.model.ctx.lib.lbt_cache_read(self.h, layer, 1 if is_v else 0, _ptr(out)))
        return out

    def free(self):
        if self.h:
            self.model.ctx.lib.lbt_cache_free(self.h)
            self.h = None


class Batch:
    """nseq sequences decoded together (lbt_batch_*)."""

    def __init__(self, model: Model, h, nseq: int):
        self.model, self.h, self.nseq = model, h, nseq

    def _check(self, rc):
        self.model.ctx.check(rc)

    def len(self, seq: int) -> int:
        return self.model.ctx.lib.lbt_batch_len(self.h, seq)

    def prefill(self, seq: int, tokens) -> int:
        t = np.ascontiguousarray(tokens, np.uint32)
        nxt = C.c_uint32()
        self._check(self.model.ctx.lib.lbt_batch_prefill(self.h, seq, _ptr(t), t.size, C.byref(nxt)))
        return int(nxt.value)

    def prefill_sample(self, seq: int, tokens, params: "LbtSampleParams", state: C.c_uint64) -> int:
        t = np.ascontiguousarray(tokens, np.uint32)
        nxt = C.c_uint32()
        self._check(self.model.ctx.lib.lbt_batch_prefill_sample(self.h, seq, _ptr(t), t.size, C.byref(params),
                                                                C.byref(state), C.byref(nxt)))
        return int(nxt.value)

    def forward_sample(self, tokens, params: list, states: np.ndarray) -> np.ndarray:
        """One step of every sequence, sequence s drawn with params[s]
        ((temperature, top_p, top_k)) and states[s] (uint64, updated)."""
        t = np.ascontiguousarray(tokens, np.uint32)
        assert t.size == self.nseq and len(params) == self.nseq and states.dtype == np.uint64
        pa = (LbtSampleParams * self.nseq)(*[LbtSampleParams(*p) for p in params])
        nxt = np.zeros(self.nseq, np.uint32)
        self._check(self.model.ctx.lib.lbt_batch_forward_sample(self.h, _ptr(t), pa, _ptr(states), _ptr(nxt)))
        return nxt

    def fill_synthetic(self, length: int, seed: int):
        self._check(self.model.ctx.lib.lbt_batch_fill_synthetic(self.h, length, C.c_uint64(seed)))

    def forward(self, tokens, want_logits: bool = True):
        t = np.ascontiguousarray(tokens, np.uint32)
        assert t.size == self.nseq
        nxt = np.zeros(self.nseq, np.uint32)
        logits = np.zeros((self.nseq, self.model.cfg.vocab_size), np.float32) if want_logits else None
        self._check(self.model.ctx.lib.lbt_batch_forward(self.h, _ptr(t), _ptr(logits) if want_logits else None,
                                                         _ptr(nxt)))
        return logits, nxt

    def decode_greedy(self, first, steps: int):
        f = np.ascontiguousarray(first, np.uint32)
        assert f.size == self.nseq
        out = np.zeros((steps, self.nseq), np.uint32)
        md = C.c_float()
        self._check(self.model.ctx.lib.lbt_batch_decode_greedy(self.h, _ptr(f), steps, _ptr(out), C.byref(md)))
        return out, float(md.value)

    def free(self):
        if self.h:
            self.model.ctx.lib.lbt_batch_free(self.h)
            self.h = None


class Sched:
    """Continuous batching of greedy requests (lbt_sched_*)."""

    NO_STOP = 0xFFFFFFFF

    def __init__(self, model: "Model", h):
        self.model, self.h = model, h

    def _check(self, rc):
        self.model.ctx.check(rc)

    def submit_sample(self, prompt, max_new: int, params, seed: int, stop: int = NO_STOP) -> int:
        """A request drawn by the device sampler: params = (temperature, top_p, top_k)."""
        t = np.ascontiguousarray(prompt, np.uint32)
        rid = C.c_uint64()
        p = LbtSampleParams(*params)
        self._check(self.model.ctx.lib.lbt_sched_submit_sample(self.h, _ptr(t), t.size, max_new, C.c_uint32(stop),
                                                               C.byref(p), C.c_uint64(seed), C.byref(rid)))
        return int(rid.value)

    def submit(self, prompt, max_new: int, stop: int = NO_STOP) -> int:
        t = np.ascontiguousarray(prompt, np.uint32)
        rid = C.c_uint64()
        self._check(self.model.ctx.lib.lbt_sched_submit(self.h, _ptr(t), t.size, max_new, C.c_uint32(stop),
                                                        C.byref(rid)))
        return int(rid.value)

    def step(self) -> int:
        p = C.c_int32()
        self._check(self.model.ctx.lib.lbt_sched_step(self.h, C.byref(p)))
        return int(p.value)

    def result(self, rid: int):
        n, done = C.c_size_t(), C.c_int32()
        self._check(self.model.ctx.lib.lbt_sched_result(self.h, C.c_uint64(rid), None, 0, C.byref(n), C.byref(done)))
        out = np.zeros(n.value, np.uint32)
        if n.value:
            self._check(self.model.ctx.lib.lbt_sched_result(self.h, C.c_uint64(rid), _ptr(out), out.size, C.byref(n),
                                                            C.byref(done)))
        return out, bool(done.value)

    def release(self, rid: int):
        self._check(self.model.ctx.lib.lbt_sched_release(self.h, C.c_uint64(rid)))

    def free(self):
        if self.h:
            self.model.ctx.lib.lbt_sched_free(self.h)
            self.h = None
