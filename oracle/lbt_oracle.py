"""ctypes wrapper of oracle/liblbt_oracle.so -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker (or the timed CPU baseline).
The product (lemonade-burn_amd/liblbt_hip.so) never uses it.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liblbt_oracle.so"

vp, sz, f32, i32, u64 = C.c_void_p, C.c_size_t, C.c_float, C.c_int, C.c_uint64


class OrConfig(C.Structure):
    _fields_ = [
        ("hidden", C.c_int), ("intermediate", C.c_int), ("heads", C.c_int), ("kv_heads", C.c_int),
        ("layers", C.c_int), ("vocab", C.c_int), ("max_pos", C.c_int),
        ("rms_norm_eps", C.c_double), ("rope_theta", C.c_double),
    ]


_SIGS = {
    "or_padded_cols": (sz, [sz]),
    "or_row_bytes": (sz, [sz]),
    "or_pack_row": (None, [vp, sz, vp]),
    "or_unpack_row": (None, [vp, sz, vp]),
    "or_pack": (None, [vp, sz, sz, vp]),
    "or_absmean": (f32, [vp, sz]),
    "or_ternarize_absmean": (f32, [vp, sz, vp]),
    "or_quantize_row": (f32, [vp, sz, vp, vp]),
    "or_quantize_acts": (None, [vp, sz, sz, vp, vp, vp]),
    "or_codes_dot": (C.c_int32, [vp, sz, vp]),
    "or_gemm_i32": (None, [vp, sz, sz, vp, vp, sz, vp]),
    "or_gemm_f32": (None, [vp, sz, sz, f32, vp, vp, vp, sz, vp]),
    "or_gemm_i32_bruteforce": (None, [vp, sz, sz, vp, sz, vp]),
    "or_bf16_to_f32": (f32, [C.c_uint16]),
    "or_f32_to_bf16": (C.c_uint16, [f32]),
    "or_bf16_dot_ref": (f32, [vp, vp, sz]),
    "or_bf16_dot_lanes": (f32, [vp, vp, sz]),
    "or_bf16_gemv_lanes": (None, [vp, sz, sz, vp, vp]),
    "or_q8head_from_bf16": (None, [vp, sz, sz, vp, vp]),
    "or_q8head_gemv_ref": (None, [vp, vp, sz, sz, vp, vp]),
    "or_q8head_gemv_lanes": (None, [vp, vp, sz, sz, vp, vp]),
    "or_model_set_head": (C.c_int, [vp, C.c_int]),
    "or_block_sum256": (f32, [vp]),
    "or_sumsq": (f32, [vp, sz]),
    "or_rmsnorm": (None, [vp, vp, sz, f32, vp]),
    "or_expf": (f32, [f32]),
    "or_argmax": (C.c_uint32, [vp, sz]),
    "or_sample": (C.c_uint32, [vp, sz, f32, f32, sz, vp]),
    "or_sample_key": (C.c_uint64, [f32, C.c_uint32]),
    "or_top_p_target": (C.c_uint64, [f32, C.c_uint64]),
    "or_sample_uniform": (C.c_uint32, [vp]),
    "or_rope_tables": (None, [sz, sz, C.c_double, vp, vp]),
    "or_synth_hash": (u64, [u64, u64, u64]),
    "or_synth_ternary": (C.c_int8, [u64, u64, u64]),
    "or_synth_packed": (None, [u64, u64, sz, sz, vp]),
    "or_synth_f32": (None, [u64, u64, sz, f32, f32, vp]),
    "or_synth_bf16": (None, [u64, u64, sz, vp]),
    "or_synth_wscale": (f32, [sz]),
    "or_model_synthetic": (vp, [C.POINTER(OrConfig), u64]),
    "or_model_wrap": (vp, [C.POINTER(OrConfig), vp, vp, vp, vp, vp]),
    "or_model_free": (None, [vp]),
    "or_model_packed": (vp, [vp, i32, i32]),
    "or_model_wscale": (f32, [vp, i32, i32]),
    "or_model_embed": (vp, [vp]),
    "or_model_reset": (None, [vp]),
    "or_model_len": (i32, [vp]),
    "or_model_forward": (i32, [vp, vp, sz, i32, vp]),
    "or_model_fill_synth_kv": (i32, [vp, u64, i32, i32, i32]),
    "or_model_hidden": (vp, [vp]),
    "or_model_kcache": (vp, [vp, i32]),
    "or_model_vcache": (vp, [vp, i32]),
    "or_model_cap": (i32, [vp]),
    "or_set_fast": (i32, [i32]),
    "or_set_threads": (i32, [i32]),
    "port_isa": (C.c_char_p, []),
    "port_gemm_i32": (None, [vp, sz, sz, vp, vp, sz, vp, i32]),
    "port_gemm_f32": (None, [vp, sz, sz, f32, vp, vp, vp, sz, vp, i32]),
    "port_quantize_row": (f32, [vp, sz, vp, vp]),
    "port_bf16_gemv": (None, [vp, sz, sz, vp, vp, i32]),
    "port_threads": (i32, []),
}

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = C.CDLL(str(LIB_PATH))
        for n, (r, a) in _SIGS.items():
            f = getattr(L, n)
            f.restype = r
            f.argtypes = a
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return C.c_void_p(a.ctypes.data)


def padded_cols(c: int) -> int:
    return (c + 127) // 128 * 128


# ---- layout --------------------------------------------------------------------
def pack(t: np.ndarray) -> np.ndarray:
    t = np.ascontiguousarray(t, dtype=np.int8)
    rows, cols = t.shape
    out = np.zeros((rows, padded_cols(cols) // 4), np.uint8)
    lib().or_pack(_p(t), rows, cols, _p(out))
    return out


def unpack(packed: np.ndarray, cols: int) -> np.ndarray:
    rows = packed.shape[0]
    kp = padded_cols(cols)
    out = np.zeros((rows, kp), np.int8)
    for r in range(rows):
        row = np.ascontiguousarray(packed[r])
        lib().or_unpack_row(_p(row), kp, _p(out[r]))
    return out[:, :cols]


def ternarize_absmean(w: np.ndarray):
    w = np.ascontiguousarray(w, dtype=np.float32).ravel()
    t = np.zeros(w.size, np.int8)
    s = lib().or_ternarize_absmean(_p(w), w.size, _p(t))
    return t, np.float32(s)


# ---- quantizer -------------------------------------------------------------------
def quantize_row(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.zeros(max(x.size, 1), np.int8)
    su = C.c_int32()
    s = lib().or_quantize_row(_p(x), x.size, _p(q), C.byref(su))
    return q[: x.size], np.float32(s), int(su.value)


def quantize_acts(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, k = x.shape
    q = np.zeros((m, padded_cols(k)), np.int8)
    s = np.zeros(m, np.float32)
    su = np.zeros(m, np.int32)
    lib().or_quantize_acts(_p(x), m, k, _p(q), _p(s), _p(su))
    return q, s, su


def port_quantize_row(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.zeros(max(x.size, 1), np.int8)
    su = C.c_int32()
    s = lib().port_quantize_row(_p(x), x.size, _p(q), C.byref(su))
    return q[: x.size], np.float32(s), int(su.value)


# ---- gemm -------------------------------------------------------------------------
def gemm_i32(packed, rows, cols, q, qsum) -> np.ndarray:
    packed = np.ascontiguousarray(packed, np.uint8)
    q = np.ascontiguousarray(q, np.int8)
    qsum = np.ascontiguousarray(qsum, np.int32)
    m = q.shape[0]
    out = np.zeros((m, rows), np.int32)
    lib().or_gemm_i32(_p(packed), rows, cols, _p(q), _p(qsum), m, _p(out))
    return out


def gemm_f32(packed, rows, cols, s_w, q, s_a, qsum) -> np.ndarray:
    packed = np.ascontiguousarray(packed, np.uint8)
    q = np.ascontiguousarray(q, np.int8)
    s_a = np.ascontiguousarray(s_a, np.float32)
    qsum = np.ascontiguousarray(qsum, np.int32)
    m = q.shape[0]
    out = np.zeros((m, rows), np.float32)
    lib().or_gemm_f32(_p(packed), rows, cols, C.c_float(s_w), _p(q), _p(s_a), _p(qsum), m, _p(out))
    return out


def gemm_i32_bruteforce(packed, rows, cols, q) -> np.ndarray:
    packed = np.ascontiguousarray(packed, np.uint8)
    q = np.ascontiguousarray(q, np.int8)
    m = q.shape[0]
    out = np.zeros((m, rows), np.int32)
    lib().or_gemm_i32_bruteforce(_p(packed), rows, cols, _p(q), m, _p(out))
    return out


def port_gemm_i32(packed, rows, cols, q, qsum, threads=0) -> np.ndarray:
    packed = np.ascontiguousarray(packed, np.uint8)
    q = np.ascontiguousarray(q, np.int8)
    qsum = np.ascontiguousarray(qsum, np.int32)
    m = q.shape[0]
    out = np.zeros((m, rows), np.int32)
    lib().port_gemm_i32(_p(packed), rows, cols, _p(q), _p(qsum), m, _p(out), threads)
    return out


# ---- bf16 -------------------------------------------------------------------------
def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_gemv_lanes(w: np.ndarray, x: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, np.uint16)
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = w.shape
    out = np.zeros(rows, np.float32)
    lib().or_bf16_gemv_lanes(_p(w), rows, cols, _p(x), _p(out))
    return out


def bf16_dot_ref(w: np.ndarray, x: np.ndarray) -> float:
    w = np.ascontiguousarray(w, np.uint16)
    x = np.ascontiguousarray(x, np.float32)
    return float(lib().or_bf16_dot_ref(_p(w), _p(x), w.size))


def port_bf16_gemv(w: np.ndarray, x: np.ndarray, threads=0) -> np.ndarray:
    w = np.ascontiguousarray(w, np.uint16)
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = w.shape
    out = np.zeros(rows, np.float32)
    lib().port_bf16_gemv(_p(w), rows, cols, _p(x), _p(out), threads)
    return out


# ---- int8 head (q8head.rs) ----------------------------------------------------------
def q8head_from_bf16(w: np.ndarray):
    """Q8Head::from_bf16 (q8head.rs:18-32) -> (q int8 [rows, cols], scale f32 [rows])."""
    w = np.ascontiguousarray(w, np.uint16)
    rows, cols = w.shape
    q = np.zeros((rows, cols), np.int8)
    s = np.zeros(rows, np.float32)
    lib().or_q8head_from_bf16(_p(w), rows, cols, _p(q), _p(s))
    return q, s


def _q8_gemv(fn, q, s, x):
    q = np.ascontiguousarray(q, np.int8)
    s = np.ascontiguousarray(s, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = q.shape
    out = np.zeros(rows, np.float32)
    fn(_p(q), _p(s), rows, cols, _p(x), _p(out))
    return out


def q8head_gemv_ref(q, s, x) -> np.ndarray:
    """Q8Head::gemv (q8head.rs:35-57) in the reference's order."""
    return _q8_gemv(lib().or_q8head_gemv_ref, q, s, x)


def q8head_gemv_lanes(q, s, x) -> np.ndarray:
    """The device int8 head's order (lane chunks, fused multiply-adds, butterfly)."""
    return _q8_gemv(lib().or_q8head_gemv_lanes, q, s, x)


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.zeros_like(x)
    lib().or_rmsnorm(_p(x), _p(w), x.size, C.c_float(eps), _p(out))
    return out


def expf(x: float) -> np.float32:
    return np.float32(lib().or_expf(C.c_float(x)))


def rope_tables(hd: int, max_pos: int, theta: float):
    c = np.zeros((max_pos, hd // 2), np.float32)
    s = np.zeros((max_pos, hd // 2), np.float32)
    lib().or_rope_tables(hd, max_pos, C.c_double(theta), _p(c), _p(s))
    return c, s


# ---- synthetic ---------------------------------------------------------------------
def synth_packed(seed, tensor, rows, cols) -> np.ndarray:
    out = np.zeros((rows, padded_cols(cols) // 4), np.uint8)
    lib().or_synth_packed(seed, tensor, rows, cols, _p(out))
    return out


def synth_bf16(seed, tensor, n) -> np.ndarray:
    out = np.zeros(n, np.uint16)
    lib().or_synth_bf16(seed, tensor, n, _p(out))
    return out


def synth_f32(seed, tensor, n, lo=0.5, span=1.0) -> np.ndarray:
    out = np.zeros(n, np.float32)
    lib().or_synth_f32(seed, tensor, n, C.c_float(lo), C.c_float(span), _p(out))
    return out


def t_layer(l: int, k: int) -> int:
    return 16 + l * 16 + k


T_EMBED, T_FINAL_NORM = 1, 2


# ---- model ----------------------------------------------------------------------------
class OracleModel:
    """BitNet::forward restated on the CPU in the device's float order."""

    def __init__(self, cfg: OrConfig, seed: int | None = None, handle=None):
        self.cfg = cfg
        self._keep = None
        if handle is None:
            handle = lib().or_model_synthetic(C.byref(cfg), seed)
        self.h = handle

    @classmethod
    def wrap(cls, cfg: OrConfig, packed: list, wscales, norms: list, final_norm, embed):
        keep = [np.ascontiguousarray(p, np.uint8) for p in packed]
        nkeep = [np.ascontiguousarray(n, np.float32) for n in norms]
        pa = (C.c_void_p * len(keep))(*[k.ctypes.data for k in keep])
        ws = np.ascontiguousarray(wscales, np.float32)
        na = (C.c_void_p * len(nkeep))(*[k.ctypes.data for k in nkeep])
        fn = np.ascontiguousarray(final_norm, np.float32)
        em = np.ascontiguousarray(embed, np.uint16)
        h = lib().or_model_wrap(C.byref(cfg), pa, _p(ws), na, _p(fn), _p(em))
        m = cls(cfg, handle=h)
        m._keep = (keep, nkeep, pa, ws, na, fn, em)
        return m

    def free(self):
        if self.h:
            lib().or_model_free(self.h)
            self.h = None

    def reset(self):
        lib().or_model_reset(self.h)

    def set_head(self, kind: int):
        if lib().or_model_set_head(self.h, kind) != 0:
            raise ValueError("head kind must be 0 (bf16) or 1 (int8)")

    def __len__(self):
        return lib().or_model_len(self.h)

    def forward(self, tokens, all_logits=False) -> np.ndarray:
        t = np.ascontiguousarray(tokens, np.uint32)
        rows = len(t) if all_logits else 1
        out = np.zeros((rows, self.cfg.vocab), np.float32)
        rc = lib().or_model_forward(self.h, _p(t), len(t), 1 if all_logits else 0, _p(out))
        if rc != 0:
            raise RuntimeError("oracle: context length exceeded")
        return out

    def fill_synth_kv(self, seed: int, nseq: int, seq: int, length: int):
        """The cache of sequence `seq` of a batch after lbt_batch_fill_synthetic(length, seed)."""
        if lib().or_model_fill_synth_kv(self.h, seed, nseq, seq, length) != 0:
            raise ValueError("fill_synth_kv: bad arguments")

    def hidden(self, n: int) -> np.ndarray:
        p = lib().or_model_hidden(self.h)
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), shape=(n, self.cfg.hidden)).copy()

    def kcache(self, layer: int, length: int, is_v=False) -> np.ndarray:
        cap = lib().or_model_cap(self.h)
        hd = self.cfg.hidden // self.cfg.heads
        fn = lib().or_model_vcache if is_v else lib().or_model_kcache
        p = fn(self.h, layer)
        a = np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint16)), shape=(self.cfg.kv_heads, cap, hd))
        return a[:, :length].copy()

    def packed(self, layer: int, which: int, rows: int, cols: int) -> np.ndarray:
        p = lib().or_model_packed(self.h, layer, which)
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint8)), shape=(rows, padded_cols(cols) // 4)).copy()


def config(hidden=2560, intermediate=6912, heads=20, kv_heads=5, layers=30, vocab=128256, max_pos=4096,
           eps=1e-5, theta=500000.0) -> OrConfig:
    return OrConfig(hidden, intermediate, heads, kv_heads, layers, vocab, max_pos, eps, theta)


def set_fast(mode: int) -> int:
    return lib().or_set_fast(mode)


def set_threads(n: int) -> int:
    """Threads of the oracle's parallel loops and the port's kernels (0 = all);
    returns the previous setting."""
    return lib().or_set_threads(n)


class Sampler:
    """Sampler (sample.rs:28-82) in the device sampler's arithmetic:
    state = seed.max(1), one draw per sample at temperature > 0."""

    def __init__(self, temperature: float, top_p: float = 1.0, top_k: int = 0, seed: int = 0x5EED):
        self.t, self.top_p, self.top_k = float(temperature), float(top_p), int(top_k)
        self.state = C.c_uint64(max(int(seed), 1))

    def sample(self, logits: np.ndarray) -> int:
        lg = np.ascontiguousarray(logits, np.float32)
        return int(lib().or_sample(_p(lg), lg.size, self.t, self.top_p, self.top_k, C.byref(self.state)))
