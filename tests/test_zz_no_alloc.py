"""lbt_ternary_linear_dev_noalloc (the entry point that allocates nothing: its
several-row activations live in a static per-device scratch) against
lbt_ternary_linear_dev and the oracle (ActQuant + ternary_gemm_multi's f32
epilogue), bit for bit, through the C ABI: two calls in a row,
the second smaller (fewer rows, a narrower padded width whose padding the
first call's rows had filled), the MFMA and the single-token paths, and the
size limit."""
import ctypes as C

import numpy as np
import pytest

import lbt_hip
import lbt_oracle as orc
from conftest import announce

pytestmark = pytest.mark.gpu


class Dev:
    """Device buffers of one call, freed together."""

    def __init__(self, ctx):
        self.ctx, self.bufs = ctx, []

    def put(self, a: np.ndarray) -> C.c_void_p:
        p = C.c_void_p()
        self.ctx.check(self.ctx.lib.lbt_dev_alloc(self.ctx.h, max(a.nbytes, 1), C.byref(p)))
        self.ctx.check(self.ctx.lib.lbt_memcpy_h2d(self.ctx.h, p, a.ctypes.data, a.nbytes))
        self.bufs.append(p)
        return p

    def zeros(self, nbytes: int) -> C.c_void_p:
        return self.put(np.full(nbytes, 0xA5, np.uint8))  # junk, every byte must be written

    def get(self, p, shape, dtype) -> np.ndarray:
        out = np.zeros(shape, dtype)
        self.ctx.check(self.ctx.lib.lbt_memcpy_d2h(self.ctx.h, out.ctypes.data, p, out.nbytes))
        return out

    def free(self):
        for p in self.bufs:
            self.ctx.lib.lbt_dev_free(self.ctx.h, p)


def run(ctx, fn, ws, x):
    m, cols = x.shape
    d = Dev(ctx)
    try:
        dx = d.put(x)
        outs = [d.zeros(m * w.rows * 4) for w in ws]
        wa = (C.c_void_p * len(ws))(*[w.h for w in ws])
        oa = (C.c_void_p * len(ws))(*[o.value for o in outs])
        ctx.check(fn(ctx.h, wa, len(ws), dx, m, cols, oa))
        ctx.sync()
        return [d.get(o, (m, w.rows), np.float32) for o, w in zip(outs, ws)]
    finally:
        d.free()


def weights(ctx, rng, shapes, cols, keep=None):
    """Uploaded ternary matrices; `keep` collects (packed, rows, scale) for the oracle."""
    out = []
    for rows, s in shapes:
        t = rng.choice(np.array([-1, 0, 1], np.int8), size=(rows, cols), p=[0.3, 0.4, 0.3])
        packed = orc.pack(t)
        out.append(ctx.upload(packed, rows, cols, s))
        if keep is not None:
            keep.append((packed, rows, s))
    return out


@pytest.mark.parametrize("cases", [[(64, 2560), (17, 1000)], [(40, 6912), (2, 2560)], [(1, 2560), (1, 1000)]])
def test_noalloc_equals_linear_dev_twice(ctx, cases):
    rng = np.random.default_rng(11)
    for i, (m, cols) in enumerate(cases):
        announce(f"noalloc call {i}: m={m} cols={cols}")
        kept = []
        ws = weights(ctx, rng, [(2560, 0.9), (640, 1.1), (640, 1.3)][: 3 if i == 0 else 1], cols, kept)
        x = rng.standard_normal((m, cols)).astype(np.float32)
        got = run(ctx, ctx.lib.lbt_ternary_linear_dev_noalloc, ws, x)
        ref = run(ctx, ctx.lib.lbt_ternary_linear_dev, ws, x)
        q, s_a, qsum = orc.quantize_acts(x)
        for g, r, (packed, rows, s_w) in zip(got, ref, kept):
            assert np.array_equal(g, r), f"call {i} m={m} cols={cols}"
            exp = orc.gemm_f32(packed, rows, cols, s_w, q, s_a, qsum)
            assert np.array_equal(g, exp), f"oracle, call {i} m={m} cols={cols}"
        for w in ws:
            w.free()


def test_noalloc_rejects_beyond_the_scratch(ctx):
    rng = np.random.default_rng(12)
    cols, m = 6912, 700  # 700 * 6912 bytes > 4 MiB
    (w,) = weights(ctx, rng, [(16, 1.0)], cols)
    x = np.zeros((m, cols), np.float32)
    d = Dev(ctx)
    try:
        dx = d.put(x)
        o = d.zeros(m * 16 * 4)
        wa = (C.c_void_p * 1)(w.h)
        oa = (C.c_void_p * 1)(o.value)
        rc = ctx.lib.lbt_ternary_linear_dev_noalloc(ctx.h, wa, 1, dx, m, cols, oa)
        assert rc == -1
        assert "scratch" in ctx.lib.lbt_last_error(ctx.h).decode()
    finally:
        d.free()
        w.free()
