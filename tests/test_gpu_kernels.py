"""GPU parity of the ternary / quantizer / bf16 kernels against the pinned
oracle, through the C ABI.  Integers and quantizer outputs are bit-exact;
f32 GEMM outputs are bit-exact to the reference's epilogue definition
(gemm.rs:141,150); the bf16 GEMV is bit-exact to the device-order oracle and
within the reference's 1e-4 of f64 (bf16.rs:126-134)."""
import ctypes as C
from pathlib import Path

import numpy as np
import pytest

import lbt_oracle as orc
from conftest import announce
from refgen import XorShiftStar, golden_case, quant_rnd_vec, ternary_iid
from test_oracle import GOLDEN_SHAPES, quant_cases

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def test_quantize_edge_cases_bitexact(ctx):
    for i, x in enumerate(quant_cases()):
        if x.size == 0:
            continue
        announce(f"quantize case {i} n={x.size}")
        q, s, su = ctx.quantize_acts(x[None, :])
        eq, es, esu = orc.quantize_acts(x[None, :])
        assert np.array_equal(q, eq) and np.array_equal(su, esu)
        assert s.tobytes() == es.tobytes()


def test_quantize_many_rows(ctx):
    rng = np.random.default_rng(3)
    for m, k in [(64, 2560), (5, 6912), (3, 100), (17, 1000)]:
        announce(f"quantize m={m} k={k}")
        x = (rng.standard_normal((m, k)) * rng.uniform(0.1, 30, (m, 1))).astype(np.float32)
        got = ctx.quantize_acts(x)
        exp = orc.quantize_acts(x)
        for g, e in zip(got, exp):
            assert np.array_equal(g, e)


def test_golden_fixtures_bitexact(ctx):
    for f in sorted(GOLDEN.glob("gemm_*.npz")):
        z = np.load(f)
        rows, cols = int(z["rows"]), int(z["cols"])
        announce(f"golden {f.name}")
        w = ctx.upload(z["packed"], rows, cols, float(z["s_w"]))
        assert np.array_equal(ctx.gemm_i32(w, z["q"], z["qsum"]), z["i32"])
        (y,) = ctx.gemm_multi([w], z["q"], z["s_a"], z["qsum"])
        assert np.array_equal(y, z["f32"])
        (y2,) = ctx.ternary_linear([w], z["x"])
        assert np.array_equal(y2, z["f32"])
        w.free()


@pytest.mark.parametrize("rows,cols,m", GOLDEN_SHAPES + [(23, 384, m) for m in range(1, 10)] +
                         [(48, 2560, 5), (37, 2560, 13), (5, 1, 3), (5, 100, 3), (5, 129, 3), (5, 300, 3)])
def test_golden_shapes(ctx, rows, cols, m):
    # golden.rs:82-105
    announce(f"golden shape {rows}x{cols} m={m}")
    t, scale, x = golden_case(rows, cols, m, rows * 31 + cols + 7 * m)
    p = orc.pack(t)
    q, sa, su = orc.quantize_acts(x)
    w = ctx.upload(p, rows, cols, float(scale))
    assert np.array_equal(ctx.gemm_i32(w, q, su), q[:, :cols].astype(np.int64) @ t.T.astype(np.int64))
    (y,) = ctx.ternary_linear([w], x)
    assert np.array_equal(y, orc.gemm_f32(p, rows, cols, scale, q, sa, su))
    w.free()


@pytest.mark.parametrize("rows,cols,m,seed", [(64, 128, 1, 1), (130, 300, 3, 2), (2560, 2560, 1, 3), (6912, 2560, 4, 4)])
def test_gpu_matches_scalar_shapes(ctx, rows, cols, m, seed):
    # crates/lb-ternary-gpu/tests/gpu_matches_scalar.rs:22-54
    announce(f"gpu_matches_scalar {rows}x{cols} m={m}")
    rng = XorShiftStar(seed)
    vals = np.array([rng.ternary() for _ in range(rows * cols)], np.int8).reshape(rows, cols)
    acts = np.array([np.float32(rng.unit() * np.float32(4.0)) for _ in range(m * cols)], np.float32).reshape(m, cols)
    p = orc.pack(vals)
    q, sa, su = orc.quantize_acts(acts)
    w = ctx.upload(p, rows, cols, 1.0)
    assert np.array_equal(ctx.gemm_i32(w, q, su), orc.gemm_i32(p, rows, cols, q, su))
    w.free()


BITNET = [(2560, 2560), (640, 2560), (6912, 2560), (2560, 6912)]


@pytest.mark.parametrize("rows,cols", BITNET)
@pytest.mark.parametrize("m", [1, 2, 5, 8, 64])
def test_bitnet_shapes_bitexact(ctx, rows, cols, m):
    # the benchmark GEMV/GEMM shapes (one decoder layer, the FFN prefill shapes), distribution P(-1,0,1)=(.3,.4,.3), N(0,1) activations
    announce(f"bitnet shape {rows}x{cols} m={m}")
    rng = np.random.default_rng(rows * 7 + cols + m)
    t = ternary_iid(rng, rows, cols)
    p = orc.pack(t)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    q, sa, su = orc.quantize_acts(x)
    sw = float(np.float32(1.0 / 0.6))
    w = ctx.upload(p, rows, cols, sw)
    assert np.array_equal(ctx.gemm_i32(w, q, su), orc.port_gemm_i32(p, rows, cols, q, su))
    (y,) = ctx.ternary_linear([w], x)
    d = orc.port_gemm_i32(p, rows, cols, q, su)
    inv = (np.float32(1.0) / (sa * np.float32(sw))).astype(np.float32)
    assert np.array_equal(y, (d.astype(np.float32) * inv[:, None]).astype(np.float32))
    w.free()


def test_extreme_values(ctx):
    # golden.rs:108-122 and :181-194
    for rows, cols, m in [(4, 6912, 1), (3, 6912 * 2, 5)]:
        announce(f"extreme {rows}x{cols} m={m}")
        p = orc.pack(np.ones((rows, cols), np.int8))
        w = ctx.upload(p, rows, cols, 1.0)
        for sign in (1.0, -1.0):
            x = np.full((m, cols), sign, np.float32)
            q, sa, su = ctx.quantize_acts(x)
            assert np.all(ctx.gemm_i32(w, q, su) == int(sign) * 127 * cols)
            (y,) = ctx.ternary_linear([w], x)
            assert np.all(y == np.float32(sign * cols))
        w.free()


def test_multi_matches_separate_bit_for_bit(ctx):
    # golden.rs:128-176 and ops.rs:27-40 (ternary_linear2/3 == separate calls)
    cols = 640
    rng = np.random.default_rng(4242)
    shapes = [(96, 0.7), (24, 1.3), (200, 2.1)]
    ws = [ctx.upload(orc.pack(ternary_iid(rng, r, cols)), r, cols, s) for r, s in shapes]
    for m in (1, 2, 5, 64):
        announce(f"multi m={m}")
        x = rng.standard_normal((m, cols)).astype(np.float32) * 3
        fused3 = ctx.ternary_linear(ws, x)
        fused2 = ctx.ternary_linear(ws[:2], x)
        for i, w in enumerate(ws):
            (single,) = ctx.ternary_linear([w], x)
            assert np.array_equal(fused3[i], single)
            if i < 2:
                assert np.array_equal(fused2[i], single)
        q, sa, su = orc.quantize_acts(x)
        pre = ctx.gemm_multi(ws, q, sa, su)
        for a, b in zip(pre, fused3):
            assert np.array_equal(a, b)
    for w in ws:
        w.free()


def test_bf16_linear(ctx):
    rng = np.random.default_rng(9)
    # m >= 9: the batched head's 16-token groups (lmhead_stream_kernel), ragged
    # groups and row tiles included
    for rows, cols, m in [(37, 2584, 1), (1000, 2560, 3), (128256 // 8, 2560, 1), (1000, 2560, 9),
                          (3001, 2560, 37), (8000, 2560, 64)]:
        announce(f"bf16 {rows}x{cols} m={m}")
        wf = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
        wb = orc.f32_to_bf16(wf).reshape(rows, cols)
        x = rng.standard_normal((m, cols)).astype(np.float32)
        w = ctx.bf16_upload(wb)
        got = ctx.bf16_linear(w, x)
        for t in range(m):
            exp = orc.bf16_gemv_lanes(wb, x[t])
            assert np.array_equal(got[t], exp)
            ref = orc.bf16_to_f32(wb).astype(np.float64) @ x[t].astype(np.float64)
            assert np.all(np.abs(got[t] - ref) < 1e-4 * max(1.0, np.abs(ref).max() / 10))
        w.free()


def test_rmsnorm_quantize_fused(ctx):
    lib = ctx.lib
    rng = np.random.default_rng(5)
    for m, k in [(1, 2560), (3, 6912), (2, 300)]:
        announce(f"rmsnorm+quant m={m} k={k}")
        x = (rng.standard_normal((m, k)) * 4).astype(np.float32)
        nw = rng.uniform(0.5, 1.5, k).astype(np.float32)
        kp = orc.padded_cols(k)
        ptrs = []
        for nbytes in (x.nbytes, nw.nbytes, m * kp, m * 4, m * 4):
            p = C.c_void_p()
            ctx.check(lib.lbt_dev_alloc(ctx.h, nbytes, C.byref(p)))
            ptrs.append(p)
        ctx.check(lib.lbt_memcpy_h2d(ctx.h, ptrs[0], x.ctypes.data, x.nbytes))
        ctx.check(lib.lbt_memcpy_h2d(ctx.h, ptrs[1], nw.ctypes.data, nw.nbytes))
        ctx.check(lib.lbt_rmsnorm_quantize_dev(ctx.h, ptrs[0], ptrs[1], C.c_float(1e-5), m, k, ptrs[2], ptrs[3],
                                               ptrs[4]))
        q = np.zeros((m, kp), np.int8)
        s = np.zeros(m, np.float32)
        su = np.zeros(m, np.int32)
        for host, dev in ((q, ptrs[2]), (s, ptrs[3]), (su, ptrs[4])):
            ctx.check(lib.lbt_memcpy_d2h(ctx.h, host.ctypes.data, dev, host.nbytes))
        normed = np.stack([orc.rmsnorm(x[i], nw, 1e-5) for i in range(m)])
        eq, es, esu = orc.quantize_acts(normed)
        assert np.array_equal(q, eq) and np.array_equal(s, es) and np.array_equal(su, esu)
        for p in ptrs:
            ctx.check(lib.lbt_dev_free(ctx.h, p))


def _rmsnorm_quantize_dev(ctx, x, nw, eps=1e-5):
    lib = ctx.lib
    m, k = x.shape
    kp = orc.padded_cols(k)
    ptrs = []
    for nbytes in (x.nbytes, nw.nbytes, m * kp, m * 4, m * 4):
        p = C.c_void_p()
        ctx.check(lib.lbt_dev_alloc(ctx.h, nbytes, C.byref(p)))
        ptrs.append(p)
    ctx.check(lib.lbt_memcpy_h2d(ctx.h, ptrs[0], x.ctypes.data, x.nbytes))
    ctx.check(lib.lbt_memcpy_h2d(ctx.h, ptrs[1], nw.ctypes.data, nw.nbytes))
    ctx.check(lib.lbt_rmsnorm_quantize_dev(ctx.h, ptrs[0], ptrs[1], C.c_float(eps), m, k, ptrs[2], ptrs[3], ptrs[4]))
    q = np.zeros((m, kp), np.int8)
    s = np.zeros(m, np.float32)
    su = np.zeros(m, np.int32)
    for host, dev in ((q, ptrs[2]), (s, ptrs[3]), (su, ptrs[4])):
        ctx.check(lib.lbt_memcpy_d2h(ctx.h, host.ctypes.data, dev, host.nbytes))
    for p in ptrs:
        ctx.check(lib.lbt_dev_free(ctx.h, p))
    return q, s, su


def absmax_cases():
    """Rows at the edges of the normed absmax: one clear maximum; equal
    maxima far apart; near-ties (one ulp) far apart and close together;
    huge and zero norm weights; tiny, huge, zero and NaN rows."""
    rng = np.random.default_rng(17)
    k = 2560
    base = rng.standard_normal(k).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, k).astype(np.float32)
    one = np.ones(k, np.float32)
    cases = [("random", base, nw), ("ones", np.ones(k, np.float32), one)]
    x = base.copy(); x[0] = 10.0; x[2000] = 10.0
    cases.append(("equal maxima, two waves", x, one))
    x = base.copy(); x[5] = 10.0; x[700] = np.nextafter(np.float32(10.0), np.float32(0.0))
    cases.append(("near tie, two waves", x, one))
    x = base.copy(); x[5] = 10.0; x[9] = np.nextafter(np.float32(10.0), np.float32(0.0))
    cases.append(("near tie, one wave", x, one))
    x = base.copy(); x[3] = -50.0
    cases.append(("negative max", x, nw))
    w = nw.copy(); w[17] = 2.0**21
    cases.append(("huge norm weight", base, w))
    cases.append(("tiny 1e-15", (base * np.float32(1e-15)).astype(np.float32), nw))
    cases.append(("tiny 1e-30", (base * np.float32(1e-30)).astype(np.float32), nw))
    cases.append(("huge 1e20", (base * np.float32(1e20)).astype(np.float32), nw))
    cases.append(("zeros", np.zeros(k, np.float32), nw))
    x = base.copy(); x[100] = np.nan
    cases.append(("nan", x, nw))
    w = nw.copy(); w[::7] = 0.0
    cases.append(("zero norm weights", base, w))
    return cases


@pytest.mark.parametrize("case", range(13))
def test_rmsnorm_quantize_absmax_edges(ctx, case):
    name, x, nw = absmax_cases()[case]
    announce(f"rmsnorm+quant absmax case {name}")
    x = x[None, :]
    q, s, su = _rmsnorm_quantize_dev(ctx, x, nw)
    normed = orc.rmsnorm(x[0], nw, 1e-5)[None, :]
    eq, es, esu = orc.quantize_acts(normed)
    assert np.array_equal(q, eq) and s.tobytes() == es.tobytes() and np.array_equal(su, esu)


def test_invalid_arguments_return_errors(ctx):
    import lbt_hip

    w = ctx.upload(np.full((4, 32), 0x55, np.uint8), 4, 128, 1.0)
    with pytest.raises(lbt_hip.LbtError):
        ctx.ternary_linear([w], np.zeros((1, 64), np.float32))  # inner dimension mismatch
    w.free()


def test_oversized_arguments_return_errors(ctx):
    # sizes the kernels could not index (int rows, columns and token counts;
    # 32-bit cache positions) are refused at the C ABI with an error, before
    # any memory behind the pointers is touched
    import lbt_hip

    lib, h = ctx.lib, ctx.h
    E_RANGE = {v: k for k, v in lbt_hip.ERRORS.items()}["LBT_E_RANGE"]
    big, huge = 1 << 31, (1 << 64) - 1
    w = ctx.upload(np.full((4, 32), 0x55, np.uint8), 4, 128, 1.0)
    x = np.zeros((1, 128), np.float32)
    out = np.zeros((1, 4), np.float32)
    wa = (C.c_void_p * 1)(w.h)
    oa = (C.c_void_p * 1)(out.ctypes.data)
    q = np.zeros((1, 128), np.int8)
    s = np.zeros(1, np.float32)
    su = np.zeros(1, np.int32)
    dummy = C.c_void_p(x.ctypes.data)
    h2 = C.c_void_p()
    calls = {
        "ternary_linear_dev m": lambda: lib.lbt_ternary_linear_dev(h, wa, 1, dummy, big, 128, oa),
        "ternary_linear m": lambda: lib.lbt_ternary_linear(h, wa, 1, dummy, big, 128, oa),
        "gemm_i32_dev m": lambda: lib.lbt_gemm_i32_dev(h, w.h, q.ctypes.data, su.ctypes.data, big, out.ctypes.data),
        "quantize_acts_dev m": lambda: lib.lbt_quantize_acts_dev(h, dummy, big, 128, q.ctypes.data, s.ctypes.data,
                                                                 su.ctypes.data),
        "quantize_acts k": lambda: lib.lbt_quantize_acts(h, dummy, 1, big, q.ctypes.data, s.ctypes.data,
                                                         su.ctypes.data),
        "weight_upload rows": lambda: lib.lbt_weight_upload(h, dummy, big, 128, C.c_float(1.0), C.byref(h2)),
        "bf16_upload rows": lambda: lib.lbt_bf16_upload(h, dummy, big, 128, C.byref(h2)),
    }
    for name, call in calls.items():
        assert call() != 0, name
    w.free()
    cfg = dict(hidden=256, intermediate=512, heads=4, kv_heads=2, layers=1, vocab=100, max_pos=64)
    m = lbt_hip.Model.synthetic(ctx, lbt_hip.make_config(**cfg), 3)
    c = m.new_cache()
    toks = np.array([1, 2, 3], np.uint32)
    nxt = np.zeros(4, np.uint32)
    assert lib.lbt_model_forward(m.h, toks.ctypes.data, (1 << 32) + 3, c.h, 0, None) == E_RANGE
    assert lib.lbt_model_forward_argmax(m.h, toks.ctypes.data, huge, c.h, nxt.ctypes.data) == E_RANGE
    assert lib.lbt_model_generate_greedy(m.h, toks.ctypes.data, 3, huge, c.h, nxt.ctypes.data, None,
                                         None) == E_RANGE
    assert lib.lbt_model_decode_greedy(m.h, c.h, 1, huge, nxt.ctypes.data, None) == E_RANGE
    assert len(c) == 0
    b = m.new_batch(2, 32)
    assert lib.lbt_batch_prefill(b.h, 0, toks.ctypes.data, (1 << 32) + 3, nxt.ctypes.data) == E_RANGE
    assert b.len(0) == 0
    b.free()
    # a valid call afterwards still gives the oracle's logits
    om = orc.OracleModel(orc.config(**cfg), 3)
    assert np.array_equal(m.forward(toks, c, all_logits=True), om.forward(toks, all_logits=True))
    om.free()
    c.free()
    m.free()


@pytest.mark.gpu
def test_fused_prologue_edge_cases_match_oracle(ctx):
    # the reference's quantizer edge cases (NaN -> 0, +-inf, denormals, ties,
    # all-zero rows) through the GEMV's fused quantize prologue
    rng = np.random.default_rng(11)
    for i, x in enumerate(quant_cases()):
        cols = x.size
        announce(f"fused prologue case {i} cols={cols}")
        rows = 24
        t = rng.integers(-1, 2, (rows, cols)).astype(np.int8)
        p = orc.pack(t)
        q, sa, su = orc.quantize_acts(x[None, :])
        w = ctx.upload(p, rows, cols, 0.75)
        (y,) = ctx.ternary_linear([w], x[None, :].copy())
        exp = orc.gemm_f32(p, rows, cols, 0.75, q, sa, su)
        assert np.array_equal(y, exp, equal_nan=True)
        w.free()


@pytest.mark.gpu
def test_memcpy_d2d_sizes(ctx):
    lib = ctx.lib
    rng = np.random.default_rng(5)
    for n, off in [(0, 0), (1, 0), (15, 0), (16, 0), (4096 + 7, 0), (1 << 20, 0), (1000, 3), (100000, 1)]:
        announce(f"memcpy_d2d n={n} off={off}")
        src_h = rng.integers(0, 256, n + 64, dtype=np.uint8)
        a, b = C.c_void_p(), C.c_void_p()
        ctx.check(lib.lbt_dev_alloc(ctx.h, n + 64, C.byref(a)))
        ctx.check(lib.lbt_dev_alloc(ctx.h, n + 64, C.byref(b)))
        ctx.check(lib.lbt_memcpy_h2d(ctx.h, a, src_h.ctypes.data, n + 64))
        zeros = np.zeros(n + 64, np.uint8)  # kept alive across the call
        ctx.check(lib.lbt_memcpy_h2d(ctx.h, b, zeros.ctypes.data, n + 64))
        ctx.check(lib.lbt_memcpy_d2d(ctx.h, C.c_void_p(b.value + off), C.c_void_p(a.value + off), n))
        ctx.sync()
        got = np.zeros(n + 64, np.uint8)
        ctx.check(lib.lbt_memcpy_d2h(ctx.h, got.ctypes.data, b, n + 64))
        exp = np.zeros(n + 64, np.uint8)
        exp[off:off + n] = src_h[off:off + n]
        assert np.array_equal(got, exp)
        lib.lbt_dev_free(ctx.h, a)
        lib.lbt_dev_free(ctx.h, b)


def test_batched_bf16_head_kernels_agree(ctx, ctx_with):
    """The batched bf16 head on the weight-streaming kernel (default) and on
    lmhead_batch_kernel (LBT_HEAD_BATCH_CLASSIC) give the same logits bit for
    bit, at the 2B head's width for 16..64 rows."""
    rng = np.random.default_rng(31)
    rows, cols = 20000, 2560
    wb = orc.f32_to_bf16((rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)).reshape(rows, cols)
    c2 = ctx_with(LBT_HEAD_BATCH_CLASSIC="1")
    w1, w2 = ctx.bf16_upload(wb), c2.bf16_upload(wb)
    for m in (16, 33, 64):
        announce(f"batched head kernels m={m}")
        x = rng.standard_normal((m, cols)).astype(np.float32)
        assert np.array_equal(ctx.bf16_linear(w1, x), c2.bf16_linear(w2, x)), m
    w1.free()
    w2.free()
