"""The opt-in int8 LM head's oracle (q8head.rs) pinned by the reference's own
tests (q8head.rs:80-128, same generator and sizes) and by known answers of
the quantizer's definition (round half to even, clamp, zero and NaN rows)."""
import numpy as np

import lbt_oracle as orc
from refgen import XorShift, q8_bf16_matrix, xorshift_f32


def bf16(vals):
    return orc.f32_to_bf16(np.asarray(vals, np.float32))


def test_known_answers():
    # amax 127 -> scale exactly 1.0, so q = rint_even(w): 2.5 -> 2, 3.5 -> 4
    w = bf16([127.0, 2.5, 3.5, -2.5, -0.5, 0.5, 1.5, -127.0]).reshape(1, 8)
    q, s = orc.q8head_from_bf16(w)
    assert s[0] == np.float32(1.0)
    assert q.tolist() == [[127, 2, 4, -2, 0, 0, 2, -127]]
    # amax 2 -> scale 2/127: w / scale = 63.5 exactly for w = 1 (ties to 64)
    w = bf16([2.0, 1.0, -1.0, 0.0]).reshape(1, 4)
    q, s = orc.q8head_from_bf16(w)
    assert s[0] == np.float32(2.0) / np.float32(127.0)
    assert q[0, 0] == 127
    assert q[0, 1] == int(np.rint(np.float32(1.0) / s[0])) and abs(q[0, 1]) == abs(q[0, 2])


def test_zero_and_nan_rows():
    w = np.zeros((3, 16), np.uint16)
    w[1] = bf16(np.linspace(-1, 1, 16))
    w[2] = bf16(np.linspace(-3, 3, 16))
    w[2, 5] = 0x7FC0  # NaN: ignored by the max, quantizes to 0
    q, s = orc.q8head_from_bf16(w)
    assert s[0] == 1.0 and not q[0].any()
    assert q[2, 5] == 0
    assert s[2] == np.float32(3.0) / np.float32(127.0)
    assert q[2, 0] == -127 and q[2, 15] == 127


def test_quantizer_matches_definition_bruteforce():
    rng = np.random.default_rng(3)
    w = bf16(rng.standard_normal((50, 130)) * 0.07).reshape(50, 130)
    q, s = orc.q8head_from_bf16(w)
    wf = orc.bf16_to_f32(w).reshape(50, 130)
    amax = np.abs(wf).max(axis=1)
    es = np.where(amax == 0, np.float32(1.0), amax / np.float32(127.0)).astype(np.float32)
    assert s.tobytes() == es.tobytes()
    eq = np.clip(np.rint(wf / es[:, None]), -127, 127).astype(np.int8)
    assert np.array_equal(q, eq)


def test_q8_matches_dequantized_reference():
    """q8head.rs:84-97: every row within 1e-4 * sum|terms| of the f64 sum."""
    rows, cols = 300, 2560
    rnd = XorShift(0x9E3779B97F4A7C15)
    w = q8_bf16_matrix(rnd, rows * cols, 0.05).reshape(rows, cols)
    x = xorshift_f32(rnd, cols)
    q, s = orc.q8head_from_bf16(w)
    terms = s[:, None].astype(np.float64) * q.astype(np.float64) * x[None, :].astype(np.float64)
    ref, mag = terms.sum(axis=1), np.abs(terms).sum(axis=1)
    for out in (orc.q8head_gemv_ref(q, s, x), orc.q8head_gemv_lanes(q, s, x)):
        assert np.all(np.abs(out.astype(np.float64) - ref) <= 1e-4 * mag)


def test_q8_argmax_agrees_with_bf16():
    """q8head.rs:99-117: argmax of the int8 head equals the bf16 head's on at
    least 190 of 200 inputs (scalar bf16 kernel, dot_scalar order)."""
    rows, cols = 2000, 512
    rnd = XorShift(42)
    w = q8_bf16_matrix(rnd, rows * cols, 0.05).reshape(rows, cols)
    q, s = orc.q8head_from_bf16(w)
    agree = 0
    for _ in range(200):
        x = xorshift_f32(rnd, cols)
        a = orc.q8head_gemv_ref(q, s, x)
        b = np.array([orc.bf16_dot_ref(w[r], x) for r in range(rows)], np.float32)
        agree += int(np.argmax(a) == np.argmax(b))
    assert agree >= 190, agree


def test_zero_row_is_safe():
    """q8head.rs:119-128."""
    rows, cols = 3, 40
    rnd = XorShift(7)
    w = q8_bf16_matrix(rnd, rows * cols, 0.05).reshape(rows, cols)
    w[1] = 0
    q, s = orc.q8head_from_bf16(w)
    assert s[1] == 1.0
    x = xorshift_f32(rnd, cols)
    assert orc.q8head_gemv_ref(q, s, x)[1] == 0.0
    assert orc.q8head_gemv_lanes(q, s, x)[1] == 0.0


def test_lane_order_against_bruteforce():
    """The device order is a fixed reassociation of the same products: the
    64-lane butterfly of per-lane fused chains, scaled; recomputed here with
    numpy on a tiny case."""
    rng = np.random.default_rng(11)
    q = rng.integers(-127, 128, (3, 1024)).astype(np.int8)
    s = rng.random(3).astype(np.float32)
    x = rng.standard_normal(1024).astype(np.float32)
    got = orc.q8head_gemv_lanes(q, s, x)
    for r in range(3):
        lane = np.zeros(64, np.float32)
        for l in range(64):
            acc = np.float32(0)
            for c in range(l, 128, 64):
                for e in range(8):
                    k = 8 * c + e
                    acc = np.float32(np.float64(q[r, k]) * np.float64(x[k]) + np.float64(acc))
            lane[l] = acc
        for m in (32, 16, 8, 4, 2, 1):
            lane = (lane + lane[np.arange(64) ^ m]).astype(np.float32)
        assert got[r] == np.float32(s[r] * lane[0])


def test_model_int8_head_close_to_bf16_head():
    cfg = orc.config(hidden=256, intermediate=512, heads=4, kv_heads=2, layers=1, vocab=700, max_pos=64)
    a = orc.OracleModel(cfg, 3)
    b = orc.OracleModel(cfg, 3)
    b.set_head(1)
    toks = [1, 5, 9, 300]
    la, lb = a.forward(toks, all_logits=True), b.forward(toks, all_logits=True)
    assert not np.array_equal(la, lb)
    scale = np.abs(la).max()
    assert np.abs(la - lb).max() < 0.02 * scale
    a.free()
    b.free()
