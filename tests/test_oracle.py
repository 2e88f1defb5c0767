"""Pins the CPU oracle (oracle/) before anything is compared against it.

Each oracle function is checked against something other than itself:
  * known answers from the reference's own unit tests;
  * closed forms (extreme values, padding, ties, special floats);
  * independent implementations: brute force over unpacked weights
    (ternary-kernels/src/reference.rs:7-16), the SIMD port (different
    instructions, same semantics), f64 evaluations;
  * the committed golden fixtures (tests/golden/).
"""
import json
import math
from pathlib import Path

import numpy as np
import pytest

import lbt_oracle as orc
from refgen import XorShift, golden_case, quant_rnd_vec

GOLDEN = Path(__file__).resolve().parent / "golden"


# ---- pack.rs ----------------------------------------------------------------
@pytest.mark.parametrize("cols", [1, 31, 128, 129, 300, 512])
def test_pack_roundtrip_with_padding(cols):
    # pack.rs:149-161
    rows = 3
    i = np.arange(rows * cols)
    vals = (((i * 7 + i // 3) % 3) - 1).astype(np.int8).reshape(rows, cols)
    p = orc.pack(vals)
    assert p.shape == (rows, orc.padded_cols(cols) // 4)
    assert np.array_equal(orc.unpack(p, cols), vals)
    full = orc.unpack(p, orc.padded_cols(cols))
    assert np.all(full[:, cols:] == 0)


def test_pack_byte_closed_form():
    # pack.rs:1-16: byte j of a block holds weight k*32+j in bits 2k..2k+1 as w+1.
    w = np.zeros((1, 128), np.int8)
    w[0, 0 * 32 + 5] = -1  # code 0 in bits 0-1
    w[0, 1 * 32 + 5] = 1  # code 2 in bits 2-3
    w[0, 2 * 32 + 5] = 0  # code 1 in bits 4-5
    w[0, 3 * 32 + 5] = 1  # code 2 in bits 6-7
    p = orc.pack(w)
    assert p[0, 5] == (0 << 0) | (2 << 2) | (1 << 4) | (2 << 6)
    assert p[0, 4] == 0x55  # all-zero weights are code 1 in all four lanes


def test_ternarize_matches_torch_semantics():
    # pack.rs:163-170
    t, s = orc.ternarize_absmean(np.array([0.5, 1.5, -0.5, -2.0, 0.0, 1.5], np.float32))
    assert s == 1.0
    assert list(t) == [0, 1, 0, -1, 0, 1]


# ---- quant.rs -----------------------------------------------------------------
def test_quantizes_like_actquant():
    # quant.rs:201-209
    q, s, su = orc.quantize_acts(np.array([[1.0, -0.5, 0.25, 0.0, -1.0]], np.float32))
    assert s[0] == 127.0
    assert list(q[0, :5]) == [127, -64, 32, 0, -127]
    assert np.all(q[0, 5:] == 0)
    assert su[0] == 127 - 64 + 32 - 127


def test_ternary_kernels_quant_known_answer():
    # crates/ternary-kernels/src/quant.rs:33-42
    q, s, su = orc.quantize_row(np.array([1.0, -2.0, 0.5, 0.0], np.float32))
    assert s == np.float32(63.5)
    assert list(q) == [64, -127, 32, 0]
    assert su == 64 - 127 + 32


def test_zero_row_is_safe():
    # quant.rs:212-216
    q, s, su = orc.quantize_acts(np.zeros((1, 4), np.float32))
    assert s[0] == np.float32(127.0) / np.float32(1e-5)
    assert np.all(q == 0) and su[0] == 0


def quant_cases():
    # quant.rs:234-264
    cases = [quant_rnd_vec(seed, n) for seed, n in [(1, 2560), (2, 6912), (3, 31), (4, 33), (5, 7), (6, 1), (7, 130)]]
    ties = np.array([(i - 48) + 0.5 for i in range(96)] + [127.0], np.float32)
    cases.append(ties)
    odd = quant_rnd_vec(9, 70)
    odd[3] = np.nan
    odd[40] = np.nan
    odd[5] = np.float32(1e-42)
    odd[6] = -0.0
    cases.append(odd)
    inf = quant_rnd_vec(10, 64)
    inf[10] = np.inf
    inf[50] = -np.inf
    cases.append(inf)
    cases.append(np.zeros(40, np.float32))
    cases.append(np.full(40, 1e-30, np.float32))
    return cases


def test_quant_scalar_matches_simd_port_on_reference_edge_cases():
    for x in quant_cases():
        a = orc.quantize_row(x)
        b = orc.port_quantize_row(x)
        assert np.float32(a[1]).tobytes() == np.float32(b[1]).tobytes()
        assert a[2] == b[2]
        assert np.array_equal(a[0], b[0])


def test_quant_ties_round_half_even():
    # amax 127 -> scale 1: values k + 0.5 round to the even neighbour
    x = np.array([(i - 48) + 0.5 for i in range(96)] + [127.0], np.float32)
    q, s, _ = orc.quantize_row(x)
    assert s == 1.0
    for v, r in zip(x[:-1], q[:-1]):
        lo = math.floor(v)
        assert r == (lo if lo % 2 == 0 else lo + 1)


def test_quant_special_values():
    x = np.array([np.nan, 2.0, -np.inf, 1.0], np.float32)
    q, s, su = orc.quantize_row(x)
    # amax ignores NaN and sees inf -> scale = 127/inf = 0; inf*0 = NaN -> 0
    assert s == 0.0
    assert list(q) == [0, 0, 0, 0]
    x = np.array([np.nan, 2.0, -1.0], np.float32)
    q, s, su = orc.quantize_row(x)
    assert s == np.float32(63.5) and list(q) == [0, 127, -64] and su == 63


# ---- gemm.rs ------------------------------------------------------------------------
GOLDEN_SHAPES = [(1, 128, 1), (7, 128, 1), (33, 256, 1), (17, 384, 1), (64, 640, 1), (40, 2560, 1), (9, 6912, 1)]


@pytest.mark.parametrize("rows,cols,m", GOLDEN_SHAPES + [(23, 384, 5), (5, 100, 3), (5, 129, 3), (5, 300, 3)])
def test_gemm_i32_equals_bruteforce_and_f64(rows, cols, m):
    # golden.rs:25-75 (integer exact, float within 1e-5 of the magnitude sum)
    t, scale, x = golden_case(rows, cols, m, rows * 31 + cols)
    p = orc.pack(t)
    q, sa, su = orc.quantize_acts(x)
    got = orc.gemm_i32(p, rows, cols, q, su)
    assert np.array_equal(got, orc.gemm_i32_bruteforce(p, rows, cols, q))
    exact = q[:, :cols].astype(np.int64) @ t.T.astype(np.int64)
    assert np.array_equal(got, exact)
    y = orc.gemm_f32(p, rows, cols, scale, q, sa, su)
    terms = (q[:, :cols].astype(np.float64) / sa[:, None].astype(np.float64))[:, None, :] * (
        t.astype(np.float64) / np.float64(scale))[None, :, :]
    ref, mag = terms.sum(-1), np.abs(terms).sum(-1)
    assert np.all(np.abs(y - ref) <= 1e-5 * np.maximum(mag, 1e-6))
    # bit-exact epilogue definition (gemm.rs:141,150; golden.rs:144-152)
    inv = (np.float32(1.0) / (sa * np.float32(scale))).astype(np.float32)
    assert np.array_equal(y, (got.astype(np.float32) * inv[:, None]).astype(np.float32))


def test_gemm_extreme_values():
    # golden.rs:108-122
    rows, cols = 4, 6912
    p = orc.pack(np.ones((rows, cols), np.int8))
    for sign in (1.0, -1.0):
        q, sa, su = orc.quantize_acts(np.full((1, cols), sign, np.float32))
        got = orc.gemm_i32(p, rows, cols, q, su)
        assert np.all(got == int(sign) * 127 * cols)


def test_prefill_extreme_long_rows():
    # golden.rs:181-194
    rows, cols, m = 3, 6912 * 2, 5
    p = orc.pack(np.ones((rows, cols), np.int8))
    for sign in (1.0, -1.0):
        q, sa, su = orc.quantize_acts(np.full((m, cols), sign, np.float32))
        y = orc.gemm_f32(p, rows, cols, 1.0, q, sa, su)
        assert np.all(y == np.float32(sign * 127.0 * cols / 127.0))


@pytest.mark.parametrize("threads", [1, 3, 8])
def test_port_gemm_matches_scalar(threads):
    # golden.rs:128-176: fused / threaded paths give the same integers
    rng = XorShift(4242)
    cols = 640
    for rows in (96, 24, 200):
        t = np.array([(rng.next() % 3) - 1 for _ in range(rows * cols)], np.int8).reshape(rows, cols)
        p = orc.pack(t)
        for m in (1, 2, 5, 64):
            x = np.array([rng.f() * (30 if i % 89 == 1 else 1) for i in range(m * cols)], np.float32).reshape(m, cols)
            q, sa, su = orc.quantize_acts(x)
            assert np.array_equal(orc.port_gemm_i32(p, rows, cols, q, su, threads), orc.gemm_i32(p, rows, cols, q, su))


# ---- bf16.rs --------------------------------------------------------------------------
def test_bf16_dots_within_reference_tolerance():
    # bf16.rs:112-136: all kernels within 1e-4 abs of f64
    rows, cols = 37, 2560 + 24
    rng = XorShift(12345)
    wf = np.array([rng.f() * np.float32(0.05) for _ in range(rows * cols)], np.float32)
    w = (wf.view(np.uint32) >> 16).astype(np.uint16).reshape(rows, cols)
    x = np.array([rng.f() for _ in range(cols)], np.float32)
    ref = orc.bf16_to_f32(w).astype(np.float64) @ x.astype(np.float64)
    lanes = orc.bf16_gemv_lanes(w, x)
    port = orc.port_bf16_gemv(w, x)
    scal = np.array([orc.bf16_dot_ref(w[r], x) for r in range(rows)], np.float32)
    for got in (lanes, port, scal):
        assert np.all(np.abs(got.astype(np.float64) - ref) < 1e-4)


def test_bf16_rounding_closed_form():
    v = np.array([1.0, 1.00390625, 1.005859375, -2.5, np.inf, np.nan], np.float32)
    b = orc.f32_to_bf16(v)
    # 1 + 2^-8 is a tie between 1 and 1 + 2^-7: even mantissa (1.0) wins
    assert list(b[:5]) == [0x3F80, 0x3F80, 0x3F81, 0xC020, 0x7F80]
    assert b[5] == 0x7FC0


# ---- float building blocks ---------------------------------------------------------------
def test_tree_and_sumsq_exact_on_integers():
    # small integers: every partial sum is exact, so any order gives the true sum
    x = (np.arange(2000) % 101 - 50).astype(np.float32)  # squares <= 2500, total < 2^24
    got = orc.lib().or_sumsq(orc._p(x), x.size)
    assert got == float(np.sum(x.astype(np.float64) ** 2))


def test_rmsnorm_vs_f64():
    rng = np.random.default_rng(1)
    for n in (7, 256, 2560, 6912):
        x = rng.standard_normal(n).astype(np.float32) * 3
        w = rng.uniform(0.5, 1.5, n).astype(np.float32)
        got = orc.rmsnorm(x, w, 1e-5)
        ref = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-5) * w
        assert np.allclose(got, ref, rtol=2e-6, atol=1e-6)


def test_expf_accuracy():
    xs = np.concatenate([np.linspace(-87, 0, 200001, dtype=np.float32), np.linspace(0, 88, 20001, dtype=np.float32)])
    got = np.array([orc.expf(float(v)) for v in xs[::7]], np.float32)
    ref = np.exp(xs[::7].astype(np.float64))
    ulp = np.abs(got.astype(np.float64) - ref) / np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert ulp.max() <= 2.0
    assert orc.expf(0.0) == 1.0
    assert orc.expf(-100.0) == 0.0
    assert np.isinf(orc.expf(100.0))


def test_rope_tables_closed_form():
    c, s = orc.rope_tables(128, 64, 500000.0)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    inv = (1.0 / 500000.0 ** (np.arange(64) * 2 / 128)).astype(np.float32)
    ang = (np.arange(64, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float32).astype(np.float64)
    assert np.array_equal(c, np.cos(ang).astype(np.float32))
    assert np.array_equal(s, np.sin(ang).astype(np.float32))


def test_argmax_first_max():
    v = np.array([1.0, 3.0, 2.0, 3.0], np.float32)
    assert orc.lib().or_argmax(orc._p(v), 4) == 1


# ---- synthetic generator -------------------------------------------------------------------
def test_synthetic_ternary_distribution_and_packing():
    rows, cols = 64, 2560
    p = orc.synth_packed(7, orc.t_layer(0, 0), rows, cols)
    t = orc.unpack(p, cols)
    frac = [(t == v).mean() for v in (-1, 0, 1)]
    assert abs(frac[0] - 0.3) < 0.01 and abs(frac[1] - 0.4) < 0.01 and abs(frac[2] - 0.3) < 0.01
    direct = np.array([[orc.lib().or_synth_ternary(7, orc.t_layer(0, 0), r * cols + c) for c in range(200)]
                       for r in range(3)], np.int8)
    assert np.array_equal(t[:3, :200], direct)


# ---- golden fixtures ------------------------------------------------------------------------
def test_golden_fixtures():
    files = sorted(GOLDEN.glob("gemm_*.npz"))
    assert files, "golden fixtures missing (tests/golden/make_golden.py)"
    for f in files:
        z = np.load(f)
        rows, cols = int(z["rows"]), int(z["cols"])
        q, sa, su = orc.quantize_acts(z["x"])
        assert np.array_equal(q, z["q"]) and np.array_equal(sa, z["s_a"]) and np.array_equal(su, z["qsum"])
        got = orc.gemm_i32(z["packed"], rows, cols, q, su)
        assert np.array_equal(got, z["i32"]), f.name
        y = orc.gemm_f32(z["packed"], rows, cols, float(z["s_w"]), q, sa, su)
        assert np.array_equal(y, z["f32"]), f.name


def test_known_answer_fixture():
    ka = json.loads((GOLDEN / "known_answers.json").read_text())
    for case in ka["quantize"]:
        x = np.array(case["x"], np.float32)
        q, s, su = orc.quantize_row(x)
        assert list(q) == case["q"] and su == case["sum"]
        assert np.float32(s) == np.float32(case["scale"])
