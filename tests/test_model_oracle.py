"""Pins the f32 model oracle (device float order) against an independent f64
restatement of BitNet::forward (tests/ref_model64.py) on small random models,
and checks the incremental-decode invariant of the KV cache."""
import numpy as np
import pytest

import lbt_oracle as orc
from ref_model64 import RefModel64, synthetic_weights

SMALL = dict(hidden=256, intermediate=512, heads=4, kv_heads=2, layers=2, vocab=512, max_pos=512)


def small_cfg(**kw):
    d = dict(SMALL, **kw)
    return orc.config(d["hidden"], d["intermediate"], d["heads"], d["kv_heads"], d["layers"], d["vocab"], d["max_pos"])


def test_model_oracle_vs_f64():
    cfg = small_cfg()
    seed = 11
    om = orc.OracleModel(cfg, seed)
    ref = RefModel64(dict(SMALL, eps=1e-5, theta=500000.0), synthetic_weights(orc, cfg, seed))
    rng = np.random.default_rng(0)
    prompt = rng.integers(0, cfg.vocab, 12).astype(np.uint32)
    a = om.forward(prompt, all_logits=True)
    b = ref.forward(prompt, all_logits=True)
    assert np.allclose(a, b, rtol=1e-3, atol=1e-2), np.abs(a - b).max()
    assert np.array_equal(a.argmax(-1), b.argmax(-1))
    tok = int(a[-1].argmax())
    for _ in range(6):
        la = om.forward([tok])
        lb = ref.forward([tok])
        assert np.allclose(la, lb, rtol=1e-3, atol=1e-2), np.abs(la - lb).max()
        assert la.argmax() == lb.argmax()
        tok = int(la.argmax())
    om.free()


def test_prefill_equals_incremental_decode_bitwise():
    cfg = small_cfg(layers=1)
    toks = np.array([3, 77, 5, 400, 9, 12, 100], np.uint32)
    a = orc.OracleModel(cfg, 5)
    la = a.forward(toks, all_logits=True)
    b = orc.OracleModel(cfg, 5)
    rows = [b.forward(toks[:3], all_logits=True)]
    for t in toks[3:]:
        rows.append(b.forward([t], all_logits=True))
    lb = np.concatenate(rows)
    assert np.array_equal(la, lb)
    assert np.array_equal(a.kcache(0, 7), b.kcache(0, 7))
    a.free()
    b.free()


def test_fast_mode_same_logits():
    cfg = small_cfg()
    toks = np.array([1, 2, 3, 4], np.uint32)
    a = orc.OracleModel(cfg, 3)
    la = a.forward(toks)
    old = orc.set_fast(1)
    try:
        b = orc.OracleModel(cfg, 3)
        lb = b.forward(toks)
    finally:
        orc.set_fast(old)
    assert np.array_equal(la, lb)
    a.free()
    b.free()


def test_cpu_baseline_mode_close_to_device_order():
    """The timed CPU baseline (fast mode 2: SIMD attention and bf16 head in the
    reference's plain order, any thread count) computes the same model: logits
    within float tolerance of the device-order oracle, same argmax."""
    cfg = small_cfg()
    toks = np.array([1, 2, 3, 4, 5, 6, 7, 8], np.uint32)
    a = orc.OracleModel(cfg, 3)
    la = a.forward(toks, all_logits=True)
    la2 = a.forward([9])
    old = orc.set_fast(2)
    try:
        for nt in (1, 0):
            orc.set_threads(nt)
            b = orc.OracleModel(cfg, 3)
            lb = b.forward(toks, all_logits=True)
            lb2 = b.forward([9])
            b.free()
            np.testing.assert_allclose(lb, la, rtol=1e-3, atol=1e-3)
            np.testing.assert_allclose(lb2, la2, rtol=1e-3, atol=1e-3)
            assert np.array_equal(lb.argmax(1), la.argmax(1))
    finally:
        orc.set_threads(0)
        orc.set_fast(old)
    a.free()
