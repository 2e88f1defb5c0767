"""Persistent decode step (one dispatch for all layers of a token, flag grid
barriers) against the oracle and against the per-kernel graph path: tokens
and the final hidden state identical bit for bit, for several grid sizes and
model shapes, including the full 2B-shaped model."""
import numpy as np
import pytest

import lbt_hip
import lbt_oracle as orc
from conftest import announce

pytestmark = pytest.mark.gpu


def run_decode(m, prompt, steps):
    c = m.new_cache()
    first = m.forward_argmax(prompt, c)
    toks, ms = m.decode_greedy(c, first, steps)
    hid = m.read_hidden(1)
    c.free()
    return first, list(toks), hid


@pytest.mark.parametrize("G", ["64", "16", "128"])
def test_persistent_matches_oracle_small(ctx, monkeypatch, G):
    cfg = dict(hidden=512, intermediate=1536, heads=4, kv_heads=1, layers=3, vocab=1000, max_pos=512)
    announce(f"persistent small G={G}")
    monkeypatch.setenv("LBT_DECODE", "persistent")
    monkeypatch.setenv("LBT_PERSIST_G", G)
    m = lbt_hip.Model.synthetic(ctx, lbt_hip.make_config(**cfg), 17)
    om = orc.OracleModel(orc.config(**cfg), 17)
    prompt = np.array([3, 1, 4, 1, 5, 9, 2, 6], np.uint32)
    first, toks, hid = run_decode(m, prompt, 20)
    tok = int(om.forward(prompt)[0].argmax())
    assert first == tok
    exp = []
    for _ in range(20):
        tok = int(om.forward([tok])[0].argmax())
        exp.append(tok)
    assert toks == exp
    assert np.array_equal(hid, om.hidden(1))
    m.free()
    om.free()


@pytest.mark.parametrize("shape", [dict(hidden=256, intermediate=512, heads=4, kv_heads=2, layers=2),
                                   dict(hidden=384, intermediate=1000, heads=3, kv_heads=3, layers=2),
                                   dict(hidden=1024, intermediate=2816, heads=8, kv_heads=2, layers=2)])
def test_persistent_equals_graph_path(ctx, monkeypatch, shape):
    cfg = dict(shape, vocab=777, max_pos=512)
    announce(f"persistent vs graph {shape}")
    m = lbt_hip.Model.synthetic(ctx, lbt_hip.make_config(**cfg), 5)
    prompt = (np.arange(11) * 13 % cfg["vocab"]).astype(np.uint32)
    monkeypatch.setenv("LBT_DECODE", "persistent")
    a = run_decode(m, prompt, 30)
    monkeypatch.setenv("LBT_DECODE", "graph")
    b = run_decode(m, prompt, 30)
    assert a[0] == b[0] and a[1] == b[1]
    assert np.array_equal(a[2], b[2])
    m.free()


def test_persistent_full_2b_equals_graph_path(ctx, monkeypatch):
    announce("persistent full 2B")
    m = lbt_hip.Model.synthetic(ctx, lbt_hip.make_config(), 2026)
    prompt = np.random.default_rng(64).integers(0, 128256, 64).astype(np.uint32)
    monkeypatch.setenv("LBT_DECODE", "persistent")
    a = run_decode(m, prompt, 48)
    monkeypatch.setenv("LBT_DECODE", "graph")
    b = run_decode(m, prompt, 48)
    assert a[1] == b[1]
    assert np.array_equal(a[2], b[2])
    m.free()
