"""One-dispatch decode step (all decoder layers of a token in one dispatch,
epoch-tagged activation words between workgroups) against the oracle and
against the multi-kernel graph step: tokens and the final hidden state
identical bit for bit, for several model shapes, including the full
2B-shaped model."""
import numpy as np
import pytest

import lbt_hip
import lbt_oracle as orc
from conftest import announce, step_built

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not step_built(), reason="one-dispatch step not built (LBT_WITH_STEP=1)")]


def run_decode(m, prompt, steps):
    c = m.new_cache()
    first = m.forward_argmax(prompt, c)
    toks, ms = m.decode_greedy(c, first, steps)
    hid = m.read_hidden(1)
    c.free()
    return first, list(toks), hid


@pytest.mark.parametrize("shape", [dict(hidden=512, intermediate=1536, heads=4, kv_heads=1, layers=3),
                                   dict(hidden=256, intermediate=512, heads=4, kv_heads=2, layers=2),
                                   dict(hidden=512, intermediate=1024, heads=2, kv_heads=1, layers=2)])
@pytest.mark.parametrize("kind", [0, 1])
def test_step_matches_oracle_small(ctx, shape, kind):
    cfg = dict(shape, vocab=1000, max_pos=512)
    announce(f"decode kind {kind} vs oracle {shape}")
    m = lbt_hip.Model.synthetic(ctx, lbt_hip.make_config(**cfg), 17)
    m.set_decode(kind)
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
                                   dict(hidden=1024, intermediate=2816, heads=8, kv_heads=2, layers=2),
                                   dict(hidden=512, intermediate=1024, heads=2, kv_heads=1, layers=2)])
def test_step_equals_graph_path(ctx, shape):
    cfg = dict(shape, vocab=777, max_pos=2048)
    announce(f"decode step vs graph {shape}")
    m = lbt_hip.Model.synthetic(ctx, lbt_hip.make_config(**cfg), 5)
    prompt = (np.arange(11) * 13 % cfg["vocab"]).astype(np.uint32)
    a = run_decode(m, prompt, 30)
    m.set_decode(1)
    b = run_decode(m, prompt, 30)
    assert a[0] == b[0] and a[1] == b[1]
    assert np.array_equal(a[2], b[2])
    m.free()


def test_step_long_context_equals_graph_path(ctx):
    """Contexts past 1024 keys: more than 64 keys per split, and more
    (head, split) items than workgroups on some shapes."""
    cfg = dict(hidden=512, intermediate=1024, heads=8, kv_heads=2, layers=2, vocab=500, max_pos=4096)
    announce("decode step long context")
    m = lbt_hip.Model.synthetic(ctx, lbt_hip.make_config(**cfg), 9)
    prompt = (np.arange(1100) * 7 % cfg["vocab"]).astype(np.uint32)
    a = run_decode(m, prompt, 40)
    m.set_decode(1)
    b = run_decode(m, prompt, 40)
    assert a[0] == b[0] and a[1] == b[1]
    assert np.array_equal(a[2], b[2])
    m.free()


def test_step_full_2b_equals_graph_path(ctx):
    announce("decode step full 2B")
    m = lbt_hip.Model.synthetic(ctx, lbt_hip.make_config(), 2026)
    prompt = np.random.default_rng(64).integers(0, 128256, 64).astype(np.uint32)
    a = run_decode(m, prompt, 48)
    m.set_decode(1)
    b = run_decode(m, prompt, 48)
    assert a[1] == b[1]
    assert np.array_equal(a[2], b[2])
    m.free()
