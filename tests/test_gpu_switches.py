"""The alternative device paths behind the environment switches give the
oracle's results bit for bit: several-token products on the VALU GEMV below
an MFMA token count (LBT_MFMA_MIN), and the batched LM head with 8-token
groups (LBT_HEAD_TG8).  The library reads the switches when a context is
created."""
import numpy as np
import pytest

import lbt_hip
import lbt_oracle as orc
from conftest import announce

pytestmark = pytest.mark.gpu

CFG = dict(hidden=256, intermediate=512, heads=4, kv_heads=2, layers=2, vocab=1000, max_pos=1024)


def models(ctx, seed):
    m = lbt_hip.Model.synthetic(ctx, lbt_hip.make_config(**CFG), seed)
    om = orc.OracleModel(orc.config(**CFG), seed)
    return m, om


@pytest.mark.parametrize("var,val", [("LBT_MFMA_MIN", "16")])
def test_switch_prefill_and_decode_match_oracle(ctx_with, var, val):
    ctx = ctx_with(**{var: val, "LBT_NO_GRAPH": "1"})
    announce(f"switch {var}={val}")
    m, om = models(ctx, 21)
    c = m.new_cache()
    prompt = np.array([5, 99, 400, 7, 12, 800, 3, 41], np.uint32)
    got = m.forward(prompt, c, all_logits=True)
    assert np.array_equal(got, om.forward(prompt, all_logits=True))
    tok = int(got[-1].argmax())
    for step in range(3):
        g = m.forward([tok], c)
        e = om.forward([tok])
        assert np.array_equal(g, e), f"step {step}"
        tok = int(e[0].argmax())
    c.free()
    m.free()
    om.free()


def test_head_tg8_batch_matches_single(ctx_with):
    ctx = ctx_with(LBT_HEAD_TG8="1")
    nseq = 17
    announce(f"switch LBT_HEAD_TG8 nseq={nseq}")
    m, om = models(ctx, 22)
    b = m.new_batch(nseq, 64)
    prompts = [np.array([2 + s, 30 + s, 500 + s], np.uint32) for s in range(nseq)]
    nxt = [b.prefill(s, prompts[s]) for s in range(nseq)]
    logits, _ = b.forward(np.array(nxt, np.uint32))
    for s in range(nseq):
        c = m.new_cache()
        m.forward(prompts[s], c)
        assert np.array_equal(logits[s], m.forward([nxt[s]], c)[0]), f"seq {s}"
        c.free()
    b.free()
    m.free()
    om.free()
