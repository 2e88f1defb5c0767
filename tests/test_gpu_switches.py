"""The alternative device paths behind the environment switches give the
oracle's results bit for bit: several-token products on the VALU GEMV below
an MFMA token count (LBT_MFMA_MIN), the batched LM head with 8-token groups
(LBT_HEAD_TG8), the one-token GEMV prologue on 16 / 4 wavefronts
(LBT_GEMV_PW, LBT_GEMV_PWO), the 1024-thread row quantizer (LBT_QUANT_WIDE),
the few-token GEMM thresholds (LBT_GEMM_SMALL_MAX, LBT_GEMM_SMALL_TILES) and
the one-wavefront attention on batched rows (LBT_ATTN_WAVE).  The library
reads the switches when a context is created."""
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


# two layers at the 2B widths (hidden 2560, FFN 6912, 20 / 5 heads of 128):
# rows wide enough for every quantizer and GEMV prologue variant
WIDE = dict(hidden=2560, intermediate=6912, heads=20, kv_heads=5, layers=2, vocab=1000, max_pos=256)


@pytest.mark.parametrize("env", [dict(LBT_GEMV_PW="16"), dict(LBT_GEMV_PWO="4"), dict(LBT_QUANT_WIDE="1"),
                                 dict(LBT_GEMM_SMALL_MAX="4", LBT_GEMM_SMALL_TILES="0"),
                                 dict(LBT_GEMM_SMALL_MAX="64"), dict(LBT_GEMM_SMALL_TILES="1000")],
                         ids=lambda e: ",".join(f"{k}={v}" for k, v in e.items()))
@pytest.mark.parametrize("graph", [False, True])
def test_switch_2b_widths_match_oracle(ctx_with, env, graph):
    # a 40-token prompt (the GEMM path and its row quantizer), then three
    # single-token steps (the one-token GEMV and its fused prologues), eager
    # and graph-replayed; logits bit-exact to the oracle
    ctx = ctx_with(**env) if graph else ctx_with(**env, LBT_NO_GRAPH="1")
    announce(f"switch {env} graph={graph}")
    m = lbt_hip.Model.synthetic(ctx, lbt_hip.make_config(**WIDE), 23)
    om = orc.OracleModel(orc.config(**WIDE), 23)
    c = m.new_cache()
    prompt = (np.arange(40) * 53 % WIDE["vocab"]).astype(np.uint32)
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


def test_batch_wave_attention_matches_oracle(ctx_with):
    # LBT_ATTN_WAVE=1 on the batched path: one wavefront per (row, KV head,
    # split) for every sequence's prefill and for the batched steps, whose
    # rows each sit at their own position (4 query heads per KV head, head_dim
    # 128); logits and greedy tokens bit-exact to the oracle per sequence
    cfg = dict(hidden=512, intermediate=1536, heads=4, kv_heads=1, layers=2, vocab=1000, max_pos=1024)
    nseq, seed = 5, 24
    announce(f"switch LBT_ATTN_WAVE=1 batch nseq={nseq}")
    m = lbt_hip.Model.synthetic(ctx_with(LBT_ATTN_WAVE="1"), lbt_hip.make_config(**cfg), seed)
    b = m.new_batch(nseq, 512)
    rng = np.random.default_rng(nseq)
    oms, nxt = [], []
    for s in range(nseq):
        prompt = rng.integers(0, cfg["vocab"], 1 + (41 * s + 9) % 150).astype(np.uint32)
        om = orc.OracleModel(orc.config(**cfg), seed)
        exp = int(om.forward(prompt)[0].argmax())
        assert b.prefill(s, prompt) == exp, f"prefill seq {s}"
        oms.append(om)
        nxt.append(exp)
    logits, nx = b.forward(np.array(nxt, np.uint32))
    for s in range(nseq):
        e = oms[s].forward([nxt[s]])
        assert np.array_equal(logits[s], e[0]), f"logits seq {s}"
    steps = 4
    toks, _ = b.decode_greedy(nx, steps)
    for s in range(nseq):
        t = int(nx[s])
        for i in range(steps):
            t = int(oms[s].forward([t])[0].argmax())
            assert toks[i, s] == t, f"seq {s} step {i}"
    for om in oms:
        om.free()
    b.free()
    m.free()
