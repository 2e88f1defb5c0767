"""Batched decode (the B = 16 / 64 benchmark path): every sequence of a batch gets
exactly the single-sequence results of the oracle model on its own tokens —
greedy next token after its prompt, logits of a batched step (bit-exact) and
the greedy continuation — for the small-M GEMV and the int8-MFMA batch
sizes and for 1, 2 and 4 query heads per KV head (grouped attention)."""
import numpy as np
import pytest

import lbt_hip
import lbt_oracle as orc
from conftest import announce

pytestmark = pytest.mark.gpu

SMALL = dict(hidden=256, intermediate=512, heads=4, kv_heads=2, layers=2, vocab=1000, max_pos=1024)


def cfgs(**kw):
    d = dict(SMALL, **kw)
    hip = lbt_hip.make_config(d["hidden"], d["intermediate"], d["heads"], d["kv_heads"], d["layers"], d["vocab"],
                              d["max_pos"])
    orcfg = orc.config(d["hidden"], d["intermediate"], d["heads"], d["kv_heads"], d["layers"], d["vocab"], d["max_pos"])
    return hip, orcfg


@pytest.mark.parametrize("shape,nseq", [(dict(), 3), (dict(heads=4, kv_heads=1, hidden=512, intermediate=1536), 5),
                                        (dict(heads=3, kv_heads=3, hidden=384, intermediate=1000), 2),
                                        (dict(), 17)])
def test_batch_matches_single_sequence_oracle(ctx, shape, nseq):
    hip_cfg, or_cfg = cfgs(**shape)
    announce(f"batch {shape} nseq={nseq}")
    seed = 33
    m = lbt_hip.Model.synthetic(ctx, hip_cfg, seed)
    b = m.new_batch(nseq, 512)
    rng = np.random.default_rng(nseq)
    oms, nxt = [], []
    for s in range(nseq):
        prompt = rng.integers(0, or_cfg.vocab, 1 + (7 * s + 3) % 23).astype(np.uint32)
        om = orc.OracleModel(or_cfg, seed)
        exp = int(om.forward(prompt)[0].argmax())
        got = b.prefill(s, prompt)
        assert got == exp, f"prefill seq {s}"
        assert b.len(s) == prompt.size
        oms.append(om)
        nxt.append(exp)
    # one batched step with logits
    logits, nx = b.forward(np.array(nxt, np.uint32))
    for s in range(nseq):
        e = oms[s].forward([nxt[s]])
        assert np.array_equal(logits[s], e[0]), f"logits seq {s}"
        assert nx[s] == int(e[0].argmax())
    # greedy continuation, all sequences at once
    steps = 5
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


def test_batch_96_matches_fewtoken_epilogue(ctx_with):
    """96 sequences: the batched GEMMs take the pipelined MFMA tiles, whose
    full wavefront blocks use the lean q/k/v epilogue (per-sequence positions
    and cache rows); logits and greedy tokens equal those of the few-token
    kernel (LBT_GEMM_MODE=6, the general epilogue) bit for bit."""
    hip_cfg, _ = cfgs()
    announce("batch 96 sequences: pipelined tiles vs few-token kernel")
    outs = []
    for c in (ctx_with(LBT_GEMM_MODE="4"), ctx_with(LBT_GEMM_MODE="6")):
        m = lbt_hip.Model.synthetic(c, hip_cfg, 57)
        b = m.new_batch(96, 256)
        rng = np.random.default_rng(96)
        nxt = []
        for s in range(96):
            prompt = rng.integers(0, hip_cfg.vocab_size, 1 + (5 * s) % 9).astype(np.uint32)
            nxt.append(b.prefill(s, prompt))
        logits, nx = b.forward(np.array(nxt, np.uint32))
        toks, _ = b.decode_greedy(nx, 4)
        outs.append((logits, nx, toks))
        b.free()
        m.free()
    for a, b_ in zip(outs[0], outs[1]):
        assert np.array_equal(a, b_)


@pytest.mark.parametrize("wide", [False, True])
def test_batch_long_context_matches_oracle(ctx, ctx_with, wide):
    """Prompts of 1100+ tokens (65-key and longer splits: the four- and, with
    LBT_ATTN_WIDE, eight-pass K/V pipelines of the grouped attention); the
    batched step's logits bit-exact to single-sequence oracles."""
    if wide:
        ctx = ctx_with(LBT_ATTN_WIDE="1")
    hip_cfg, or_cfg = cfgs(max_pos=2048, layers=1)
    announce(f"batch long context wide={wide}")
    seed = 41
    m = lbt_hip.Model.synthetic(ctx, hip_cfg, seed)
    b = m.new_batch(3, 2048)
    oms, nxt = [], []
    for s in range(3):
        prompt = (np.arange(1100 + 97 * s, dtype=np.uint32) * (31 + s)) % or_cfg.vocab
        om = orc.OracleModel(or_cfg, seed)
        exp = int(om.forward(prompt)[0].argmax())
        assert b.prefill(s, prompt) == exp, f"prefill seq {s}"
        oms.append(om)
        nxt.append(exp)
    logits, _ = b.forward(np.array(nxt, np.uint32))
    for s in range(3):
        assert np.array_equal(logits[s], oms[s].forward([nxt[s]])[0]), f"seq {s}"
    for om in oms:
        om.free()
    b.free()
    m.free()


def test_batch_capacity_and_synthetic_fill(ctx):
    hip_cfg, _ = cfgs()
    announce("batch capacity / synthetic fill")
    m = lbt_hip.Model.synthetic(ctx, hip_cfg, 3)
    b = m.new_batch(4, 64)
    b.fill_synthetic(60, 7)
    assert all(b.len(s) == 60 for s in range(4))
    toks, _ = b.decode_greedy(np.array([1, 2, 3, 4], np.uint32), 4)
    assert toks.shape == (4, 4) and (toks < hip_cfg.vocab_size).all()
    assert all(b.len(s) == 64 for s in range(4))
    with pytest.raises(lbt_hip.LbtError, match="capacity"):
        b.forward(np.array([1, 2, 3, 4], np.uint32))
    with pytest.raises(lbt_hip.LbtError):
        m.new_batch(2, hip_cfg.max_position_embeddings + 1)
    b.free()
    m.free()
