"""Batched decode at its benchmark workload: the 2B-shaped model decoding B = 16
and 64 sequences together, each over a 4096-position bf16 KV cache filled to
4087 positions with the synthetic fill; sampled sequences' step logits are
bit-exact to the single-sequence oracle holding the same cache contents."""
import numpy as np
import pytest

import lbt_hip
import lbt_oracle as orc
from conftest import announce

pytestmark = pytest.mark.gpu

SEED = 2026
FILL_SEED = 5
CTX = 4087


@pytest.mark.parametrize("nseq,check", [(16, (0, 7, 15)), (64, (0, 33, 63))])
def test_batched_decode_2b_context4096_matches_oracle(ctx, nseq, check):
    announce(f"config 5: 2B batch {nseq} at {CTX} cached positions")
    cfg = lbt_hip.make_config()
    m = lbt_hip.Model.synthetic(ctx, cfg, SEED)
    b = m.new_batch(nseq, 4096)
    b.fill_synthetic(CTX, FILL_SEED)
    toks = np.random.default_rng(nseq).integers(0, cfg.vocab_size, nseq).astype(np.uint32)
    logits, nxt = b.forward(toks)
    b.free()
    m.free()
    assert np.isfinite(logits).all()
    assert (nxt == logits.argmax(axis=1)).all()
    old = orc.set_fast(1)
    try:
        om = orc.OracleModel(orc.config(), SEED)
        for s in check:
            om.fill_synth_kv(FILL_SEED, nseq, s, CTX)
            exp = om.forward([int(toks[s])])
            assert np.array_equal(logits[s], exp[0]), f"sequence {s}"
        om.free()
    finally:
        orc.set_fast(old)
