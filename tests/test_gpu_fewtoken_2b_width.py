"""The few-token MFMA GEMM at the 2B model's widths (hidden 2560, FFN 6912:
the fused gate/up has 13824 rows, so 32-row tiles by default), through every
fused epilogue -- q/k/v + RoPE + KV append at per-sequence positions, the
residual add of o and down, relu^2 * up -- at 2..32 tokens, with the 32-row
tile forced on the narrower products too, and the per-token epilogue
prefetch on and off: each sequence's batched-step logits bit-exact to the
oracle's single-sequence forward."""
import numpy as np
import pytest

import lbt_hip
import lbt_oracle as orc
from conftest import announce

pytestmark = pytest.mark.gpu

WIDE = dict(hidden=2560, intermediate=6912, heads=20, kv_heads=5, layers=1, vocab=1000, max_pos=512)


@pytest.mark.parametrize("nseq", [2, 5, 16, 17, 32])
@pytest.mark.parametrize("env", [{}, {"LBT_GEMM_SMALL_NS": "2"}, {"LBT_GEMM_SMALL_PF": "0"},
                                 {"LBT_GEMM_SMALL_NS": "2", "LBT_GEMM_SMALL_PF": "0"}])
def test_batched_step_at_2b_width_matches_oracle(ctx_with, nseq, env):
    ctx = ctx_with(**env)
    announce(f"few-token 2B width nseq={nseq} env={env}")
    seed = 44
    m = lbt_hip.Model.synthetic(ctx, lbt_hip.make_config(**WIDE), seed)
    om = orc.OracleModel(orc.config(**WIDE), seed)
    b = m.new_batch(nseq, 128)
    rng = np.random.default_rng(nseq)
    prompts = [rng.integers(0, WIDE["vocab"], 1 + (5 * s + 2) % 19).astype(np.uint32) for s in range(nseq)]
    nxt = [b.prefill(s, prompts[s]) for s in range(nseq)]
    logits, _ = b.forward(np.array(nxt, np.uint32))
    for s in range(nseq):
        om.reset()
        om.forward(prompts[s])
        e = om.forward([nxt[s]])
        assert np.array_equal(logits[s], e[0]), f"seq {s}"
    b.free()
    m.free()
    om.free()
