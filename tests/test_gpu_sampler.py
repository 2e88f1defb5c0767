"""Device sampler (lbt_sample, lbt_model_forward_sample / decode_sample)
against the sampler oracle (or_sample, sample.rs:45-82 with exact integer
masses): the same ids and the same sampler states, over seeds, parameter
sets, vocabulary sizes (candidates in LDS and in the global scratch) and the
reference's edge cases (ties, NaN, infinities, temperature <= 0)."""
import ctypes as C

import numpy as np
import pytest

import lbt_hip
import lbt_oracle as orc
from conftest import announce

pytestmark = pytest.mark.gpu

PARAMS = [(1.0, 1.0, 0), (0.7, 0.9, 0), (1.3, 1.0, 40), (0.5, 0.8, 50), (2.0, 0.95, 10), (0.05, 0.5, 0),
          (1.0, 1e-6, 0), (1.0, 0.0, 7), (0.8, 1.0, 1), (0.0, 0.9, 5), (-1.0, 1.0, 0), (1e30, 1.0, 3)]


def oracle_rows(lg, t, top_p, top_k, states):
    out = []
    for r in range(lg.shape[0]):
        st = C.c_uint64(int(states[r]))
        out.append(int(orc.lib().or_sample(orc._p(np.ascontiguousarray(lg[r])), lg.shape[1], t, top_p, top_k,
                                           C.byref(st))))
        states[r] = st.value
    return np.array(out, np.uint32)


@pytest.mark.parametrize("V,scale", [(50, 3.0), (1000, 3.0), (128256, 1.0), (128256, 12.0), (5000, 0.0)])
def test_sample_rows_match_oracle(ctx, V, scale):
    rng = np.random.default_rng(V)
    rows = 4
    for pi, (t, top_p, top_k) in enumerate(PARAMS):
        announce(f"sample V={V} scale={scale} params={t},{top_p},{top_k}")
        lg = (rng.standard_normal((rows, V)) * scale).astype(np.float32)
        if scale == 0.0:
            lg[:, ::7] = 1.0  # many exact ties
        st = rng.integers(1, 2**63, rows).astype(np.uint64)
        st_o = st.copy()
        got = ctx.sample(lg, t, top_p, top_k, st)
        exp = oracle_rows(lg, t, top_p, top_k, st_o)
        assert np.array_equal(got, exp), (pi, got, exp)
        assert np.array_equal(st, st_o), pi


@pytest.mark.parametrize("V", [2047, 2048, 2049, 4096, 4097, 6145])
def test_sample_chunk_and_lds_boundaries_match_oracle(ctx, V):
    """Rows around the candidate pass's 2048-logit chunks and the 4096
    candidates kept in LDS: flat logits (every logit a candidate), so the
    candidate count is V itself."""
    rng = np.random.default_rng(V + 1)
    rows = 3
    for t, top_p, top_k in [(1.0, 1.0, 0), (0.9, 0.95, 0), (1.2, 1.0, 4000), (0.7, 0.5, 2049)]:
        announce(f"sample boundaries V={V} params={t},{top_p},{top_k}")
        lg = (rng.standard_normal((rows, V)) * 0.5).astype(np.float32)
        lg[1, ::3] = lg[1, 0]  # exact ties across chunks
        st = rng.integers(1, 2**63, rows).astype(np.uint64)
        st_o = st.copy()
        got = ctx.sample(lg, t, top_p, top_k, st)
        exp = oracle_rows(lg, t, top_p, top_k, st_o)
        assert np.array_equal(got, exp), (V, t, top_p, top_k, got, exp)
        assert np.array_equal(st, st_o)


def test_sample_edge_cases_match_oracle(ctx):
    nan = np.float32("nan")
    neg_nan = np.frombuffer(np.uint32(0xFFC00000).tobytes(), np.float32)[0]
    base = np.random.default_rng(5).standard_normal(300).astype(np.float32)
    cases = []
    a = base.copy(); a[17] = nan; cases.append(a)
    a = base.copy(); a[3] = neg_nan; cases.append(a)
    a = base.copy(); a[9] = np.inf; cases.append(a)
    a = base.copy(); a[:] = -np.inf; cases.append(a)
    a = base.copy(); a[100:] = -np.inf; cases.append(a)
    a = base.copy(); a[5] = a[6] = a.max() + 1; cases.append(a)
    a = base.copy(); a[0] = nan; cases.append(a)
    a = np.zeros(300, np.float32); a[::2] = -0.0; cases.append(a)
    # -NaN past a top-k set that holds every candidate (far below the max)
    a = np.full(300, -200.0, np.float32); a[:5] = [3, 2, 1, 0, -1]; a[299] = neg_nan; cases.append(a)
    for ci, lg in enumerate(cases):
        for t, top_p, top_k in PARAMS + [(float("nan"), 1.0, 0), (1.0, float("nan"), 0), (1.0, 1.0, 299),
                                         (1.0, 1.0, 300), (1.0, 1.0, 1000), (1.0, 0.9, 20)]:
            announce(f"sample edge case {ci} params={t},{top_p},{top_k}")
            st = np.array([0x9E3779B97F4A7C15], np.uint64)
            st_o = st.copy()
            got = ctx.sample(lg[None], t, top_p, top_k, st)
            exp = oracle_rows(lg[None], t, top_p, top_k, st_o)
            assert got[0] == exp[0], (ci, t, top_p, top_k, got, exp)
            assert st[0] == st_o[0]


CFG = dict(hidden=256, intermediate=512, heads=4, kv_heads=2, layers=2, vocab=1000, max_pos=1024)


def run_model(m, om, params, seed, prompt, steps):
    """Device: forward_sample + decode_sample; oracle: forward + or_sample with
    the same sampler state (the lb-server job loop, main.rs:102-160)."""
    p = lbt_hip.LbtSampleParams(*params)
    st = C.c_uint64(max(seed, 1))
    c = m.new_cache()
    first = m.forward_sample(prompt, c, p, st)
    toks, _ = m.decode_sample(c, first, steps, p, st)
    c.free()
    smp = orc.Sampler(*params, seed)
    om.reset()
    exp = [smp.sample(om.forward(prompt)[0])]
    for _ in range(steps):
        exp.append(smp.sample(om.forward([exp[-1]])[0]))
    return [first] + list(toks), exp, st.value, smp.state.value


@pytest.mark.parametrize("params", [(0.8, 0.9, 0), (1.2, 1.0, 20), (0.0, 1.0, 0), (0.6, 0.7, 5)])
@pytest.mark.parametrize("path", ["graph", "eager"])
def test_model_sampling_matches_oracle(ctx, ctx_with, params, path):
    c_ = ctx_with(LBT_NO_GRAPH="1") if path == "eager" else ctx
    announce(f"model sampling {path} {params}")
    m = lbt_hip.Model.synthetic(c_, lbt_hip.make_config(**CFG), 31)
    om = orc.OracleModel(orc.config(**CFG), 31)
    prompt = np.array([5, 99, 400, 7, 12, 800], np.uint32)
    for seed in (1, 0xDEADBEEF12345, 2**63 + 7):
        got, exp, st, st_o = run_model(m, om, params, seed, prompt, 40)
        assert got == exp, (seed, got, exp)
        assert st == st_o
    m.free()
    om.free()


def test_full_2b_sampling_matches_oracle(ctx):
    """The 2B-shaped model (vocab 128256: candidates past the LDS list) with
    top-p sampling, 24 steps, against the oracle's logits and sampler."""
    announce("2B sampling")
    cfg = lbt_hip.make_config()
    m = lbt_hip.Model.synthetic(ctx, cfg, 2026)
    old = orc.set_fast(1)
    try:
        om = orc.OracleModel(orc.config(), 2026)
        prompt = np.random.default_rng(64).integers(0, cfg.vocab_size, 16).astype(np.uint32)
        got, exp, st, st_o = run_model(m, om, (0.9, 0.95, 0), 0x5EED, prompt, 24)
        assert got == exp
        assert st == st_o
        om.free()
    finally:
        orc.set_fast(old)
    m.free()
