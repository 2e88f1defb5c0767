"""Per-request sampling in batched decode and continuous batching
(lbt_batch_prefill_sample / lbt_batch_forward_sample / lbt_sched_submit_sample):
each sequence draws with its own SamplingParams and sampler state
(sample.rs:28-82), and its tokens and final state equal the oracle's for that
sequence alone — the oracle model's logits fed to the sampler oracle, one job
at a time as lb-server runs them (main.rs:102-160).  Greedy sequences in the
same batch keep the argmax."""
import ctypes as C

import numpy as np
import pytest

import lbt_hip
import lbt_oracle as orc
from conftest import announce

pytestmark = pytest.mark.gpu

SMALL = dict(hidden=256, intermediate=512, heads=4, kv_heads=2, layers=2, vocab=1000, max_pos=1024)
# per-sequence (temperature, top_p, top_k); temperature 0 is greedy
PARAMS = [(0.8, 0.95, 0), (0.0, 1.0, 0), (1.3, 1.0, 40), (0.6, 0.7, 5), (1.0, 1.0, 1), (-1.0, 0.9, 0),
          (2.0, 0.5, 0)]


def cfgs():
    d = SMALL
    hip = lbt_hip.make_config(d["hidden"], d["intermediate"], d["heads"], d["kv_heads"], d["layers"], d["vocab"],
                              d["max_pos"])
    orcfg = orc.config(d["hidden"], d["intermediate"], d["heads"], d["kv_heads"], d["layers"], d["vocab"], d["max_pos"])
    return hip, orcfg


def oracle_job(om, prompt, params, seed, n, stop=0xFFFFFFFF):
    """The oracle's tokens for one job: prompt, then up to n sampled tokens."""
    smp = orc.Sampler(*params, seed)
    om.reset()
    out = [smp.sample(om.forward(prompt)[0])]
    while len(out) < n and out[-1] != stop:
        out.append(smp.sample(om.forward([out[-1]])[0]))
    return out, smp.state.value


@pytest.mark.parametrize("nseq", [3, 7, 17])
def test_batch_sampling_matches_oracle(ctx, nseq):
    hip_cfg, or_cfg = cfgs()
    announce(f"batch sampling nseq={nseq}")
    seed = 41
    m = lbt_hip.Model.synthetic(ctx, hip_cfg, seed)
    om = orc.OracleModel(or_cfg, seed)
    b = m.new_batch(nseq, 256)
    rng = np.random.default_rng(100 + nseq)
    params = [PARAMS[s % len(PARAMS)] for s in range(nseq)]
    seeds = [int(x) for x in rng.integers(0, 2**63, nseq)]
    seeds[0] = 0  # Sampler::new keeps seed.max(1)
    prompts = [rng.integers(0, or_cfg.vocab, 1 + (5 * s + 2) % 19).astype(np.uint32) for s in range(nseq)]
    steps = 12
    states = np.zeros(nseq, np.uint64)
    toks = np.zeros((steps + 1, nseq), np.uint32)
    for s in range(nseq):
        st = C.c_uint64(max(seeds[s], 1))
        toks[0, s] = b.prefill_sample(s, prompts[s], lbt_hip.LbtSampleParams(*params[s]), st)
        states[s] = st.value
    for i in range(steps):
        toks[i + 1] = b.forward_sample(toks[i], params, states)
    for s in range(nseq):
        exp, st_o = oracle_job(om, prompts[s], params[s], seeds[s], steps + 1)
        assert list(toks[:, s]) == exp, f"seq {s} params {params[s]}"
        assert int(states[s]) == st_o, f"seq {s} sampler state"
    b.free()
    m.free()
    om.free()


def test_sched_mixed_greedy_and_sampled_matches_oracle(ctx):
    hip_cfg, or_cfg = cfgs()
    announce("continuous batching, sampled and greedy requests, 3 slots")
    seed = 23
    m = lbt_hip.Model.synthetic(ctx, hip_cfg, seed)
    om = orc.OracleModel(or_cfg, seed)
    rng = np.random.default_rng(8)
    reqs = []
    for i, (n, max_new) in enumerate([(4, 6), (17, 9), (2, 1), (11, 14), (7, 5), (1, 8), (9, 10)]):
        prompt = rng.integers(0, or_cfg.vocab, n).astype(np.uint32)
        params = PARAMS[i % len(PARAMS)]
        s0 = int(rng.integers(0, 2**63))
        exp, _ = oracle_job(om, prompt, params, s0, max_new)
        stop = lbt_hip.Sched.NO_STOP
        if i == 3:  # ends at its fourth token
            stop = exp[3]
            exp = exp[: exp.index(stop) + 1]
        reqs.append((prompt, max_new, stop, params, s0, exp))
    s = m.new_sched(3, 64)

    def submit(r):
        prompt, max_new, stop, params, s0, _ = r
        if params[0] == 0.0:
            return s.submit(prompt, max_new, stop)
        return s.submit_sample(prompt, max_new, params, s0, stop)

    ids = [submit(r) for r in reqs[:4]]
    pending, steps = 1, 0
    while pending and steps < 100:
        pending = s.step()
        steps += 1
        if steps == 3:  # late arrivals join while others run
            ids += [submit(r) for r in reqs[4:]]
            pending = 1
    assert pending == 0, "requests left after 100 steps"
    for rid, r in zip(ids, reqs):
        got, done = s.result(rid)
        assert done and list(got) == r[-1], f"request {rid} params {r[3]}: {list(got)} vs {r[-1]}"
    s.free()
    m.free()
    om.free()
