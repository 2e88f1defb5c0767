"""Continuous batching (lbt_sched_*): requests of different prompt lengths
and lengths of output share three slots, joining as others finish; each
request's tokens equal the oracle's greedy generation for it alone (the stop
token ends a request early)."""
import numpy as np
import pytest

import lbt_hip
import lbt_oracle as orc
from conftest import announce

pytestmark = pytest.mark.gpu

SMALL = dict(hidden=256, intermediate=512, heads=4, kv_heads=2, layers=2, vocab=1000, max_pos=1024)


def greedy(om, prompt, max_new, stop):
    om.reset()
    t = int(om.forward(prompt)[0].argmax())
    out = [t]
    while len(out) < max_new and t != stop:
        t = int(om.forward([t])[0].argmax())
        out.append(t)
    return out


def test_sched_matches_single_sequence_oracle(ctx):
    d = SMALL
    hip_cfg = lbt_hip.make_config(d["hidden"], d["intermediate"], d["heads"], d["kv_heads"], d["layers"], d["vocab"],
                                  d["max_pos"])
    or_cfg = orc.config(d["hidden"], d["intermediate"], d["heads"], d["kv_heads"], d["layers"], d["vocab"],
                        d["max_pos"])
    announce("continuous batching, 3 slots, 6 requests")
    seed = 19
    m = lbt_hip.Model.synthetic(ctx, hip_cfg, seed)
    om = orc.OracleModel(or_cfg, seed)
    rng = np.random.default_rng(4)
    reqs = []
    for i, (n, max_new) in enumerate([(3, 1), (20, 7), (9, 12), (1, 5), (14, 9), (6, 4)]):
        prompt = rng.integers(0, or_cfg.vocab, n).astype(np.uint32)
        exp = greedy(om, prompt, max_new, 0xFFFFFFFF)
        stop = exp[2] if i == 2 else lbt_hip.Sched.NO_STOP  # request 2 ends at its third token
        if i == 2:
            exp = exp[: exp.index(stop) + 1]
        reqs.append((prompt, max_new, stop, exp))
    s = m.new_sched(3, 64)
    ids = [s.submit(p, mn, st) for p, mn, st, _ in reqs[:4]]
    pending, steps = 1, 0
    while pending and steps < 100:
        pending = s.step()
        steps += 1
        if steps == 2:  # late arrivals join while others run
            ids += [s.submit(p, mn, st) for p, mn, st, _ in reqs[4:]]
            pending = 1
    assert pending == 0, "requests left after 100 steps"
    for rid, (_, _, _, exp) in zip(ids, reqs):
        got, done = s.result(rid)
        assert done and list(got) == exp, f"request {rid}: {list(got)} vs {exp}"
    s.free()
    m.free()
    om.free()


def test_sched_rejects_requests_beyond_capacity(ctx):
    d = SMALL
    hip_cfg = lbt_hip.make_config(d["hidden"], d["intermediate"], d["heads"], d["kv_heads"], d["layers"], d["vocab"],
                                  d["max_pos"])
    announce("sched capacity")
    m = lbt_hip.Model.synthetic(ctx, hip_cfg, 3)
    s = m.new_sched(2, 16)
    with pytest.raises(lbt_hip.LbtError, match="capacity"):
        s.submit(np.arange(10, dtype=np.uint32), 8)
    rid = s.submit(np.arange(10, dtype=np.uint32), 7)
    while s.step():
        pass
    got, done = s.result(rid)
    assert done and len(got) == 7
    s.release(rid)
    with pytest.raises(lbt_hip.LbtError, match="unknown"):
        s.result(rid)
    s.free()
    m.free()
