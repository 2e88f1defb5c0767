"""The sampler oracle (or_sample: sample.rs:45-82 with exact integer masses)
pinned against a plain f32 restatement of the reference's steps, brute-force
special cases and the softmax distribution it draws from."""
import math

import numpy as np
import pytest

import lbt_oracle as orc


def ref_sample(logits, t, top_p, top_k, state):
    """sample.rs:45-82 step by step in f32 (sequential sums in sorted order);
    returns (id, new state, the smallest distance of the draw from a
    cumulative boundary, which says how close a call was)."""
    lg = np.asarray(logits, np.float32)
    if t <= 0.0:
        return int(np.argmax(lg)), state, 1.0
    s = state
    idx = sorted(range(lg.size), key=lambda i: orc.lib().or_sample_key(float(lg[i]), i))
    if top_k > 0:
        idx = idx[:top_k]
    mx = lg[idx[0]]
    t32 = np.float32(t)
    with np.errstate(all="ignore"):
        probs = [np.float32(math.exp(np.float32((lg[i] - mx) / t32))) if not math.isnan((lg[i] - mx) / t32)
                 else np.float32("nan") for i in idx]
        tot = np.float32(0)
        for p in probs:
            tot = np.float32(tot + p)
        probs = [np.float32(p / tot) for p in probs]
        if np.float32(top_p) < 1.0:
            c, keep = np.float32(0), len(probs)
            for i, p in enumerate(probs):
                c = np.float32(c + p)
                if c >= np.float32(top_p):
                    keep = i + 1
                    break
            probs = probs[:keep]
            s2 = np.float32(0)
            for p in probs:
                s2 = np.float32(s2 + p)
            probs = [np.float32(p / s2) for p in probs]
    s ^= (s << 13) & (2**64 - 1)
    s ^= s >> 7
    s ^= (s << 17) & (2**64 - 1)
    r = np.float32((s >> 40) / float(1 << 24))
    c, gap = np.float32(0), 1.0
    with np.errstate(all="ignore"):
        for i, p in enumerate(probs):
            c = np.float32(c + p)
            gap = min(gap, abs(float(c) - float(r))) if not math.isnan(c) else gap
            if r < c:
                return idx[i], s, gap
    return idx[len(probs) - 1], s, gap


def oracle(logits, t, top_p, top_k, seed):
    smp = orc.Sampler(t, top_p, top_k, seed)
    return smp.sample(logits), smp.state.value


@pytest.mark.parametrize("V,t,top_p,top_k", [(50, 1.0, 1.0, 0), (300, 0.7, 0.9, 0), (300, 1.3, 1.0, 40),
                                              (1000, 0.5, 0.8, 50), (64, 2.0, 0.95, 10), (200, 0.05, 0.5, 0)])
def test_oracle_matches_f32_reference_steps(V, t, top_p, top_k):
    """Over many seeds the ids equal the f32 restatement's, except draws that
    land within 1e-5 of a cumulative boundary (the f32 sums and the exact
    integer masses round differently there)."""
    rng = np.random.default_rng(V + top_k)
    same = close = 0
    for trial in range(200):
        lg = (rng.standard_normal(V) * 3).astype(np.float32)
        seed = int(rng.integers(1, 2**63))
        got, st = oracle(lg, t, top_p, top_k, seed)
        exp, st_ref, gap = ref_sample(lg, t, top_p, top_k, max(seed, 1))
        assert st == st_ref
        if got == exp:
            same += 1
        else:
            assert gap < 1e-5, (trial, got, exp, gap)
            close += 1
    assert same >= 195


def test_greedy_and_special_cases():
    lg = np.array([0.5, 2.0, 2.0, -1.0], np.float32)
    # temperature <= 0: argmax, first of equal maxima, state untouched
    for t in (0.0, -1.0):
        smp = orc.Sampler(t, 0.3, 1, 9)
        assert smp.sample(lg) == 1 and smp.state.value == 9
    # top_k = 1 is the argmax (the tie goes to the lower index) whatever the draw
    for seed in range(1, 50):
        assert orc.Sampler(1.0, 1.0, 1, seed).sample(lg) == 1
    # tiny top_p keeps only the first element
    for seed in range(1, 50):
        assert orc.Sampler(1.0, 1e-6, 0, seed).sample(lg) == 1
        assert orc.Sampler(1.0, 0.0, 0, seed).sample(lg) == 1
    # a huge temperature makes every element equally likely: top_k = 2 keeps
    # the tied pair, each drawn about half the time
    # (large seeds: one xorshift step of a small seed leaves the top 24 bits zero)
    seeds = np.random.default_rng(1).integers(1, 2**63, 2000)
    picks = [orc.Sampler(1e30, 1.0, 2, int(seed)).sample(lg) for seed in seeds]
    assert set(picks) == {1, 2} and abs(picks.count(1) - 1000) < 120
    # seed 0 behaves as seed 1 (seed.max(1))
    assert orc.Sampler(1.0, 1.0, 0, 0).sample(lg) == orc.Sampler(1.0, 1.0, 0, 1).sample(lg)


def test_nan_and_infinities_return_last_of_set():
    nan = np.float32("nan")
    lg = np.array([1.0, nan, 3.0, 2.0], np.float32)
    # total order: +NaN first (then every p is NaN), so the last of the set
    assert orc.Sampler(1.0, 1.0, 0, 5).sample(lg) == oracle_last(lg, 0)
    assert orc.Sampler(1.0, 1.0, 2, 5).sample(lg) == oracle_last(lg, 2)
    neg_nan = np.frombuffer(np.uint32(0xFFC00000).tobytes(), np.float32)[0]
    lg2 = np.array([1.0, neg_nan, 3.0, 2.0], np.float32)
    # -NaN sorts last: outside a top-3 set it changes nothing
    a = [orc.Sampler(1.0, 1.0, 3, s).sample(lg2) for s in range(1, 40)]
    b = [orc.Sampler(1.0, 1.0, 3, s).sample(np.array([1.0, -np.inf, 3.0, 2.0], np.float32)) for s in range(1, 40)]
    assert a == b and 1 not in a
    assert orc.Sampler(1.0, 1.0, 0, 5).sample(lg2) == 1  # inside the set: the last element
    assert orc.Sampler(1.0, 1.0, 0, 5).sample(np.array([0.0, np.inf, 1.0], np.float32)) == 0
    assert orc.Sampler(1.0, 1.0, 0, 5).sample(np.full(3, -np.inf, np.float32)) == 2
    assert orc.Sampler(float("nan"), 1.0, 0, 5).sample(np.array([0.0, 1.0, 2.0], np.float32)) == 0
    for lgx, k in ((lg, 0), (lg, 2)):
        exp, _, _ = ref_sample(lgx, 1.0, 1.0, k, 5)
        assert orc.Sampler(1.0, 1.0, k, 5).sample(lgx) == exp


def oracle_last(lg, k):
    idx = sorted(range(lg.size), key=lambda i: orc.lib().or_sample_key(float(lg[i]), i))
    return idx[(k if 0 < k < lg.size else lg.size) - 1]


def test_draws_follow_the_softmax():
    rng = np.random.default_rng(3)
    lg = rng.standard_normal(8).astype(np.float32)
    t = 0.8
    p = np.exp((lg - lg.max()) / t)
    p /= p.sum()
    smp = orc.Sampler(t, 1.0, 0, 12345)
    n = 20000
    counts = np.bincount([smp.sample(lg) for _ in range(n)], minlength=8)
    chi2 = float((((counts - n * p) ** 2) / (n * p)).sum())
    assert chi2 < 30.0  # 7 degrees of freedom: p < 1e-4


def test_top_p_target_is_exact_ceiling():
    for top_p in (0.9, 0.5, 1e-3, 0.999999, 2.0**-30, 1e-45):
        for W in (1, 2**45, 2**62 - 1, 123456789012345):
            from fractions import Fraction

            exp = math.ceil(Fraction(float(np.float32(top_p))) * W)
            assert orc.lib().or_top_p_target(top_p, W) == exp
    assert orc.lib().or_top_p_target(0.0, 5) == 0
    assert orc.lib().or_top_p_target(-0.5, 5) == 0
