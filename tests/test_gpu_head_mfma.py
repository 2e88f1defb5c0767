"""Head kind 2: the tied bf16 LM head of 33..64 rows on the bf16 matrix cores
(activations split into bf16 hi + lo, f32 accumulation in the matrix core's
order).  Its logits cannot equal the exact head's bits, so they are checked
to the tolerance the north star sets for float outputs (1e-3 relative /
1e-2 absolute) against the exact head (kind 0, itself bit-exact to the
oracle), with the same argmax wherever the exact top-1/top-2 margin exceeds
that tolerance; greedy batched decode gives the same tokens; heads of up to
32 rows (kind 2 leaves them on the exact kernel) stay bit-exact."""
import numpy as np
import pytest

import lbt_hip
from conftest import announce

pytestmark = pytest.mark.gpu

SHAPE = dict(layers=1, max_pos=512)  # the 2B head: vocab 128256 x hidden 2560


def _close(got, exp):
    assert np.allclose(got, exp, rtol=1e-3, atol=1e-2)
    top2 = np.sort(exp, axis=1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 2e-2
    assert (got.argmax(1) == exp.argmax(1))[clear].all()


@pytest.mark.parametrize("nseq", [2, 16, 33, 64])
def test_batched_head_on_matrix_cores_within_tolerance(ctx, nseq):
    announce(f"bf16 matrix-core head, 2B head, nseq={nseq}")
    m = lbt_hip.Model.synthetic(ctx, lbt_hip.make_config(**SHAPE), 17)
    toks = np.random.default_rng(nseq).integers(0, 128256, nseq).astype(np.uint32)
    out = {}
    for kind in (0, 2):
        m.set_head(kind)
        b = m.new_batch(nseq, 64)
        b.fill_synthetic(40, 5)
        out[kind] = b.forward(toks)
        b.free()
    (l0, n0), (l2, n2) = out[0], out[2]
    if nseq <= 32:
        assert np.array_equal(l2, l0)  # the exact kernel
    else:
        assert not np.array_equal(l2, l0)  # the matrix-core path ran (its sum order differs)
        _close(l2, l0)
    assert np.array_equal(n0, l0.argmax(1))
    assert np.array_equal(n2, l2.argmax(1))
    m.free()


def test_batched_greedy_decode_same_tokens(ctx):
    announce("bf16 matrix-core head, 48 sequences x 12 greedy steps")
    m = lbt_hip.Model.synthetic(ctx, lbt_hip.make_config(**SHAPE), 23)
    first = np.random.default_rng(3).integers(0, 128256, 48).astype(np.uint32)
    toks = {}
    for kind in (0, 2):
        m.set_head(kind)
        b = m.new_batch(48, 64)
        b.fill_synthetic(20, 9)
        toks[kind], _ = b.decode_greedy(first, 12)
        b.free()
    assert np.array_equal(toks[0], toks[2])
    m.free()


def test_one_row_head_stays_exact(ctx):
    announce("bf16 matrix-core head: one-row heads exact")
    m = lbt_hip.Model.synthetic(ctx, lbt_hip.make_config(**SHAPE), 29)
    prompt = np.array([5, 900, 77, 128000], np.uint32)
    res = []
    for kind in (0, 2):
        m.set_head(kind)
        c = m.new_cache()
        res.append((m.forward(prompt, c), m.forward([11], c)))
        c.free()
    assert np.array_equal(res[0][0], res[1][0]) and np.array_equal(res[0][1], res[1][1])
    with pytest.raises(lbt_hip.LbtError):
        m.set_head(3)
    m.free()
