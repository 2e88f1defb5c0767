"""GPU int8 LM head (q8head.rs) against the oracle through the C ABI: the
device quantizer is bit-exact to Q8Head::from_bf16; the head's logits are
bit-exact to the device-order oracle and within the reference's bound of
1e-4 * sum|terms| of the f64 sum (q8head.rs:84-97); the model with the int8
head matches the oracle model with the int8 head bit for bit, and a batched
step equals the single-sequence steps."""
import numpy as np
import pytest

import lbt_hip
import lbt_oracle as orc
from conftest import announce
from refgen import XorShift, q8_bf16_matrix, xorshift_f32

pytestmark = pytest.mark.gpu


def edge_matrix(rows, cols, rng):
    w = orc.f32_to_bf16((rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)).reshape(rows, cols)
    w[0] = 0  # all-zero row: scale 1
    w[1, : min(cols, 8)] = orc.f32_to_bf16(np.array([127, 2.5, 3.5, -2.5, -0.5, 0.5, 1.5, -127], np.float32))[
        : min(cols, 8)
    ]
    w[1, 8:] = 0
    w[2, 3] = 0x7FC0  # NaN
    return w


@pytest.mark.parametrize("rows,cols", [(300, 2560), (37, 40), (1000, 4104), (128256 // 16, 2560)])
def test_quantizer_bitexact(ctx, rows, cols):
    announce(f"q8 quantize {rows}x{cols}")
    w = edge_matrix(rows, cols, np.random.default_rng(rows))
    bw = ctx.bf16_upload(w)
    h = ctx.q8head_from_bf16(bw)
    q, s = h.read()
    eq, es = orc.q8head_from_bf16(w)
    assert np.array_equal(q, eq)
    assert s.tobytes() == es.tobytes()
    h.free()
    bw.free()


@pytest.mark.parametrize("rows,cols,m", [(300, 2560, 1), (37, 40, 1), (1000, 4104, 2), (2048, 2560, 3),
                                         (5000, 2560, 8), (777, 2560, 9), (1500, 512, 17)])
def test_head_bitexact_to_device_order(ctx, rows, cols, m):
    announce(f"q8 head {rows}x{cols} m={m}")
    rng = np.random.default_rng(rows + m)
    w = edge_matrix(rows, cols, rng)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    bw = ctx.bf16_upload(w)
    h = ctx.q8head_from_bf16(bw)
    got = ctx.q8head_linear(h, x)
    q, s = orc.q8head_from_bf16(w)
    for t in range(m):
        assert np.array_equal(got[t], orc.q8head_gemv_lanes(q, s, x[t])), f"token {t}"
        terms = s[:, None].astype(np.float64) * q.astype(np.float64) * x[t][None, :].astype(np.float64)
        ref, mag = terms.sum(axis=1), np.abs(terms).sum(axis=1)
        assert np.all(np.abs(got[t].astype(np.float64) - ref) <= 1e-4 * mag + 1e-30)
    h.free()
    bw.free()


def test_reference_case_q8_matches_dequantized(ctx):
    """q8head.rs:84-97 on the device, with the reference's inputs."""
    rows, cols = 300, 2560
    rnd = XorShift(0x9E3779B97F4A7C15)
    w = q8_bf16_matrix(rnd, rows * cols, 0.05).reshape(rows, cols)
    x = xorshift_f32(rnd, cols)
    announce("q8 reference case")
    bw = ctx.bf16_upload(w)
    h = ctx.q8head_from_bf16(bw)
    out = ctx.q8head_linear(h, x[None, :])[0]
    q, s = h.read()
    terms = s[:, None].astype(np.float64) * q.astype(np.float64) * x[None, :].astype(np.float64)
    ref, mag = terms.sum(axis=1), np.abs(terms).sum(axis=1)
    assert np.all(np.abs(out.astype(np.float64) - ref) <= 1e-4 * mag)
    h.free()
    bw.free()


SMALL = dict(hidden=256, intermediate=512, heads=4, kv_heads=2, layers=2, vocab=1000, max_pos=1024)


def test_model_int8_head_matches_oracle(ctx):
    d = SMALL
    hip_cfg = lbt_hip.make_config(d["hidden"], d["intermediate"], d["heads"], d["kv_heads"], d["layers"], d["vocab"],
                                  d["max_pos"])
    or_cfg = orc.config(d["hidden"], d["intermediate"], d["heads"], d["kv_heads"], d["layers"], d["vocab"],
                        d["max_pos"])
    announce("model int8 head")
    m = lbt_hip.Model.synthetic(ctx, hip_cfg, 8)
    m.set_head(1)
    om = orc.OracleModel(or_cfg, 8)
    om.set_head(1)
    cache = m.new_cache()
    prompt = np.array([3, 77, 500, 12, 999, 4], np.uint32)
    got = m.forward(prompt, cache, all_logits=True)
    exp = om.forward(prompt, all_logits=True)
    assert np.array_equal(got, exp)
    tok = int(exp[-1].argmax())
    for step in range(4):
        g = m.forward([tok], cache)
        e = om.forward([tok])
        assert np.array_equal(g, e), f"step {step}"
        tok = int(e[0].argmax())
    # greedy decode on the device (graph path) against the oracle's tokens
    cache.free()
    om.reset()
    cache = m.new_cache()
    toks, _, _ = m.generate_greedy(prompt, 6, cache)
    etoks = [int(om.forward(prompt)[0].argmax())]
    for _ in range(6):
        etoks.append(int(om.forward([etoks[-1]])[0].argmax()))
    assert list(toks) == etoks
    # back to the bf16 head: the oracle's bf16 logits again
    m.set_head(0)
    om2 = orc.OracleModel(or_cfg, 8)
    c2 = m.new_cache()
    assert np.array_equal(m.forward(prompt, c2, all_logits=True), om2.forward(prompt, all_logits=True))
    c2.free()
    cache.free()
    m.free()
    om.free()
    om2.free()


@pytest.mark.parametrize("nseq", [5, 17])
def test_batch_int8_head_equals_single(ctx, nseq):
    d = SMALL
    hip_cfg = lbt_hip.make_config(d["hidden"], d["intermediate"], d["heads"], d["kv_heads"], d["layers"], d["vocab"],
                                  d["max_pos"])
    announce(f"batch int8 head nseq={nseq}")
    m = lbt_hip.Model.synthetic(ctx, hip_cfg, 9)
    m.set_head(1)
    b = m.new_batch(nseq, 64)
    prompts = [np.array([1 + s, 20 + s, 300 + s], np.uint32) for s in range(nseq)]
    nxt = [b.prefill(s, prompts[s]) for s in range(nseq)]
    logits, _ = b.forward(np.array(nxt, np.uint32))
    for s in range(nseq):
        c = m.new_cache()
        m.forward(prompts[s], c)
        e = m.forward([nxt[s]], c)
        assert np.array_equal(logits[s], e[0]), f"seq {s}"
        c.free()
    b.free()
    m.free()


def test_graph_step_survives_head_switches_and_regrowth(ctx):
    """The captured decode-step graph across everything that frees a buffer it
    refers to: head switches (bf16 -> int8 -> bf16), growth of the token
    slots, of the workspace (a longer prompt) and of the cache, and a cache
    freed and replaced.  Every decode is checked against the oracle's greedy
    tokens with the same head."""
    d = SMALL
    hip_cfg = lbt_hip.make_config(d["hidden"], d["intermediate"], d["heads"], d["kv_heads"], d["layers"], d["vocab"],
                                  d["max_pos"])
    or_cfg = orc.config(d["hidden"], d["intermediate"], d["heads"], d["kv_heads"], d["layers"], d["vocab"],
                        d["max_pos"])
    announce("graph step across head switches and regrowth")
    m = lbt_hip.Model.synthetic(ctx, hip_cfg, 21)

    def oracle_tokens(head, prompt, steps):
        om = orc.OracleModel(or_cfg, 21)
        om.set_head(head)
        out = [int(om.forward(prompt)[0].argmax())]
        for _ in range(steps):
            out.append(int(om.forward([out[-1]])[0].argmax()))
        om.free()
        return out

    short = np.array([5, 6, 7], np.uint32)
    longp = (np.arange(40) * 11 % d["vocab"]).astype(np.uint32)
    for head, prompt, steps in [(0, short, 4), (1, short, 9), (1, longp, 30), (0, longp, 12), (0, short, 300)]:
        m.set_head(head)
        cache = m.new_cache()
        toks, _, _ = m.generate_greedy(prompt, steps, cache)
        assert list(toks) == oracle_tokens(head, prompt, steps), f"head {head}, prompt {len(prompt)}, {steps} steps"
        cache.free()
    m.free()
