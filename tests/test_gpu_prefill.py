"""Prefill GEMM on the int8 matrix cores (v_mfma_i32_16x16x64_i8): exact
integers and bit-identical f32 outputs vs the oracle on the prefill benchmark shapes
(FFN shapes 2560->6912 and 6912->2560 at M = 128, 512, 2048), ragged tiles,
the reference's prefill overflow case, and the model prefill through the
MFMA path equal to the decode GEMV path."""
import numpy as np
import pytest

import lbt_hip
import lbt_oracle as orc
from conftest import announce
from refgen import golden_case, ternary_iid

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,cols", [(6912, 2560), (2560, 6912)])
@pytest.mark.parametrize("m", [128, 512, 2048])
def test_config3_ffn_shapes_bitexact(ctx, rows, cols, m):
    announce(f"prefill {rows}x{cols} m={m}")
    rng = np.random.default_rng(rows + cols + m)
    t = ternary_iid(rng, rows, cols)
    p = orc.pack(t)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    q, sa, su = orc.quantize_acts(x)
    sw = float(np.float32(1.7))
    w = ctx.upload(p, rows, cols, sw)
    d = orc.port_gemm_i32(p, rows, cols, q, su)
    assert np.array_equal(ctx.gemm_i32(w, q, su), d)
    (y,) = ctx.ternary_linear([w], x)
    inv = (np.float32(1.0) / (sa * np.float32(sw))).astype(np.float32)
    assert np.array_equal(y, (d.astype(np.float32) * inv[:, None]).astype(np.float32))
    w.free()


@pytest.mark.parametrize("rows,cols,m", [(23, 384, 17), (37, 2560, 33), (130, 300, 65), (5, 129, 16), (100, 1000, 200),
                                         (130, 2560, 129), (300, 512, 257), (1, 256, 128), (257, 768, 1000)])
def test_ragged_tiles(ctx, rows, cols, m):
    announce(f"prefill ragged {rows}x{cols} m={m}")
    t, scale, x = golden_case(rows, cols, m, rows + cols + m)
    p = orc.pack(t)
    q, sa, su = orc.quantize_acts(x)
    w = ctx.upload(p, rows, cols, float(scale))
    assert np.array_equal(ctx.gemm_i32(w, q, su), q[:, :cols].astype(np.int64) @ t.T.astype(np.int64))
    (y,) = ctx.ternary_linear([w], x)
    assert np.array_equal(y, orc.gemm_f32(p, rows, cols, scale, q, sa, su))
    w.free()


@pytest.mark.parametrize("rows,cols,m", [(23, 384, 17), (300, 512, 257), (257, 768, 1000), (1000, 2560, 129),
                                         (600, 1280, 300)])
@pytest.mark.parametrize("mode", ["7", "8"])
def test_ragged_tiles_one_workgroup_per_cu(ctx_with, rows, cols, m, mode):
    # the 128 x 256 (8 wavefronts) and 64 x 320 (10 wavefronts) tiles forced
    # at sizes that leave partial token and row tiles (and a partial
    # wavefront block inside a tile)
    ctx = ctx_with(LBT_GEMM_MODE=mode)
    announce(f"prefill one-wg-per-cu mode {mode} ragged {rows}x{cols} m={m}")
    t, scale, x = golden_case(rows, cols, m, rows + cols + m)
    p = orc.pack(t)
    q, sa, su = orc.quantize_acts(x)
    w = ctx.upload(p, rows, cols, float(scale))
    assert np.array_equal(ctx.gemm_i32(w, q, su), q[:, :cols].astype(np.int64) @ t.T.astype(np.int64))
    (y,) = ctx.ternary_linear([w], x)
    assert np.array_equal(y, orc.gemm_f32(p, rows, cols, scale, q, sa, su))
    w.free()


@pytest.mark.parametrize("rows,cols,m", [(130, 2560, 129), (300, 1280, 257), (256, 6912, 96), (1000, 2560, 70),
                                         (77, 1024, 200)])
@pytest.mark.parametrize("mode,ks", [("4", "2"), ("4", "3"), ("4", "7"), ("5", "2"), ("5", "5")])
def test_split_k_ranges(ctx_with, rows, cols, m, mode, ks):
    # k cut into ks ranges (workgroups of one tile meet at a counter; the
    # last adds the int32 partials): the same integers and f32 bits as one
    # range, three calls in a row (the counters return to zero), the last on
    # fewer tokens
    ctx = ctx_with(LBT_GEMM_MODE=mode, LBT_GEMM_KSPLIT=ks)
    announce(f"prefill split-k mode {mode} ks {ks} {rows}x{cols} m={m}")
    t, scale, x = golden_case(rows, cols, m, rows + cols + m)
    p = orc.pack(t)
    w = ctx.upload(p, rows, cols, float(scale))
    for mm in (m, m, m - 33):
        q, sa, su = orc.quantize_acts(x[:mm])
        assert np.array_equal(ctx.gemm_i32(w, q, su), q[:, :cols].astype(np.int64) @ t.T.astype(np.int64))
        (y,) = ctx.ternary_linear([w], x[:mm])
        assert np.array_equal(y, orc.gemm_f32(p, rows, cols, scale, q, sa, su))
    w.free()


def test_split_k_alternating_inputs(ctx_with):
    # the default split of 2560 x 6912 at M = 128 (three k ranges), twelve
    # calls alternating two inputs: each call's partials land at the same
    # scratch addresses as the previous call's, so a reader that saw an
    # earlier call's values (a stale cache line on its XCD) would fail here
    ctx = ctx_with(LBT_GEMM_KSPLIT="3")
    rows, cols, m = 2560, 6912, 128
    announce(f"prefill split-k alternating inputs {rows}x{cols} m={m}")
    rng = np.random.default_rng(77)
    t = ternary_iid(rng, rows, cols)
    p = orc.pack(t)
    w = ctx.upload(p, rows, cols, 1.0)
    xs = [rng.standard_normal((m, cols)).astype(np.float32) for _ in range(2)]
    want = []
    for x in xs:
        q, sa, su = orc.quantize_acts(x)
        want.append(orc.gemm_f32(p, rows, cols, 1.0, q, sa, su))
    for i in range(12):
        (y,) = ctx.ternary_linear([w], xs[i % 2])
        assert np.array_equal(y, want[i % 2]), f"call {i}"
    w.free()


@pytest.mark.parametrize("rows,cols", [(6912, 2560), (2560, 6912), (640, 2560), (13824, 2560)])
@pytest.mark.parametrize("m", [2, 7, 16, 17, 32, 48, 64])
def test_few_token_gemm_bitexact(ctx, rows, cols, m):
    # batched-decode sizes through the few-token kernel (16-row tiles, K split
    # over four wavefronts)
    announce(f"few-token gemm {rows}x{cols} m={m}")
    rng = np.random.default_rng(rows + 3 * cols + m)
    t = ternary_iid(rng, rows, cols)
    p = orc.pack(t)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    q, sa, su = orc.quantize_acts(x)
    sw = float(np.float32(0.8))
    w = ctx.upload(p, rows, cols, sw)
    d = q[:, :cols].astype(np.int64) @ t.T.astype(np.int64)
    assert np.array_equal(ctx.gemm_i32(w, q, su), d)
    (y,) = ctx.ternary_linear([w], x)
    assert np.array_equal(y, orc.gemm_f32(p, rows, cols, sw, q, sa, su))
    w.free()


@pytest.mark.parametrize("rows,cols,m", [(23, 384, 17), (37, 2560, 33), (130, 300, 65), (5, 129, 16), (100, 1000, 200),
                                         (1, 256, 20), (257, 768, 130), (31, 8192, 64)])
@pytest.mark.parametrize("ms,ns", [("1", "1"), ("2", "1"), ("3", "2"), ("4", "1"), ("1", "2"), ("4", "2")])
def test_few_token_kernel_ragged(ctx_with, rows, cols, m, ms, ns):
    # LBT_GEMM_MODE=6 forces the few-token kernel at any token count;
    # LBT_GEMM_SMALL_MS / _NS its tile (16 * ms tokens x 16 * ns rows)
    ctx = ctx_with(LBT_GEMM_MODE="6", LBT_GEMM_SMALL_MS=ms, LBT_GEMM_SMALL_NS=ns)
    announce(f"few-token ragged {rows}x{cols} m={m} ms={ms} ns={ns}")
    t, scale, x = golden_case(rows, cols, m, 7 * rows + cols + m)
    p = orc.pack(t)
    q, sa, su = orc.quantize_acts(x)
    w = ctx.upload(p, rows, cols, float(scale))
    assert np.array_equal(ctx.gemm_i32(w, q, su), q[:, :cols].astype(np.int64) @ t.T.astype(np.int64))
    (y,) = ctx.ternary_linear([w], x)
    assert np.array_equal(y, orc.gemm_f32(p, rows, cols, scale, q, sa, su))
    w.free()


def test_prefill_extreme_long_rows_mfma(ctx):
    # golden.rs:181-194 at an MFMA-sized token count
    rows, cols, m = 3, 6912 * 2, 32
    announce("prefill extreme")
    w = ctx.upload(orc.pack(np.ones((rows, cols), np.int8)), rows, cols, 1.0)
    for sign in (1.0, -1.0):
        x = np.full((m, cols), sign, np.float32)
        q, sa, su = ctx.quantize_acts(x)
        assert np.all(ctx.gemm_i32(w, q, su) == int(sign) * 127 * cols)
        (y,) = ctx.ternary_linear([w], x)
        assert np.all(y == np.float32(sign * cols))
    w.free()


@pytest.mark.parametrize("m", [3, 8, 24, 96, 200])
def test_fused_multi_mfma_equals_separate(ctx, m):
    cols = 2560
    rng = np.random.default_rng(77)
    ws = [ctx.upload(orc.pack(ternary_iid(rng, r, cols)), r, cols, s) for r, s in [(2560, 0.9), (640, 1.1), (640, 1.3)]]
    x = rng.standard_normal((m, cols)).astype(np.float32)
    announce(f"prefill fused multi m={m}")
    fused = ctx.ternary_linear(ws, x)
    for i, w in enumerate(ws):
        (single,) = ctx.ternary_linear([w], x)
        assert np.array_equal(fused[i], single)
    for w in ws:
        w.free()


@pytest.mark.parametrize("n", [2, 5, 16, 40, 130])
def test_model_prefill_mfma_matches_oracle_and_gemv(ctx, ctx_with, n):
    cfg = dict(hidden=512, intermediate=1536, heads=4, kv_heads=1, layers=2, vocab=1000, max_pos=1024)
    hip_cfg = lbt_hip.make_config(**cfg)
    or_cfg = orc.config(**cfg)
    announce(f"model prefill mfma n={n}")
    m = lbt_hip.Model.synthetic(ctx, hip_cfg, 3)
    om = orc.OracleModel(or_cfg, 3)
    toks = (np.arange(n) * 31 % cfg["vocab"]).astype(np.uint32)
    c = m.new_cache()
    got = m.forward(toks, c, all_logits=True)
    assert np.array_equal(got, om.forward(toks, all_logits=True))
    c.free()
    m.free()
    m = lbt_hip.Model.synthetic(ctx_with(LBT_NO_MFMA="1"), hip_cfg, 3)
    c = m.new_cache()
    assert np.array_equal(m.forward(toks, c, all_logits=True), got)
    c.free()
    m.free()
    om.free()


@pytest.mark.parametrize("n,force", [(1100, None), (130, "1"), (9, "1")])
def test_model_long_prefill_attention_matches_oracle(ctx, ctx_with, n, force):
    # the one-wavefront-per-split attention kernel (4 query heads per KV
    # head, head_dim 128): by default past 1024 tokens (splits of more than
    # 64 keys), forced on short prompts; logits bit-exact to the oracle
    cfg = dict(hidden=512, intermediate=1536, heads=4, kv_heads=1, layers=2, vocab=1000, max_pos=2048)
    announce(f"model long prefill n={n} wave={force}")
    c0 = ctx_with(LBT_ATTN_WAVE=force) if force else ctx
    m = lbt_hip.Model.synthetic(c0, lbt_hip.make_config(**cfg), 5)
    om = orc.OracleModel(orc.config(**cfg), 5)
    toks = (np.arange(n) * 37 % cfg["vocab"]).astype(np.uint32)
    c = m.new_cache()
    got = m.forward(toks, c, all_logits=True)
    want = om.forward(toks, all_logits=True)
    assert np.array_equal(got[-64:], want[-64:])
    assert np.array_equal(got, want)
    c.free()
    m.free()
    om.free()


def test_model_chunked_long_prefill_matches_oracle(ctx):
    # a 1100-token prompt in two chunks (700 then 400 tokens): the second
    # chunk's rows start at position 700 over a cache the first wrote, on the
    # one-wavefront-per-split attention; logits bit-exact to the oracle's
    # same two calls
    cfg = dict(hidden=512, intermediate=1536, heads=4, kv_heads=1, layers=2, vocab=1000, max_pos=2048)
    announce("model chunked long prefill 700 + 400")
    m = lbt_hip.Model.synthetic(ctx, lbt_hip.make_config(**cfg), 6)
    om = orc.OracleModel(orc.config(**cfg), 6)
    toks = (np.arange(1100) * 41 % cfg["vocab"]).astype(np.uint32)
    c = m.new_cache()
    for part in (toks[:700], toks[700:]):
        got = m.forward(part, c, all_logits=True)
        assert np.array_equal(got, om.forward(part, all_logits=True))
    c.free()
    m.free()
    om.free()


def test_model_prefill_wide_hidden_matches_oracle(ctx):
    # hidden 4096: the q/k/v GEMM at 128 tokens has 32 k steps over 192
    # 64 x 64 tiles, so it splits k in two (the RoPE / KV-append epilogue
    # after the partials' hand-off), and the attention takes the
    # one-wavefront-per-split kernel; logits bit-exact to the oracle
    cfg = dict(hidden=4096, intermediate=1024, heads=32, kv_heads=8, layers=1, vocab=1000, max_pos=512)
    announce("model prefill hidden 4096, 128 tokens")
    m = lbt_hip.Model.synthetic(ctx, lbt_hip.make_config(**cfg), 9)
    om = orc.OracleModel(orc.config(**cfg), 9)
    toks = (np.arange(128) * 13 % cfg["vocab"]).astype(np.uint32)
    c = m.new_cache()
    got = m.forward(toks, c, all_logits=True)
    assert np.array_equal(got, om.forward(toks, all_logits=True))
    c.free()
    m.free()
    om.free()


@pytest.mark.parametrize("n", [2, 63, 65, 700, 1024, 1025, 1040, 4096, 4100])
def test_prefill_attention_kernels_agree(ctx, ctx_with, n):
    # the 2B shape's attention (20 query heads over 5 KV heads, head_dim 128)
    # at prefill lengths across the split-size steps (64-key splits up to
    # 1024 keys, then ceil(vis / 16); past 4096 two keys per virtual thread):
    # one wavefront per split against the workgroup-per-split kernel (both
    # forced), logits and KV cache bit for bit
    cfg = lbt_hip.make_config(layers=1, vocab=1000, max_pos=4224)
    announce(f"prefill attention wavefront vs workgroup kernel n={n}")
    toks = np.random.default_rng(n + 7).integers(0, 1000, n).astype(np.uint32)
    outs = []
    for c in (ctx_with(LBT_ATTN_WAVE="1"), ctx_with(LBT_ATTN_WAVE="0")):
        m = lbt_hip.Model.synthetic(c, cfg, 17)
        cache = m.new_cache()
        logits = m.forward(toks, cache, all_logits=True)
        outs.append((logits, cache.read(0, False), cache.read(0, True)))
        cache.free()
        m.free()
    for a, b in zip(outs[0], outs[1]):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("mode", ["4", "5", "6", "7", "8"])
def test_model_prefill_every_gemm_tiling_matches_oracle(ctx_with, mode):
    # every epilogue (q/k/v + RoPE + KV append, residual add, relu^2*up) through
    # each MFMA tiling: 64x64 and 128x128 tiles of the 32x32x32 GEMM, the
    # few-token kernel, the 128x256 and 64x320 tiles of the one-workgroup-per-CU
    # kernel
    cfg = dict(hidden=512, intermediate=1536, heads=4, kv_heads=1, layers=2, vocab=1000, max_pos=1024)
    n = 200
    ctx = ctx_with(LBT_GEMM_MODE=mode)
    announce(f"model prefill gemm mode {mode} n={n}")
    m = lbt_hip.Model.synthetic(ctx, lbt_hip.make_config(**cfg), 5)
    om = orc.OracleModel(orc.config(**cfg), 5)
    toks = (np.arange(n) * 17 % cfg["vocab"]).astype(np.uint32)
    c = m.new_cache()
    got = m.forward(toks, c, all_logits=True)
    assert np.array_equal(got, om.forward(toks, all_logits=True))
    c.free()
    m.free()
    om.free()


@pytest.mark.parametrize("n", [1024, 2048])
def test_2b_width_long_prefill_tilings_agree(ctx, ctx_with, n):
    # a 2B-width prefill of n tokens takes the one-workgroup-per-CU tilings
    # for q/k/v, o, gate/up and down (every fused epilogue at full width);
    # its logits and KV cache equal the 128 x 128 tiling's bit for bit (that
    # path is checked against the oracle above)
    cfg = lbt_hip.make_config(layers=2, vocab=1000, max_pos=4096)
    announce(f"2B-width prefill n={n}: default tilings vs LBT_GEMM_MODE=5")
    toks = np.random.default_rng(n + 1).integers(0, 1000, n).astype(np.uint32)
    outs = []
    for c in (ctx, ctx_with(LBT_GEMM_MODE="5")):
        m = lbt_hip.Model.synthetic(c, cfg, 13)
        cache = m.new_cache()
        logits = m.forward(toks, cache, all_logits=True)
        outs.append((logits, cache.read(1, False), cache.read(1, True)))
        cache.free()
        m.free()
    for a, b in zip(outs[0], outs[1]):
        assert np.array_equal(a, b)
