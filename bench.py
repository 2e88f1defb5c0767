"""Benchmark: batch-1 greedy decode of a BitNet-b1.58-2B4T-shaped model on one
MI355X (the decode benchmark: 30 layers, hidden 2560, FFN 6912 ReLU^2-gated,
20/5 heads, head_dim 128, vocab 128256 bf16 tied head, random-init weights,
64-token uniform-random prompt, then greedy decode).

A step is one decode token (one pass of the whole token loop).  Prints one
JSON line: decode tok/s, the roofline of the dominant kernel class (the
ternary decode GEMV, HBM-bound) measured with HIP events on the library's
stream, and the CPU baseline (the SIMD restatement of the reference's CPU
path, timed on this host).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "lemonade-burn_amd"))

HBM_PEAK_GBS = 8000.0
SEED = 2026
PROMPT_LEN = 64
CALIB_BYTES = 256 << 20  # the copy kernel of known size that calibrates the HBM counters
TRAFFIC_SUMMARY = REPO / "profiles" / "decode_gemv_hbm_traffic.md"


def gemv_traffic() -> float | None:
    """HBM bytes per decode-GEMV launch from the committed rocprofv3 counter
    summary (FETCH_SIZE + WRITE_SIZE per dispatch, each scaled by the same
    counter's reading on the copy kernel of known size), or None."""
    try:
        for ln in TRAFFIC_SUMMARY.read_text().splitlines():
            if ln.startswith("traffic_bytes_per_launch:"):
                return float(ln.split(":", 1)[1])
    except OSError:
        pass
    return None


def batched_decode(model, cfg, batch: int, cap: int = 4096, steps: int = 8) -> dict:
    """Batched decode: `batch` sequences, each with a `cap`-position bf16
    KV cache (the model's max_position_embeddings) pre-filled with synthetic
    values (approximately N(0,1)) up to cap - steps - 1, decoded together;
    greedy steps timed on the device after one untimed step.  Bytes per step:
    every sequence's K and V over all layers plus one pass over the weights."""
    ctx_len = cap - steps - 1
    b = model.new_batch(batch, cap)
    try:
        b.fill_synthetic(ctx_len, 5)
        first = np.random.default_rng(batch).integers(0, cfg.vocab_size, batch).astype(np.uint32)
        toks, _ = b.decode_greedy(first, 1)
        out, ms = b.decode_greedy(toks[-1], steps)
    finally:
        b.free()
    hd = cfg.hidden_size // cfg.num_attention_heads
    kv = batch * cfg.num_hidden_layers * 2 * cfg.num_key_value_heads * (ctx_len + 1 + steps / 2) * hd * 2
    weights = 521_011_200 + cfg.vocab_size * cfg.hidden_size * 2
    ms_step = ms / steps
    gbs = (kv + weights) / (ms_step / 1e3) / 1e9
    return {"batch": batch, "ctx": ctx_len, "steps": steps, "tok_s": round(batch * steps / (ms / 1e3), 1),
            "ms_per_step": round(ms_step, 3), "hbm_GBs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}


MFMA_INT8_PEAK_TOPS = 5000.0


def batched_mfma_head(model, cfg) -> list:
    """The batched-decode figures with head kind 2 (the bf16 head of the
    batch's rows on the matrix cores, logits within tolerance of the exact
    head); reported beside `batched_decode`, never as it."""
    model.set_head(2)
    try:
        return [batched_decode(model, cfg, b) for b in (16, 64)]
    finally:
        model.set_head(0)


def int8_head_decode(model, ctx, prompt, steps: int = 128) -> dict:
    """Decode tok/s with the opt-in int8 LM head (q8head.rs), the same loop as
    `value`; its logits are not the exact bf16 head's, so it is reported
    beside the headline figure, never as it."""
    model.set_head(1)
    try:
        cache = model.new_cache()
        first = model.forward_argmax(prompt, cache)
        model.decode_greedy(cache, first, 8)  # builds the step graph
        cache.free()
        cache = model.new_cache()
        first = model.forward_argmax(prompt, cache)
        _, ms_dev = model.decode_greedy(cache, first, steps)
        cache.free()
        cache = model.new_cache()
        first = model.forward_argmax(prompt, cache)
        ctx.prof_read(reset=True)
        ctx.prof_enable(True)
        model.decode_greedy(cache, first, 16)
        prof = ctx.prof_read(reset=True)
        ctx.prof_enable(False)
        cache.free()
    finally:
        model.set_head(0)
    h = prof["head"]
    return {"tok_s": round(steps / (ms_dev / 1e3), 2), "ms_per_step": round(ms_dev / steps, 4),
            "head_us": round(h["ms"] * 1e3 / max(h["launches"], 1), 2),
            "head_GBs": round(h["bytes"] / (h["ms"] / 1e3) / 1e9, 1) if h["ms"] > 0 else 0.0}


def sampled_decode(model, prompt, steps: int = 128) -> dict:
    """The same decode loop with the device sampler (temperature 0.8, top-p
    0.95; and top-k 40) instead of the argmax: the lb-server job loop with
    its Sampler (main.rs:102-160, sample.rs:45-82), ids only over PCIe."""
    import ctypes as C

    import lbt_hip

    out = {}
    for name, p in (("t0.8_p0.95", (0.8, 0.95, 0)), ("t0.8_k40", (0.8, 1.0, 40))):
        params = lbt_hip.LbtSampleParams(*p)
        st = C.c_uint64(0x5EED)
        cache = model.new_cache()
        first = model.forward_sample(prompt, cache, params, st)
        model.decode_sample(cache, first, 8, params, st)  # builds the step graph
        cache.free()
        cache = model.new_cache()
        first = model.forward_sample(prompt, cache, params, st)
        _, ms = model.decode_sample(cache, first, steps, params, st)
        cache.free()
        out[name] = {"tok_s": round(steps / (ms / 1e3), 2), "ms_per_step": round(ms / steps, 4)}
    return out


def sched_throughput(model, cfg, slots: int = 16, requests: int = 32, prompt_len: int = 64, new: int = 64) -> dict:
    """Continuous batching (lbt_sched_*): `requests` greedy requests of a
    `prompt_len`-token prompt and `new` tokens each through `slots` slots;
    generated tokens per second of host wall time (prefills included)."""
    rng = np.random.default_rng(7)
    s = model.new_sched(slots, prompt_len + new)
    ids = [s.submit(rng.integers(0, cfg.vocab_size, prompt_len).astype(np.uint32), new) for _ in range(requests)]
    t0 = time.perf_counter()
    steps = 0
    while s.step():
        steps += 1
    wall = time.perf_counter() - t0
    total = sum(len(s.result(i)[0]) for i in ids)
    s.free()
    return {"slots": slots, "requests": requests, "prompt": prompt_len, "new_tokens": new, "steps": steps + 1,
            "tok_s": round(total / wall, 1), "wall_s": round(wall, 3)}


def long_prefill(model, ctx, cfg, lengths=(512, 2048)) -> list:
    """Prefill of one long prompt (uniform-random ids) on the 2B-shaped model:
    host wall time of lbt_model_forward (argmax of the last row) between two
    synchronizations, best of three after a warm-up, and the device time of
    its attention, GEMM and head kernels from one profiled run."""
    res = []
    for n in lengths:
        toks = np.random.default_rng(n).integers(0, cfg.vocab_size, n).astype(np.uint32)
        ts = []
        for _ in range(4):
            c = model.new_cache()
            ctx.sync()
            t0 = time.perf_counter()
            model.forward_argmax(toks, c)
            ctx.sync()
            ts.append(time.perf_counter() - t0)
            c.free()
        ctx.prof_read(reset=True)
        ctx.prof_enable(True)
        c = model.new_cache()
        model.forward_argmax(toks, c)
        ctx.sync()
        c.free()
        p = ctx.prof_read(reset=True)
        ctx.prof_enable(False)
        best = min(ts[1:])
        res.append({"tokens": n, "ms": round(best * 1e3, 2), "tok_s": round(n / best, 1),
                    "attn_ms": round(p["attn"]["ms"], 2), "gemm_ms": round(p["gemm"]["ms"], 2)})
    return res


def prefill_gemm(ctx, reps: int = 10) -> list:
    """The prefill GEMM benchmark: the prefill GEMM (int8 MFMA) on the FFN shapes
    2560->6912 and 6912->2560 at M = 128, 512, 2048 tokens; seeded ternary
    weights (P = 0.3/0.4/0.3) and int8 activations resident on the device;
    HIP events around each launch (the library's profiling pass)."""
    import ctypes as C

    lib = ctx.lib
    rng = np.random.default_rng(3)
    res = []
    for rows, cols in [(6912, 2560), (2560, 6912)]:
        kp = (cols + 127) // 128 * 128
        codes = rng.choice(np.array([0, 1, 2], np.uint8), size=(rows, kp), p=[0.3, 0.4, 0.3])
        c4 = codes.reshape(rows, kp // 128, 4, 32)  # block, code group k, byte j
        packed = (c4[:, :, 0] | (c4[:, :, 1] << 2) | (c4[:, :, 2] << 4) | (c4[:, :, 3] << 6)).reshape(rows, kp // 4)
        w = ctx.upload(packed, rows, cols, 1.0)
        for m in (128, 512, 2048):
            q = rng.integers(-127, 128, (m, kp)).astype(np.int8)
            q[:, cols:] = 0
            qs = q.astype(np.int32).sum(1).astype(np.int32)
            sa = np.full(m, 0.05, np.float32)
            dq, ds, dsum, dout = C.c_void_p(), C.c_void_p(), C.c_void_p(), C.c_void_p()
            for p_, n in ((dq, q.nbytes), (ds, sa.nbytes), (dsum, qs.nbytes), (dout, m * rows * 4)):
                ctx.check(lib.lbt_dev_alloc(ctx.h, n, C.byref(p_)))
            ctx.check(lib.lbt_memcpy_h2d(ctx.h, dq, q.ctypes.data, q.nbytes))
            ctx.check(lib.lbt_memcpy_h2d(ctx.h, ds, sa.ctypes.data, sa.nbytes))
            ctx.check(lib.lbt_memcpy_h2d(ctx.h, dsum, qs.ctypes.data, qs.nbytes))
            wa = (C.c_void_p * 1)(w.h)
            oa = (C.c_void_p * 1)(dout.value)
            ctx.check(lib.lbt_gemm_multi_dev(ctx.h, wa, 1, dq, ds, dsum, m, oa))
            ctx.sync()
            ctx.prof_read(reset=True)
            ctx.prof_enable(True)
            for _ in range(reps):
                ctx.check(lib.lbt_gemm_multi_dev(ctx.h, wa, 1, dq, ds, dsum, m, oa))
            p = ctx.prof_read(reset=True)
            ctx.prof_enable(False)
            us = p["gemm"]["ms"] * 1e3 / max(p["gemm"]["launches"], 1)
            tops = 2.0 * m * rows * kp / (us * 1e-6) / 1e12
            res.append({"rows": rows, "cols": cols, "m": m, "us": round(us, 2), "TOPS": round(tops, 1),
                        "frac": round(tops / MFMA_INT8_PEAK_TOPS, 4)})
            for p_ in (dq, ds, dsum, dout):
                lib.lbt_dev_free(ctx.h, p_)
        w.free()
    return res


LAYER_SHAPES = [("q", 2560, 2560), ("k", 640, 2560), ("v", 640, 2560), ("o", 2560, 2560),
                ("gate", 6912, 2560), ("up", 6912, 2560), ("down", 2560, 6912)]
COLD_BYTES = 288 << 20  # rotated weight bytes per shape: more than the 256 MB MALL holds


def synth_packed(rng, rows: int, cols: int) -> np.ndarray:
    """Packed LB2 rows (pack.rs:1-116) of i.i.d. ternary weights, P(-1, 0, +1)
    = 0.3 / 0.4 / 0.3; padded columns carry code 1 (weight 0)."""
    kp = (cols + 127) // 128 * 128
    codes = rng.choice(np.array([0, 1, 2], np.uint8), size=(rows, kp), p=[0.3, 0.4, 0.3])
    codes[:, cols:] = 1
    c4 = codes.reshape(rows, kp // 128, 4, 32)  # block, code group k, byte j
    return (c4[:, :, 0] | (c4[:, :, 1] << 2) | (c4[:, :, 2] << 4) | (c4[:, :, 3] << 6)).reshape(rows, kp // 4)


def gemv_shapes(ctx, reps: int = 4) -> dict:
    """The per-shape GEMV benchmark (one shape, then every decoder-layer shape) on the device: each decode-layer shape at M = 1
    (f32 N(0,1) activation, absmax-quantized inside the op, f32 out) through
    lbt_ternary_linear_dev -- the product decode GEMV with its fused quantizer.
    "cold": enough distinct copies of the matrix (>= 288 MB) are rotated that
    none is in the MALL when its turn comes; "warm": one copy called again and
    again (the reference kbench's method, kbench.rs:44-63).  Per-launch
    device time from HIP events on the library's stream; bytes = packed
    weights + the f32 activation row."""
    import ctypes as C

    lib = ctx.lib
    rng = np.random.default_rng(1)
    out = {}
    for name, rows, cols in LAYER_SHAPES:
        packed = synth_packed(rng, rows, cols)
        ncopy = max(64, -(-COLD_BYTES // packed.nbytes))
        ws = [ctx.upload(packed, rows, cols, 1.0) for _ in range(ncopy)]
        x = rng.standard_normal(cols).astype(np.float32)
        dx, do = C.c_void_p(), C.c_void_p()
        ctx.check(lib.lbt_dev_alloc(ctx.h, x.nbytes, C.byref(dx)))
        ctx.check(lib.lbt_dev_alloc(ctx.h, rows * 4, C.byref(do)))
        ctx.check(lib.lbt_memcpy_h2d(ctx.h, dx, x.ctypes.data, x.nbytes))
        oa = (C.c_void_p * 1)(do.value)
        was = [(C.c_void_p * 1)(w.h) for w in ws]

        def run(seq):
            ctx.prof_read(reset=True)
            ctx.prof_enable(True)
            for wa in seq:
                ctx.check(lib.lbt_ternary_linear_dev(ctx.h, wa, 1, dx, 1, cols, oa))
            p = ctx.prof_read(reset=True)["gemv"]
            ctx.prof_enable(False)
            return p["ms"] * 1e3 / max(p["launches"], 1)

        run(was[:4])  # code objects, clocks
        cold = run(was * reps)
        warm = run([was[0]] * 256)
        # the host-pointer entry point (the reference's slice API): the row
        # copied in, the product, the outputs copied back and the stream
        # synchronized, per call by the host clock (PCIe-inclusive; warm
        # matrix)
        y = np.zeros(rows, np.float32)
        ha = (C.c_void_p * 1)(y.ctypes.data)
        for _ in range(8):
            ctx.check(lib.lbt_ternary_linear(ctx.h, was[0], 1, x.ctypes.data, 1, cols, ha))
        t0 = time.perf_counter()
        for _ in range(200):
            ctx.check(lib.lbt_ternary_linear(ctx.h, was[0], 1, x.ctypes.data, 1, cols, ha))
        host = (time.perf_counter() - t0) / 200 * 1e6
        bytes_ = packed.nbytes + cols * 4
        rec = {"rows": rows, "cols": cols, "copies": ncopy}
        for k, us in (("cold", cold), ("warm", warm), ("host_pointers", host)):
            gbs = bytes_ / (us * 1e-6) / 1e9
            rec[k] = {"us": round(us, 3), "GBs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
        out[name] = rec
        for w in ws:
            w.free()
        lib.lbt_dev_free(ctx.h, dx)
        lib.lbt_dev_free(ctx.h, do)
    return out


def pmc_pass() -> int:
    """The command profiled for the HBM counters (under rocprofv3 --pmc):
    one copy of CALIB_BYTES with the library's copy kernel (the calibration
    dispatch), then the 2B model's 64-token prefill and 8 decode steps with
    per-kernel launches (no graph), so every GEMV is its own dispatch."""
    import ctypes as C

    import lbt_hip

    os.environ["LBT_NO_GRAPH"] = "1"
    ctx = lbt_hip.Ctx(0)
    lib = ctx.lib
    a, b = C.c_void_p(), C.c_void_p()
    ctx.check(lib.lbt_dev_alloc(ctx.h, CALIB_BYTES, C.byref(a)))
    ctx.check(lib.lbt_dev_alloc(ctx.h, CALIB_BYTES, C.byref(b)))
    ctx.check(lib.lbt_memcpy_d2d(ctx.h, b, a, CALIB_BYTES))
    ctx.sync()
    lib.lbt_dev_free(ctx.h, a)
    lib.lbt_dev_free(ctx.h, b)
    cfg = lbt_hip.make_config()
    model = lbt_hip.Model.synthetic(ctx, cfg, SEED)
    prompt = np.random.default_rng(64).integers(0, cfg.vocab_size, PROMPT_LEN).astype(np.uint32)
    cache = model.new_cache()
    first = model.forward_argmax(prompt, cache)
    model.decode_greedy(cache, first, 8)
    ctx.sync()
    cache.free()
    model.free()
    ctx.close()
    print("pmc pass done", flush=True)
    return 0


def _loop(fn, min_s: float = 0.3) -> float:
    """kbench's timing (kbench.rs:44-63): one warm-up call, then calls until
    at least `min_s` seconds have passed; seconds per call."""
    fn()
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el >= min_s:
            return el / n


def cpu_baseline(decode_s: float = 12.0, decode_s1: float = 8.0) -> dict:
    """Reference CPU path restated (VNNI/AVX-512BW/AVX2 ternary GEMV/GEMM +
    AVX-512 bf16 LM head, OpenMP over rows) timed on this host, on all cores
    and on one: (1) the decode benchmark, the 2B-shaped model (same shape and
    seed as the device run) prefilling the 64-token prompt and then decoding
    greedily for about `decode_s` (`decode_s1` on one core) seconds; (2) the
    config-1/2 GEMV shapes at M = 1 (kbench.rs:44-63: warm, >= 0.3 s loop),
    plus one pass over a 520 MB matrix (kbench.rs:75-127, cold); (3) the
    config-3 prefill GEMM at M = 128 / 512 / 2048 (one core: M = 128)."""
    sys.path.insert(0, str(REPO / "oracle"))
    import lbt_oracle as orc

    allc = int(orc.lib().port_threads())
    rng = np.random.default_rng(1)
    shapes = {}
    for name, rows, cols in LAYER_SHAPES:
        packed = synth_packed(rng, rows, cols)
        x = rng.standard_normal((1, cols)).astype(np.float32)
        q, sa, qs = orc.quantize_acts(x)
        rec = {}
        for nt in (allc, 1):
            dt = _loop(lambda: orc.port_gemm_i32(packed, rows, cols, q, qs, threads=nt))
            rec["all" if nt == allc else "one"] = {"us": round(dt * 1e6, 1), "GBs": round(packed.nbytes / dt / 1e9, 2)}
        shapes[name] = rec
    # the 520 MB stream: a 2560-column matrix of ~520 MB, read once per call
    tile = synth_packed(rng, 6912, 2560)
    reps_ = -(-520_000_000 // tile.nbytes)
    big = np.tile(tile, (reps_, 1))
    x = rng.standard_normal((1, 2560)).astype(np.float32)
    q, sa, qs = orc.quantize_acts(x)
    stream = {}
    for nt in (allc, 1):
        t0 = time.perf_counter()
        orc.port_gemm_i32(big, big.shape[0], 2560, q, qs, threads=nt)
        dt = time.perf_counter() - t0
        stream["all" if nt == allc else "one"] = {"ms": round(dt * 1e3, 1), "GBs": round(big.nbytes / dt / 1e9, 2)}
    del big
    prefill = []
    for rows, cols in [(6912, 2560), (2560, 6912)]:
        packed = synth_packed(rng, rows, cols)
        for m, nts in ((128, (allc, 1)), (512, (allc,)), (2048, (allc,))):
            x = rng.standard_normal((m, cols)).astype(np.float32)
            q, sa, qs = orc.quantize_acts(x)
            for nt in nts:
                dt = _loop(lambda: orc.port_gemm_i32(packed, rows, cols, q, qs, threads=nt))
                prefill.append({"rows": rows, "cols": cols, "m": m, "threads": nt,
                                "GOPS": round(2.0 * m * rows * cols / dt / 1e9, 1)})

    old = orc.set_fast(2)
    decode = {}
    try:
        t0 = time.perf_counter()
        om = orc.OracleModel(orc.config(), SEED)
        build_s = time.perf_counter() - t0
        prompt = np.random.default_rng(64).integers(0, 128256, PROMPT_LEN).astype(np.uint32)
        for nt, budget in ((allc, decode_s), (1, decode_s1)):
            orc.set_threads(nt)
            om.reset()
            t0 = time.perf_counter()
            tok = int(om.forward(prompt)[-1].argmax())
            pf = time.perf_counter() - t0
            n, t0 = 0, time.perf_counter()
            while True:
                tok = int(om.forward([tok])[0].argmax())
                n += 1
                el = time.perf_counter() - t0
                if el > budget or n >= 256:
                    break
            decode["all" if nt == allc else "one"] = {"tok_s": round(n / el, 3), "steps": n,
                                                      "prefill64_s": round(pf, 2)}
        om.free()
    finally:
        orc.set_threads(0)
        orc.set_fast(old)
    return {
        "value": decode["all"]["tok_s"],
        "unit": "tok/s",
        "cores": allc,
        "kind": "port",
        "sample": f"2B-shaped synthetic model (seed {SEED}), the 64-token prompt then "
                  f"{decode['all']['steps']} greedy decode steps on {allc} threads; ternary "
                  f"{orc.lib().port_isa().decode()} + AVX-512 bf16 head (model build {build_s:.1f}s)",
        "decode_one_core": decode["one"],
        "decode_all_cores": decode["all"],
        "gemv_shapes_warm": shapes,
        "gemv_520MB_stream": stream,
        "prefill_gemm": prefill,
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--prof-steps", type=int, default=32)
    ap.add_argument("--pmc-pass", action="store_true", help="the workload profiled for the HBM counters")
    ap.add_argument("--no-batched", action="store_true", help="skip the batched-decode (config 5) figures")
    ap.add_argument("--no-int8-head", action="store_true", help="skip the opt-in int8 LM head figure")
    ap.add_argument("--no-shapes", action="store_true", help="skip the config-1/2 per-shape GEMV figures")
    ap.add_argument("--no-sampled", action="store_true", help="skip the device-sampling decode figure")
    ap.add_argument("--shapes-only", action="store_true",
                    help="only the config-1/2 per-shape GEMV figures (the workload profiled for them)")
    ap.add_argument("--int8-head-only", action="store_true",
                    help="only the opt-in int8 LM head decode figure (the workload profiled for its kernel)")
    ap.add_argument("--no-long-prefill", action="store_true", help="skip the 512 / 2048-token prefills")
    ap.add_argument("--long-prefill-only", action="store_true",
                    help="only the 512 / 2048-token prefills (the workload profiled for the prefill attention)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the config-3 prefill GEMM sweep (the workload profiled for the MFMA counters)")
    ap.add_argument("--batched-only", action="store_true",
                    help="only the config-5 batched-decode figures (the workload profiled for its kernels)")
    args = ap.parse_args()
    if args.pmc_pass:
        return pmc_pass()
    if args.prefill_only:
        import lbt_hip

        print(json.dumps({"prefill_gemm": prefill_gemm(lbt_hip.Ctx(0))}), flush=True)
        return 0
    if args.shapes_only:
        import lbt_hip

        print(json.dumps({"gemv_shapes": gemv_shapes(lbt_hip.Ctx(0))}), flush=True)
        return 0
    if args.batched_only:
        import lbt_hip

        ctx = lbt_hip.Ctx(0)
        cfg = lbt_hip.make_config()
        model = lbt_hip.Model.synthetic(ctx, cfg, SEED)
        print(json.dumps({"batched_decode": [batched_decode(model, cfg, b) for b in (16, 64)],
                          "batched_decode_mfma_head": batched_mfma_head(model, cfg)}), flush=True)
        return 0
    if args.long_prefill_only:
        import lbt_hip

        ctx = lbt_hip.Ctx(0)
        cfg = lbt_hip.make_config()
        model = lbt_hip.Model.synthetic(ctx, cfg, SEED)
        print(json.dumps({"long_prefill": long_prefill(model, ctx, cfg)}), flush=True)
        return 0
    if args.int8_head_only:
        import lbt_hip

        ctx = lbt_hip.Ctx(0)
        cfg = lbt_hip.make_config()
        model = lbt_hip.Model.synthetic(ctx, cfg, SEED)
        prompt = np.random.default_rng(64).integers(0, cfg.vocab_size, PROMPT_LEN).astype(np.uint32)
        print(json.dumps({"int8_head_decode": int8_head_decode(model, ctx, prompt)}), flush=True)
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU; a multi-GPU figure is not part of it "
              "(rows of the ternary GEMVs would shard across GPUs with no exchange).", file=sys.stderr)
        return 2

    import lbt_hip

    ctx = lbt_hip.Ctx(0)
    cfg = lbt_hip.make_config()
    model = lbt_hip.Model.synthetic(ctx, cfg, SEED)
    prompt = np.random.default_rng(64).integers(0, cfg.vocab_size, PROMPT_LEN).astype(np.uint32)

    # warmup: prefill + W decode steps
    cache = model.new_cache()
    toks, _, _ = model.generate_greedy(prompt, max(args.warmup, 1), cache)
    cache.free()
    # the 64-token prefill's device time, after the first (which also loads code objects)
    cache = model.new_cache()
    _, ms_pf, _ = model.generate_greedy(prompt, 1, cache)
    cache.free()

    # timed: prefill (untimed) then exactly K decode steps
    cache = model.new_cache()
    first = model.forward_argmax(prompt, cache)
    ctx.sync()
    t0 = time.perf_counter()
    out, ms_dev = model.decode_greedy(cache, first, args.steps)
    ctx.sync()
    wall = time.perf_counter() - t0
    cache.free()
    ms_step = ms_dev / args.steps
    tok_s = args.steps / (ms_dev / 1e3)

    # roofline pass: HIP events around every kernel launch of a decode run
    cache = model.new_cache()
    first = model.forward_argmax(prompt, cache)
    ctx.prof_read(reset=True)
    ctx.prof_enable(True)
    model.decode_greedy(cache, first, args.prof_steps)
    prof = ctx.prof_read(reset=True)
    ctx.prof_enable(False)
    cache.free()
    g = prof["gemv"]
    achieved = g["bytes"] / (g["ms"] / 1e3) / 1e9 if g["ms"] > 0 else 0.0
    head = prof["head"]
    head_gbs = head["bytes"] / (head["ms"] / 1e3) / 1e9 if head["ms"] > 0 else 0.0

    line = {
        "metric": "decode tok/s @2B ternary batch 1; GEMV HBM GB/s as % of peak",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8xternary/i32 (bf16 head, f32 norms)",
        "data": "synthetic (random-init weights, uniform-random prompt ids)",
        "config": {
            "workload": "BitNet-b1.58-2B4T-shaped decoder (30 layers, hidden 2560, FFN 6912, 20/5 heads, "
                        "vocab 128256), 64-token prompt then greedy decode, batch 1",
            "global_batch": 1,
            "seq_len": PROMPT_LEN + args.steps,
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": gemv_traffic(),
            "kernel": "tgemv_cu_kernel (ternary decode GEMV, all 4 per-layer groups)",
            "bytes_per_launch": round(g["bytes"] / max(g["launches"], 1)),
            "avg_launch_us": round(g["ms"] * 1e3 / max(g["launches"], 1), 3),
            "launches": g["launches"],
        },
        "breakdown_ms_per_step": {k: round(v["ms"] / args.prof_steps, 4) for k, v in prof.items()},
        "lm_head_GBs": round(head_gbs, 1),
        "prefill_ms": round(ms_pf, 3),
        "wall_tok_s": round(args.steps / wall, 2),
        "tokens_head": [int(t) for t in out[:8]],
    }
    if not args.no_int8_head:
        line["int8_head_decode"] = int8_head_decode(model, ctx, prompt)
    if not args.no_sampled:
        line["sampled_decode"] = sampled_decode(model, prompt)
    if not args.no_long_prefill:
        line["long_prefill"] = long_prefill(model, ctx, cfg)
    if not args.no_batched:
        line["batched_decode"] = [batched_decode(model, cfg, bsz) for bsz in (16, 64)]
        line["batched_decode_mfma_head"] = batched_mfma_head(model, cfg)
        line["continuous_batching"] = sched_throughput(model, cfg)
        line["prefill_gemm"] = prefill_gemm(ctx)
    if not args.no_shapes:
        line["gemv_shapes"] = gemv_shapes(ctx)
    model.free()
    ctx.close()
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
