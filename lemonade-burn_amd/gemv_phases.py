"""Phase breakdown of the batch-1 decode GEMV (tgemv_cu_kernel) inside a
2B-shaped decode step, from the phase stamps of the trace build of the
library (``python lemonade-burn_amd/build.py trace`` writes
liblbt_hip_trace.so; the product library has no stamps).

For each of the four per-layer GEMVs (q/k/v, o, gate/up, down) it runs
decode steps as separate launches (LBT_NO_GRAPH=1), keeps the stamps of the
last layer's launch of that GEMV (one per workgroup, thread 0, 100 MHz
wall clock) and prints the median over workgroups and steps of each phase:
  ramp        first workgroup start -> this workgroup's start
  issue       start -> every row and weight load issued
  arrive+norm -> row arrived, RMSNorm sum of squares reduced and applied
                 (o: the attention combine first, then its subln norm)
  absmax      -> block absmax
  quant+LDS   -> quantized row in LDS, barrier passed
  dots        -> the row's dot products reduced
  stores      -> epilogue stores issued, then completed
  span        first start -> last store completed (all workgroups)
and when the last of the 16 wavefronts of a workgroup starts.
Run on the GPU box from the repository root:
  python3 lemonade-burn_amd/gemv_phases.py
"""
from __future__ import annotations

import ctypes as C
import os
import sys
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
os.environ["LBT_LIB"] = str(PKG / "liblbt_hip_trace.so")
os.environ["LBT_NO_GRAPH"] = "1"
sys.path.insert(0, str(PKG))
import lbt_hip  # noqa: E402

# (OUT, IN) template codes of the four decode GEMVs
KINDS = {"q/k/v": (4, 1), "o": (2, 2), "gate/up": (3, 1), "down": (2, 1)}
TICK_US = 0.01  # 100 MHz


def phases(tr: np.ndarray, kind: str) -> dict:
    rows = tr[(tr[:, 0] != 0) & (tr[:, 12] != 0)].astype(np.int64)
    s = lambda i: rows[:, i]
    out = {"wgs": len(rows), "ramp": s(0) - s(0).min(), "issue": s(1) - s(0)}
    if kind == "o":
        out["arrive+norm"] = s(4) - s(1)
        out["(combine)"] = s(3) - s(1)
    else:
        out["arrive+norm"] = s(4) - s(1)
    out["absmax"] = s(6) - s(4)
    out["quant+LDS"] = s(9) - s(6)
    out["dots"] = s(10) - s(9)
    out["stores issue"] = s(11) - s(10)
    out["stores drain"] = s(12) - s(11)
    out["span"] = np.array([s(12).max() - s(0).min()])
    out["last wave start"] = s(13) - s(0)
    out["last wave rows out"] = s(14) - s(0)
    return out


def main(steps: int = 8) -> None:
    ctx = lbt_hip.Ctx(0)
    lib = ctx.lib
    for fn, args in (("lbt_debug_gemvcu_select", [C.c_int, C.c_int]), ("lbt_debug_gemvcu_clear", []),
                     ("lbt_debug_gemvcu_trace", [C.c_void_p])):
        getattr(lib, fn).argtypes = args
        getattr(lib, fn).restype = C.c_int
    cfg = lbt_hip.make_config()
    m = lbt_hip.Model.synthetic(ctx, cfg, 7)
    prompt = np.random.default_rng(64).integers(0, cfg.vocab_size, 64).astype(np.uint32)
    cache = m.new_cache()
    tok = m.forward_argmax(prompt, cache)
    tr = np.zeros((1024, 16), np.uint64)
    print("| GEMV | workgroups | ramp | issue | arrive+norm | absmax | quant+LDS | dots | stores issue | stores drain"
          " | span (us) |\n|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|")
    extra = []
    for kind, (o, i) in KINDS.items():
        acc: dict = {}
        for _ in range(steps):
            assert lib.lbt_debug_gemvcu_select(o, i) == 0 and lib.lbt_debug_gemvcu_clear() == 0
            toks, _ = m.decode_greedy(cache, tok, 1)
            tok = int(toks[0])
            ctx.sync()
            assert lib.lbt_debug_gemvcu_trace(tr.ctypes.data) == 0
            for k, v in phases(tr, kind).items():
                acc.setdefault(k, []).append(v)
        med = {k: float(np.median(np.concatenate([np.atleast_1d(x) for x in v]))) * TICK_US
               for k, v in acc.items() if k != "wgs"}
        wgs = acc["wgs"][0]
        arrive = f"{med['arrive+norm']:.2f}" + (f" (combine {med['(combine)']:.2f})" if kind == "o" else "")
        print(f"| {kind} | {wgs} | {med['ramp']:.2f} | {med['issue']:.2f} | {arrive} | {med['absmax']:.2f} | "
              f"{med['quant+LDS']:.2f} | {med['dots']:.2f} | {med['stores issue']:.2f} | {med['stores drain']:.2f} | "
              f"{med['span']:.2f} |", flush=True)
        extra.append(f"{kind}: the last of the 16 wavefronts starts {med['last wave start']:.2f} us after the first "
                     f"and has its row loads out at {med['last wave rows out']:.2f} us")
    print()
    for line in extra:
        print(line)
    cache.free()
    m.free()
    ctx.close()


if __name__ == "__main__":
    main()
