"""Writes the committed golden fixtures of tests/golden/.

gemm_<rows>x<cols>_m<m>.npz: inputs generated exactly like the reference's
golden tests (crates/lb-ternary/tests/golden.rs:25-35, restated in
tests/refgen.py), packed in the LB2 layout, quantized by the oracle, with
expected i32 accumulators and f32 outputs.  Every expected i32 is
cross-checked against brute force over unpacked weights and an int64 matmul
before it is written.

known_answers.json: the hand-written known answers of the reference's unit
tests (quant.rs:201-216, ternary-kernels/src/quant.rs:33-42).

Run: python tests/golden/make_golden.py
"""
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
sys.path.insert(0, str(HERE.parent.parent / "oracle"))

import lbt_oracle as orc  # noqa: E402
from refgen import golden_case  # noqa: E402

SHAPES = [(1, 128, 1), (7, 128, 1), (33, 256, 1), (17, 384, 1), (64, 640, 1), (40, 2560, 1), (9, 6912, 1),
          (23, 384, 9), (48, 2560, 5), (37, 2560, 13), (5, 100, 3), (5, 300, 3)]


def main():
    for rows, cols, m in SHAPES:
        t, scale, x = golden_case(rows, cols, m, rows * 31 + cols + m)
        p = orc.pack(t)
        q, sa, su = orc.quantize_acts(x)
        i32 = orc.gemm_i32(p, rows, cols, q, su)
        assert np.array_equal(i32, orc.gemm_i32_bruteforce(p, rows, cols, q))
        assert np.array_equal(i32, q[:, :cols].astype(np.int64) @ t.T.astype(np.int64))
        f = orc.gemm_f32(p, rows, cols, scale, q, sa, su)
        np.savez_compressed(HERE / f"gemm_{rows}x{cols}_m{m}.npz", rows=rows, cols=cols, m=m, packed=p, s_w=scale,
                            x=x, q=q, s_a=sa, qsum=su, i32=i32, f32=f)
    ka = {
        "source": "crates/lb-ternary/src/quant.rs:201-216; crates/ternary-kernels/src/quant.rs:33-42",
        "quantize": [
            {"x": [1.0, -0.5, 0.25, 0.0, -1.0], "q": [127, -64, 32, 0, -127], "scale": 127.0, "sum": -32},
            {"x": [1.0, -2.0, 0.5, 0.0], "q": [64, -127, 32, 0], "scale": 63.5, "sum": -31},
            {"x": [0.0, 0.0, 0.0, 0.0], "q": [0, 0, 0, 0], "scale": float(np.float32(127.0) / np.float32(1e-5)),
             "sum": 0},
        ],
    }
    (HERE / "known_answers.json").write_text(json.dumps(ka, indent=1) + "\n")
    print("wrote", len(SHAPES), "gemm fixtures")


if __name__ == "__main__":
    main()
