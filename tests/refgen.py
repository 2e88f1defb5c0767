"""Input generators restated from the reference's own tests.

xorshift64 (crates/lb-ternary/tests/golden.rs:12-23, quant.rs:218-229) and
xorshift64* (crates/lb-ternary-gpu/tests/gpu_matches_scalar.rs:6-20), with the
reference's float conversions: `(s >> 11) as f32 / (1u64 << 53) as f32 * 2 - 1`.
"""
from __future__ import annotations

import numpy as np

M64 = (1 << 64) - 1
F2_53 = np.float32(2.0**53)


class XorShift:
    """golden.rs:12-23."""

    def __init__(self, seed: int):
        self.s = seed & M64

    def next(self) -> int:
        s = self.s
        s ^= (s << 13) & M64
        s ^= s >> 7
        s ^= (s << 17) & M64
        self.s = s
        return s

    def f(self) -> np.float32:
        # (next >> 11) as f32 / (1 << 53) as f32 * 2.0 - 1.0, all in f32
        v = np.float32(self.next() >> 11) / F2_53
        return np.float32(np.float32(v * np.float32(2.0)) - np.float32(1.0))


def xorshift_f32(rng: XorShift, n: int) -> np.ndarray:
    """n successive XorShift.f() values (vectorized float conversion)."""
    s, out = rng.s, np.empty(n, np.uint64)
    for i in range(n):
        s ^= (s << 13) & M64
        s ^= s >> 7
        s ^= (s << 17) & M64
        out[i] = s >> 11
    rng.s = s
    v = out.astype(np.float64).astype(np.float32) / F2_53
    return (v * np.float32(2.0)).astype(np.float32) - np.float32(1.0)


def q8_bf16_matrix(rng: XorShift, n: int, amp: float) -> np.ndarray:
    """bf16_matrix of q8head.rs:76-78: the bf16 bits of rnd() * amp by truncation."""
    v = (xorshift_f32(rng, n) * np.float32(amp)).astype(np.float32)
    return (v.view(np.uint32) >> 16).astype(np.uint16)


class XorShiftStar:
    """gpu_matches_scalar.rs:6-20."""

    def __init__(self, seed: int):
        self.s = seed & M64

    def next(self) -> int:
        s = self.s
        s ^= s >> 12
        s ^= (s << 25) & M64
        s ^= s >> 27
        self.s = s
        return (s * 0x2545F4914F6CDD1D) & M64

    def ternary(self) -> int:
        return int(self.next() % 3) - 1

    def unit(self) -> np.float32:
        v = np.float32(self.next() >> 40) / np.float32(1 << 24)
        return np.float32(np.float32(v * np.float32(2.0)) - np.float32(1.0))


def golden_case(rows: int, cols: int, m: int, seed: int):
    """golden.rs:25-35: Gaussian-ish weights (sum of three uniforms * 0.02),
    absmean ternarisation, activations with an outlier (x20) at i % 97 == 3."""
    import lbt_oracle as orc

    rng = XorShift(seed)
    wf = np.empty(rows * cols, np.float32)
    for i in range(rows * cols):
        a, b, c = rng.f(), rng.f(), rng.f()
        wf[i] = np.float32(np.float32(np.float32(a + b) + c) * np.float32(0.02))
    t, scale = orc.ternarize_absmean(wf)
    x = np.empty(m * cols, np.float32)
    for i in range(m * cols):
        v = rng.f()
        x[i] = np.float32(v * np.float32(20.0)) if i % 97 == 3 else v
    return t.reshape(rows, cols), scale, x.reshape(m, cols)


def quant_rnd_vec(seed: int, n: int) -> np.ndarray:
    """quant.rs:218-229: uniform(-1,1) with every 53rd element (i % 53 == 7) x40."""
    rng = XorShift(seed)
    out = np.empty(n, np.float32)
    for i in range(n):
        u = rng.f()
        out[i] = np.float32(u * np.float32(40.0)) if i % 53 == 7 else u
    return out


def ternary_iid(rng: np.random.Generator, rows: int, cols: int) -> np.ndarray:
    """i.i.d. ternary with P(-1, 0, +1) = (0.3, 0.4, 0.3) (the benchmark distribution)."""
    u = rng.random((rows, cols))
    return np.where(u < 0.3, -1, np.where(u < 0.7, 0, 1)).astype(np.int8)
