"""Independent float64 numpy restatement of BitNet::forward
(crates/lb-model/src/model.rs:305-374) used to pin the f32 oracle model to the
north-star tolerance (1e-3 relative / 1e-2 absolute on logits).

Vectorised, float64 everywhere except where the reference's semantics are
integer (ActQuant codes, ternary dot): activations are quantized per row
(quant.rs:100-113) from the f64 values rounded to f32, the ternary dot is
exact, RoPE tables follow model.rs:213-230, the KV cache is rounded to bf16 as
the device path stores it.
"""
from __future__ import annotations

import numpy as np


def bf16_round(x: np.ndarray) -> np.ndarray:
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    r = (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16).astype(np.uint32)
    return r.view(np.float32).astype(np.float64)


def actquant(x: np.ndarray):
    x32 = x.astype(np.float32)
    amax = np.max(np.abs(x32), axis=-1, keepdims=True)
    s = (np.float32(127.0) / np.maximum(amax, np.float32(1e-5))).astype(np.float32)
    q = np.clip(np.rint(x32 * s), -128, 127).astype(np.int64)
    return q, s.astype(np.float64)


class RefModel64:
    def __init__(self, cfg, weights):
        """weights: dict with 'lin' [layers][7] -> (ternary int8 [rows, cols], s_w),
        'norm' [layers][4] f32, 'final_norm', 'embed' (f32 values of bf16)."""
        self.c = cfg
        self.w = weights
        hd = cfg["hidden"] // cfg["heads"]
        inv = (1.0 / cfg["theta"] ** (np.arange(hd // 2) * 2 / hd)).astype(np.float32)
        pos = np.arange(cfg["max_pos"], dtype=np.float32)
        ang = (pos[:, None] * inv[None, :]).astype(np.float32).astype(np.float64)
        self.cos = np.cos(ang).astype(np.float32).astype(np.float64)
        self.sin = np.sin(ang).astype(np.float32).astype(np.float64)
        L, kvh = cfg["layers"], cfg["kv_heads"]
        self.K = [np.zeros((kvh, 0, hd)) for _ in range(L)]
        self.V = [np.zeros((kvh, 0, hd)) for _ in range(L)]

    def rms(self, x, w):
        return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + self.c["eps"]) * w

    def lin(self, x, layer, which):
        t, sw = self.w["lin"][layer][which]
        q, s = actquant(x)
        dot = q @ t.astype(np.int64).T
        return dot.astype(np.float64) / (s * np.float64(sw))

    def rope(self, x, pos):
        hd = x.shape[-1]
        c = np.concatenate([self.cos[pos], self.cos[pos]], -1)
        s = np.concatenate([self.sin[pos], self.sin[pos]], -1)
        rot = np.concatenate([-x[..., hd // 2:], x[..., : hd // 2]], -1)
        return x * c + rot * s

    def forward(self, tokens, all_logits=False):
        c = self.c
        nh, kvh = c["heads"], c["kv_heads"]
        hd = c["hidden"] // nh
        g = nh // kvh
        m = len(tokens)
        pos0 = self.K[0].shape[1]
        pos = np.arange(pos0, pos0 + m)
        x = self.w["embed"][np.asarray(tokens)].astype(np.float64)
        for l in range(c["layers"]):
            nw = self.w["norm"][l]
            n1 = self.rms(x, nw[0])
            q = self.lin(n1, l, 0).reshape(m, nh, hd).transpose(1, 0, 2)
            k = self.lin(n1, l, 1).reshape(m, kvh, hd).transpose(1, 0, 2)
            v = self.lin(n1, l, 2).reshape(m, kvh, hd).transpose(1, 0, 2)
            q = self.rope(q, pos)
            k = self.rope(k, pos)
            self.K[l] = np.concatenate([self.K[l], bf16_round(k)], 1)
            self.V[l] = np.concatenate([self.V[l], bf16_round(v)], 1)
            total = pos0 + m
            out = np.zeros((nh, m, hd))
            for h in range(nh):
                sc = q[h] @ self.K[l][h // g].T * np.float64(np.float32(hd) ** np.float32(-0.5))
                mask = np.arange(total)[None, :] > pos[:, None]
                sc = np.where(mask, -np.inf, sc)
                sc = sc - sc.max(-1, keepdims=True)
                p = np.exp(sc)
                p /= p.sum(-1, keepdims=True)
                out[h] = p @ self.V[l][h // g]
            att = out.transpose(1, 0, 2).reshape(m, nh * hd)
            x = x + self.lin(self.rms(att, nw[2]), l, 3)
            n2 = self.rms(x, nw[1])
            gg = np.maximum(self.lin(n2, l, 4), 0.0)
            u = self.lin(n2, l, 5)
            x = x + self.lin(self.rms(gg * gg * u, nw[3]), l, 6)
        xs = x if all_logits else x[-1:]
        xn = self.rms(xs, self.w["final_norm"])
        return xn @ self.w["embed"].astype(np.float64).T


def synthetic_weights(orc, cfg_or, seed):
    """Unpacked weights of the oracle's synthetic model (same generator)."""
    H, I = cfg_or.hidden, cfg_or.intermediate
    hd = H // cfg_or.heads
    kv = cfg_or.kv_heads * hd
    shapes = [(H, H), (kv, H), (kv, H), (H, H), (I, H), (I, H), (H, I)]
    lin, norm = [], []
    for l in range(cfg_or.layers):
        row = []
        for w, (r, c) in enumerate(shapes):
            p = orc.synth_packed(seed, orc.t_layer(l, w), r, c)
            row.append((orc.unpack(p, c), np.float32(orc.lib().or_synth_wscale(c))))
        lin.append(row)
        norm.append([orc.synth_f32(seed, orc.t_layer(l, 7 + k), I if k == 3 else H).astype(np.float64)
                     for k in range(4)])
    embed = orc.bf16_to_f32(orc.synth_bf16(seed, orc.T_EMBED, cfg_or.vocab * H)).reshape(cfg_or.vocab, H)
    final = orc.synth_f32(seed, orc.T_FINAL_NORM, H).astype(np.float64)
    return {"lin": lin, "norm": norm, "final_norm": final, "embed": embed}
