"""Writes tests/golden/hf_bitnet_tiny.npz: logits of a tiny random BitNet b1.58
built with HF transformers' own BitNet implementation (an independent
implementation of the model the reference runs; transformers 5.15.0,
models/bitnet/modeling_bitnet.py with the online-quantized linear of
integrations/bitnet.py: WeightQuant = round(w / mean|w|) clamped to [-1, 1]
times mean|w|, ActQuant = per-token round(x * 127 / absmax) / that scale).

Run in the build container only (transformers is not used by any product or
GPU code):  python tests/golden/make_hf_fixture.py

The weights are not stored: `tiny_weights(seed)` regenerates them from the
seed with numpy's PCG64 generator, and the test builds the oracle model from
the same arrays.  Linear weights are exact ternary * a per-matrix scale, so
WeightQuant returns them unchanged up to the scale 1/mean|w| (the s_w of the
LB2 layout); the tied embedding holds bf16-representable values.  The model
runs in float64 (its RMSNorm computes in float32, as HF writes it).  K (after
RoPE) and V are rounded to bf16 as the device's KV cache stores them: without
that rounding HF and an f64 restatement of the same semantics agree to ~1e-5,
with it the cache rounding alone moves the logits by ~0.08, more than a wrong
RoPE convention does.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np

CFG = dict(vocab=300, hidden=256, intermediate=512, heads=4, kv_heads=2, layers=2, max_pos=2048, eps=1e-5,
           theta=500000.0)
SEED = 20260
PROMPT = [3, 77, 150, 299, 1, 42, 42, 208, 9, 120, 64, 255, 17, 5, 180, 91]
# a long prompt (uniform ids from this seed): RoPE at large positions and
# attention over more than 1024 keys; only the rows LONG_ROWS are stored
LONG_LEN, LONG_SEED = 1100, 11
LONG_ROWS = list(range(8)) + list(range(1020, 1030)) + list(range(1090, 1100))
OUT = Path(__file__).with_name("hf_bitnet_tiny.npz")


def long_prompt() -> list:
    return [int(t) for t in np.random.default_rng(LONG_SEED).integers(0, CFG["vocab"], LONG_LEN)]


def tiny_weights(seed: int = SEED):
    """Per layer the 7 linears (q, k, v, o, gate, up, down) as int8 ternary
    [rows, cols] with a positive scale a (w = t * a), the 4 norms (input,
    post-attention, attention sub-norm, FFN sub-norm), then the final norm and
    the embedding (float32 values of bf16)."""
    c = CFG
    rng = np.random.default_rng(seed)
    H, I = c["hidden"], c["intermediate"]
    kv = c["kv_heads"] * (H // c["heads"])
    shapes = [(H, H), (kv, H), (kv, H), (H, H), (I, H), (I, H), (H, I)]
    layers = []
    for _ in range(c["layers"]):
        lin = []
        for r, k in shapes:
            t = rng.choice(np.array([-1, 0, 1], np.int8), size=(r, k), p=[0.3, 0.4, 0.3])
            a = float(rng.uniform(0.01, 0.05))
            lin.append((t, a))
        norms = [rng.uniform(0.5, 1.5, n).astype(np.float32) for n in (H, H, H, I)]
        layers.append((lin, norms))
    final = rng.uniform(0.5, 1.5, H).astype(np.float32)
    emb = (0.05 * rng.standard_normal((c["vocab"], H))).astype(np.float32)
    u = emb.view(np.uint32).astype(np.uint64)
    emb = ((((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16).astype(np.uint32)).view(np.float32)  # bf16 round
    return layers, final, emb


def hf_logits(prompt=PROMPT) -> np.ndarray:
    import torch
    import transformers.models.bitnet.modeling_bitnet as mb
    from transformers import BitNetConfig, BitNetForCausalLM
    from transformers.integrations.bitnet import ActQuant, WeightQuant

    def bf16(x):
        return x.to(torch.bfloat16).to(x.dtype)  # round to nearest even

    rope = mb.apply_rotary_pos_emb

    def rope_bf16_k(q, k, cos, sin, *a, **kw):
        qe, ke = rope(q, k, cos, sin, *a, **kw)
        return qe, bf16(ke)

    mb.apply_rotary_pos_emb = rope_bf16_k

    c = CFG
    cfg = BitNetConfig(vocab_size=c["vocab"], hidden_size=c["hidden"], intermediate_size=c["intermediate"],
                       num_hidden_layers=c["layers"], num_attention_heads=c["heads"],
                       num_key_value_heads=c["kv_heads"], max_position_embeddings=c["max_pos"],
                       rms_norm_eps=c["eps"], hidden_act="relu2", tie_word_embeddings=True,
                       rope_parameters={"rope_theta": c["theta"], "rope_type": "default"}, bos_token_id=None,
                       eos_token_id=None)
    cfg._attn_implementation = "eager"
    model = BitNetForCausalLM(cfg).double().eval()

    class OnlineQuantLinear(torch.nn.Module):
        def __init__(self, weight, round_out=False):
            super().__init__()
            self.weight = torch.nn.Parameter(weight, requires_grad=False)
            self.round_out = round_out

        def forward(self, x):
            y = torch.nn.functional.linear(ActQuant.apply(x), WeightQuant.apply(self.weight))
            return bf16(y) if self.round_out else y

    layers, final, emb = tiny_weights()
    names = [("self_attn", "q_proj"), ("self_attn", "k_proj"), ("self_attn", "v_proj"), ("self_attn", "o_proj"),
             ("mlp", "gate_proj"), ("mlp", "up_proj"), ("mlp", "down_proj")]
    with torch.no_grad():
        for dl, (lin, norms) in zip(model.model.layers, layers):
            for (blk, name), (t, a) in zip(names, lin):
                w = torch.from_numpy(t.astype(np.float64) * a)
                setattr(getattr(dl, blk), name, OnlineQuantLinear(w, round_out=name == "v_proj"))
            dl.input_layernorm.weight.copy_(torch.from_numpy(norms[0].astype(np.float64)))
            dl.post_attention_layernorm.weight.copy_(torch.from_numpy(norms[1].astype(np.float64)))
            dl.self_attn.attn_sub_norm.weight.copy_(torch.from_numpy(norms[2].astype(np.float64)))
            dl.mlp.ffn_sub_norm.weight.copy_(torch.from_numpy(norms[3].astype(np.float64)))
        model.model.norm.weight.copy_(torch.from_numpy(final.astype(np.float64)))
        model.model.embed_tokens.weight.copy_(torch.from_numpy(emb.astype(np.float64)))
        assert model.lm_head.weight.data_ptr() == model.model.embed_tokens.weight.data_ptr(), "tied head"
        ids = torch.tensor([prompt], dtype=torch.long)
        out = model(input_ids=ids, use_cache=False)
    mb.apply_rotary_pos_emb = rope
    return out.logits[0].numpy()


if __name__ == "__main__":
    lg = hf_logits()
    ll = hf_logits(long_prompt())[LONG_ROWS]
    np.savez_compressed(OUT, logits=lg.astype(np.float64), prompt=np.array(PROMPT, np.int64), seed=np.int64(SEED),
                        long_logits=ll.astype(np.float32), long_rows=np.array(LONG_ROWS, np.int64))
    print(f"wrote {OUT}: logits {lg.shape}, long-prompt rows {ll.shape}, max |logit| {np.abs(lg).max():.3f}")
