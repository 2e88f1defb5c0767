"""The tiny BitNet of tests/golden/make_hf_fixture.py as oracle weights and as
an lb-convert v1 directory (crates/lb-convert/src/lib.rs:1-16), for the
parity tests against HF transformers' BitNet logits."""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

sys.path.insert(0, str(Path(__file__).with_name("golden")))
import make_hf_fixture as mk  # noqa: E402

FIXTURE = Path(__file__).with_name("golden") / "hf_bitnet_tiny.npz"
TOL = 0.05  # max |logit - HF|; see test_hf_parity.py
TOL_LONG = 0.1  # the same for the rows of the 1100-token prompt


def load_fixture():
    fx = np.load(FIXTURE)
    return fx["logits"], [int(t) for t in fx["prompt"]], int(fx["seed"])


def load_long():
    """(HF logits of the stored rows, their row indices, the 1100-token prompt)."""
    fx = np.load(FIXTURE)
    return fx["long_logits"].astype(np.float64), [int(r) for r in fx["long_rows"]], mk.long_prompt()


def weights(orc, seed):
    """(packed, s_w, norms) in the oracle's order: linears q, k, v, o, gate, up,
    down per layer; norms input, post-attention, attention sub-norm, FFN sub-norm;
    then the final norm and the embedding as bf16 bits.  s_w = 1 / mean|w|
    (the scale WeightQuant divides by)."""
    layers, final, emb = mk.tiny_weights(seed)
    packed, ws, norms, tern = [], [], [], []
    for lin, nrm in layers:
        for t, a in lin:
            packed.append(orc.pack(t))
            tern.append(t)
            ws.append(np.float32(1.0 / np.abs(t.astype(np.float64) * a).mean()))
        norms += nrm
    emb16 = (emb.view(np.uint32) >> 16).astype(np.uint16)
    return packed, np.array(ws, np.float32), norms, final, emb16, tern


def oracle_config(orc):
    c = mk.CFG
    return orc.config(c["hidden"], c["intermediate"], c["heads"], c["kv_heads"], c["layers"], c["vocab"],
                      c["max_pos"])


def write_lbt_dir(orc, path: Path, seed: int):
    c = mk.CFG
    packed, ws, norms, final, emb16, _ = weights(orc, seed)
    names = ["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj",
             "mlp.up_proj", "mlp.down_proj"]
    nnames = ["input_layernorm.weight", "post_attention_layernorm.weight", "self_attn.attn_sub_norm.weight",
              "mlp.ffn_sub_norm.weight"]
    import torch
    from safetensors.torch import save_file

    t = {}
    for l in range(c["layers"]):
        for w, n in enumerate(names):
            t[f"model.layers.{l}.{n}.qweight"] = torch.from_numpy(np.ascontiguousarray(packed[l * 7 + w]))
            t[f"model.layers.{l}.{n}.wscale"] = torch.from_numpy(np.array([ws[l * 7 + w]], np.float32))
        for k, n in enumerate(nnames):
            t[f"model.layers.{l}.{n}"] = torch.from_numpy(np.ascontiguousarray(norms[l * 4 + k]))
    t["model.norm.weight"] = torch.from_numpy(final)
    t["model.embed_tokens.weight"] = torch.from_numpy(emb16.view(np.int16)).view(torch.bfloat16)
    save_file(t, str(path / "model.lbt.safetensors"), metadata={"format": "lemonade-burn-ternary", "version": "1"})
    (path / "config.json").write_text(json.dumps({
        "hidden_size": c["hidden"], "intermediate_size": c["intermediate"], "num_attention_heads": c["heads"],
        "num_key_value_heads": c["kv_heads"], "num_hidden_layers": c["layers"], "vocab_size": c["vocab"],
        "rms_norm_eps": c["eps"], "rope_theta": c["theta"], "max_position_embeddings": c["max_pos"],
        "hidden_act": "relu2", "tie_word_embeddings": True, "bos_token_id": 1}))
