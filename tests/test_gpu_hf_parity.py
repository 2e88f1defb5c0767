"""The HIP library against HF transformers' BitNet logits (the independent
implementation of test_hf_parity.py): the tiny model written as an
lb-convert v1 directory and loaded with lbt_model_load, prefill logits of
every row and single-token decode within the same 0.05 bound (0.1 for the
1100-token prompt's rows), and bit for bit equal to the oracle built from the
same weights."""
import numpy as np
import pytest

import hf_tiny
import lbt_hip
import lbt_oracle as orc
from conftest import announce

pytestmark = pytest.mark.gpu


def test_hip_model_matches_hf_bitnet(ctx, tmp_path):
    announce("tiny BitNet vs HF transformers logits")
    exp, prompt, seed = hf_tiny.load_fixture()
    hf_tiny.write_lbt_dir(orc, tmp_path, seed)
    m = lbt_hip.Model.load(ctx, tmp_path)
    c = m.new_cache()
    got = m.forward(np.array(prompt, np.uint32), c, all_logits=True)
    c.free()
    c = m.new_cache()
    rows = [m.forward(np.array(prompt[:10], np.uint32), c, all_logits=True)]
    for t in prompt[10:]:
        rows.append(m.forward(np.array([t], np.uint32), c))
    dec = np.concatenate(rows)
    c.free()
    m.free()
    for g in (got, dec):
        assert np.abs(g - exp).max() <= hf_tiny.TOL
    packed, ws, norms, final, emb16, _ = hf_tiny.weights(orc, seed)
    om = orc.OracleModel.wrap(hf_tiny.oracle_config(orc), packed, ws, norms, final, emb16)
    assert np.array_equal(got, om.forward(np.array(prompt, np.uint32), all_logits=True))
    om.free()


def test_hip_long_prompt_matches_hf_bitnet(ctx, tmp_path):
    announce("tiny BitNet vs HF transformers logits, 1100-token prompt")
    _, _, seed = hf_tiny.load_fixture()
    exp, rows, prompt = hf_tiny.load_long()
    hf_tiny.write_lbt_dir(orc, tmp_path, seed)
    m = lbt_hip.Model.load(ctx, tmp_path)
    c = m.new_cache()
    got = m.forward(np.array(prompt, np.uint32), c, all_logits=True)
    c.free()
    m.free()
    assert np.abs(got[rows] - exp).max() <= hf_tiny.TOL_LONG
    packed, ws, norms, final, emb16, _ = hf_tiny.weights(orc, seed)
    om = orc.OracleModel.wrap(hf_tiny.oracle_config(orc), packed, ws, norms, final, emb16)
    assert np.array_equal(got, om.forward(np.array(prompt, np.uint32), all_logits=True))
    om.free()
