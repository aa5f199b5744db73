"""Pins the CPU restatement's forward to the reference's own PyTorch port.

The fixtures in tests/golden/torchport_forward.npz hold logits that the
reference's `GELU_GPT(mlp="relu2")` (flaxchat/torch_port/torch_gpt.py:268-375)
computed on weights converted by its `build_torch_state_dict`
(torch_port/convert_flax_to_torch.py:155-265); tests/golden/
make_torchport_golden.py wrote them. Here:

* oracle/full.py `gpt_call` (flaxchat/gpt.py:407-454) matches them for every
  case (smear on and off, GQA, value embeddings, windows, tied / untied head,
  head_dim 16 and 128) within 1e-5 max-abs; the port's own bar is 1e-4
  (torch_port/validate_parity.py:187);
* oracle/model.py `OracleModel.step`, the per-token decode forward
  (flaxchat/engine.py:51-177), matches them at every position when
  smear_lambda is 0, where the decode recurrence and the full-sequence smear
  coincide; with the smear on it matches at positions 0 and 1 and differs
  from position 2 on;
* flaxchat_amd/checkpoint.py `load_torch_port` reads the converter-written
  file tests/golden/torchport_tiny.pt back to the same weights, and the
  model it returns reproduces the port's logits;
* planted mistakes in the oracle (VE gate reading the un-normalised stream,
  backout taken before the MLP, an exclusive window, interleaved GQA
  grouping, x0 taken before the smear) each move the logits far outside the
  tolerance, so the fixtures do pin those choices.
"""
import os

import numpy as np
import pytest

from flaxchat_amd.checkpoint import load_torch_port
from oracle.full import gpt_call
from oracle.model import OracleModel
from tests.golden.torchport_cases import CASES, build_model, weight_checksum

HERE = os.path.dirname(os.path.abspath(__file__))
FIX = os.path.join(HERE, "golden", "torchport_forward.npz")
PT = os.path.join(HERE, "golden", "torchport_tiny.pt")
TOL = 1e-5


@pytest.fixture(scope="module")
def fixtures():
    return np.load(FIX, allow_pickle=False)


def _model(name, fixtures):
    m = build_model(CASES[name])
    np.testing.assert_array_equal(weight_checksum(m), fixtures[f"{name}/checksum"],
                                  err_msg=f"{name}: regenerated weights differ from the fixture's")
    return m


@pytest.mark.parametrize("name", list(CASES))
def test_full_forward_matches_port(name, fixtures):
    m = _model(name, fixtures)
    ids, ref = fixtures[f"{name}/ids"], fixtures[f"{name}/logits"]
    got = gpt_call(m, ids)
    assert got.shape == ref.shape
    err = float(np.abs(got - ref).max())
    assert err <= TOL, f"{name}: max-abs {err:.3g} against the reference port"


@pytest.mark.parametrize("name", ["nosmear", "d128_nosmear"])
def test_decode_step_matches_port_every_position(name, fixtures):
    m = _model(name, fixtures)
    assert float(m.smear_lambda[0]) == 0.0
    ids, ref = fixtures[f"{name}/ids"], fixtures[f"{name}/logits"]
    om = OracleModel(m)
    for b in range(ids.shape[0]):
        st = om.new_state(ids.shape[1])
        for t in range(ids.shape[1]):
            lg = om.step(int(ids[b, t]), t, st)
            err = float(np.abs(lg - ref[b, t]).max())
            assert err <= TOL, f"{name} row {b} position {t}: max-abs {err:.3g}"


@pytest.mark.parametrize("name", ["smear", "d128_smear"])
def test_decode_step_smear_semantics(name, fixtures):
    """The decode step adds the previous *smeared* embedding
    (flaxchat/engine.py:84-89); the full forward the previous *normalised* one
    (flaxchat/gpt.py:418-421). They agree at positions 0 and 1 only."""
    m = _model(name, fixtures)
    ids, ref = fixtures[f"{name}/ids"], fixtures[f"{name}/logits"]
    om = OracleModel(m)
    st = om.new_state(ids.shape[1])
    errs = [float(np.abs(om.step(int(ids[0, t]), t, st) - ref[0, t]).max()) for t in range(ids.shape[1])]
    assert max(errs[:2]) <= TOL
    assert min(errs[2:]) > 1e-3


def test_torch_port_checkpoint_loads(fixtures):
    """The converter's payload {"config", "state_dict"} (convert_flax_to_torch.py:
    329-331) with (out, in) Linear weights comes back as the NNX tree."""
    ref_model = _model("tiny_pt", fixtures)
    m = load_torch_port(PT)
    c, rc = m.config, ref_model.config
    assert (c.vocab_size, c.n_layer, c.n_head, c.n_kv_head, c.n_embd, c.window_pattern, c.tie_embeddings) == \
        (rc.vocab_size, rc.n_layer, rc.n_head, rc.n_kv_head, rc.n_embd, rc.window_pattern, rc.tie_embeddings)
    assert m.window_sizes == ref_model.window_sizes
    np.testing.assert_array_equal(m.wte.embedding, ref_model.wte.embedding)
    np.testing.assert_array_equal(m.lm_head.kernel, ref_model.lm_head.kernel)
    for a, b in zip(m.blocks, ref_model.blocks):
        for n in ("c_q", "c_k", "c_v", "c_proj"):
            np.testing.assert_array_equal(getattr(a.attn, n).kernel, getattr(b.attn, n).kernel)
        np.testing.assert_array_equal(a.mlp.c_fc.kernel, b.mlp.c_fc.kernel)
        np.testing.assert_array_equal(a.mlp.c_proj.kernel, b.mlp.c_proj.kernel)
    ids, ref = fixtures["tiny_pt/ids"], fixtures["tiny_pt/logits"]
    assert float(np.abs(gpt_call(m, ids) - ref).max()) <= TOL


@pytest.mark.parametrize("mistake", ["ve_gate_reads_x", "backout_before_mlp", "window_exclusive",
                                     "gqa_interleaved", "x0_unsmeared"])
def test_planted_mistakes_are_caught(mistake, fixtures):
    name = "smear"
    m = _model(name, fixtures)
    ids, ref = fixtures[f"{name}/ids"], fixtures[f"{name}/logits"]
    err = float(np.abs(gpt_call(m, ids, mutate=(mistake,)) - ref).max())
    assert err > 100 * TOL, f"planting {mistake} moved the logits by only {err:.3g}"
