"""Weight-file loaders (flaxchat_amd/checkpoint.py): the reference's pickle
export and the PyTorch port's checkpoint, written here in the layouts the
reference's scripts produce, read back parameter for parameter."""
import os
import pickle
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

from flaxchat_amd.checkpoint import load_pickle_export, load_torch_port, torch_port_state_dict  # noqa: E402
from flaxchat_amd.config import GPTConfig  # noqa: E402
from flaxchat_amd.gpt import GPT, to_pure_dict  # noqa: E402


def _model(tied=False):
    cfg = GPTConfig(sequence_len=64, vocab_size=250, n_layer=3, n_head=2, n_kv_head=1, n_embd=64,
                    window_pattern="SL", tie_embeddings=tied)
    return GPT.init_normal(cfg, seed=4, std=0.1).perturb_scalars()


def _flat(tree, prefix=""):
    out = {}
    if isinstance(tree, dict):
        for k, v in tree.items():
            out.update(_flat(v, f"{prefix}/{k}"))
    else:
        out[prefix] = np.asarray(tree, np.float32)
    return out


def _same(a: GPT, b: GPT):
    fa, fb = _flat(to_pure_dict(a)), _flat(to_pure_dict(b))
    assert fa.keys() == fb.keys()
    for k in fa:
        np.testing.assert_array_equal(fa[k], fb[k], err_msg=k)
    assert a.config.vocab_size == b.config.vocab_size and a.config.n_layer == b.config.n_layer


@pytest.mark.parametrize("tied", [False, True])
def test_pickle_export_roundtrip(tmp_path, tied):
    """The payload of flaxchat/scripts/run_tinystories.py:328-345: numpy
    parameter tree (block indices as ints) + architecture fields."""
    m = _model(tied)
    c = m.config
    payload = {"params": to_pure_dict(m),
               "config": {"sequence_len": c.sequence_len, "vocab_size": c.vocab_size, "n_layer": c.n_layer,
                          "n_head": c.n_head, "n_kv_head": c.n_kv_head, "n_embd": c.n_embd,
                          "window_pattern": c.window_pattern},
               "training": {"steps": 10}}
    p = tmp_path / "model.pkl"
    with open(p, "wb") as f:
        pickle.dump(payload, f)
    _same(m, load_pickle_export(str(p)))


class _Evil:
    def __reduce__(self):
        return (os.system, ("echo should-not-run",))


def test_pickle_export_refuses_code(tmp_path):
    p = tmp_path / "evil.pkl"
    with open(p, "wb") as f:
        pickle.dump({"params": _Evil(), "config": {}}, f)
    with pytest.raises(pickle.UnpicklingError):
        load_pickle_export(str(p))


def _port_sd_from_reference_mapping(m: GPT):
    """State dict built by the key table of
    flaxchat/torch_port/convert_flax_to_torch.py:158-175 (Linear kernels
    transposed to (out, in), embeddings as they are), independently of
    torch_port_state_dict."""
    import torch
    d = to_pure_dict(m)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(np.asarray(a, np.float32).T))  # noqa: E731
    N = lambda a: torch.from_numpy(np.ascontiguousarray(np.asarray(a, np.float32)))  # noqa: E731
    sd = {"wte.weight": N(d["wte"]["embedding"]), "resid_lambdas": N(d["resid_lambdas"]),
          "x0_lambdas": N(d["x0_lambdas"]), "smear_gate.weight": T(d["smear_gate"]["kernel"]),
          "smear_lambda": N(d["smear_lambda"]), "backout_lambda": N(d["backout_lambda"])}
    for i, b in d["blocks"].items():
        for n, v in b["attn"].items():
            sd[f"blocks.{i}.attn.{n}.weight"] = T(v["kernel"])
        for n, v in b["mlp"].items():
            sd[f"blocks.{i}.mlp.{n}.weight"] = T(v["kernel"])
    for i, v in d["value_embeds"].items():
        sd[f"value_embeds.{i}.weight"] = N(v["embedding"])
    if "lm_head" in d:
        sd["lm_head.weight"] = T(d["lm_head"]["kernel"])
    return sd


@pytest.mark.parametrize("tied", [False, True])
def test_torch_port_roundtrip(tmp_path, tied):
    torch = pytest.importorskip("torch")
    m = _model(tied)
    c = m.config
    cfg = {"sequence_len": c.sequence_len, "vocab_size": c.vocab_size, "n_layer": c.n_layer, "n_head": c.n_head,
           "n_kv_head": c.n_kv_head, "n_embd": c.n_embd, "window_pattern": c.window_pattern,
           "tie_embeddings": tied, "rope_base": 100000.0, "pad_vocab_size_to": 64, "mlp": "relu2"}
    p = tmp_path / "port.pt"
    torch.save({"config": cfg, "state_dict": _port_sd_from_reference_mapping(m)}, p)
    _same(m, load_torch_port(str(p)))
    # the writer here produces the same payload
    mine = torch_port_state_dict(m)
    ref = _port_sd_from_reference_mapping(m)
    assert mine["state_dict"].keys() == ref.keys()
    for k in ref:
        assert torch.equal(mine["state_dict"][k], ref[k]), k


def test_torch_port_rejects_gelu(tmp_path):
    torch = pytest.importorskip("torch")
    m = _model()
    payload = torch_port_state_dict(m)
    payload["config"]["mlp"] = "gelu"
    p = tmp_path / "gelu.pt"
    torch.save(payload, p)
    with pytest.raises(ValueError, match="relu"):
        load_torch_port(str(p))
