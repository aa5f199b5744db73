"""Loaders for the weight files the reference writes.

* The training scripts' pickle export: ``{"params": nnx.to_pure_dict(params)
  as numpy arrays, "config": {...}, ...}`` (flaxchat/scripts/run_tinystories.py:
  328-345, flaxchat/scripts/train_local.py:184-195). It is read with a
  restricted unpickler that rebuilds numpy arrays and plain containers and
  refuses anything else, so a file cannot run code on load.
* The PyTorch port's checkpoint: ``torch.save({"config": asdict(GPTConfig),
  "state_dict": sd})`` where ``sd`` holds the NNX kernels transposed to
  PyTorch's (out, in) orientation under ``blocks.{i}.attn.c_q.weight``-style
  keys (flaxchat/torch_port/convert_flax_to_torch.py:155-265, 329-331). It is
  read with ``torch.load(weights_only=True)``.
* The in-memory NNX parameter tree (``from_pure_dict``) and this package's
  own ``.npz`` (``save_npz`` / ``load_npz``) live in ``gpt.py``.

Orbax checkpoints (flaxchat/checkpoint.py:47-137) need orbax / tensorstore,
which are not available here; export them to one of the formats above.
"""

from __future__ import annotations

import io
import pickle
from typing import Any, Dict

import numpy as np

from .config import GPTConfig, has_ve, padded_vocab
from .gpt import GPT, from_pure_dict

__all__ = ["load_pickle_export", "load_torch_port", "torch_port_state_dict"]

# numpy's pickle reconstruction entry points (numpy 1.x and 2.x module paths)
_NUMPY_OK = {
    ("numpy.core.multiarray", "_reconstruct"), ("numpy._core.multiarray", "_reconstruct"),
    ("numpy.core.multiarray", "scalar"), ("numpy._core.multiarray", "scalar"),
    ("numpy", "ndarray"), ("numpy", "dtype"),
    ("numpy.core.numeric", "_frombuffer"), ("numpy._core.numeric", "_frombuffer"),
}
_BUILTINS_OK = {("builtins", n) for n in ("dict", "list", "tuple", "set", "frozenset", "int", "float", "str",
                                          "bytes", "bytearray", "bool", "complex", "slice")}
_BUILTINS_OK |= {("collections", "OrderedDict"), ("_codecs", "encode")}


class _ArrayUnpickler(pickle.Unpickler):
    """Unpickler limited to numpy arrays / scalars / dtypes and builtin
    containers; any other global (a function, a class with side effects) is
    refused before it is touched."""

    def find_class(self, module: str, name: str):
        if (module, name) in _NUMPY_OK or (module, name) in _BUILTINS_OK:
            return super().find_class(module, name)
        raise pickle.UnpicklingError(f"refusing to load {module}.{name} from a weight file")


def _config_from(d: Dict[str, Any], **over) -> GPTConfig:
    keys = ("sequence_len", "vocab_size", "n_layer", "n_head", "n_kv_head", "n_embd", "window_pattern",
            "tie_embeddings")
    kw = {k: d[k] for k in keys if k in d}
    kw.update(over)
    return GPTConfig(**kw)


def load_pickle_export(path: str) -> GPT:
    """Model from the training scripts' ``model.pkl`` export
    (flaxchat/scripts/run_tinystories.py:328-345): the NNX parameter tree as
    numpy arrays plus the architecture fields of GPTConfig. The lm_head is
    taken as tied when the tree has none (GPTConfig.tie_embeddings)."""
    with open(path, "rb") as f:
        payload = _ArrayUnpickler(io.BufferedReader(f)).load()
    if not isinstance(payload, dict) or "params" not in payload or "config" not in payload:
        raise ValueError(f"{path}: expected a dict with 'params' and 'config' (the reference's pickle export)")
    params = payload["params"]
    cfg = _config_from(payload["config"], tie_embeddings="lm_head" not in params)
    return from_pure_dict(cfg, params)


def _tensor_np(t) -> np.ndarray:
    return t.detach().to("cpu").float().numpy()


def load_torch_port(path: str) -> GPT:
    """Model from the PyTorch port's checkpoint
    (flaxchat/torch_port/convert_flax_to_torch.py:155-265, 329-331): Linear
    weights are stored (out, in) and transposed back to the NNX (in, out)
    kernels; embeddings are stored as they are. Only checkpoints the flaxchat
    engine can run are accepted: ReLU^2 MLP (flaxchat/gpt.py:161) and RoPE
    base 100000 (flaxchat/engine.py:76-78)."""
    import torch
    payload = torch.load(path, map_location="cpu", weights_only=True)
    if not isinstance(payload, dict) or "state_dict" not in payload or "config" not in payload:
        raise ValueError(f"{path}: expected a dict with 'config' and 'state_dict' (the PyTorch port's format)")
    c = payload["config"]
    mlp = c.get("mlp", "relu2")
    if mlp != "relu2":
        raise ValueError(f"{path}: MLP '{mlp}' — flaxchat's engine computes relu(x)^2 (flaxchat/gpt.py:161)")
    if float(c.get("rope_base", 100000.0)) != 100000.0:
        raise ValueError(f"{path}: rope_base {c.get('rope_base')} — flaxchat's engine uses 100000")
    sd = payload["state_dict"]
    cfg = _config_from(c, tie_embeddings=bool(c.get("tie_embeddings", "lm_head.weight" not in sd)))
    L = cfg.n_layer

    def W(key):  # Linear: (out, in) -> kernel (in, out)
        return np.ascontiguousarray(_tensor_np(sd[key]).T)

    params: Dict[str, Any] = {"wte": {"embedding": _tensor_np(sd["wte.weight"])}, "blocks": {},
                              "resid_lambdas": _tensor_np(sd["resid_lambdas"]),
                              "x0_lambdas": _tensor_np(sd["x0_lambdas"]),
                              "smear_gate": {"kernel": W("smear_gate.weight")},
                              "smear_lambda": _tensor_np(sd["smear_lambda"]),
                              "backout_lambda": _tensor_np(sd["backout_lambda"]), "value_embeds": {}}
    for i in range(L):
        attn = {n: {"kernel": W(f"blocks.{i}.attn.{n}.weight")} for n in ("c_q", "c_k", "c_v", "c_proj")}
        if has_ve(i, L):
            attn["ve_gate"] = {"kernel": W(f"blocks.{i}.attn.ve_gate.weight")}
            params["value_embeds"][str(i)] = {"embedding": _tensor_np(sd[f"value_embeds.{i}.weight"])}
        params["blocks"][i] = {"attn": attn, "mlp": {n: {"kernel": W(f"blocks.{i}.mlp.{n}.weight")}
                                                      for n in ("c_fc", "c_proj")}}
    if not cfg.tie_embeddings:
        k = W("lm_head.weight")  # (D, V_pad') with the port's padding
        vp = padded_vocab(cfg)
        if k.shape[1] != vp:  # re-pad the real vocabulary columns to this package's multiple of 64
            lm = np.zeros((k.shape[0], vp), np.float32)
            n = min(cfg.vocab_size, k.shape[1])
            lm[:, :n] = k[:, :n]
            k = lm
        params["lm_head"] = {"kernel": k}
    return from_pure_dict(cfg, params)


def torch_port_state_dict(model: GPT) -> Dict[str, Any]:
    """The PyTorch port's payload for `model` (the inverse of load_torch_port:
    the key names and transposes of flaxchat/torch_port/convert_flax_to_torch.py:
    155-265), fp32 tensors."""
    import torch
    from dataclasses import asdict
    t = lambda a: torch.from_numpy(np.ascontiguousarray(np.asarray(a, np.float32)))  # noqa: E731
    sd = {"wte.weight": t(model.wte.embedding), "resid_lambdas": t(model.resid_lambdas),
          "x0_lambdas": t(model.x0_lambdas), "smear_gate.weight": t(model.smear_gate.kernel.T),
          "smear_lambda": t(model.smear_lambda), "backout_lambda": t(model.backout_lambda)}
    for i, b in enumerate(model.blocks):
        for n in ("c_q", "c_k", "c_v", "c_proj"):
            sd[f"blocks.{i}.attn.{n}.weight"] = t(getattr(b.attn, n).kernel.T)
        if b.attn.ve_gate is not None:
            sd[f"blocks.{i}.attn.ve_gate.weight"] = t(b.attn.ve_gate.kernel.T)
        sd[f"blocks.{i}.mlp.c_fc.weight"] = t(b.mlp.c_fc.kernel.T)
        sd[f"blocks.{i}.mlp.c_proj.weight"] = t(b.mlp.c_proj.kernel.T)
    for k, v in model.value_embeds.items():
        sd[f"value_embeds.{k}.weight"] = t(v.embedding)
    if model.lm_head is not None:
        sd["lm_head.weight"] = t(model.lm_head.kernel.T)
    cfg = {k: v for k, v in asdict(model.config).items() if k not in ("use_scan", "short_window")}
    cfg.update(rope_base=100000.0, pad_vocab_size_to=64, mlp="relu2")
    return {"config": cfg, "state_dict": sd}
