"""Writes tests/golden/cfg1_oracle.json: BASELINE configs[0] token streams
and per-round accept records from the CPU restatement (oracle/), plus a
digest of the first prefill logits. Regression anchors for the oracle and
the GPU engine (the reference's own tests hold no numeric vectors for this
path). Run from the repository root: python tests/golden/make_golden.py"""
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from flaxchat_amd.config import GPTConfig  # noqa: E402
from flaxchat_amd.gpt import GPT  # noqa: E402
from oracle.model import OracleModel  # noqa: E402
from oracle.spec import spec_literal  # noqa: E402


def cfg1_models():
    cfg = GPTConfig(sequence_len=512, vocab_size=8192, n_layer=4, n_head=2, n_kv_head=2, n_embd=256,
                    window_pattern="SSSL", short_window=256)
    tgt = GPT.init_normal(cfg, seed=0, std=0.02)
    return tgt, tgt.make_draft(2)


def main():
    tgt, draft = cfg1_models()
    prompt = np.random.default_rng(0).integers(0, 8192, 32).tolist()
    out = {"config": "BASELINE configs[0]: d4 D256 H2 G2 V8192 seq512 SSSL sw256, draft 2 layers, "
                     "N(0,0.02) seed 0, prompt = default_rng(0).integers(0, 8192, 32)",
           "prompt": prompt, "cases": []}
    for T, top_k, seed in ((0.0, 40, 42), (0.8, None, 2), (1.0, 40, 7)):
        rec = []
        toks = spec_literal(tgt, draft, prompt, max_tokens=64, temperature=T, top_k=top_k, seed=seed,
                            draft_steps=4, record=rec)
        out["cases"].append({"temperature": T, "top_k": top_k, "seed": seed, "draft_steps": 4,
                             "tokens": toks, "rounds": [{k: r[k] for k in ("drafts", "emitted", "accepted", "rej")}
                                                        for r in rec]})
    om = OracleModel(tgt)
    lg = om.prefill(prompt, om.new_state(40))
    order = np.argsort(-lg)[:8]
    out["prefill_logits"] = {"top8_ids": order.tolist(), "top8_vals": [float(lg[i]) for i in order],
                             "sum": float(lg.astype(np.float64).sum()), "sumsq": float((lg.astype(np.float64) ** 2).sum())}
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cfg1_oracle.json")
    with open(path, "w") as f:
        json.dump(out, f)
    print("wrote", path)


if __name__ == "__main__":
    main()
