"""Writes tests/golden/configs_oracle.json: token streams of the CPU
restatement (oracle/, fp32) on BASELINE configs[1] at full size and on the
architectures of configs[3] and configs[4] (2 rows, short prompts), which
the fp32 GPU engine must reproduce token for token
(tests/test_gpu_configs.py). Weights come from GPT.init_normal_parallel at
each config's seed, so the GPU box regenerates them in seconds; prompts from
numpy's default_rng at the same seed.

The streams come from oracle.spec.spec_rollback, the engine's state machine
on the numpy forward, which tests/test_oracle.py holds equal to
spec_literal (the line-by-line restatement of flaxchat/engine.py:410-608)
token for token; it needs far fewer forward steps at these sizes.

Run from the repository root (about 3 minutes, ~20 GB of host memory):
    python tests/golden/make_config_golden.py
"""
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from flaxchat_amd.config import GPTConfig  # noqa: E402
from flaxchat_amd.gpt import GPT  # noqa: E402

# name: (config kwargs, seed, draft layers, prompt lengths, max_tokens, draft_steps, [(T, top_k), ...])
CASES = {
    "cfg2": (dict(sequence_len=2048, vocab_size=65536, n_layer=12, n_head=6, n_kv_head=6, n_embd=768,
                  window_pattern="SSSL", short_window=1024), 0, 2, (512,), 256, 4, [(0.0, 40)]),
    "cfg4_arch": (dict(sequence_len=2048, vocab_size=65536, n_layer=24, n_head=12, n_kv_head=12, n_embd=1536,
                       window_pattern="SSSL", short_window=1024), 2, 4, (24, 17), 40, 6,
                  [(0.0, 40), (0.8, None)]),
    "cfg5_arch": (dict(sequence_len=8192, vocab_size=65536, n_layer=24, n_head=12, n_kv_head=4, n_embd=1536,
                       window_pattern="SSSL", short_window=2048), 3, 4, (20, 9), 40, 8, [(0.0, 40)]),
}


def models(name):
    kw, seed, n_draft = CASES[name][:3]
    tgt = GPT.init_normal_parallel(GPTConfig(**kw), seed=seed)
    return tgt, tgt.make_draft(n_draft)


def prompts(name):
    kw, seed, _, lens = CASES[name][:4]
    rng = np.random.default_rng(seed)
    return [rng.integers(0, kw["vocab_size"], n).tolist() for n in lens]


def main(names=None):
    from oracle.spec import spec_rollback
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "configs_oracle.json")
    out = json.load(open(path)) if os.path.exists(path) else {}
    for name in names or CASES:
        kw, seed, n_draft, lens, max_tokens, k, modes = CASES[name]
        t0 = time.time()
        tgt, draft = models(name)
        rows = prompts(name)
        entry = {"config": kw, "seed": seed, "draft_layers": n_draft, "prompt_lens": list(lens),
                 "max_tokens": max_tokens, "draft_steps": k, "cases": []}
        for T, top_k in modes:
            toks, recs = [], []
            for b, p in enumerate(rows):
                rec = []
                toks.append(spec_rollback(tgt, draft, p, max_tokens=max_tokens, temperature=T, top_k=top_k,
                                          seed=seed, draft_steps=k, row=b, record=rec))
                recs.append(rec)
            n_rej = sum(1 for rec in recs for r in rec if r["accepted"] < len(r["drafts"]))
            entry["cases"].append({"temperature": T, "top_k": top_k, "tokens": toks, "rounds": [len(r) for r in recs],
                                   "mid_round_rejections": n_rej})
        out[name] = entry
        print(f"{name}: {time.time() - t0:.0f} s", flush=True)
        del tgt, draft
    with open(path, "w") as f:
        json.dump(out, f)
    print("wrote", path)


if __name__ == "__main__":
    main(sys.argv[1:] or None)
