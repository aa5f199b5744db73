"""bench.py's contract on the CPU: one GPU only, and its workloads are the
BASELINE.json configurations the GPU tests run."""

import json
import os
import re
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""


def test_workloads_match_the_gpu_tests():
    from tests.test_gpu_configs import FULL
    for name, row in bench.CONFIGS.items():
        full = FULL[name]
        assert full[:7] == row[:7], name          # model, draft layers, batch, prompt, new, k, T
        assert full[8] == row[7], name            # seed
        assert full[7] is None, name              # the headline runs without a top-k filter


def _numbers(text):
    return [int(x) for x in re.findall(r"(?<![\w.])(\d+)(?![\w.])", text)]


def test_workloads_match_baseline():
    """Each bench workload's sizes appear in the BASELINE.json configuration it names."""
    with open(os.path.join(ROOT, "BASELINE.json")) as f:
        configs = json.load(f)["configs"]
    for name, idx in (("cfg2", 1), ("cfg4", 3), ("cfg5", 4)):
        kw, n_draft, B, P, new, k, T, seed = bench.CONFIGS[name]
        text = configs[idx]
        nums = set(_numbers(text))
        for v in (kw["n_layer"], kw["n_embd"], kw["n_head"], kw["vocab_size"], kw["sequence_len"],
                  kw["short_window"], n_draft, P, new, seed):
            assert v in nums, (name, v)
        assert f"draft_steps={k}" in text, name
        assert f"batch {B}" in text or (B == 1 and "batch 1" in text), name
        assert kw["window_pattern"] in text, name
        if T > 0:
            assert f"temperature {T}" in text, name
        else:
            assert "greedy" in text, name
        if kw["n_kv_head"] != kw["n_head"]:
            assert f"{kw['n_kv_head']} KV heads" in text, name
