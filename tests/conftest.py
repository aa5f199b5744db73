"""Shared fixtures. GPU tests are marked `gpu` and run only on a ROCm box."""

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm) GPU; runs the HIP kernels")


def _has_gpu():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _has_gpu():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU in this environment")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)


@pytest.fixture(scope="session")
def tiny_pair():
    """Reference-style tiny target (2 layers, SL) and a 1-layer draft with
    non-trivial smear / lambdas (cf. reference tests/conftest.py:32-43)."""
    from flaxchat_amd.config import GPTConfig
    from flaxchat_amd.gpt import GPT
    cfg = GPTConfig(sequence_len=64, vocab_size=256, n_layer=2, n_head=2, n_kv_head=2, n_embd=64,
                    window_pattern="SL", short_window=8)
    tgt = GPT.init_normal(cfg, seed=0, std=0.1).perturb_scalars()
    draft = tgt.make_draft(1)
    return tgt, draft


@pytest.fixture(scope="session")
def cfg1_pair():
    """d4 target (D256, 2 heads of 128, V8192, seq 512,
    SSSL, short window 256), 2-layer draft copying target layers 0-1 with
    shared wte / lm_head; N(0, 0.02), seed 0."""
    from flaxchat_amd.config import GPTConfig
    from flaxchat_amd.gpt import GPT
    cfg = GPTConfig(sequence_len=512, vocab_size=8192, n_layer=4, n_head=2, n_kv_head=2, n_embd=256,
                    window_pattern="SSSL", short_window=256)
    tgt = GPT.init_normal(cfg, seed=0, std=0.02)
    return tgt, tgt.make_draft(2)
