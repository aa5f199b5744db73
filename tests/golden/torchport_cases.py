"""Model and input recipes of the fixtures in torchport_forward.npz.

Shared by the fixture writer (make_torchport_golden.py, which runs the
reference's PyTorch port on them) and the tests (which rebuild the same
weights and compare the CPU restatement and the HIP engine with the port's
logits). Weights come from GPT.init_normal(config, seed, std); a checksum
stored with each case catches a change of the random stream.
"""
import numpy as np

from flaxchat_amd.config import GPTConfig
from flaxchat_amd.gpt import GPT


def _ids(seed, B, T, V):
    return np.random.default_rng(seed).integers(0, V, (B, T)).astype(np.int64)


# d = 16, GQA 4 query heads on 2 KV heads, value embeddings on layers 1 and 3,
# backout after layer 2, S window of 8 keys (+1) inside a 40-token sequence.
_SMALL = GPTConfig(sequence_len=64, vocab_size=300, n_layer=4, n_head=4, n_kv_head=2, n_embd=64,
                   window_pattern="SSSL", short_window=8)
# head_dim 128 (the HIP engine's bf16 path), GQA 2 on 1, 3 layers (VE on 0 and 2).
_D128 = GPTConfig(sequence_len=64, vocab_size=256, n_layer=3, n_head=2, n_kv_head=1, n_embd=256,
                  window_pattern="SL", short_window=6)
# the checkpoint-file case: windows from the reference rule (sequence_len 64 -> S = 128).
_TINY = GPTConfig(sequence_len=64, vocab_size=128, n_layer=2, n_head=2, n_kv_head=1, n_embd=32,
                  window_pattern="SL")

CASES = {
    # perturbed lambdas, smear_lambda 0.7: pins the full forward (gpt.py:407-454)
    "smear": dict(config=_SMALL, seed=11, std=0.1, perturb=True, smear=0.7, ids=_ids(5, 2, 40, 300)),
    # same weights with the smear off: the full forward equals the per-token decode
    # recurrence at every position, so this pins OracleModel.step (engine.py:51-177)
    "nosmear": dict(config=_SMALL, seed=11, std=0.1, perturb=True, smear=0.0, ids=_ids(5, 2, 40, 300)),
    # tied head (lm_head = wte^T, gpt.py:441-444)
    "tied": dict(config=_SMALL.with_(tie_embeddings=True), seed=12, std=0.1, perturb=True, smear=0.5,
                 ids=_ids(6, 1, 33, 300)),
    # head_dim 128, smear on and off
    "d128_smear": dict(config=_D128, seed=13, std=0.05, perturb=True, smear=0.7, ids=_ids(7, 2, 24, 256)),
    "d128_nosmear": dict(config=_D128, seed=13, std=0.05, perturb=True, smear=0.0, ids=_ids(7, 2, 24, 256)),
    # the converter-written checkpoint file (torchport_tiny.pt)
    "tiny_pt": dict(config=_TINY, seed=14, std=0.2, perturb=True, smear=0.6, ids=_ids(8, 2, 20, 128),
                    write_pt=True),
}


def build_model(case) -> GPT:
    m = GPT.init_normal(case["config"], seed=case["seed"], std=case["std"])
    if case.get("perturb"):
        m.perturb_scalars(seed=case["seed"], smear=case["smear"])
    return m


def weight_checksum(model: GPT) -> np.ndarray:
    """A few raw weights plus float64 sums, enough to tell a different draw."""
    w = model.wte.embedding
    lm = model.lm_head_kernel()
    b0 = model.blocks[0]
    return np.array([w[0, 0], w[1, 3], lm[2, 5], b0.attn.c_q.kernel[0, 1], b0.mlp.c_fc.kernel[3, 2],
                     float(np.sum(w, dtype=np.float64)), float(np.sum(b0.attn.c_v.kernel, dtype=np.float64)),
                     float(np.sum(model.blocks[-1].mlp.c_proj.kernel, dtype=np.float64)),
                     float(model.smear_lambda[0]), float(np.sum(model.resid_lambdas, dtype=np.float64))],
                    np.float64)
