"""The full-sequence forward GPT.__call__ (flaxchat/gpt.py:407-454): the
oracle restatement (oracle/full.py) pinned against an independent float64
torch formulation written here (whole-sequence matrices, the non-recursive
smear x_t = n_t + gate_t n_{t-1}), against the per-token decode oracle when
the smear is off, and its loss against torch's cross_entropy."""

import os
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

torch = pytest.importorskip("torch")

from flaxchat_amd.config import GPTConfig  # noqa: E402
from flaxchat_amd.gpt import GPT  # noqa: E402
from oracle.full import gpt_call  # noqa: E402
from oracle.model import OracleModel  # noqa: E402


def _cfg(**kw):
    base = dict(sequence_len=64, vocab_size=256, n_layer=3, n_head=4, n_kv_head=2, n_embd=128,
                window_pattern="SSL", short_window=8)
    base.update(kw)
    return GPTConfig(**base)


def _f64_forward(m: GPT, ids):
    """Float64 torch forward written from flaxchat/gpt.py:101-163, 407-454."""
    T64 = lambda a: torch.tensor(np.asarray(a, np.float64))  # noqa: E731
    c = m.config
    H, G, d = c.n_head, c.n_kv_head, c.n_embd // c.n_head
    T = len(ids)
    ids_t = torch.tensor(ids)

    def rms(x):
        return x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-6)

    inv = 1.0 / (100000.0 ** (torch.arange(0, d, 2, dtype=torch.float64) / d))
    ang = torch.arange(T, dtype=torch.float64)[:, None] * inv[None, :]
    cos, sin = torch.cos(ang)[:, None, :], torch.sin(ang)[:, None, :]

    def rope(x):
        x1, x2 = x[..., : d // 2], x[..., d // 2:]
        return torch.cat([x1 * cos + x2 * sin, -x1 * sin + x2 * cos], -1)

    n = rms(T64(m.wte.embedding)[ids_t])
    g = float(np.ravel(m.smear_lambda)[0]) * torch.sigmoid(n[1:, :24] @ T64(m.smear_gate.kernel))
    x = torch.cat([n[:1], n[1:] + g * n[:-1]], 0)
    x0 = x
    xb = None
    for i, blk in enumerate(m.blocks):
        x = float(m.resid_lambdas[i]) * x + float(m.x0_lambdas[i]) * x0
        h = rms(x)
        q = (h @ T64(blk.attn.c_q.kernel)).view(T, H, d)
        k = (h @ T64(blk.attn.c_k.kernel)).view(T, G, d)
        v = (h @ T64(blk.attn.c_v.kernel)).view(T, G, d)
        if str(i) in m.value_embeds:
            gate = 3.0 * torch.sigmoid(h[:, :12] @ T64(blk.attn.ve_gate.kernel))
            v = v + gate[..., None] * T64(m.value_embeds[str(i)].embedding)[ids_t].view(T, G, d)
        q, k = rms(rope(q)) * 1.2, rms(rope(k)) * 1.2
        k, v = k.repeat_interleave(H // G, 1), v.repeat_interleave(H // G, 1)
        W = m.window_sizes[i][0]
        r_, c_ = torch.arange(T)[:, None], torch.arange(T)[None, :]
        mask = c_ <= r_
        if 0 < W < T:
            mask &= (r_ - c_) <= W
        s = torch.einsum("thd,shd->hts", q, k) / np.sqrt(d)
        s = s.masked_fill(~mask, float("-inf"))
        y = torch.einsum("hts,shd->thd", torch.softmax(s, -1), v).reshape(T, H * d)
        x = x + y @ T64(blk.attn.c_proj.kernel)
        x = x + torch.relu(rms(x) @ T64(blk.mlp.c_fc.kernel)) ** 2 @ T64(blk.mlp.c_proj.kernel)
        if i == c.n_layer // 2:
            xb = x
    x = x - float(np.ravel(m.backout_lambda)[0]) * xb
    z = (rms(x) @ T64(m.lm_head_kernel()))[:, : c.vocab_size]
    return (15.0 * torch.tanh(z / 15.0)).numpy()


@pytest.mark.parametrize("tied", [False, True])
def test_oracle_full_vs_float64(tied):
    m = GPT.init_normal(_cfg(tie_embeddings=tied), seed=3, std=0.1).perturb_scalars(smear=0.8)
    ids = np.random.default_rng(1).integers(0, 256, (2, 24))
    got = gpt_call(m, ids)
    for b in range(2):
        ref = _f64_forward(m, ids[b].tolist())
        assert np.abs(got[b] - ref).max() < 2e-4


def test_oracle_full_equals_decode_without_smear():
    m = GPT.init_normal(_cfg(), seed=4, std=0.1)
    assert float(np.ravel(m.smear_lambda)[0]) == 0.0
    ids = np.random.default_rng(2).integers(0, 256, (1, 30))
    om = OracleModel(m)
    st = om.new_state(32)
    dec = np.stack([om.step(int(t), i, st) for i, t in enumerate(ids[0])])
    assert np.abs(gpt_call(m, ids)[0] - dec).max() < 1e-5


def test_oracle_full_smear_differs_from_decode():
    """With the smear on, GPT.__call__ and the decode step give different
    logits from the third position on (the decode recurrence carries the
    smeared value), the same for the first two."""
    m = GPT.init_normal(_cfg(), seed=4, std=0.1).perturb_scalars(smear=0.9)
    ids = np.random.default_rng(2).integers(0, 256, (1, 12))
    om = OracleModel(m)
    st = om.new_state(16)
    dec = np.stack([om.step(int(t), i, st) for i, t in enumerate(ids[0])])
    full = gpt_call(m, ids)[0]
    assert np.abs(full[:2] - dec[:2]).max() < 1e-5
    assert np.abs(full[2:] - dec[2:]).max() > 1e-3


def test_oracle_loss_vs_torch():
    m = GPT.init_normal(_cfg(), seed=5, std=0.1).perturb_scalars()
    rng = np.random.default_rng(3)
    ids = rng.integers(0, 256, (2, 16))
    tg = rng.integers(0, 256, (2, 16))
    tg[0, :5] = -1
    tg[1, -3:] = -1
    loss = gpt_call(m, ids, tg)
    z = torch.tensor(gpt_call(m, ids), dtype=torch.float64)
    ref = torch.nn.functional.cross_entropy(z.view(-1, 256), torch.tensor(tg).view(-1), ignore_index=-1).item()
    assert abs(loss - ref) < 1e-9 * max(1.0, abs(ref)) + 1e-12
    assert gpt_call(m, ids, np.full((2, 16), -1)) == 0.0
