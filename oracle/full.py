"""GPT.__call__, the full-sequence forward, restated in numpy fp32 — TEST
INFRASTRUCTURE (parity oracle; see oracle/__init__.py for who may import it).

Follows flaxchat/gpt.py:407-454 (embedding, smear, layer loop, backout,
head, softcap, masked cross-entropy) with Attention / MLP from
flaxchat/gpt.py:101-163. It differs from the per-token decode forward
(oracle/model.py) in the smear only: x_t = n_t + gate_t * n_{t-1} with n the
normalised embeddings (gpt.py:418-421), where the decode step adds the
previous smeared value. Causal mask with the window (t - j <= W) applied
when 0 < W < T (gpt.py:133-139); the -1e9 fill of masked scores is exactly
zero after the softmax in fp32, so masked keys are left out.
"""

from __future__ import annotations

import numpy as np

from .model import F32, OracleModel, apply_rotary_emb, rms_norm, sigmoid, softcap


def _seq_forward(om: OracleModel, ids, mutate=()):
    """`mutate` plants a known mistake (tests use it to show that the
    fixtures pinning this function would catch it); empty in every real use."""
    m, L, H, G, d = om.m, om.L, om.H, om.G, om.d
    T = len(ids)
    n = rms_norm(m.wte.embedding[ids])                                        # (T, D)
    x = n.copy()
    if T > 1:
        gate = m.smear_lambda * sigmoid(n[1:, :24] @ m.smear_gate.kernel)    # (T-1, 1)
        x[1:] = (n[1:] + gate * n[:-1]).astype(F32)
    x0 = n if "x0_unsmeared" in mutate else x
    cos, sin = om.cos[:T], om.sin[:T]                                         # (T, d/2)
    scale = F32(1.0 / np.sqrt(d))
    rep = H // G
    x_backout = None
    for i, blk in enumerate(m.blocks):
        x = (m.resid_lambdas[i] * x + m.x0_lambdas[i] * x0).astype(F32)
        a = blk.attn
        h = rms_norm(x)
        q = (h @ a.c_q.kernel).reshape(T, H, d)
        k = (h @ a.c_k.kernel).reshape(T, G, d)
        v = (h @ a.c_v.kernel).reshape(T, G, d)
        ve = m.value_embeds.get(str(i))
        if ve is not None:
            gin = x if "ve_gate_reads_x" in mutate else h
            gv = F32(3.0) * sigmoid(gin[:, :12] @ a.ve_gate.kernel)            # (T, G)
            v = (v + gv[:, :, None] * ve.embedding[ids].reshape(T, G, d)).astype(F32)
        q = rms_norm(apply_rotary_emb(q, cos[:, None, :], sin[:, None, :])) * F32(1.2)
        k = rms_norm(apply_rotary_emb(k, cos[:, None, :], sin[:, None, :])) * F32(1.2)
        W = om.windows[i]
        tt = np.arange(T)
        vis = tt[None, :] <= tt[:, None]
        if 0 < W < T:
            off = 1 if "window_exclusive" in mutate else 0
            vis &= (tt[:, None] - tt[None, :]) <= W - off
        y = np.empty((T, H, d), F32)
        for hh in range(H):
            g = hh % G if "gqa_interleaved" in mutate else hh // rep
            s = (q[:, hh, :] @ k[:, g, :].T) * scale                           # (T, T)
            s = np.where(vis, s, -np.inf)
            s = s - s.max(axis=1, keepdims=True)
            p = np.exp(s)
            p = p / p.sum(axis=1, keepdims=True, dtype=F32)
            y[:, hh, :] = p @ v[:, g, :]
        x = (x + y.reshape(T, H * d) @ a.c_proj.kernel).astype(F32)
        if i == L // 2 and "backout_before_mlp" in mutate:
            x_backout = x
        hid = np.maximum(rms_norm(x) @ blk.mlp.c_fc.kernel, F32(0.0)) ** 2
        x = (x + hid @ blk.mlp.c_proj.kernel).astype(F32)
        if i == L // 2 and "backout_before_mlp" not in mutate:
            x_backout = x
    if x_backout is not None:
        x = (x - m.backout_lambda * x_backout).astype(F32)
    logits = (rms_norm(x) @ om.lm)[:, : om.config.vocab_size].astype(F32)
    return softcap(logits)


def gpt_call(model, idx, targets=None, mutate=()):
    """logits (B, T, V) fp32, or the masked mean cross-entropy (float) with
    targets (flaxchat/gpt.py:446-452)."""
    om = model if isinstance(model, OracleModel) else OracleModel(model)
    idx = np.asarray(idx)
    logits = np.stack([_seq_forward(om, row, mutate) for row in idx])
    if targets is None:
        return logits
    targets = np.asarray(targets)
    z = logits.astype(np.float64)
    mx = z.max(axis=-1, keepdims=True)
    logp = z - (mx + np.log(np.exp(z - mx).sum(axis=-1, keepdims=True)))
    mask = targets >= 0
    nll = -np.take_along_axis(logp, np.where(mask, targets, 0)[..., None], axis=-1)[..., 0]
    return float((nll * mask).sum() / max(mask.sum(), 1))
