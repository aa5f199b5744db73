"""numpy fp32 per-token forward with an explicit KV cache — TEST INFRASTRUCTURE
(parity oracle; see oracle/__init__.py for who may import it).

Restates flaxchat/engine.py:51-177 (`_single_step_forward`) for one sequence
in float32, and flaxchat/engine.py:382-393 (`_init_kv_cache`).
Primitives follow flaxchat/gpt.py:44-71.
"""

from __future__ import annotations

import numpy as np

F32 = np.float32


def rms_norm(x):
    """x * rsqrt(mean(x^2) + 1e-6) over the last axis (flaxchat/gpt.py:44-46)."""
    x = np.asarray(x, dtype=F32)
    ms = np.mean(x * x, axis=-1, keepdims=True, dtype=F32)
    return (x * (F32(1.0) / np.sqrt(ms + F32(1e-6)))).astype(F32)


def apply_rotary_emb(x, cos, sin):
    """x: (..., d); cos/sin: (d/2,) (flaxchat/gpt.py:65-71)."""
    h = x.shape[-1] // 2
    x1, x2 = x[..., :h], x[..., h:]
    y1 = x1 * cos + x2 * sin
    y2 = x1 * (-sin) + x2 * cos
    return np.concatenate([y1, y2], axis=-1).astype(F32)


def sigmoid(x):
    x = np.asarray(x, dtype=F32)
    return (F32(1.0) / (F32(1.0) + np.exp(-x))).astype(F32)


def softcap(z):
    """15 * tanh(z / 15) in fp32 (flaxchat/engine.py:173-174)."""
    z = np.asarray(z, dtype=F32)
    return (F32(15.0) * np.tanh(z / F32(15.0))).astype(F32)


class SeqState:
    """KV cache + smear state of one sequence (flaxchat/engine.py:382-393):
    k, v of shape (n_layer, cap, n_kv_head, head_dim) and prev_emb (n_embd,)."""

    def __init__(self, model, cap: int):
        c = model.config
        d = c.n_embd // c.n_head
        self.k = np.zeros((c.n_layer, cap, c.n_kv_head, d), F32)
        self.v = np.zeros((c.n_layer, cap, c.n_kv_head, d), F32)
        self.prev_emb = np.zeros(c.n_embd, F32)
        self.cap = cap


class OracleModel:
    """Caches the fp32 views and the RoPE table of a host GPT container."""

    def __init__(self, model, rope_len: int = None):
        from flaxchat_amd.gpt import precompute_rotary_embeddings
        self.m = model
        c = model.config
        self.config = c
        self.L, self.D, self.H, self.G = c.n_layer, c.n_embd, c.n_head, c.n_kv_head
        self.d = self.D // self.H
        # the reference precomputes 10 * sequence_len positions (flaxchat/gpt.py:254-258)
        n = rope_len or c.sequence_len * 10
        self.cos, self.sin = precompute_rotary_embeddings(n, self.d)
        self.windows = [w for (w, _) in model.window_sizes]
        self.lm = model.lm_head_kernel().astype(F32)

    def new_state(self, cap: int) -> SeqState:
        return SeqState(self.m, cap)

    def step(self, token: int, pos: int, st: SeqState, need_logits: bool = True):
        """One token through the model at position `pos`; updates `st` in
        place. Returns (V,) softcapped fp32 logits or None
        (flaxchat/engine.py:51-177)."""
        m, L, H, G, d = self.m, self.L, self.H, self.G, self.d
        if not 0 <= pos < st.cap:
            raise IndexError(f"position {pos} outside cache of {st.cap}")
        cos, sin = self.cos[pos], self.sin[pos]
        x = rms_norm(m.wte.embedding[token])
        gate = m.smear_lambda * sigmoid(x[:24] @ m.smear_gate.kernel)          # (1,)
        x = (x + gate * st.prev_emb).astype(F32)
        st.prev_emb = x
        x0 = x
        backout_layer = L // 2
        x_backout = np.zeros_like(x)
        scale = F32(1.0 / np.sqrt(d))
        for i, blk in enumerate(m.blocks):
            x = (m.resid_lambdas[i] * x + m.x0_lambdas[i] * x0).astype(F32)
            a = blk.attn
            h = rms_norm(x)
            q = (h @ a.c_q.kernel).reshape(H, d)
            k = (h @ a.c_k.kernel).reshape(G, d)
            v = (h @ a.c_v.kernel).reshape(G, d)
            ve = m.value_embeds.get(str(i))
            if ve is not None:
                gv = F32(3.0) * sigmoid(h[:12] @ a.ve_gate.kernel)              # (G,)
                v = (v + gv[:, None] * ve.embedding[token].reshape(G, d)).astype(F32)
            q = rms_norm(apply_rotary_emb(q, cos, sin)) * F32(1.2)
            k = rms_norm(apply_rotary_emb(k, cos, sin)) * F32(1.2)
            st.k[i, pos] = k
            st.v[i, pos] = v
            W = self.windows[i]
            lo = max(0, pos - W) if W > 0 else 0
            ks = st.k[i, lo:pos + 1]                                           # (n, G, d)
            vs = st.v[i, lo:pos + 1]
            rep = H // G
            y = np.empty((H, d), F32)
            for hh in range(H):
                g = hh // rep
                s = (ks[:, g, :] @ q[hh]) * scale
                s = s - s.max()
                p = np.exp(s)
                p = p / p.sum(dtype=F32)
                y[hh] = p @ vs[:, g, :]
            x = (x + y.reshape(-1) @ a.c_proj.kernel).astype(F32)
            hid = rms_norm(x) @ blk.mlp.c_fc.kernel
            hid = np.maximum(hid, F32(0.0)) ** 2
            x = (x + hid @ blk.mlp.c_proj.kernel).astype(F32)
            if i == backout_layer:
                x_backout = x
        x = (x - m.backout_lambda * x_backout).astype(F32)
        if not need_logits:
            return None
        x = rms_norm(x)
        logits = (x @ self.lm)[: self.config.vocab_size].astype(F32)
        return softcap(logits)

    def prefill(self, tokens, st: SeqState, start: int = 0):
        """Token-by-token feed of `tokens` at positions start.. (flaxchat/engine.py:396-407).
        Returns the logits after the last token."""
        logits = None
        n = len(tokens)
        for t, tok in enumerate(tokens):
            logits = self.step(int(tok), start + t, st, need_logits=(t == n - 1))
        return logits
