"""generate_speculative / generate_fast / generate_with_cache restated on the
numpy forward — TEST INFRASTRUCTURE (parity oracle; see oracle/__init__.py).

`spec_literal` follows flaxchat/engine.py:410-608 statement by statement:
token-by-token prefill of both models, k' draft steps, sequential verify,
accept/reject, bonus on `accepted == k'` (including the last-index
rejection quirk) and full re-prefill of both models on any other rejection.

`spec_rollback` is the state machine the HIP engine runs: both caches are
length pointers; each model keeps a list of fed-but-pending tokens; the
verify is one chunk of (pending + k) tokens; a rejection rolls the pointer
back to min(accept point, dirty_from) instead of re-prefilling. It must
reproduce `spec_literal` token for token (tests/test_oracle.py).
"""

from __future__ import annotations

import numpy as np

from .model import OracleModel
from .sampling import accept_round, draft_sample, get_probs, fast_sample

INF = 1 << 62


def _as_oracle(m):
    return m if isinstance(m, OracleModel) else OracleModel(m)


def spec_literal(model, draft_model, tokens, max_tokens=256, temperature=1.0, top_k=40,
                 seed=42, draft_steps=4, row=0, record=None):
    """flaxchat/engine.py:410-608 on the numpy forward. `record`, if a list,
    receives one dict per round (drafts, emitted, accepted)."""
    M, Dm = _as_oracle(model), _as_oracle(draft_model)
    assert M.config.vocab_size == Dm.config.vocab_size
    total_len = len(tokens) + max_tokens + draft_steps
    ms, ds = M.new_state(total_len), Dm.new_state(total_len)
    main_logits = M.prefill(tokens, ms)
    draft_logits = Dm.prefill(tokens, ds)
    main_pos = draft_pos = len(tokens)
    generated = list(tokens)
    ng = 0
    rnd = 0
    while ng < max_tokens:
        kp = min(draft_steps, max_tokens - ng)
        drafts, q_rows = [], []
        cur = draft_logits
        for i in range(kp):
            q_rows.append(cur)
            t = draft_sample(cur, temperature, top_k, seed, row, rnd, i)
            drafts.append(t)
            cur = Dm.step(t, draft_pos, ds)
            draft_pos += 1
        p_rows = [main_logits]
        vl = main_logits
        for dt in drafts:
            vl = M.step(dt, main_pos, ms)
            main_pos += 1
            p_rows.append(vl)
        emitted, accepted, rej, bonus = accept_round(
            np.stack(p_rows), np.stack(q_rows), drafts, temperature, top_k, seed, row, rnd)
        generated.extend(emitted[:accepted])
        ng += accepted
        if accepted == kp:
            bt = emitted[-1]
            generated.append(bt)
            ng += 1
            main_logits = M.step(bt, main_pos, ms)
            main_pos += 1
            draft_logits = Dm.step(bt, draft_pos, ds)
            draft_pos += 1
        else:
            ds = Dm.new_state(total_len)
            draft_logits = Dm.prefill(generated, ds)
            draft_pos = len(generated)
            ms = M.new_state(total_len)
            main_logits = M.prefill(generated, ms)
            main_pos = len(generated)
        if record is not None:
            record.append(dict(drafts=drafts, emitted=emitted, accepted=accepted, rej=rej))
        rnd += 1
    return generated[:len(tokens) + max_tokens]


class _Side:
    """One model's cache pointer, pending tokens and dirty mark."""

    def __init__(self, om, cap):
        self.om = om
        self.st = om.new_state(cap)
        self.hist = np.zeros((cap, om.D), np.float32)   # smeared embedding per position
        self.L = 0                                       # valid cache length
        self.pending = []                                # tokens to feed before the next round
        self.dirty = INF                                 # earliest position fed != emitted

    def rollback(self, new_len):
        self.L = new_len
        self.st.prev_emb = self.hist[new_len - 1].copy() if new_len > 0 else np.zeros(self.om.D, np.float32)

    def feed(self, toks):
        logits = None
        for t in toks:
            logits = self.om.step(int(t), self.L, self.st)
            self.hist[self.L] = self.st.prev_emb
            self.L += 1
        return logits


def spec_rollback(model, draft_model, tokens, max_tokens=256, temperature=1.0, top_k=40,
                  seed=42, draft_steps=4, row=0, record=None):
    """The engine's state machine on the numpy forward (see module docstring).

    Per round (k' = min(k, max_tokens - ng)):
      draft: feed pending_d, sample d_1 from its last logits, then feed
             d_1..d_{k-1} one at a time, sampling d_2..d_k;
      verify: feed pending_t + d_1..d_k; p_i = logits before d_i, bonus row
             = logits after d_k';
      accept (flaxchat/engine.py:525-592), then
        a == k' : target keeps pending+d_1..d_k' (pointer at +k'), draft keeps
                  what it was fed up to d_k' (d_k is pending when k' == k);
                  if the last draft was rejected the emitted token differs
                  from the cached one -> dirty mark; pending = [bonus].
        a <  k' : both pointers roll back to min(dirty, position of d_a);
                  pending = generated[pointer:]; dirty cleared.
    """
    M, Dm = _as_oracle(model), _as_oracle(draft_model)
    k = draft_steps
    P = len(tokens)
    cap = P + max_tokens + 2 * k + 8
    T, D = _Side(M, cap), _Side(Dm, cap)
    T.feed(tokens[:-1])
    D.feed(tokens[:-1])
    T.pending = [tokens[-1]]
    D.pending = [tokens[-1]]
    generated = list(tokens)
    ng, rnd = 0, 0
    while ng < max_tokens:
        kp = min(k, max_tokens - ng)
        d_base = D.L
        n_pd = len(D.pending)
        cur = D.feed(D.pending)
        D.pending = []
        drafts, q_rows = [], []
        for i in range(k):
            q_rows.append(cur)
            t = draft_sample(cur, temperature, top_k, seed, row, rnd, i)
            drafts.append(t)
            if i < k - 1:
                cur = D.feed([t])
        t_base = T.L
        n_pt = len(T.pending)
        p_rows = []
        for j, t in enumerate(list(T.pending) + drafts):
            lg = T.om.step(int(t), T.L, T.st)
            T.hist[T.L] = T.st.prev_emb
            T.L += 1
            if j >= n_pt - 1:
                p_rows.append(lg)
        T.pending = []
        emitted, accepted, rej, bonus = accept_round(
            np.stack(p_rows[:kp + 1]), np.stack(q_rows[:kp]), drafts[:kp],
            temperature, top_k, seed, row, rnd)
        generated.extend(emitted)
        ng += len(emitted)
        if bonus:
            T.rollback(t_base + n_pt + kp)
            if kp == k:
                D.rollback(d_base + n_pd + k - 1)
                D.pending = [drafts[k - 1], emitted[-1]]
            else:
                D.rollback(d_base + n_pd + kp)
                D.pending = [emitted[-1]]
            if rej >= 0:   # last-index rejection: cache holds d_k', output holds the correction
                pos = t_base + n_pt + kp - 1
                T.dirty = min(T.dirty, pos)
                D.dirty = min(D.dirty, pos)
            T.pending = [emitted[-1]]
        else:
            a = accepted
            t_new = min(T.dirty, t_base + n_pt + a - 1)
            d_new = min(D.dirty, d_base + n_pd + a - 1)
            T.rollback(t_new)
            D.rollback(d_new)
            T.pending = generated[t_new:]
            D.pending = generated[d_new:]
            T.dirty = D.dirty = INF
        if record is not None:
            record.append(dict(drafts=drafts[:kp], emitted=emitted, accepted=accepted, rej=rej))
        rnd += 1
    return generated[:P + max_tokens]


def generate_with_cache(model, tokens, max_tokens=256, temperature=1.0, top_k=40, seed=42, row=0):
    """flaxchat/engine.py:209-253 (top-k filter, then categorical or argmax).
    Uses generate_fast's draw ids (round = step index, slot 0)."""
    M = _as_oracle(model)
    st = M.new_state(len(tokens) + max_tokens)
    logits = M.prefill(tokens, st)
    generated = list(tokens)
    pos = len(tokens)
    for s in range(max_tokens):
        t = fast_sample(logits, temperature, top_k, seed, row, s)
        generated.append(t)
        if pos < st.cap:
            logits = M.step(t, pos, st)
        pos += 1
    return generated


def generate_fast(model, tokens, max_tokens=256, temperature=1.0, top_k=40, seed=42,
                  eos_token=0, row=0):
    """flaxchat/engine.py:259-376: sample from prefill logits, then loop while
    pos < total_len - 1 and not done; output includes the EOS token."""
    if top_k is None:
        raise TypeError("generate_fast requires an integer top_k (flaxchat/engine.py:310)")
    M = _as_oracle(model)
    P = len(tokens)
    total_len = P + max_tokens
    st = M.new_state(total_len)
    logits = M.prefill(tokens, st)
    buf = list(tokens)
    t = fast_sample(logits, temperature, top_k, seed, row, 0)
    buf.append(t)
    done = t == eos_token
    pos = P
    step = 1
    while pos < total_len - 1 and not done:
        logits = M.step(buf[pos], pos, st)
        pos += 1
        t = fast_sample(logits, temperature, top_k, seed, row, step)
        step += 1
        buf.append(t)
        done = done or t == eos_token
    return buf[:min(pos + 1, total_len)]
