"""Sampling primitives and the accept/reject step — TEST INFRASTRUCTURE
(parity oracle; see oracle/__init__.py for who may import it).

Restates flaxchat/engine.py:461-482 (`_apply_top_k`, `_get_probs`,
`_sample_from_probs`) and :525-592 (accept / reject / bonus) with the
engine's random stream:

  Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as
  easy as 1, 2, 3", SC'11), key = (seed lo32, seed hi32),
  counter = (element group, row, round, slot).

Slots within a round: draft sample i -> i; accept uniform i -> 16 + i;
rejection draw (q == 0 branch or residual) -> 48; bonus draw -> 49.
generate_fast uses round = step index, slot 0.

A categorical draw is Gumbel-max, like jax.random.categorical:
  argmax_v (log(max(p_v, 1e-10)) + G_v),  G_v = -log(-log(u_v)),
  u_v = ((bits >> 9) + 0.5) * 2^-23 from word v % 4 of counter (v // 4, ...)
  (23 bits keep u < 1 exactly in fp32).
An accept uniform is (bits >> 8) * 2^-24 from word 0 of counter (0, ...).
"""

from __future__ import annotations

import numpy as np

F32 = np.float32
U32 = np.uint32
M0, M1 = 0xD2511F53, 0xCD9E8D57
W0, W1 = 0x9E3779B9, 0xBB67AE85
SLOT_ACCEPT = 16
SLOT_REJECT = 48
SLOT_BONUS = 49
NEG_FILL = F32(-1e9)


def philox4x32_10(ctr, key):
    """Vectorised Philox4x32 with 10 rounds. ctr: (..., 4) uint32; key: (2,) ints.
    Round: (hi0,lo0)=M0*c0, (hi1,lo1)=M1*c2; c' = (hi1^c1^k0, lo1, hi0^c3^k1, lo0);
    key bump k += (W0, W1) between rounds."""
    c = np.asarray(ctr, dtype=np.uint64) & 0xFFFFFFFF
    c0, c1, c2, c3 = c[..., 0], c[..., 1], c[..., 2], c[..., 3]
    k0 = np.uint64(int(key[0]) & 0xFFFFFFFF)
    k1 = np.uint64(int(key[1]) & 0xFFFFFFFF)
    mask = np.uint64(0xFFFFFFFF)
    for r in range(10):
        if r:
            k0 = (k0 + np.uint64(W0)) & mask
            k1 = (k1 + np.uint64(W1)) & mask
        p0 = np.uint64(M0) * c0
        p1 = np.uint64(M1) * c2
        hi0, lo0 = p0 >> np.uint64(32), p0 & mask
        hi1, lo1 = p1 >> np.uint64(32), p1 & mask
        c0, c1, c2, c3 = hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0
    return np.stack([c0, c1, c2, c3], axis=-1).astype(U32)


def seed_key(seed: int):
    s = int(seed) & 0xFFFFFFFFFFFFFFFF
    return (s & 0xFFFFFFFF, s >> 32)


def vocab_bits(V: int, seed: int, row: int, rnd: int, slot: int):
    """uint32 bits for elements 0..V-1 of draw (row, round, slot)."""
    n = (V + 3) // 4
    ctr = np.zeros((n, 4), np.uint64)
    ctr[:, 0] = np.arange(n)
    ctr[:, 1] = row
    ctr[:, 2] = rnd
    ctr[:, 3] = slot
    return philox4x32_10(ctr, seed_key(seed)).reshape(-1)[:V]


def gumbel(V, seed, row, rnd, slot):
    bits = vocab_bits(V, seed, row, rnd, slot)
    u = (((bits >> U32(9)).astype(F32) + F32(0.5)) * F32(2.0 ** -23)).astype(F32)
    return (-np.log(-np.log(u))).astype(F32)


def accept_uniform(seed, row, rnd, i) -> float:
    bits = philox4x32_10(np.array([[0, row, rnd, SLOT_ACCEPT + i]], np.uint64), seed_key(seed))[0, 0]
    return float(F32((int(bits) >> 8) * 2.0 ** -24))


def topk_keep(z, top_k):
    """Boolean mask of the entries lax.top_k keeps: exactly k, larger value
    first, lower index first among equal values (flaxchat/engine.py:461-466)."""
    V = z.shape[-1]
    if top_k is None or top_k <= 0 or top_k >= V:
        return np.ones(V, bool)
    order = np.lexsort((np.arange(V), -z.astype(np.float64)))
    keep = np.zeros(V, bool)
    keep[order[:top_k]] = True
    return keep


def get_probs(z, temperature, top_k):
    """(V,) probabilities from (V,) logits (flaxchat/engine.py:468-476):
    top-k fill with -1e9, softmax(z / T) if T > 0 else one-hot argmax."""
    z = np.asarray(z, F32)
    keep = topk_keep(z, top_k)
    filt = np.where(keep, z, NEG_FILL).astype(F32)
    if temperature > 0:
        x = (filt / F32(temperature)).astype(F32)
        e = np.exp(x - x.max()).astype(F32)
        return (e / e.sum(dtype=F32)).astype(F32)
    p = np.zeros(z.shape[-1], F32)
    p[int(np.argmax(filt))] = 1.0
    return p


def sample_from_probs(p, seed, row, rnd, slot) -> int:
    """categorical(log(max(p, 1e-10))) as Gumbel-max (flaxchat/engine.py:478-482)."""
    lp = np.log(np.maximum(p.astype(F32), F32(1e-10))).astype(F32)
    g = gumbel(p.shape[-1], seed, row, rnd, slot)
    return int(np.argmax((lp + g).astype(F32)))


def fast_sample(z, temperature, top_k, seed, row, step) -> int:
    """generate_fast's `_sample` (flaxchat/engine.py:308-324): greedy picks
    the argmax of the top-k values (their first index); otherwise a
    categorical over the k kept values at temperature T, with no floor."""
    z = np.asarray(z, F32)
    if temperature <= 0:
        return int(np.argmax(z))
    keep = topk_keep(z, top_k)
    g = gumbel(z.shape[-1], seed, row, step, 0)
    sc = np.where(keep, (z / F32(temperature)).astype(F32) + g, -np.inf)
    return int(np.argmax(sc))


def accept_round(p_logits, q_logits, drafts, temperature, top_k, seed, row, rnd):
    """One accept/reject pass (flaxchat/engine.py:525-592).

    p_logits: (k'+1, V) target logits; row i is the target's prediction
      for draft i (row k' follows the last draft, for the bonus).
    q_logits: (k', V) draft logits that produced drafts[i].
    Returns (emitted tokens, accepted count, rejected index or -1,
    bonus emitted flag). `accepted` counts the correction token, so a
    rejection at the last index still leads to a bonus (engine.py:573).
    """
    kp = len(drafts)
    emitted, accepted, rej = [], 0, -1
    for i in range(kp):
        dt = int(drafts[i])
        if temperature == 0 or temperature < 0:
            am = int(np.argmax(get_probs(p_logits[i], 0.0, top_k)))
            if am == dt:
                emitted.append(dt)
                accepted += 1
            else:
                emitted.append(am)
                accepted += 1
                rej = i
                break
        else:
            mp = get_probs(p_logits[i], temperature, top_k)
            dp = get_probs(q_logits[i], temperature, top_k)
            p_main, p_draft = float(mp[dt]), float(dp[dt])
            if p_draft == 0:
                emitted.append(sample_from_probs(mp, seed, row, rnd, SLOT_REJECT))
                accepted += 1
                rej = i
                break
            accept_prob = min(1.0, p_main / p_draft)
            u = accept_uniform(seed, row, rnd, i)
            if u < accept_prob:
                emitted.append(dt)
                accepted += 1
            else:
                adj = np.maximum(mp - dp, F32(0.0)).astype(F32)
                s = adj.sum(dtype=F32)
                adj = (adj / s).astype(F32) if s > 0 else mp
                emitted.append(sample_from_probs(adj, seed, row, rnd, SLOT_REJECT))
                accepted += 1
                rej = i
                break
    bonus = False
    if accepted == kp:
        bp = get_probs(p_logits[kp], temperature, top_k)
        if temperature > 0:
            emitted.append(sample_from_probs(bp, seed, row, rnd, SLOT_BONUS))
        else:
            emitted.append(int(np.argmax(bp)))
        bonus = True
    return emitted, accepted, rej, bonus


def draft_sample(q_logits_row, temperature, top_k, seed, row, rnd, i) -> int:
    """Draft proposal i of a round (flaxchat/engine.py:493-499)."""
    if temperature > 0:
        return sample_from_probs(get_probs(q_logits_row, temperature, top_k), seed, row, rnd, i)
    return int(np.argmax(get_probs(q_logits_row, 0.0, top_k)))
