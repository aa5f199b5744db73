"""The BASELINE configurations on the GPU engine.

* fp32 token identity with the CPU restatement (oracle/, fixtures written by
  tests/golden/make_config_golden.py): configs[1] (d12, V65536, prompt 512,
  256 new, k 4, greedy) at full size; the d24 architectures of configs[3]
  (k 6, greedy and T 0.8) and configs[4] (GQA 12 / 4, k 8, greedy) on two
  rows with short prompts.
* The bench workloads at full size in bf16 (configs[3]: 32 rows x 1024-token
  prompts, k 6, T 0.8; configs[4]: 128 rows x 6144-token prompts, k 8,
  greedy; configs[1]): the first round's device logits, drafts and
  accept records against the oracle's accept_round (flaxchat/engine.py:
  525-592) for every row, the draft's chunk-merged row statistics against
  a host recomputation, and two fresh sessions giving identical streams.
* bf16 greedy decoding on a reduced configs[3] shape (head_dim 128, V 65536,
  k 6, 8 rows) against the fp32 oracle, teacher-forced on the device's own
  stream: every emitted token is the oracle's argmax or within the bf16
  logits error of it.
* The first emitted token's distribution under the drop-in default top_k 40
  at T 0.8, V 65536, bf16: chi-square against the target's own probabilities
  (speculative-sampling theorem).
"""

import ctypes
import json
import os
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from flaxchat_amd import _lib  # noqa: E402
from flaxchat_amd._lib import FcRowstat  # noqa: E402
from flaxchat_amd.config import GPTConfig  # noqa: E402
from flaxchat_amd.engine import SpecSession, generate_speculative  # noqa: E402
from flaxchat_amd.runtime import DeviceModel  # noqa: E402

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _golden():
    return json.load(open(os.path.join(HERE, "golden", "configs_oracle.json")))


# ---------------------------------------------------------------- fp32 token identity
_MODELS = {}


@pytest.mark.parametrize("name,case", [("cfg2", 0), ("cfg4_arch", 0), ("cfg4_arch", 1), ("cfg5_arch", 0)])
def test_config_streams_fp32(name, case):
    from tests.golden.make_config_golden import models, prompts
    g = _golden()[name]
    if _MODELS.get("name") != name:  # one architecture held at a time (the d24 ones are 8 GB fp32)
        _MODELS.clear()
        _MODELS.update(name=name, pair=models(name))
    tgt, draft = _MODELS["pair"]
    c = g["cases"][case]
    _say(f"{name} fp32 T={c['temperature']} top_k={c['top_k']}: {len(c['tokens'])} rows, "
         f"{g['max_tokens']} new, k={g['draft_steps']}")
    rows = prompts(name)
    got = generate_speculative(tgt, draft, rows, max_tokens=g["max_tokens"], temperature=c["temperature"],
                               top_k=c["top_k"], seed=g["seed"], draft_steps=g["draft_steps"], dtype="fp32")
    assert c["mid_round_rejections"] > 0, "fixture no longer exercises a rollback"
    for b in range(len(rows)):
        ref = c["tokens"][b]
        if got[b] != ref:
            first = next(i for i, (x, y) in enumerate(zip(got[b], ref)) if x != y)
            pytest.fail(f"row {b}: first difference at position {first} ({got[b][first]} vs {ref[first]})")


# ---------------------------------------------------------------- full-size bf16 workloads
FULL = {
    # name: (config kwargs, draft layers, batch, prompt, new, k, temperature, top_k, seed)  == bench.py CONFIGS
    "cfg2": (dict(sequence_len=2048, vocab_size=65536, n_layer=12, n_head=6, n_kv_head=6, n_embd=768,
                  window_pattern="SSSL", short_window=1024), 2, 1, 512, 256, 4, 0.0, None, 0),
    "cfg4": (dict(sequence_len=2048, vocab_size=65536, n_layer=24, n_head=12, n_kv_head=12, n_embd=1536,
                  window_pattern="SSSL", short_window=1024), 4, 32, 1024, 512, 6, 0.8, None, 2),
    "cfg4_topk40": (dict(sequence_len=2048, vocab_size=65536, n_layer=24, n_head=12, n_kv_head=12, n_embd=1536,
                         window_pattern="SSSL", short_window=1024), 4, 32, 1024, 512, 6, 0.8, 40, 2),
    "cfg5": (dict(sequence_len=8192, vocab_size=65536, n_layer=24, n_head=12, n_kv_head=4, n_embd=1536,
                  window_pattern="SSSL", short_window=2048), 4, 128, 6144, 1024, 8, 0.0, None, 3),
}


def _session(target, draft, name):
    kw, _, B, P, new, k, T, top_k, seed = FULL[name]
    prompts = np.random.default_rng(seed).integers(0, kw["vocab_size"], (B, P)).tolist()
    s = SpecSession(target, draft, prompts, new, T, top_k, seed, k)
    s.prefill()
    return s


def _check_first_round(s, name):
    """Round 1's device inputs to the accept step, replayed on the host."""
    from oracle.sampling import accept_round, draft_sample, get_probs
    _, _, B, P, new, k, T, top_k, seed = FULL[name]
    rnd0 = s.bufs["round"].cpu().numpy().copy()
    assert (rnd0 == 0).all()
    s.run(max_rounds=1)
    s.stream.synchronize()
    res = s.bufs["result"].cpu().numpy()
    drafts = s.bufs["drafts"].cpu().numpy()
    n_acc = n_bonus = 0
    stats_err = 0.0
    for b in range(B):
        p = s.bufs["p_logits"][b].cpu().numpy()
        q = s.bufs["q_logits"][b].cpu().numpy()
        # the drafts are the oracle's draws from the device's draft logits
        # (flaxchat/engine.py:492-499: the multi-workgroup vocab pass of each
        # draft step and its per-row merge)
        if b < 8:
            ref_d = [draft_sample(q[i], T, top_k, seed, b, 0, i) for i in range(k)]
            assert drafts[b].tolist() == ref_d, f"row {b}: drafts {drafts[b].tolist()} vs oracle {ref_d}"
        em, acc, rej, bonus = accept_round(p, q, drafts[b], T, top_k, seed, b, 0)
        n = int(res[b, 0])
        assert res[b, 8:8 + n].tolist() == em, f"row {b}: device {res[b, 8:8 + n].tolist()} vs oracle {em}"
        assert (int(res[b, 1]), int(res[b, 2])) == (acc, rej), f"row {b}"
        n_acc += acc - (0 if rej < 0 else 1)
        n_bonus += int(bonus)
        if T > 0 and b < 4:
            # the draft's row statistics come from the multi-workgroup vocab
            # passes merged per row: max of z / T exact, exp-sum to fp32
            # rounding of a different summation order
            raw = s.bufs["q_stats"].cpu().numpy().tobytes()
            for i in range(k):
                st = FcRowstat.from_buffer_copy(raw[(b * k + i) * 32:(b * k + i + 1) * 32])
                keep = np.ones(q.shape[1], bool)
                if top_k:
                    from oracle.sampling import topk_keep
                    keep = topk_keep(q[i], top_k)
                x = (q[i][keep] / np.float32(T)).astype(np.float32)
                assert np.float32(st.mx) == x.max(), f"row {b} draft {i}: max"
                ref = np.exp(x.astype(np.float64) - float(x.max())).sum()
                stats_err = max(stats_err, abs(st.sum - ref) / ref)
                # the probabilities the oracle's accept step used
                assert np.isclose(get_probs(q[i], T, top_k)[drafts[b, i]],
                                  np.exp(q[i][drafts[b, i]] / T - st.mx) / st.sum if keep[drafts[b, i]] else 0.0,
                                  rtol=1e-5, atol=1e-12)
    _say(f"  round 1: accepted drafts {n_acc} of {B * k}, bonus rows {n_bonus}, q_stats rel err {stats_err:.2e}")
    assert stats_err < 1e-5
    return res


def _gen_state(s):
    s.stream.synchronize()
    return s.bufs["gen"].cpu().numpy().copy(), s.bufs["gen_n"].cpu().numpy().copy()


@pytest.mark.parametrize("name", ["cfg2", "cfg4", "cfg4_topk40", "cfg5"])
def test_full_size_bf16(name):
    kw, n_draft, B, P, new, k, T, top_k, seed = FULL[name]
    _say(f"{name} full size bf16: batch {B}, prompt {P}, k={k}, T={T}, top_k={top_k}")
    target = DeviceModel.random_init(GPTConfig(**kw), seed=seed, dtype="bf16")
    draft = target.make_draft(n_draft)
    runs = []
    for rep in range(2):
        s = _session(target, draft, name)
        if rep == 0:
            _check_first_round(s, name)
            s.run(max_rounds=4)
        else:
            s.run(max_rounds=5)
        runs.append(_gen_state(s))
        _say(f"  run {rep}: {int((runs[-1][1] - P).sum())} tokens after 5 rounds")
        s.close()
        del s
        torch.cuda.empty_cache()
    assert np.array_equal(runs[0][1], runs[1][1]), "generated lengths differ between identical runs"
    assert np.array_equal(runs[0][0], runs[1][0]), "token streams differ between identical runs"
    assert (runs[0][1] > P).all()


# ---------------------------------------------------------------- bf16 greedy vs the fp32 oracle
def _bf16(a):
    b = np.ascontiguousarray(a, np.float32).view(np.uint32)
    r = ((b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)).view(np.float32)
    return r.reshape(a.shape)


def _bf16_weights(m):
    """Round every matrix and embedding to bf16 (round to nearest even), so
    the device's bf16 copy holds the oracle's fp32 weights exactly and the
    comparison sees only the engine's own bf16 arithmetic."""
    m.wte.embedding = _bf16(m.wte.embedding)
    if m.lm_head is not None:
        m.lm_head.kernel = _bf16(m.lm_head.kernel)
    for blk in m.blocks:
        for lin in (blk.attn.c_q, blk.attn.c_k, blk.attn.c_v, blk.attn.c_proj, blk.mlp.c_fc, blk.mlp.c_proj):
            lin.kernel = _bf16(lin.kernel)
    for ve in m.value_embeds.values():
        ve.embedding = _bf16(ve.embedding)
    return m


def test_bf16_greedy_vs_oracle_reduced_cfg4():
    """bf16 speculative greedy decoding on the configs[3] width (D 1536,
    12 heads of 128, V 65536, 4 target / 2 draft layers, k 6, 8 rows) against
    the fp32 oracle teacher-forced on the device's stream. Greedy
    speculative decoding emits the target's argmax at every position, so
    each device token must be the oracle's argmax, or within the bf16 logits
    error of it (a near-tie the rounding can flip)."""
    from flaxchat_amd.gpt import GPT
    from oracle.model import OracleModel
    cfg = GPTConfig(sequence_len=2048, vocab_size=65536, n_layer=4, n_head=12, n_kv_head=12, n_embd=1536,
                    window_pattern="SSSL", short_window=1024)
    tgt = _bf16_weights(GPT.init_normal_parallel(cfg, seed=4))
    draft = tgt.make_draft(2)
    rng = np.random.default_rng(4)
    B, P, new = 8, 24, 40
    rows = [rng.integers(0, 65536, P).tolist() for _ in range(B)]
    got = generate_speculative(tgt, draft, rows, max_tokens=new, temperature=0.0, top_k=40, seed=4, draft_steps=6,
                               dtype="bf16")
    om = OracleModel(tgt)
    worst, exact = 0.0, 0
    for b in range(B):
        st = om.new_state(P + new + 8)
        for i in range(P - 1):
            om.step(rows[b][i], i, st)
        for j in range(new):
            pos = P - 1 + j
            lg = om.step(got[b][pos], pos, st)
            tok = got[b][pos + 1]
            gap = float(lg.max() - lg[tok])
            worst = max(worst, gap)
            exact += int(gap == 0.0)
    _say(f"bf16 greedy: {exact} of {B * new} tokens are the fp32 argmax; worst logit gap {worst:.3e}")
    assert worst < 1e-2  # measured 2.4e-3
    assert exact >= 0.95 * B * new


def test_chi_square_topk40_bf16_v65536():
    """First emitted token under top_k 40, T 0.8 (generate_speculative's
    default top-k; flaxchat/engine.py:411, 461-482) in bf16 at V 65536:
    8192 rows with one prompt, k 2. The expected distribution is the
    target's: softmax over its 40 largest logits / T, from the device's own
    verify logits of that position."""
    from scipy.stats import chisquare
    from oracle.sampling import get_probs
    cfg = GPTConfig(sequence_len=256, vocab_size=65536, n_layer=2, n_head=2, n_kv_head=2, n_embd=256,
                    window_pattern="SL", short_window=128)
    target = DeviceModel.random_init(cfg, seed=6, dtype="bf16", std=0.3)
    draft = target.make_draft(1)
    prompt = [11, 4099, 65000, 7]
    B = 8192
    s = SpecSession(target, draft, [prompt] * B, 1, 0.8, 40, 6, 2)
    s.prefill()
    s.run()
    s.stream.synchronize()
    first = s.bufs["gen"][:, len(prompt)].cpu().numpy()
    z = s.bufs["p_logits"][0, 0].cpu().numpy()
    assert np.array_equal(s.bufs["p_logits"][B - 1, 0].cpu().numpy(), z), "rows saw different target logits"
    s.close()
    p = get_probs(z, 0.8, 40).astype(np.float64)
    support = np.flatnonzero(p)
    assert len(support) == 40
    assert np.isin(first, support).all(), "a token outside the target's top 40 was emitted"
    counts = np.bincount(first, minlength=65536)[support].astype(np.float64)
    exp = p[support] * B
    big = exp >= 5
    obs, ex = counts[big], exp[big]
    if (~big).any():
        obs, ex = np.append(obs, counts[~big].sum()), np.append(ex, exp[~big].sum())
    stat, pval = chisquare(obs, ex * obs.sum() / ex.sum())
    _say(f"chi-square top_k 40 T 0.8 V 65536: {stat:.1f} p={pval:.3g} bins={len(obs)}, "
         f"top prob {p.max():.3f}")
    assert pval > 1e-4
