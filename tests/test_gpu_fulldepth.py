"""bf16 numerics at full depth against the fp32 oracle, on the architectures
of the bench workloads: configs[3] (d24, D 1536, 12 heads of 128, V 65536,
SSSL window 1024, draft = the first 4 layers) and configs[4]'s GQA 12 / 4
layout (window 2048).

The weights are drawn by GPT.init_normal_parallel and rounded to bf16, so
the device's bf16 copy holds the oracle's fp32 weights exactly and every
difference is the engine's own bf16 arithmetic (bf16 activations and
caches, fp32 accumulation). The reference init keeps smear_lambda at 0
(flaxchat/gpt.py:300-303), where the decode step's smear and the
full-sequence forward's coincide, so oracle.full.gpt_call over a row's whole
sequence gives the per-token forward's logits at every position (the
teacher-forced oracle) in one batched pass.

* A verify chunk with the cfg4 verify kernel plans: 32 cache rows, chunk
  capacity 704 with 22 tokens per row at most, typical 224 tokens (the
  GEMM tiles, the split-K MLP c_proj, the folded RMSNorm, the fused QKV
  epilogue and the decode attention all chosen as in the cfg4 round); 4
  rows carry 7 tokens each after prompts of 256-1100 positions, the other
  28 feed nothing. Logits of the 28 live tokens against the oracle.
* A draft step with the draft's plans (1 token per row, typical 32).
* generate_speculative, greedy, k 6, 4 rows of 256-token prompts, 32 new
  tokens: every emitted token is the oracle's argmax at its position or
  within the bf16 logits error of it.

The logits bounds are about twice the errors these tests print on MI355X
(BOUNDS below).
"""

import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from flaxchat_amd.config import GPTConfig  # noqa: E402
from flaxchat_amd.engine import generate_speculative  # noqa: E402
from flaxchat_amd.runtime import DeviceCache, DeviceModel, Workspace, forward_packed, pack_rows, prefill_rows  # noqa: E402

pytestmark = pytest.mark.gpu

ARCH = {
    "cfg4": (dict(sequence_len=2048, vocab_size=65536, n_layer=24, n_head=12, n_kv_head=12, n_embd=1536,
                  window_pattern="SSSL", short_window=1024), 2),
    "cfg5": (dict(sequence_len=8192, vocab_size=65536, n_layer=24, n_head=12, n_kv_head=4, n_embd=1536,
                  window_pattern="SSSL", short_window=2048), 3),
}
# (max |logits - oracle|, worst oracle-argmax gap of the device's argmax): bounds.
# Measured on MI355X: verify chunk 1.18e-2 (cfg4) / 1.20e-2 (cfg5), draft step
# 1.08e-2 / 1.04e-2; every argmax equal but one near-tie of 1.8e-4 (cfg5); all
# 128 greedy tokens of each architecture the oracle's argmax. The logits bounds
# are about twice that; a flipped argmax costs at most twice the logits error,
# which bounds the gap.
BOUNDS = {"verify": (2.5e-2, 5e-2), "draft": (2.2e-2, 4.4e-2), "generate": (None, 5e-2)}

def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _round_bf16(a):
    """a rounded to bf16 (round to nearest even) in place, fp32 storage
    (torch's vectorised conversion: the d24 model holds ~2.8e9 values)."""
    t = torch.from_numpy(np.ascontiguousarray(a, np.float32))
    return t.to(torch.bfloat16).to(torch.float32).numpy()


def _models(name):
    """(host fp32 GPT whose matrices and embeddings are bf16-representable,
    its DeviceModel in bf16)."""
    from flaxchat_amd.gpt import GPT
    kw, seed = ARCH[name]
    _say(f"{name}: drawing the d24 weights (seed {seed})")
    m = GPT.init_normal_parallel(GPTConfig(**kw), seed=seed)
    m.wte.embedding = _round_bf16(m.wte.embedding)
    if m.lm_head is not None:
        m.lm_head.kernel = _round_bf16(m.lm_head.kernel)
    for blk in m.blocks:
        for lin in (blk.attn.c_q, blk.attn.c_k, blk.attn.c_v, blk.attn.c_proj, blk.mlp.c_fc, blk.mlp.c_proj):
            lin.kernel = _round_bf16(lin.kernel)
    for ve in m.value_embeds.values():
        ve.embedding = _round_bf16(ve.embedding)
    assert float(m.smear_lambda[0]) == 0.0, "the teacher-forcing shortcut needs smear_lambda 0"
    _say(f"{name}: uploading")
    return m, DeviceModel.from_host(m, dtype="bf16")


def _oracle_logits(host, seq):
    from oracle.full import gpt_call
    return gpt_call(host, np.asarray([seq], np.int64))[0]


def _compare(tag, got, ref):
    """max |got - ref| and the oracle's max logit minus its logit at the
    device's argmax, per position."""
    err = float(np.abs(got - ref).max())
    am = got.argmax(-1)
    gap = (ref.max(-1) - np.take_along_axis(ref, am[..., None], -1)[..., 0])
    _say(f"  {tag}: max |logits - oracle| {err:.3e} (max |oracle| {np.abs(ref).max():.2f}), "
         f"argmax gap {gap.max():.3e}, {(gap == 0).sum()} of {gap.size} argmax equal")
    return err, float(gap.max())


def _chunk_logits(dm, rows_live, toks_live, B, cap, max_tokens, max_per_row, typ, n_out):
    """Prefill the live rows' prompts, then feed one chunk of `toks_live`
    tokens per live row (the other rows feed nothing) with the given chunk
    capacity and typical size; logits [B][n_out][V] of the chunk."""
    dev = dm.device
    cache = DeviceCache(dm, B, cap)
    ws = Workspace(dev)
    prefill_rows(dm, cache, [rows_live.get(b, []) for b in range(B)], [0] * B, ws)
    tok, off, _ = pack_rows([toks_live.get(b, []) for b in range(B)])
    tokens = torch.zeros(max_tokens, dtype=torch.int32, device=dev)
    tokens[:len(tok)] = torch.from_numpy(tok).to(dev)
    starts = [len(rows_live.get(b, [])) for b in range(B)]
    logits = torch.zeros(B, n_out, dm.V, dtype=torch.float32, device=dev)
    forward_packed(dm, cache, tokens, torch.from_numpy(off).to(dev),
                   torch.from_numpy(np.asarray(starts, np.int32)).to(dev), max_per_row, n_out, logits, ws,
                   typ_tokens=typ)
    torch.cuda.synchronize()
    return logits.cpu().numpy()


def _check_verify_chunk(name, host, dm):
    rng = np.random.default_rng(7)
    V = dm.V
    # cfg4: one row past the 1024-position window of the S layers
    lens = {0: 256, 9: 300, 18: 1100, 31: 257} if name == "cfg4" else {0: 256, 9: 300, 18: 420, 31: 257}
    rows = {b: rng.integers(0, V, n).tolist() for b, n in lens.items()}
    new = {b: rng.integers(0, V, 7).tolist() for b in lens}
    _say(f"{name} verify chunk: 32 rows (4 live, 7 tokens each), capacity 704, typical 224")
    lg = _chunk_logits(dm, rows, new, 32, 1152, 704, 22, 224, 7)
    worst = (0.0, 0.0)
    for b in lens:
        ref = _oracle_logits(host, rows[b] + new[b])[-7:]
        e, g = _compare(f"row {b} (prompt {lens[b]})", lg[b], ref)
        worst = (max(worst[0], e), max(worst[1], g))
    _say(f"{name} verify chunk: worst |diff| {worst[0]:.3e}, worst argmax gap {worst[1]:.3e}")
    return worst


def _check_draft_step(name, host, dm):
    draft_host, draft = host.make_draft(4), dm.make_draft(4)
    rng = np.random.default_rng(8)
    V = dm.V
    lens = {3: 256, 14: 700, 22: 1030, 30: 400}
    rows = {b: rng.integers(0, V, n).tolist() for b, n in lens.items()}
    new = {b: rng.integers(0, V, 1).tolist() for b in lens}
    _say(f"{name} draft step: 32 rows (4 live, 1 token each), typical 32")
    lg = _chunk_logits(draft, rows, new, 32, 1152, 32, 1, 32, 1)
    worst = (0.0, 0.0)
    for b in lens:
        ref = _oracle_logits(draft_host, rows[b] + new[b])[-1:]
        e, g = _compare(f"row {b} (prompt {lens[b]})", lg[b], ref)
        worst = (max(worst[0], e), max(worst[1], g))
    _say(f"{name} draft step: worst |diff| {worst[0]:.3e}, worst argmax gap {worst[1]:.3e}")
    return worst


def _check_generate(name, host, dm):
    """generate_speculative(target, draft, 4 rows, greedy, k 6): greedy
    speculative decoding emits the target's argmax at every position, so the
    teacher-forced oracle's argmax must be each emitted token, or within the
    bf16 logits error of it (a near-tie the rounding can flip)."""
    rng = np.random.default_rng(9)
    B, P, new = 4, 256, 32
    prompts = [rng.integers(0, dm.V, P).tolist() for _ in range(B)]
    _say(f"{name} generate_speculative: {B} rows, prompt {P}, {new} new, k 6, greedy, bf16")
    got = generate_speculative(dm, dm.make_draft(4), prompts, max_tokens=new, temperature=0.0, top_k=40, seed=9,
                               draft_steps=6)
    worst, exact = 0.0, 0
    for b in range(B):
        assert got[b][:P] == prompts[b] and len(got[b]) == P + new
        ref = _oracle_logits(host, got[b])                 # position t: logits after got[b][:t + 1]
        z = ref[P - 1:P - 1 + new]                          # the logits each emitted token was drawn from
        tok = np.asarray(got[b][P:P + new])
        gap = z.max(-1) - z[np.arange(new), tok]
        worst = max(worst, float(gap.max()))
        exact += int((gap == 0).sum())
        _say(f"  row {b}: {(gap == 0).sum()} of {new} emitted tokens are the oracle's argmax, worst gap {gap.max():.3e}")
    _say(f"{name} generate: {exact} of {B * new} tokens are the fp32 argmax; worst logit gap {worst:.3e}")
    return worst, exact / (B * new)


@pytest.mark.parametrize("name", ["cfg4", "cfg5"])
def test_fulldepth_bf16_vs_oracle(name):
    host, dm = _models(name)
    v = _check_verify_chunk(name, host, dm)
    d = _check_draft_step(name, host, dm)
    g, frac = _check_generate(name, host, dm)
    assert v[0] <= BOUNDS["verify"][0] and v[1] <= BOUNDS["verify"][1], f"verify chunk {v}"
    assert d[0] <= BOUNDS["draft"][0] and d[1] <= BOUNDS["draft"][1], f"draft step {d}"
    assert g <= BOUNDS["generate"][1] and frac >= 0.95, f"generate: gap {g}, argmax fraction {frac}"


def test_verify_chunk_rows_past_one_query_block():
    """A verify-size chunk whose typical row fills one 16-column query block
    (7 tokens) while some rows feed 20 (a long rollback's backlog), so the
    decode attention's second query block holds queries for those rows
    only. Logits of the live tokens of long and short rows against the fp32
    oracle (2 layers at the cfg4 width, bf16-rounded weights)."""
    from flaxchat_amd.gpt import GPT
    cfg = GPTConfig(sequence_len=1024, vocab_size=8192, n_layer=2, n_head=12, n_kv_head=12, n_embd=1536,
                    window_pattern="SL", short_window=64)
    host = GPT.init_normal_parallel(cfg, seed=12)
    host.wte.embedding = _round_bf16(host.wte.embedding)
    host.lm_head.kernel = _round_bf16(host.lm_head.kernel)
    for blk in host.blocks:
        for lin in (blk.attn.c_q, blk.attn.c_k, blk.attn.c_v, blk.attn.c_proj, blk.mlp.c_fc, blk.mlp.c_proj):
            lin.kernel = _round_bf16(lin.kernel)
    for ve in host.value_embeds.values():
        ve.embedding = _round_bf16(ve.embedding)
    dm = DeviceModel.from_host(host, dtype="bf16")
    rng = np.random.default_rng(13)
    B, n_out = 32, 20
    lens = {b: int(rng.integers(1, 200)) for b in range(B)}
    n_new = {b: (20 if b in (3, 17, 30) else 7) for b in range(B)}
    rows = {b: rng.integers(0, 8192, n).tolist() for b, n in lens.items()}
    new = {b: rng.integers(0, 8192, n_new[b]).tolist() for b in range(B)}
    _say("verify chunk: 32 rows, 3 of them with 20 tokens, typical 7 per row")
    dev = dm.device
    cache = DeviceCache(dm, B, 512)
    ws = Workspace(dev)
    prefill_rows(dm, cache, [rows[b] for b in range(B)], [0] * B, ws)
    tok, off, _ = pack_rows([new[b] for b in range(B)])
    max_tokens = 704
    tokens = torch.zeros(max_tokens, dtype=torch.int32, device=dev)
    tokens[:len(tok)] = torch.from_numpy(tok).to(dev)
    starts = np.asarray([lens[b] for b in range(B)], np.int32)
    logits = torch.zeros(B, n_out, dm.V, dtype=torch.float32, device=dev)
    forward_packed(dm, cache, tokens, torch.from_numpy(off).to(dev), torch.from_numpy(starts).to(dev), 22, n_out,
                   logits, ws, typ_tokens=B * 7)
    torch.cuda.synchronize()
    lg = logits.cpu().numpy()
    worst = 0.0
    for b in (0, 3, 17, 21, 30):
        k = n_new[b]
        ref = _oracle_logits(host, rows[b] + new[b])[-k:]
        e, g = _compare(f"row {b} ({k} tokens)", lg[b, n_out - k:], ref)
        worst = max(worst, e)
        assert g <= 4e-2, f"row {b}: argmax gap {g}"
    assert worst <= 2e-2
