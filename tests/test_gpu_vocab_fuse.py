"""Draft steps whose logits GEMM also writes the vocab-pass partials.

Without top-k, a draft step of 17-32 rows (the LDS-shared GEMM's 32 x 64
tiles) or of 128+ rows (128 x 128 tiles) gets each logits row's argmax,
max / exp-sum of z / T and Gumbel-max terms per column tile from the lm_head
GEMM's epilogue, merged per row by one workgroup (flaxchat/engine.py:
492-499: the draft's probabilities and its draw). Checked on the first
round of a bf16 session at V 65536 against the oracle: every draft is the
oracle's draw from the device's own draft logits (oracle/sampling.py
draft_sample, the Philox / Gumbel-max restatement), the row statistics
match a host recomputation, and the partials left in the buffer by the last
row's last draft step are per-tile ones (each argmax inside its own tile),
so the fused path is the one that ran (from 17 rows on)."""

import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from flaxchat_amd._lib import FcRowstat  # noqa: E402
from flaxchat_amd.config import GPTConfig  # noqa: E402
from flaxchat_amd.engine import SpecSession  # noqa: E402
from flaxchat_amd.runtime import DeviceModel  # noqa: E402

pytestmark = pytest.mark.gpu

_DECISION_BYTES = 128  # the partials buffer starts with one 128-byte decision record per row


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("B,T,tile", [(4, 0.8, None), (32, 0.8, 64), (128, 0.0, 128), (128, 0.8, 128)])
def test_draft_vocab_partials_from_lm_head(B, T, tile):
    """tile None: at 16 rows or fewer the lm_head runs on the K-split kernel
    and the separate vocab pass serves the draft step (the control case)."""
    from oracle.sampling import draft_sample
    _say(f"draft vocab partials in the lm_head epilogue: batch {B}, T {T}, {tile}-column tiles")
    V, k, seed = 65536, 3, 21
    cfg = GPTConfig(sequence_len=256, vocab_size=V, n_layer=2, n_head=2, n_kv_head=2, n_embd=256,
                    window_pattern="SL", short_window=128)
    target = DeviceModel.random_init(cfg, seed=seed, dtype="bf16", std=0.3)
    draft = target.make_draft(1)
    rng = np.random.default_rng(seed)
    prompts = rng.integers(0, V, (B, 12)).tolist()
    s = SpecSession(target, draft, prompts, 8, T, None, seed, k)
    s.prefill()
    s.run(max_rounds=1)
    s.stream.synchronize()
    drafts = s.bufs["drafts"].cpu().numpy()
    q_all = s.bufs["q_logits"].cpu().numpy()
    raw = s.bufs["q_stats"].cpu().numpy().tobytes()
    part = s.bufs["part"].cpu().numpy()
    s.close()
    stats_err = 0.0
    for b in range(B):
        q = q_all[b]
        ref = [draft_sample(q[i], T, None, seed, b, 0, i) for i in range(k)]
        assert drafts[b].tolist() == ref, f"row {b}: drafts {drafts[b].tolist()} vs oracle {ref}"
        for i in range(k):
            st = FcRowstat.from_buffer_copy(raw[(b * k + i) * 32:(b * k + i + 1) * 32])
            assert st.argmax == int(np.argmax(q[i])), f"row {b} step {i}: argmax"
            if T > 0:
                x = (q[i] / np.float32(T)).astype(np.float32)
                assert np.float32(st.mx) == x.max(), f"row {b} step {i}: max"
                ref_s = np.exp(x.astype(np.float64) - float(x.max())).sum()
                stats_err = max(stats_err, abs(st.sum - ref_s) / ref_s)
    _say(f"  {B * k} drafts equal the oracle's draws; row-sum rel err {stats_err:.2e}")
    assert stats_err < 1e-5
    if tile is None:
        return
    # the last row's partials of the last draft step (the verify's own pass
    # writes fewer entries, from the start of the region)
    nt = V // tile
    o_vp = (B * _DECISION_BYTES + 255) // 256 * 256
    rec = part[o_vp:o_vp + B * nt * 32].view(np.int32).reshape(B, nt, 8)[B - 1]
    assert (rec[:, 1] // tile == np.arange(nt)).all(), "the last row's partials are not per-tile ones"
    zmax = rec[:, 0].view(np.float32)
    q_last = q_all[B - 1, k - 1]
    assert np.array_equal(zmax, q_last.reshape(nt, tile).max(axis=1)), "per-tile maxima"
