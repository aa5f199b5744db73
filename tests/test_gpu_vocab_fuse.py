"""Draft steps whose logits GEMM also writes the vocab-pass partials.

Without top-k, a draft step of 17-32 rows (the LDS-shared GEMM's 32 x 64
tiles) or of 128+ rows (128 x 128 tiles) gets each logits row's argmax,
max / exp-sum of z / T and Gumbel-max terms per column tile from the lm_head
GEMM's epilogue, merged per row by one workgroup (flaxchat/engine.py:
492-499: the draft's probabilities and its draw): for steps 0..k-2 at the
start of the next step's embedding kernel, which takes the merged draft as
its token, for the last step by its own merge kernel. Checked on the first
round of a bf16 session at V 65536 against the oracle: every draft is the
oracle's draw from the device's own draft logits (oracle/sampling.py
draft_sample, the Philox / Gumbel-max restatement), the draft and target
row statistics match a host recomputation from the device's logits, and
the partials the last row's last draft step left in the buffer are
per-tile ones (each argmax inside its own tile, each maximum its tile's),
so the fused path is the one that ran.
"""

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


def _check_stats(raw, logits, T, what):
    """Row statistics (fc_rowstat records) against the logits rows."""
    err = 0.0
    for r, z in enumerate(logits):
        st = FcRowstat.from_buffer_copy(raw[r * 32:(r + 1) * 32])
        assert st.argmax == int(np.argmax(z)), f"{what} row {r}: argmax"
        if T > 0:
            x = (z / np.float32(T)).astype(np.float32)
            assert np.float32(st.mx) == x.max(), f"{what} row {r}: max"
            ref = np.exp(x.astype(np.float64) - float(x.max())).sum()
            err = max(err, abs(st.sum - ref) / ref)
    assert err < 1e-5, f"{what}: row-sum rel err {err:.2e}"
    return err


def _tile_parts(part, B, first, n, tile, z):
    """The n partials of one logits row z starting at VPart index `first`:
    each a tile's argmax and maximum."""
    o_vp = (B * _DECISION_BYTES + 255) // 256 * 256 + first * 32
    rec = part[o_vp:o_vp + n * 32].view(np.int32).reshape(n, 8)
    assert (rec[:, 1] // tile == np.arange(n)).all(), "the partials are not per-tile ones"
    assert np.array_equal(rec[:, 0].view(np.float32), z.reshape(n, tile).max(axis=1)), "per-tile maxima"


# (batch, T, k, draft tile): None = 16 rows or fewer, where the lm_head runs
# on the K-split GEMM and the separate vocab pass serves the draft step (the
# verify's own pass writes fewer partials than the draft's, from the start
# of the region, so the last row's draft partials are left to check)
@pytest.mark.parametrize("B,T,k,dtile", [(4, 0.8, 3, None), (20, 0.8, 3, 64), (32, 0.8, 6, 64),
                                         (128, 0.0, 3, 128), (128, 0.8, 3, 128)])
def test_draft_vocab_partials_from_lm_head(B, T, k, dtile):
    from oracle.sampling import draft_sample
    _say(f"draft vocab partials in the lm_head epilogue: batch {B}, T {T}, k {k}, {dtile}-column tiles")
    V, seed = 65536, 21
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
    p_all = s.bufs["p_logits"].cpu().numpy()
    q_raw = s.bufs["q_stats"].cpu().numpy().tobytes()
    p_raw = s.bufs["p_stats"].cpu().numpy().tobytes()
    part = s.bufs["part"].cpu().numpy()
    s.close()
    for b in range(B):
        ref = [draft_sample(q_all[b, i], T, None, seed, b, 0, i) for i in range(k)]
        assert drafts[b].tolist() == ref, f"row {b}: drafts {drafts[b].tolist()} vs oracle {ref}"
    eq = _check_stats(q_raw, q_all.reshape(B * k, V), T, "draft")
    ep = _check_stats(p_raw, p_all.reshape(B * (k + 1), V), T, "verify")
    _say(f"  {B * k} drafts equal the oracle's draws; row-sum rel err draft {eq:.2e}, verify {ep:.2e}")
    if dtile is not None:  # the last row's partials of the last draft step
        n = V // dtile
        _tile_parts(part, B, (B - 1) * n, n, dtile, q_all[B - 1, k - 1])
