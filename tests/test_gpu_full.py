"""GPT.__call__ on the HIP engine (flaxchat_amd.engine.gpt_forward) against
the oracle's full-sequence forward (oracle/full.py). Tolerances as the rest
of the suite: fp32 logits within 1e-3 max-abs,
bf16 within 2e-2 (measured errors are printed; about 5e-3 at these
widths); the loss within 1e-4 relative in fp32."""

import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from flaxchat_amd.engine import gpt_forward  # noqa: E402
from oracle.full import gpt_call  # noqa: E402

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("which", ["tiny", "cfg1"])
def test_full_forward_fp32(which, tiny_pair, cfg1_pair):
    _say(f"full forward fp32 {which}")
    m = (tiny_pair if which == "tiny" else cfg1_pair)[0]
    ids = np.random.default_rng(7).integers(0, m.config.vocab_size, (3, 37))
    got = gpt_forward(m, ids, dtype="fp32").cpu().numpy()
    ref = gpt_call(m, ids)
    assert got.shape == ref.shape
    assert np.abs(got - ref).max() < 1e-3


def test_full_forward_smear_is_the_full_sequence_one(tiny_pair):
    """tiny_pair's target has a non-zero smear: the device result follows
    GPT.__call__, not the decode recurrence."""
    from oracle.model import OracleModel
    m = tiny_pair[0]
    ids = np.random.default_rng(8).integers(0, m.config.vocab_size, (1, 12))
    got = gpt_forward(m, ids, dtype="fp32").cpu().numpy()[0]
    om = OracleModel(m)
    st = om.new_state(16)
    dec = np.stack([om.step(int(t), i, st) for i, t in enumerate(ids[0])])
    assert np.abs(got - gpt_call(m, ids)[0]).max() < 1e-3
    assert np.abs(got[2:] - dec[2:]).max() > 1e-2


def test_full_forward_chunks(tiny_pair):
    """Several chunks per row (the smear history carries n_{t-1} across a
    chunk boundary) equal one chunk."""
    _say("full forward chunked")
    m = tiny_pair[0]
    ids = np.random.default_rng(9).integers(0, m.config.vocab_size, (2, 45))
    one = gpt_forward(m, ids, dtype="fp32").cpu().numpy()
    many = gpt_forward(m, ids, dtype="fp32", chunk=16).cpu().numpy()
    assert np.abs(one - many).max() < 1e-5


def test_full_forward_bf16_prefill_kernels(cfg1_pair):
    """bf16 at > 1024 tokens per chunk (256 x 256 GEMM tiles, chunk attention)."""
    _say("full forward bf16 cfg1 4 x 300")
    m = cfg1_pair[0]
    ids = np.random.default_rng(10).integers(0, m.config.vocab_size, (4, 300))
    got = gpt_forward(m, ids, dtype="bf16").cpu().numpy()
    ref = gpt_call(m, ids)
    err = float(np.abs(got - ref).max())
    _say(f"  max abs err {err:.3e}")
    assert err < 2e-2


def test_full_forward_bf16_big_tiles():
    """n_embd 1024 at 4 x 900 tokens: the QKV (fused prologue) and c_fc
    GEMMs take the 256-row tiles, Wo / MLP c_proj the 64-row kernels."""
    from flaxchat_amd.config import GPTConfig
    from flaxchat_amd.gpt import GPT
    _say("full forward bf16 d1024 4 x 900")
    cfg = GPTConfig(sequence_len=1024, vocab_size=1024, n_layer=2, n_head=8, n_kv_head=8, n_embd=1024,
                    window_pattern="SL", short_window=256)
    m = GPT.init_normal(cfg, seed=12, std=0.02).perturb_scalars()
    ids = np.random.default_rng(12).integers(0, cfg.vocab_size, (4, 900))
    got = gpt_forward(m, ids, dtype="bf16").cpu().numpy()
    ref = gpt_call(m, ids)
    err = float(np.abs(got - ref).max())
    _say(f"  max abs err {err:.3e}")
    assert err < 2e-2


def test_full_forward_loss(tiny_pair):
    _say("full forward loss")
    m = tiny_pair[0]
    rng = np.random.default_rng(11)
    ids = rng.integers(0, m.config.vocab_size, (3, 20))
    tg = rng.integers(0, m.config.vocab_size, (3, 20))
    tg[0, :4] = -1
    tg[2, -6:] = -1
    got = float(gpt_forward(m, ids, tg, dtype="fp32"))
    ref = gpt_call(m, ids, tg)
    assert abs(got - ref) < 1e-4 * max(1.0, abs(ref))
    assert float(gpt_forward(m, ids, np.full((3, 20), -1), dtype="fp32")) == 0.0
    # the container's __call__ is the same entry point
    assert abs(float(m(ids, tg, dtype="fp32")) - got) < 1e-6


def test_full_forward_rejects_bad_input(tiny_pair):
    m = tiny_pair[0]
    with pytest.raises(ValueError):
        gpt_forward(m, [[1, 2, m.config.vocab_size]], dtype="fp32")
    with pytest.raises(ValueError):
        gpt_forward(m, [[1, 2, 3]], [[1, 2]], dtype="fp32")


def test_full_forward_bf16_mid_rows():
    """n_embd 1024 at 6 x 150 tokens (M = 900, a large-batch verify chunk's
    size, below the 256 x 256 kernel's tile count): c_fc on the LDS-shared
    128 x 128 tile reading the folded norm, the attention c_proj's folded
    norm on 32 x 64 tiles, the MLP c_proj (K = 4096) unsplit on the LDS-ring
    64 x 64 tile with the residual / lambda / backout epilogue."""
    from flaxchat_amd.config import GPTConfig
    from flaxchat_amd.gpt import GPT
    _say("full forward bf16 d1024 6 x 150")
    cfg = GPTConfig(sequence_len=256, vocab_size=1024, n_layer=2, n_head=8, n_kv_head=8, n_embd=1024,
                    window_pattern="SL", short_window=64)
    m = GPT.init_normal(cfg, seed=14, std=0.02).perturb_scalars()
    ids = np.random.default_rng(14).integers(0, cfg.vocab_size, (6, 150))
    got = gpt_forward(m, ids, dtype="bf16", chunk=150).cpu().numpy()
    ref = gpt_call(m, ids)
    err = float(np.abs(got - ref).max())
    _say(f"  max abs err {err:.3e}")
    assert err < 2e-2


def test_full_forward_bf16_verify_size_split():
    """n_embd 1024 at 8 x 25 tokens (M = 200, a verify-size chunk): the MLP
    c_proj (K = 4096) takes the split-K path (32 x 64 tiles, 3 splits) whose
    partials the RMSNorm kernel sums with the residual update."""
    from flaxchat_amd.config import GPTConfig
    from flaxchat_amd.gpt import GPT
    _say("full forward bf16 d1024 8 x 25")
    cfg = GPTConfig(sequence_len=256, vocab_size=1024, n_layer=2, n_head=8, n_kv_head=8, n_embd=1024,
                    window_pattern="SL", short_window=64)
    m = GPT.init_normal(cfg, seed=13, std=0.02).perturb_scalars()
    ids = np.random.default_rng(13).integers(0, cfg.vocab_size, (8, 25))
    got = gpt_forward(m, ids, dtype="bf16").cpu().numpy()
    ref = gpt_call(m, ids)
    err = float(np.abs(got - ref).max())
    _say(f"  max abs err {err:.3e}")
    assert err < 2e-2


def test_full_forward_bf16_large_verify_split_big_tiles():
    """n_embd 1536 at 8 x 150 tokens (M = 1200, a large-batch verify chunk
    like cfg5's 128 rows x 9-10 tokens): the MLP c_proj (K = 6144) takes the
    256 x 256 tiles with an 8-way K split, one split per XCD (30 tiles x 8 =
    240 workgroups), whose partials the RMSNorm kernel sums with the
    residual / lambda / backout update (the second layer is the last:
    backout applied there)."""
    from flaxchat_amd.config import GPTConfig
    from flaxchat_amd.gpt import GPT
    _say("full forward bf16 d1536 8 x 150 (split 256-row tiles)")
    cfg = GPTConfig(sequence_len=256, vocab_size=1024, n_layer=2, n_head=12, n_kv_head=12, n_embd=1536,
                    window_pattern="SL", short_window=64)
    m = GPT.init_normal(cfg, seed=15, std=0.02).perturb_scalars()
    ids = np.random.default_rng(15).integers(0, cfg.vocab_size, (8, 150))
    got = gpt_forward(m, ids, dtype="bf16", chunk=150).cpu().numpy()
    ref = gpt_call(m, ids)
    err = float(np.abs(got - ref).max())
    _say(f"  max abs err {err:.3e}")
    assert err < 2e-2
