"""torch.ops.flaxchat_mi355x without a GPU: the operators are registered,
their fake implementations propagate shapes on meta tensors, and the
fragment-order view used for bf16 outputs inverts the documented layout."""

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import flaxchat_amd.torch_ops as ops  # noqa: E402
from flaxchat_amd.runtime import frag_pack  # noqa: E402


def test_registered():
    for name in ("pack_operand", "linear", "attention", "cross_entropy", "forward", "attn_prologue", "attn_qkv",
                 "row_stats", "spec_accept", "spec_round"):
        assert hasattr(torch.ops.flaxchat_mi355x, name)


def test_fake_shapes():
    m = dict(device="meta")
    x = torch.empty(5, 128, dtype=torch.bfloat16, **m)
    w = torch.empty(96, 128, dtype=torch.bfloat16, **m)
    assert torch.ops.flaxchat_mi355x.pack_operand(x).shape == (16, 128)
    y = torch.ops.flaxchat_mi355x.linear(x, w, True)
    assert y.shape == (5, 96) and y.dtype == torch.float32
    q = torch.empty(7, 6, 128, dtype=torch.bfloat16, **m)
    kc = torch.empty(2, 3, 64, 128, dtype=torch.bfloat16, **m)
    ro = torch.empty(3, dtype=torch.int32, **m)
    st = torch.empty(2, dtype=torch.int32, **m)
    o = torch.ops.flaxchat_mi355x.attention(q, kc, kc, ro, st, 4, 0)
    assert o.shape == (7, 768) and o.dtype == torch.bfloat16
    lg = torch.empty(9, 1000, **m)
    assert torch.ops.flaxchat_mi355x.cross_entropy(lg, torch.empty(9, dtype=torch.int64, **m)).shape == (9,)


@pytest.mark.parametrize("R,K", [(16, 32), (21, 96), (3, 64)])
def test_frag_to_rows_inverts_frag_pack(R, K):
    a = np.arange(R * K, dtype=np.float32).reshape(R, K)
    packed = torch.from_numpy(frag_pack(a))
    np.testing.assert_array_equal(ops.frag_to_rows(packed, R).numpy(), a)


def _cpu_model(**kw):
    """An fp32 DeviceModel whose weights sit in host memory: enough for the
    operators' host-side checks and fake implementations (no kernel runs)."""
    from flaxchat_amd.config import GPTConfig
    from flaxchat_amd.gpt import GPT
    from flaxchat_amd.runtime import DeviceModel
    cfg = GPTConfig(sequence_len=64, vocab_size=256, n_layer=2, n_head=6, n_kv_head=2, n_embd=768,
                    window_pattern="SL", short_window=32)
    cfg.__dict__.update(kw)
    return DeviceModel.from_host(GPT.init_normal(cfg, seed=0, std=0.02), dtype="fp32", device=torch.device("cpu"))


def test_engine_op_fakes():
    """Shape propagation of the engine operators on meta tensors (the model
    descriptor is host memory; nothing is launched)."""
    import ctypes
    dm = _cpu_model()
    addr = ctypes.addressof(dm.desc)
    meta = dict(device="meta")
    kc = torch.empty(2, 3, 2, 64, 128, **meta)
    i = torch.empty(9, dtype=torch.int32, **meta)
    h = torch.empty(9, 768, **meta)
    q = torch.ops.flaxchat_mi355x.attn_qkv(addr, 0, kc, kc, h, i, i, i, 0)
    assert q.shape == (9, 6, 128) and q.dtype == torch.float32
    qkv = torch.empty(9, 1280, **meta)
    assert torch.ops.flaxchat_mi355x.attn_prologue(addr, 1, kc, kc, qkv, h, i, i, i).shape == (9, 6, 128)
    mx, s, tau, tie, am = torch.ops.flaxchat_mi355x.row_stats(torch.empty(5, 100, **meta), 1.0, 0)
    assert mx.shape == (5,) and am.dtype == torch.int32


def test_engine_ops_refuse_foreign_and_stale_descriptors():
    """Only the descriptor of a live DeviceModel is accepted: a hand-built
    fc_model, an arbitrary integer and the address of a collected model are
    refused with ValueError before any pointer reaches the library."""
    import ctypes
    import gc
    from flaxchat_amd import _lib
    kc = torch.zeros(2, 3, 2, 64, 128)
    i = torch.zeros(9, dtype=torch.int32)
    h = torch.zeros(9, 768)
    raw = _lib.FcModel()
    raw.n_layer, raw.n_head, raw.head_dim, raw.n_kv_head = 2, 6, 128, 2
    for addr in (ctypes.addressof(raw), 0x7F0000001000, 0):
        with pytest.raises(ValueError, match="live DeviceModel"):
            torch.ops.flaxchat_mi355x.attn_qkv(addr, 0, kc, kc, h, i, i, i, 0)
    dm = _cpu_model()
    addr = ctypes.addressof(dm.desc)
    del dm
    gc.collect()
    with pytest.raises(ValueError, match="live DeviceModel"):
        torch.ops.flaxchat_mi355x.attn_qkv(addr, 0, kc, kc, h, i, i, i, 0)


def test_engine_ops_check_tensors_against_the_model():
    """Each mismatch between a tensor and the model descriptor raises
    ValueError on the host: cache layers, KV heads, head_dim, dtype and
    capacity, the GEMM input's size and dtype, the layer index, and every
    speculative-state buffer's size."""
    import ctypes
    dm = _cpu_model()
    addr = ctypes.addressof(dm.desc)
    op = torch.ops.flaxchat_mi355x
    i = torch.zeros(9, dtype=torch.int32)
    h = torch.zeros(9, 768)
    good = torch.zeros(2, 3, 2, 64, 128)
    bad_caches = {
        "n_layer": torch.zeros(1, 3, 2, 64, 128),
        "n_kv_head": torch.zeros(2, 3, 6, 64, 128),
        "head_dim": torch.zeros(2, 3, 2, 64, 64),
        "dtype": torch.zeros(2, 3, 2, 64, 128, dtype=torch.bfloat16),
        "cap": torch.zeros(2, 3, 2, 40, 128),
    }
    for what, kc in bad_caches.items():
        with pytest.raises(ValueError):
            op.attn_qkv(addr, 0, kc, kc, h, i, i, i, 0)
    with pytest.raises(ValueError):  # v_cache of a different size
        op.attn_qkv(addr, 0, good, good[:, :2].contiguous(), h, i, i, i, 0)
    with pytest.raises(ValueError):  # h holds fewer than 9 x 768 values
        op.attn_qkv(addr, 0, good, good, torch.zeros(8, 768), i, i, i, 0)
    with pytest.raises(ValueError):  # h in the wrong dtype
        op.attn_qkv(addr, 0, good, good, h.to(torch.bfloat16), i, i, i, 0)
    with pytest.raises(ValueError):  # layer past the model
        op.attn_qkv(addr, 2, good, good, h, i, i, i, 0)
    with pytest.raises(ValueError):  # qkv of the wrong width
        op.attn_prologue(addr, 0, good, good, torch.zeros(9, 1024), h, i, i, i)
    with pytest.raises(ValueError):  # hist of the wrong width
        op.forward(addr, good, good, torch.zeros(3, 64, 512), i, torch.zeros(4, dtype=torch.int32),
                   torch.zeros(3, dtype=torch.int32), 3, 0, torch.zeros(1), torch.zeros(1, dtype=torch.uint8))
    # speculative state: one buffer short of its size for batch 3, k 4, vocab 256
    from flaxchat_amd.torch_ops import SPEC_BUFFERS, _spec_bytes
    need = _spec_bytes(3, 4, 100, 256)
    bufs = [torch.zeros(max(need[n], 1), dtype=torch.uint8) for n in SPEC_BUFFERS]
    hist = torch.zeros(3, 64, 768)
    for short in ("gen", "p_logits", "q_stats", "part"):
        b = list(bufs)
        b[SPEC_BUFFERS.index(short)] = torch.zeros(max(need[short] - 4, 1), dtype=torch.uint8)
        with pytest.raises(ValueError, match=short):
            op.spec_round(addr, addr, good, good, hist, good, good, hist, b, 3, 4, 100, 100, 256, 1.0, 0, 1,
                          torch.zeros(1, dtype=torch.uint8))
    with pytest.raises(ValueError, match="vocab"):
        op.spec_round(addr, addr, good, good, hist, good, good, hist, bufs, 3, 4, 100, 100, 512, 1.0, 0, 1,
                      torch.zeros(1, dtype=torch.uint8))
