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


def test_engine_op_fakes():
    """Shape propagation of the engine operators on meta tensors (the model
    descriptor is host memory; nothing is launched)."""
    import ctypes
    from flaxchat_amd import _lib
    m = _lib.FcModel()
    m.n_head, m.head_dim, m.dtype = 6, 128, _lib.FC_BF16
    addr = ctypes.addressof(m)
    meta = dict(device="meta")
    kc = torch.empty(2, 3, 2, 64, 128, dtype=torch.bfloat16, **meta)
    i = torch.empty(9, dtype=torch.int32, **meta)
    h = torch.empty(16, 768, dtype=torch.bfloat16, **meta)
    q = torch.ops.flaxchat_mi355x.attn_qkv(addr, 0, kc, kc, h, i, i, i, 0)
    assert q.shape == (9, 6, 128) and q.dtype == torch.bfloat16
    qkv = torch.empty(9, 1280, **meta)
    assert torch.ops.flaxchat_mi355x.attn_prologue(addr, 1, kc, kc, qkv, h, i, i, i).shape == (9, 6, 128)
    mx, s, tau, tie, am = torch.ops.flaxchat_mi355x.row_stats(torch.empty(5, 100, **meta), 1.0, 0)
    assert mx.shape == (5,) and am.dtype == torch.int32
