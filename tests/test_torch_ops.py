"""torch.ops.flaxchat_mi355x without a GPU: the operators are registered,
their fake implementations propagate shapes on meta tensors, and the
fragment-order view used for bf16 outputs inverts the documented layout."""

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import flaxchat_amd.torch_ops as ops  # noqa: E402
from flaxchat_amd.runtime import frag_pack  # noqa: E402


def test_registered():
    for name in ("pack_operand", "linear", "attention", "cross_entropy"):
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
