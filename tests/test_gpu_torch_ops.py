"""torch.ops.flaxchat_mi355x on the GPU against float64 references (the same
references and tolerances as the C-ABI kernel tests: fp32 1e-4, bf16 2e-4
for fp32 GEMM outputs and 2e-2 for bf16 attention outputs)."""

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import flaxchat_amd.torch_ops  # noqa: E402,F401
from flaxchat_amd.runtime import frag_pack  # noqa: E402
from tests.test_gpu_kernels import _attn_ref, _to_kblocked, _to_vblocked, _say, bf  # noqa: E402

pytestmark = pytest.mark.gpu
OPS = torch.ops.flaxchat_mi355x


def dev():
    return torch.device("cuda", 0)


def test_pack_operand():
    _say("torch op pack_operand")
    a = bf(np.random.default_rng(0).standard_normal((40, 128)).astype(np.float32))
    got = OPS.pack_operand(torch.from_numpy(a).to(dev(), torch.bfloat16))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.float().cpu().numpy(), frag_pack(a))


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("M,N,K,softcap", [(5, 96, 128, False), (37, 256, 192, True), (300, 512, 256, False)])
def test_linear(dtype, M, N, K, softcap):
    _say(f"torch op linear {dtype} M={M} N={N} K={K} softcap={softcap}")
    rng = np.random.default_rng(M + N)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    tdt = torch.float32
    if dtype == "bf16":
        x, w, tdt = bf(x), bf(w), torch.bfloat16
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    if softcap:
        ref = 15 * np.tanh(ref / 15)
    got = OPS.linear(torch.from_numpy(x).to(dev(), tdt), torch.from_numpy(w).to(dev(), tdt), softcap)
    torch.cuda.synchronize()
    tol = 1e-4 if dtype == "fp32" else 2e-4
    np.testing.assert_allclose(got.cpu().numpy(), ref, rtol=tol, atol=tol * max(1.0, np.abs(ref).max()))


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("B,W,H,G,window,lmax", [(4, 5, 6, 6, 0, 700), (3, 9, 12, 4, 300, 900)])
def test_attention(dtype, B, W, H, G, window, lmax):
    _say(f"torch op attention {dtype} B={B} W={W} H={H} G={G} window={window}")
    rng = np.random.default_rng(B + W + H)
    d = 128
    cap = ((lmax + W + 31) // 32) * 32 + 32
    L = rng.integers(W, lmax, size=B)
    nvalid = np.minimum(rng.integers(1, W + 1, size=B), L).astype(np.int32)
    start = (L - nvalid).astype(np.int32)
    q = rng.standard_normal((B, W, H, d)).astype(np.float32)
    K = rng.standard_normal((B, G, cap, d)).astype(np.float32)
    V = rng.standard_normal((B, G, cap, d)).astype(np.float32)
    tdt = torch.float32
    if dtype == "bf16":
        q, K, V, tdt = bf(q), bf(K), bf(V), torch.bfloat16
    ref = _attn_ref(q.astype(np.float64), K.astype(np.float64), V.astype(np.float64), start, nvalid, W, H, G, window)
    off = np.zeros(B + 1, np.int32)
    off[1:] = np.cumsum(nvalid)
    qp = np.concatenate([q[b, W - nvalid[b]:] for b in range(B)])
    refp = np.concatenate([ref[b, W - nvalid[b]:] for b in range(B)]).reshape(int(off[-1]), H * d)
    kc = torch.from_numpy(_to_kblocked(K) if dtype == "bf16" else K).to(dev(), tdt)
    vc = torch.from_numpy(_to_vblocked(V)).to(dev(), tdt)
    got = OPS.attention(torch.from_numpy(qp).to(dev(), tdt), kc, vc, torch.from_numpy(off).to(dev()),
                        torch.from_numpy(start).to(dev()), W, window)
    torch.cuda.synchronize()
    tol = 1e-5 if dtype == "fp32" else 2e-2
    np.testing.assert_allclose(got.float().cpu().numpy(), refp, rtol=tol, atol=tol)


def test_cross_entropy():
    _say("torch op cross_entropy")
    rng = np.random.default_rng(5)
    z = (rng.standard_normal((33, 5000)) * 3).astype(np.float32)
    t = rng.integers(0, 5000, 33)
    t[[3, 17]] = -1
    got = OPS.cross_entropy(torch.from_numpy(z).to(dev()), torch.from_numpy(t).to(dev()))
    torch.cuda.synchronize()
    zz = z.astype(np.float64)
    mx = zz.max(axis=1)
    ref = mx + np.log(np.exp(zz - mx[:, None]).sum(axis=1)) - zz[np.arange(33), np.maximum(t, 0)]
    ref[t < 0] = 0.0
    np.testing.assert_allclose(got.cpu().numpy(), ref, rtol=1e-5, atol=1e-5)
    with pytest.raises(ValueError):
        OPS.cross_entropy(torch.from_numpy(z).to(dev()), torch.full((33,), 5000, device=dev()))
