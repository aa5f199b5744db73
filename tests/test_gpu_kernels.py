"""Kernel-level parity through the C-ABI against float64 / oracle references.

Tolerances: fp32 kernels 1e-4 relative to the float64 result; bf16 kernels
are compared with float64 math on the same bf16-rounded inputs, with the
tolerance each case states (the kernels accumulate in fp32; bf16 output
rounding is 2^-9 relative).
"""

import ctypes
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from flaxchat_amd import _lib  # noqa: E402
from flaxchat_amd._lib import check, lib, FcRowstat  # noqa: E402

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def dev():
    return torch.device("cuda", 0)


def stream():
    return torch.cuda.current_stream().cuda_stream


def bf(x):
    """round a float32 numpy array to bf16 and back (torch RNE)."""
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16).float().numpy()


# ---------------------------------------------------------------- GEMM
@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("M", [1, 3, 5, 16, 32, 64, 100, 224, 300])
@pytest.mark.parametrize("epi", [0, 1, 2, 4])
@pytest.mark.parametrize("NK", [(256, 384), (1536, 6144)])
def test_gemm_parity(dtype, M, epi, NK):
    """Small and model-sized shapes through every kernel family (VALU GEMV,
    streaming MFMA, LDS-tiled MFMA with 64-row and full-M tiles)."""
    _say(f"gemm dtype={dtype} M={M} epi={epi} NK={NK}")
    rng = np.random.default_rng(M * 10 + epi)
    N, K = NK
    if N * K > 1e6 and (epi in (1, 4) or (dtype == "fp32" and M > 64)):
        pytest.skip("covered by the small shape; keeps the run short")
    A = rng.standard_normal((M, K)).astype(np.float32)
    W = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    if dtype == "bf16":
        A, W = bf(A), bf(W)
        tdt, code = torch.bfloat16, _lib.FC_BF16
    else:
        tdt, code = torch.float32, _lib.FC_F32
    ref = A.astype(np.float64) @ W.astype(np.float64).T
    base = rng.standard_normal((M, N)).astype(np.float32)
    At = torch.from_numpy(A).to(dev(), tdt)
    Wt = torch.from_numpy(W).to(dev(), tdt)
    if epi == 2:
        out = torch.zeros(M, N, device=dev(), dtype=tdt)
        ref = np.maximum(ref, 0) ** 2
    elif epi == 1:
        out = torch.from_numpy(base).to(dev())
        ref = ref + base
    else:
        out = torch.zeros(M, N, device=dev(), dtype=torch.float32)
        if epi == 4:
            ref = 15 * np.tanh(ref / 15)
    check(lib().fc_gemm(At.data_ptr(), Wt.data_ptr(), out.data_ptr(), M, N, K, code, epi, stream()), "gemm")
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    tol = 1e-4 if dtype == "fp32" else (1e-2 if epi == 2 else 2e-4)
    np.testing.assert_allclose(got, ref, rtol=tol, atol=tol * max(1.0, np.abs(ref).max()))


# ---------------------------------------------------------------- attention
def _attn_ref(q, K, V, start, nvalid, W, H, G, window):
    """float64 brute force: q [B][W][H][d], K/V [B][G][cap][d] (natural layout)."""
    B, _, _, d = q.shape
    rep = H // G
    y = np.zeros((B, W, H, d))
    for b in range(B):
        off = W - nvalid[b]
        for j in range(off, W):
            p = start[b] + j - off
            lo = max(0, p - window) if window > 0 else 0
            for h in range(H):
                g = h // rep
                s = K[b, g, lo:p + 1] @ q[b, j, h] / np.sqrt(d)
                s = np.exp(s - s.max())
                s /= s.sum()
                y[b, j, h] = s @ V[b, g, lo:p + 1]
    return y


def _to_vblocked(V):
    B, G, cap, d = V.shape
    return np.ascontiguousarray(V.reshape(B, G, cap // 32, 32, d).transpose(0, 1, 2, 4, 3))


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("B,W,H,G,window,lmax", [
    (4, 5, 6, 6, 0, 700),       # verify chunk, full layer
    (4, 5, 6, 6, 256, 700),     # sliding window
    (3, 9, 12, 4, 300, 900),    # GQA 3:1
    (5, 1, 6, 6, 0, 1500),      # draft step
    (2, 40, 2, 2, 64, 300),     # prefill-like chunk, many query blocks
    (3, 3, 4, 2, 0, 70),        # ragged, short rows
])
def test_attention_parity(dtype, B, W, H, G, window, lmax):
    _say(f"attention dtype={dtype} B={B} W={W} H={H} G={G} window={window} lmax={lmax}")
    rng = np.random.default_rng(B * 1000 + W * 7 + H + window)
    d = 128
    cap = ((lmax + W + 31) // 32) * 32 + 32
    L = rng.integers(max(1, W), lmax, size=B)
    nvalid = np.minimum(rng.integers(1, W + 1, size=B), L).astype(np.int32)
    nvalid[0] = W if W <= L[0] else nvalid[0]
    start = (L - nvalid).astype(np.int32)
    q = rng.standard_normal((B, W, H, d)).astype(np.float32)
    K = rng.standard_normal((B, G, cap, d)).astype(np.float32)
    V = rng.standard_normal((B, G, cap, d)).astype(np.float32)
    if dtype == "bf16":
        q, K, V = bf(q), bf(K), bf(V)
        tdt, code = torch.bfloat16, _lib.FC_BF16
    else:
        tdt, code = torch.float32, _lib.FC_F32
    ref = _attn_ref(q.astype(np.float64), K.astype(np.float64), V.astype(np.float64), start, nvalid, W, H, G, window)
    qt = torch.from_numpy(q).to(dev(), tdt)
    Kt = torch.from_numpy(K).to(dev(), tdt)
    Vt = torch.from_numpy(_to_vblocked(V)).to(dev(), tdt)
    y = torch.full((B, W, H, d), 7.0, device=dev(), dtype=tdt)
    st = torch.from_numpy(start).to(dev())
    nv = torch.from_numpy(nvalid).to(dev())
    max_keys = min(cap, window + W) if window > 0 else cap
    nb = lib().fc_attention_workspace_bytes(B, W, H, G, d, max_keys)
    ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=dev())
    check(lib().fc_attention(qt.data_ptr(), Kt.data_ptr(), Vt.data_ptr(), y.data_ptr(), B, W, H, G, d, cap,
                             st.data_ptr(), nv.data_ptr(), window, max_keys, code, ws.data_ptr(), ws.numel(),
                             stream()), "attention")
    torch.cuda.synchronize()
    got = y.float().cpu().numpy()
    for b in range(B):
        got_inv = got[b, :W - nvalid[b]]
        assert np.all(got_inv == 0), "invalid slots must be zero"
    tol = 1e-5 if dtype == "fp32" else 2e-2
    np.testing.assert_allclose(got, ref, rtol=tol, atol=tol)


# ---------------------------------------------------------------- row stats / top-k
@pytest.mark.parametrize("V,top_k,T", [(8192, 40, 1.0), (65536, 40, 0.8), (1000, 1, 1.0), (4096, 0, 0.7),
                                       (300, 299, 1.3), (64, 5, 1.0)])
def test_row_stats(V, top_k, T):
    _say(f"row_stats V={V} top_k={top_k} T={T}")
    from oracle.sampling import topk_keep
    rng = np.random.default_rng(V + top_k)
    rows = 6
    z = (rng.standard_normal((rows, V)) * 2).astype(np.float32)
    z = (15 * np.tanh(z / 15)).astype(np.float32)
    # ties at and around the cut, lower index must win
    z[1, :] = np.round(z[1, :] * 2) / 2
    z[2, 10:20] = 5.0
    z[3, :] = 0.0
    zt = torch.from_numpy(z).to(dev())
    stats = torch.zeros(rows * ctypes.sizeof(FcRowstat), dtype=torch.uint8, device=dev())
    check(lib().fc_row_stats(zt.data_ptr(), rows, V, T, top_k, stats.data_ptr(), stream()), "row_stats")
    torch.cuda.synchronize()
    raw = stats.cpu().numpy().tobytes()
    for r in range(rows):
        rs = FcRowstat.from_buffer_copy(raw[r * 32:(r + 1) * 32])
        assert rs.argmax == int(np.argmax(z[r]))
        keep = topk_keep(z[r], top_k)
        tau = np.float32(rs.tau)
        got_keep = (z[r] > tau) | ((z[r] == tau) & (np.arange(V) <= rs.tie_idx))
        assert np.array_equal(got_keep, keep), f"row {r}: keep-set differs"
        x = (z[r][keep] / np.float32(T)).astype(np.float32)
        assert np.float32(rs.mx) == x.max()
        np.testing.assert_allclose(rs.sum, np.exp(x.astype(np.float64) - x.max()).sum(), rtol=1e-5)
