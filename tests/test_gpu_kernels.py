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
def _gemm_cases():
    """Small shapes for every (dtype, M, epilogue); model-sized shapes for the
    kernel paths they add (split tiles, 6144-deep K) without repeating the
    epilogue checks."""
    cases = []
    for NK in [(256, 384), (1536, 6144)]:
        for M in [1, 3, 5, 16, 32, 40, 64, 100, 224, 300]:
            for epi in [0, 1, 2, 4]:
                for dtype in ["fp32", "bf16"]:
                    big = NK[0] * NK[1] > 1e6
                    if big and (epi in (1, 4) or (dtype == "fp32" and M > 64)):
                        continue
                    cases.append((dtype, M, epi, NK))
    # draft-size rows with a vocabulary-wide output (the LDS-shared 32 x 64 tiles of the draft lm_head)
    for M in [20, 32]:
        for epi in [0, 4]:
            cases.append(("bf16", M, epi, (16384, 256)))
    # row counts >= 1024 with few output tiles (the 64-row kernels)
    for NK in [(512, 256), (768, 1536)]:
        for M in [1024, 1100, 2304]:
            for epi in [0, 1, 2, 4]:
                if NK[1] > 256 and M != 1100:
                    continue
                cases.append(("bf16", M, epi, NK))
    # prefill-size GEMMs with >= 224 tiles (the 256 x 256 / 256 x 192 tile kernel)
    for M, NK, epis in [(3000, (4608, 256), [0, 1, 2]), (4100, (4096, 128), [0, 2, 4])]:
        for epi in epis:
            cases.append(("bf16", M, epi, NK))
    return cases


@pytest.mark.parametrize("dtype,M,epi,NK", _gemm_cases())
def test_gemm_parity(dtype, M, epi, NK):
    """Every kernel family (VALU GEMV in fp32; matrix-core tiles of 16, 32 and
    64 rows on fragment-order operands in bf16) against float64."""
    from flaxchat_amd.runtime import frag_pack, frag_unpack
    _say(f"gemm dtype={dtype} M={M} epi={epi} NK={NK}")
    rng = np.random.default_rng(M * 10 + epi)
    N, K = NK
    A = rng.standard_normal((M, K)).astype(np.float32)
    W = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    if dtype == "bf16":
        A, W = bf(A), bf(W)
        tdt, code = torch.bfloat16, _lib.FC_BF16
        A_dev, W_dev = frag_pack(A), frag_pack(W)
    else:
        tdt, code = torch.float32, _lib.FC_F32
        A_dev, W_dev = A, W
    ref = A.astype(np.float64) @ W.astype(np.float64).T
    base = rng.standard_normal((M, N)).astype(np.float32)
    At = torch.from_numpy(A_dev).to(dev(), tdt)
    Wt = torch.from_numpy(W_dev).to(dev(), tdt)
    if epi == 2:
        out = torch.zeros((M + 15) // 16 * 16 if dtype == "bf16" else M, N, device=dev(), dtype=tdt)
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
    if epi == 2 and dtype == "bf16":
        got = frag_unpack(got, M)
    tol = 1e-4 if dtype == "fp32" else (1e-2 if epi == 2 else 2e-4)
    np.testing.assert_allclose(got, ref, rtol=tol, atol=tol * max(1.0, np.abs(ref).max()))


@pytest.mark.parametrize("M", [3, 32, 224, 1100, 4100])
def test_gemm_softcap_range(M):
    """The bf16 kernels' softcap (exponential / reciprocal form, series below
    |x| = 1/16) against 15 tanh(z / 15) in float64 over pre-cap values from
    2^-14 to 2^13 of both signs: z = A[m, 0] W[n, 0] is exact in fp32
    (bf16 x bf16), so the error is the softcap's alone. Row counts route to
    the K-split, LDS-shared, 64-row and 256 x 256 tile kernels."""
    from flaxchat_amd.runtime import frag_pack
    _say(f"gemm softcap range M={M}")
    N, K = 4096, 128
    e = np.arange(M) % 24 - 12                      # 2^-12 .. 2^11
    s = np.where(np.arange(M) % 2 == 0, 1.0, -1.0) * np.exp2(e)
    c = ((np.arange(N) % 64) - 32) / 4.0            # -8 .. 7.75 in steps of 1/4
    A = np.zeros((M, K), np.float32)
    A[:, 0] = s
    W = np.zeros((N, K), np.float32)
    W[:, 0] = c
    z = s[:, None] * c[None, :]
    ref = 15 * np.tanh(z / 15)
    At = torch.from_numpy(frag_pack(A)).to(dev(), torch.bfloat16)
    Wt = torch.from_numpy(frag_pack(W)).to(dev(), torch.bfloat16)
    out = torch.zeros(M, N, device=dev(), dtype=torch.float32)
    check(lib().fc_gemm(At.data_ptr(), Wt.data_ptr(), out.data_ptr(), M, N, K, _lib.FC_BF16, 4, stream()), "gemm")
    torch.cuda.synchronize()
    got = out.cpu().numpy().astype(np.float64)
    err = np.abs(got - ref)
    _say(f"  max abs error {err.max():.2e}; max relative error where |z| < 1: "
         f"{(err / np.maximum(np.abs(ref), 1e-30))[np.abs(z) < 1].max():.2e}")
    assert err.max() <= 1e-5
    small = (np.abs(z) < 1) & (z != 0)
    assert (err[small] / np.abs(ref[small])).max() <= 1e-5
    assert np.all(got[z == 0] == 0)


def test_pack_operand_matches_host_layout():
    """fc_pack_operand reproduces the documented fragment order (host
    restatement frag_pack), including the zero padding rows."""
    from flaxchat_amd.runtime import frag_pack
    rng = np.random.default_rng(7)
    a = bf(rng.standard_normal((40, 96)).astype(np.float32))
    src = torch.from_numpy(a).to(dev(), torch.bfloat16)
    dst = torch.full((48, 96), 3.0, device=dev(), dtype=torch.bfloat16)
    check(lib().fc_pack_operand(src.data_ptr(), dst.data_ptr(), 40, 96, stream()), "pack")
    torch.cuda.synchronize()
    assert np.array_equal(dst.float().cpu().numpy(), frag_pack(a))


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


def _to_kblocked(K):
    """K cache of the matrix-core attention (include/flaxchat_amd.h): in each
    32-position block, element (kk, d) at ((2*(d//32) + (kk//4)%2)*64 +
    4*(kk//8) + kk%4 + 16*((d//8)%4))*8 + d%8."""
    B, G, cap, d = K.shape
    assert d == 128
    out = np.zeros((B, G, cap // 32, 4096), K.dtype)
    kk = np.arange(32)[:, None]
    dd = np.arange(128)[None, :]
    idx = ((2 * (dd // 32) + (kk // 4) % 2) * 64 + 4 * (kk // 8) + kk % 4 + 16 * ((dd // 8) % 4)) * 8 + dd % 8
    blocks = K.reshape(B, G, cap // 32, 32, 128)
    out[..., idx.reshape(-1)] = blocks.reshape(B, G, cap // 32, 32 * 128)
    return out.reshape(B, G, cap, d)


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("B,W,H,G,window,lmax", [
    (4, 5, 6, 6, 0, 700),       # verify chunk, full layer
    (4, 5, 6, 6, 256, 700),     # sliding window
    (3, 9, 12, 4, 300, 900),    # GQA 3:1
    (5, 1, 6, 6, 0, 1500),      # draft step
    (2, 40, 2, 2, 64, 300),     # prefill-like chunk, many query blocks
    (3, 3, 4, 2, 0, 70),        # ragged, short rows
    (32, 2, 8, 8, 0, 300),      # >= 256 row x group units: one key split, output written directly
    (32, 3, 16, 8, 100, 300),   # the same with GQA 2:1 and a window
    (1, 12, 12, 4, 0, 1500),    # GQA 3:1, 36 columns: two query blocks per workgroup with key splits
    (2, 160, 2, 2, 0, 600),     # prefill-width chunk (>= 128 columns per row): per-wave query blocks
    (3, 130, 12, 4, 300, 900),  # the same, GQA 3:1 (390 columns) and a window
    (2, 256, 4, 4, 64, 700),    # short window: blocks skip the tiles they cannot see
    (4, 200, 6, 2, 0, 500),     # ragged rows, GQA 3:1
    (64, 5, 6, 6, 1024, 2048),  # the config-3 microbenchmark shape: 64 rows x 5 queries, sliding-window layer
    (64, 5, 6, 6, 0, 2048),     # the same, full layer
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
    # packed layout: row b's nvalid[b] queries (its last slots) at row_off[b]..
    off = np.zeros(B + 1, np.int32)
    off[1:] = np.cumsum(nvalid)
    tot = int(off[-1])
    qp = np.concatenate([q[b, W - nvalid[b]:] for b in range(B)])
    refp = np.concatenate([ref[b, W - nvalid[b]:] for b in range(B)])
    qt = torch.from_numpy(qp).to(dev(), tdt)
    Kt = torch.from_numpy(_to_kblocked(K) if dtype == "bf16" else K).to(dev(), tdt)
    Vt = torch.from_numpy(_to_vblocked(V)).to(dev(), tdt)
    # bf16 output is the c_proj GEMM operand: fragment order, whole 16-row blocks
    rows = (tot + 3 + 15) // 16 * 16 if dtype == "bf16" else tot + 3
    y = torch.full((rows, H * d), 7.0, device=dev(), dtype=tdt)
    st = torch.from_numpy(start).to(dev())
    ro = torch.from_numpy(off).to(dev())
    max_keys = min(cap, window + W) if window > 0 else cap
    nb = lib().fc_attention_workspace_bytes(B, W, H, G, d, max_keys)
    ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=dev())
    check(lib().fc_attention(qt.data_ptr(), Kt.data_ptr(), Vt.data_ptr(), y.data_ptr(), B, tot, W, H, G, d, cap,
                             ro.data_ptr(), st.data_ptr(), window, max_keys, code, ws.data_ptr(), ws.numel(),
                             stream()), "attention")
    torch.cuda.synchronize()
    got = y.float().cpu().numpy()
    if dtype == "bf16":
        from flaxchat_amd.runtime import frag_unpack
        got = frag_unpack(got, rows)
    got = got.reshape(rows, H, d)
    assert np.all(got[tot:] == 7.0), "rows past the chunk total must be untouched"
    tol = 1e-5 if dtype == "fp32" else 2e-2
    np.testing.assert_allclose(got[:tot], refp, rtol=tol, atol=tol)


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


# ---------------------------------------------------------------- accept at full vocabulary
def _run_accept(P, Q, drafts, rnd, T, top_k, seed):
    """fc_spec_accept on host-made logits / drafts (the state of a round
    whose rows each fed one pending token at position 10); the draft's row
    statistics from fc_row_stats with the round's top-k. Returns the
    device's result rows and the final round counters."""
    B, k1, V = P.shape
    k = k1 - 1
    i32 = dict(dtype=torch.int32, device=dev())
    z = lambda *s: torch.zeros(*s, **i32)  # noqa: E731
    gen_cap, P_MAX = 64, _lib.PMAX
    bufs = dict(t_len=torch.full((B,), 10, **i32), d_len=torch.full((B,), 10, **i32), t_pend=z(B, P_MAX),
                d_pend=z(B, P_MAX), t_pend_n=torch.ones(B, **i32), d_pend_n=torch.ones(B, **i32),
                t_dirty=torch.full((B,), 1 << 30, **i32), d_dirty=torch.full((B,), 1 << 30, **i32),
                gen=z(B, gen_cap), gen_n=torch.full((B,), 11, **i32), prompt_len=torch.full((B,), 11, **i32),
                round=torch.from_numpy(rnd).to(dev()), stall=z(B), result=z(B, _lib.RES_STRIDE),
                tok_d0=z(B * P_MAX), off_d0=z(B + 1), start_d=z(k, B), tok_ds=z(k, B), off_ds=z(B + 1),
                tok_v=z(B * (P_MAX + k)), off_v=z(B + 1), start_v=z(B), drafts=torch.from_numpy(drafts).to(dev()),
                q_logits=torch.from_numpy(Q).to(dev()), p_logits=torch.from_numpy(P).to(dev()),
                q_stats=torch.zeros(B * k * ctypes.sizeof(FcRowstat), dtype=torch.uint8, device=dev()),
                p_stats=torch.zeros(B * (k + 1) * ctypes.sizeof(FcRowstat), dtype=torch.uint8, device=dev()),
                part=torch.zeros(lib().fc_spec_part_bytes(B, k, V), dtype=torch.uint8, device=dev()))
    st = _lib.FcSpecState(B, k, 40, gen_cap, V, T, top_k or 0, seed, *[bufs[n].data_ptr() for n in _lib._SPEC_PTRS],
                          bufs["part"].data_ptr(), bufs["part"].numel())
    check(lib().fc_row_stats(bufs["q_logits"].data_ptr(), B * k, V, T, top_k or 0, bufs["q_stats"].data_ptr(),
                             stream()), "row stats")
    check(lib().fc_spec_accept(ctypes.byref(st), stream()), "spec accept")
    torch.cuda.synchronize()
    return bufs["result"].cpu().numpy(), bufs["round"].cpu().numpy()


def _check_accept(P, Q, drafts, rnd, T, top_k, seed):
    from oracle import sampling as S
    res, rnd_after = _run_accept(P, Q, drafts, rnd, T, top_k, seed)
    assert np.array_equal(rnd_after, rnd + 1)
    recs = []
    for b in range(P.shape[0]):
        em, acc, rej, bonus = S.accept_round(P[b], Q[b], drafts[b], T, top_k, seed, b, int(rnd[b]))
        n = int(res[b, 0])
        assert res[b, 8:8 + n].tolist() == em, f"row {b}: {res[b, 8:8 + n].tolist()} vs oracle {em}"
        assert (int(res[b, 1]), int(res[b, 2])) == (acc, rej), f"row {b}"
        recs.append((em, acc, rej, bonus))
    return recs


def _cfg3_logits(B, k, V, seed_np=11):
    rng = np.random.default_rng(seed_np)
    P = (15 * np.tanh(rng.standard_normal((B, k + 1, V)) * 2 / 15)).astype(np.float32)
    Q = (15 * np.tanh((P[:, :k] + rng.standard_normal((B, k, V)) * 0.5) / 15)).astype(np.float32)
    return P, Q


@pytest.mark.parametrize("T,top_k", [(1.0, None), (0.0, None), (0.8, 40), (0.0, 40)])
def test_spec_accept_cfg3_vs_oracle(T, top_k):
    """fc_spec_accept on the config-3 sampling shape (64 rows, k = 4, V =
    65536) against the oracle's accept_round (flaxchat/engine.py:525-592) on
    the same logits, drafts and Philox counters. Without top-k the
    vocab-wide passes run in 64 chunks per row and merge their partials;
    with top_k 40 (generate_speculative's default, engine.py:411, 461-466)
    each 1024-entry chunk keeps its exact top-k candidates (k_topk_cand),
    one workgroup per row selects the keep set among them (k_topk_stats),
    and the accept decision and its draws run split over the vocabulary as
    without top-k (k_accept_decide_st, k_draw_part). Target logits
    are 15 tanh(N(0, 2^2) / 15), the draft's the target's plus N(0, 0.5^2)
    noise (softcapped again); drafts are the oracle's own draws from the
    draft logits. The emitted tokens must match exactly."""
    from oracle import sampling as S
    _say(f"spec accept cfg3 T={T} top_k={top_k}")
    B, k, V, seed = 64, 4, 65536, 1234
    P, Q = _cfg3_logits(B, k, V)
    rnd = (np.arange(B) % 5).astype(np.int32)
    drafts = np.array([[S.draft_sample(Q[b, i], T, top_k, seed, b, int(rnd[b]), i) for i in range(k)]
                       for b in range(B)], np.int32)
    recs = _check_accept(P, Q, drafts, rnd, T, top_k, seed)
    n_acc = sum(r[1] for r in recs)
    n_bonus = sum(int(r[3]) for r in recs)
    _say(f"accepted {n_acc} of {B * k}, bonus rows {n_bonus}")
    assert 0 < n_bonus < B  # both the bonus and the rejection paths ran


@pytest.mark.parametrize("T", [1.0, 0.8])
def test_spec_accept_draft_outside_topk(T):
    """The q == 0 branch (flaxchat/engine.py:548-552): a draft token outside
    the draft's top-k has draft probability exactly 0, so the target samples
    from p at once. Rows put such a draft at index 1 (a mid-round
    rejection, then re-prefill) or at the last index k - 1 (accepted ==
    k', so a bonus follows: the quirk of engine.py:573); top_k 4 at V =
    65536. Bit-exact against the oracle."""
    _say(f"accept q == 0 branch T={T}")
    B, k, V, seed, top_k = 16, 4, 65536, 77, 4
    P, Q = _cfg3_logits(B, k, V, seed_np=12)
    from oracle import sampling as S
    rnd = np.zeros(B, np.int32)
    drafts = np.array([[S.draft_sample(Q[b, i], T, top_k, seed, b, 0, i) for i in range(k)] for b in range(B)],
                      np.int32)
    # make the target agree with the draft before the planted index, so the
    # rows reach it: copy the draft logits into the target rows
    for b in range(B):
        at = 1 if b % 2 == 0 else k - 1
        P[b, :at] = Q[b, :at]
        outside = np.argsort(-Q[b, at], kind="stable")[top_k + 3 + b]
        drafts[b, at] = outside
    recs = _check_accept(P, Q, drafts, rnd, T, top_k, seed)
    hit_mid = sum(1 for b, r in enumerate(recs) if b % 2 == 0 and r[2] == 1 and not r[3])
    hit_last = sum(1 for b, r in enumerate(recs) if b % 2 == 1 and r[2] == k - 1 and r[3])
    _say(f"q == 0 at index 1: {hit_mid} of {B // 2} rows; at the last index (+ bonus): {hit_last} of {B // 2}")
    assert hit_mid == B // 2 and hit_last == B // 2


def test_spec_accept_topk_ties_v65536():
    """top_k 40 at V = 65536 with ties across the cut: logits rounded to a
    coarse grid so the 40th largest value repeats; the kept set is exactly
    40 entries, lower index first among equals (lax.top_k,
    flaxchat/engine.py:461-466). Sampled (T 0.8) and greedy."""
    from oracle import sampling as S
    B, k, V, seed, top_k = 32, 4, 65536, 5, 40
    P, Q = _cfg3_logits(B, k, V, seed_np=13)
    P = (np.round(P * 2) / 2).astype(np.float32)
    Q = (np.round(Q * 2) / 2).astype(np.float32)
    for b in range(B):  # at least one tie straddling the cut in every row
        v = np.sort(P[b, 0])[::-1][top_k - 1]
        assert (P[b, 0] == v).sum() > 1
    rnd = (np.arange(B) % 3).astype(np.int32)
    for T in (0.8, 0.0):
        drafts = np.array([[S.draft_sample(Q[b, i], T, top_k, seed, b, int(rnd[b]), i) for i in range(k)]
                           for b in range(B)], np.int32)
        recs = _check_accept(P, Q, drafts, rnd, T, top_k, seed)
        _say(f"top-k ties T={T}: accepted {sum(r[1] for r in recs)} of {B * k}")


def _topk_path_rows(V, seed_np=17):
    """Target logits rows that drive each branch of the chunked top-k passes
    (k_topk_cand: the lanes' maxima bound a chunk's top-k from below and at
    most 128 entries at or above it are searched narrowly; k_topk_stats /
    k_topk_draft: the chunks' maxima bound the row's, at most 256 candidates
    searched narrowly; more take the search over every entry)."""
    rng = np.random.default_rng(seed_np)
    base = lambda: (15 * np.tanh(rng.standard_normal(V) * 2 / 15)).astype(np.float32)  # noqa: E731
    rows = []
    rows.append(base())                                    # smooth: narrow everywhere
    r = base() - 20.0                                      # chunk 3: 2 entries per lane at L = 5 -> exactly
    for lane in range(64):                                 # 128 at the bound (narrow); the row's top 40 tie at L
        r[3 * 1024 + 16 * lane: 3 * 1024 + 16 * lane + 2] = 5.0
    rows.append(r)
    r = rows[-1].copy()                                    # one more at L: 129 (chunk search over every entry)
    r[3 * 1024 + 2] = 5.0
    rows.append(r)
    r = base()                                             # chunk 5: 200 tied maxima (chunk fallback, row narrow)
    r[5 * 1024: 5 * 1024 + 200] = 16.0
    rows.append(r)
    rows.append(np.full(V, 0.25, np.float32))              # all equal: both passes search every entry
    rows.append((np.round(base() * 2) / 2).astype(np.float32))  # coarse grid: ties at many cuts
    return np.stack(rows)


@pytest.mark.parametrize("V", [65536, 65000])
def test_spec_accept_topk_search_paths(V):
    """The top-k accept path (k_topk_cand, k_topk_stats, k_accept) on rows
    crafted to take the narrow and the full threshold searches of both passes,
    with ties at the cut, against the oracle's accept_round (flaxchat/engine.py:
    461-466, 525-592); V = 65000 leaves a 488-entry last chunk with fewer lanes
    than top_k (no lower bound there). Sampled and greedy."""
    from oracle import sampling as S
    _say(f"top-k search paths V={V}")
    rows = _topk_path_rows(V)
    B, k, seed, top_k = rows.shape[0], 2, 9, 40
    rng = np.random.default_rng(3)
    P = np.stack([np.stack([rows[b]] * (k + 1)) for b in range(B)]).astype(np.float32)
    P[:, 1:] += (rng.standard_normal((B, k, V)) * 1e-3).astype(np.float32) * (np.arange(B) != 4)[:, None, None]
    Q = (15 * np.tanh((P[:, :k] + rng.standard_normal((B, k, V)) * 0.5) / 15)).astype(np.float32)
    rnd = (np.arange(B) % 3).astype(np.int32)
    for T in (0.8, 0.0):
        drafts = np.array([[S.draft_sample(Q[b, i], T, top_k, seed, b, int(rnd[b]), i) for i in range(k)]
                           for b in range(B)], np.int32)
        recs = _check_accept(P, Q, drafts, rnd, T, top_k, seed)
        _say(f"  T={T}: accepted {sum(r[1] for r in recs)} of {B * k}")


# ---------------------------------------------------------------- attention prologue
@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_attn_prologue_vs_oracle(dtype):
    """fc_attn_prologue against the oracle's per-token prologue
    (oracle/model.py Oracle.step: apply_rotary_emb, rms_norm * 1.2, the
    value-embedding gate 3 sigmoid(h[:12] . ve_gate)) on GQA heads (4 q, 2
    kv), for a layer without a value embedding (0) and one with (1); cache
    positions at both ends, and one at cap (q written, nothing appended).
    bf16: the inputs the device holds in bf16 (h, the VE table) are rounded
    first; tolerance 2e-2 (outputs rounded to bf16), fp32 1e-5."""
    from flaxchat_amd.config import GPTConfig
    from flaxchat_amd.gpt import GPT
    from flaxchat_amd.runtime import DeviceCache, DeviceModel
    from oracle.model import apply_rotary_emb, rms_norm, sigmoid
    _say(f"attention prologue {dtype}")
    H, G, d, D, V = 4, 2, 128, 512, 512
    cfg = GPTConfig(sequence_len=128, vocab_size=V, n_layer=2, n_head=H, n_kv_head=G, n_embd=D,
                    window_pattern="SL", short_window=64)
    host = GPT.init_normal(cfg, seed=3, std=0.1)
    dm = DeviceModel.from_host(host, dtype=dtype, device=dev())
    B, cap = 3, 96
    cache = DeviceCache(dm, B, cap)
    rows = np.array([0, 0, 1, 2, 2, 2, 1, 0], np.int32)
    pos = np.array([5, 6, 40, 0, 1, 95, 41, 96], np.int32)
    M = len(rows)
    rng = np.random.default_rng(7)
    tokens = rng.integers(0, V, M).astype(np.int32)
    qkv = rng.standard_normal((M, (H + 2 * G) * d)).astype(np.float32)
    hrow = rng.standard_normal((M, D)).astype(np.float32)
    tdt = torch.float32 if dtype == "fp32" else torch.bfloat16
    if dtype == "bf16":
        from flaxchat_amd.runtime import frag_pack
        hrow = bf(hrow)
        h_t = torch.from_numpy(frag_pack(hrow)).to(dev(), tdt)
    else:
        h_t = torch.from_numpy(hrow).to(dev())
    cos, sin = dm.t["rope_cos"].cpu().numpy(), dm.t["rope_sin"].cpu().numpy()
    i32 = lambda a: torch.from_numpy(a).to(dev())  # noqa: E731
    qkv_t, tok_t, row_t, pos_t = i32(qkv), i32(tokens), i32(rows), i32(pos)
    tol = 1e-5 if dtype == "fp32" else 2e-2
    for layer in range(2):
        q = torch.zeros(M, H, d, dtype=tdt, device=dev())
        check(lib().fc_attn_prologue(ctypes.byref(dm.desc), layer, ctypes.byref(cache.desc), qkv_t.data_ptr(),
                                     h_t.data_ptr(), tok_t.data_ptr(), row_t.data_ptr(), pos_t.data_ptr(), M,
                                     q.data_ptr(), stream()), "attn prologue")
        torch.cuda.synchronize()
        ve = host.value_embeds.get(str(layer))
        assert (ve is not None) == (layer == 1)
        q_ref = np.zeros((M, H, d), np.float32)
        k_nat = np.zeros((B, G, cap, d), np.float32)
        v_nat = np.zeros((B, G, cap, d), np.float32)
        for m in range(M):
            c, s_ = cos[pos[m]], sin[pos[m]]
            q_ref[m] = rms_norm(apply_rotary_emb(qkv[m, :H * d].reshape(H, d), c, s_)) * np.float32(1.2)
            k = rms_norm(apply_rotary_emb(qkv[m, H * d:(H + G) * d].reshape(G, d), c, s_)) * np.float32(1.2)
            v = qkv[m, (H + G) * d:].reshape(G, d).copy()
            if ve is not None:
                emb = ve.embedding[tokens[m]].reshape(G, d).astype(np.float32)
                if dtype == "bf16":
                    emb = bf(emb)
                gv = np.float32(3.0) * sigmoid(hrow[m, :12] @ host.blocks[layer].attn.ve_gate.kernel)
                v = (v + gv[:, None] * emb).astype(np.float32)
            if pos[m] < cap:
                k_nat[rows[m], :, pos[m]] = k
                v_nat[rows[m], :, pos[m]] = v
        np.testing.assert_allclose(q.float().cpu().numpy(), q_ref, rtol=tol, atol=tol)
        k_got = cache.k[layer].float().cpu().numpy()
        v_got = cache.v[layer].float().cpu().numpy()
        k_exp = _to_kblocked(k_nat) if dtype == "bf16" else k_nat
        np.testing.assert_allclose(k_got, k_exp, rtol=tol, atol=tol)
        np.testing.assert_allclose(v_got, _to_vblocked(v_nat), rtol=tol, atol=tol)


# ---------------------------------------------------------------- fused QKV epilogue
@pytest.mark.parametrize("dtype,M", [("fp32", 40), ("bf16", 40), ("bf16", 24)])
def test_attn_qkv_unfused_fallback(dtype, M):
    """fc_attn_qkv between the fused-epilogue row counts (bf16 with 24 or 40
    tokens: above the one-row decode sizes, below the verify sizes) and for
    fp32 models takes the unfused path: the QKV GEMM into
    the caller's workspace, then the prologue kernel. Its q, K and V must
    equal fc_gemm followed by fc_attn_prologue on the same inputs exactly
    (the same kernels with the same plan), GQA 12 / 4 with a value-embedding
    layer and one without, including a skipped token (row -1) and one at
    position cap."""
    from flaxchat_amd.config import GPTConfig
    from flaxchat_amd.gpt import GPT
    from flaxchat_amd.runtime import DeviceCache, DeviceModel
    from flaxchat_amd.torch_ops import pack_operand
    _say(f"unfused attn_qkv dtype={dtype} M={M}")
    D, V, d, H, G = 1536, 4096, 128, 12, 4
    cfg = GPTConfig(sequence_len=1024, vocab_size=V, n_layer=2, n_head=H, n_kv_head=G, n_embd=D,
                    window_pattern="SL", short_window=256)
    dm = DeviceModel.from_host(GPT.init_normal_parallel(cfg, seed=11, std=0.05), dtype=dtype, device=dev())
    B, cap = 3, 256
    rng = np.random.default_rng(M + (7 if dtype == "fp32" else 0))
    slots = rng.permutation(B * cap)[:M]
    rows, pos = (slots // cap).astype(np.int32), (slots % cap).astype(np.int32)
    rows[3] = -1
    pos[5] = cap
    i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev())  # noqa: E731
    tok_t, row_t, pos_t = i32(rng.integers(0, V, M)), i32(rows), i32(pos)
    hrows = torch.from_numpy(rng.standard_normal((M, D)).astype(np.float32)).to(dev())
    h = pack_operand(hrows.to(torch.bfloat16)) if dtype == "bf16" else hrows.contiguous()
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    code = _lib.FC_BF16 if dtype == "bf16" else _lib.FC_F32
    NQKV = (H + 2 * G) * d
    L = _lib.lib()
    for layer in range(2):
        ca, cb = DeviceCache(dm, B, cap), DeviceCache(dm, B, cap)
        qa = torch.zeros(M, H, d, dtype=tdt, device=dev())
        qb = torch.zeros_like(qa)
        need = L.fc_attn_qkv_workspace_bytes(ctypes.byref(dm.desc), M, M)
        assert need >= M * NQKV * 4, "this case should take the unfused path"
        ws = torch.zeros(need, dtype=torch.uint8, device=dev())
        check(L.fc_attn_qkv(ctypes.byref(dm.desc), layer, ctypes.byref(ca.desc), h.data_ptr(), tok_t.data_ptr(),
                            row_t.data_ptr(), pos_t.data_ptr(), M, M, qa.data_ptr(), ws.data_ptr(), ws.numel(),
                            stream()), "attn_qkv")
        qkv = torch.zeros(M, NQKV, dtype=torch.float32, device=dev())
        check(L.fc_gemm(h.data_ptr(), dm.t["layers"][layer]["wqkv"].data_ptr(), qkv.data_ptr(), M, NQKV, D, code, 0,
                        stream()), "gemm")
        check(L.fc_attn_prologue(ctypes.byref(dm.desc), layer, ctypes.byref(cb.desc), qkv.data_ptr(), h.data_ptr(),
                                 tok_t.data_ptr(), row_t.data_ptr(), pos_t.data_ptr(), M, qb.data_ptr(), stream()),
              "prologue")
        torch.cuda.synchronize()
        for name, a, b in (("q", qa, qb), ("k", ca.k[layer], cb.k[layer]), ("v", ca.v[layer], cb.v[layer])):
            assert b.float().abs().max().item() > 0, f"layer {layer} {name}: reference is all zero"
            assert torch.equal(a, b), f"layer {layer} {name}: differs from fc_gemm + fc_attn_prologue"
        assert qa[3].float().abs().sum().item() == 0, "the skipped token wrote q"


@pytest.mark.parametrize("H,G,M", [(12, 4, 6), (12, 12, 16), (12, 4, 130), (12, 12, 224), (12, 4, 1000),
                                   (12, 12, 3400)])
def test_attn_qkv_fused_vs_prologue(H, G, M):
    """fc_attn_qkv at one-row decode sizes (up to 16 tokens), verify and
    prefill row counts runs the attention prologue inside the QKV GEMM's
    epilogue (the 32 x 128 tile of the LDS-shared kernel; its 64 x 128
    tile, two 32-token passes, from 832 rows; at 3400 rows the 256 x 256
    tile's quadrants). Its q
    and the K / V it appends (RoPE, 1.2 * RMSNorm, the value-embedding gate
    on the V heads) must equal fc_gemm's fp32 projection of the same input
    followed by fc_attn_prologue, element by element within 1e-2 relative
    (the outputs are bf16), for a layer with a value embedding and one
    without. Includes a skipped token (row -1) and one at position cap
    (q written, nothing appended)."""
    from flaxchat_amd.config import GPTConfig
    from flaxchat_amd.gpt import GPT
    from flaxchat_amd.runtime import DeviceCache, DeviceModel
    from flaxchat_amd.torch_ops import pack_operand
    _say(f"fused QKV epilogue H={H} G={G} M={M}")
    D, V, d = 1536, 4096, 128
    cfg = GPTConfig(sequence_len=1024, vocab_size=V, n_layer=2, n_head=H, n_kv_head=G, n_embd=D,
                    window_pattern="SL", short_window=256)
    host = GPT.init_normal_parallel(cfg, seed=9, std=0.05)
    dm = DeviceModel.from_host(host, dtype="bf16", device=dev())
    B, cap = 4, 1024
    rng = np.random.default_rng(M)
    slots = rng.permutation(B * cap)[:M]
    rows, pos = (slots // cap).astype(np.int32), (slots % cap).astype(np.int32)
    rows[3] = -1
    pos[5] = cap
    i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev())  # noqa: E731
    tok_t, row_t, pos_t = i32(rng.integers(0, V, M)), i32(rows), i32(pos)
    hrows = torch.from_numpy(rng.standard_normal((M, D)).astype(np.float32)).to(dev(), torch.bfloat16)
    h = pack_operand(hrows)
    NQKV = (H + 2 * G) * d
    L = _lib.lib()
    for layer in range(2):
        ca, cb = DeviceCache(dm, B, cap), DeviceCache(dm, B, cap)
        qa = torch.zeros(M, H, d, dtype=torch.bfloat16, device=dev())
        qb = torch.zeros_like(qa)
        need = L.fc_attn_qkv_workspace_bytes(ctypes.byref(dm.desc), M, M)
        assert need == 0, "this row count should take the fused epilogue"
        check(L.fc_attn_qkv(ctypes.byref(dm.desc), layer, ctypes.byref(ca.desc), h.data_ptr(), tok_t.data_ptr(),
                            row_t.data_ptr(), pos_t.data_ptr(), M, M, qa.data_ptr(), None, 0, stream()), "attn_qkv")
        qkv = torch.zeros(M, NQKV, dtype=torch.float32, device=dev())
        check(L.fc_gemm(h.data_ptr(), dm.t["layers"][layer]["wqkv"].data_ptr(), qkv.data_ptr(), M, NQKV, D,
                        _lib.FC_BF16, 0, stream()), "gemm")
        check(L.fc_attn_prologue(ctypes.byref(dm.desc), layer, ctypes.byref(cb.desc), qkv.data_ptr(), h.data_ptr(),
                                 tok_t.data_ptr(), row_t.data_ptr(), pos_t.data_ptr(), M, qb.data_ptr(), stream()),
              "prologue")
        torch.cuda.synchronize()
        for name, a, b in (("q", qa, qb), ("k", ca.k[layer], cb.k[layer]), ("v", ca.v[layer], cb.v[layer])):
            a, b = a.float(), b.float()
            scale = b.abs().max().item()
            err = (a - b).abs().max().item()
            rel = ((a - b).abs() / (b.abs() + 1e-2 * scale)).max().item()
            _say(f"  layer {layer} {name}: max |diff| {err:.3e} (max |ref| {scale:.3f}), max rel {rel:.3e}")
            assert scale > 0 and rel <= 1e-2, f"layer {layer} {name}"
        # the skipped token (row -1) wrote no q either
        assert qa[3].abs().sum().item() == 0 and qb[3].abs().sum().item() == 0


# ---------------------------------------------------------------- measurement probes
def test_walk_probe_reads_each_units_tiles():
    """fc_walk_probe (the attention's load walk, timed by bench.py): every
    thread's output word is the XOR of the 16-byte groups it loaded, so a
    host recomputation over the expected addresses (unit u's tiles at
    u * tiles * 16 KB, wave w taking tiles w, w + 4, ..., lane l the groups
    l + 64 i of a tile) checks that it reads exactly its units' bytes."""
    units, tiles = 5, 6
    rng = np.random.default_rng(31)
    words = rng.integers(0, 2**32, units * tiles * 4096, dtype=np.uint64).astype(np.uint32)
    src = torch.from_numpy(words.view(np.int32)).to(dev())
    out = torch.zeros(256 * units, dtype=torch.int32, device=dev())
    check(_lib.lib().fc_walk_probe(src.data_ptr(), units, tiles, out.data_ptr(), stream()), "fc_walk_probe")
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint32).reshape(units, 4, 64)
    g16 = words.reshape(units, tiles, 1024, 4)  # 16-byte groups of each tile
    want = np.zeros((units, 4, 64), np.uint32)
    for w in range(4):
        for t in range(w, tiles, 4):
            for i in range(16):
                grp = g16[:, t, np.arange(64) + 64 * i, :]  # [units, lane, 4 words]
                want[:, w, :] ^= np.bitwise_xor.reduce(grp, axis=-1)
    assert np.array_equal(got, want)
    assert _lib.lib().fc_walk_probe(src.data_ptr(), 0, tiles, out.data_ptr(), stream()) != 0  # refused


@pytest.mark.parametrize("reg_loads", [0, 1])
def test_gemm_walk_probe_reads_each_tiles_blocks(reg_loads):
    """fc_gemm_walk_probe (the GEMM operand walk bench.py times): workgroup g
    takes tile t = (g % 8) per_xcd + g / 8, decoded M tile fastest, then K
    split, then N tile; wave w walks the split's 64-deep k chunks w, w + 4,
    ..., per chunk the tile's W blocks then its A blocks (row blocks clamped
    to the last live one), each block's two k steps in turn. Its word is
    the XOR (each lane's 16 bytes, every word) of the last min(loads, 16)
    blocks it landed in LDS (direct loads) or of every block it loaded
    (register loads), recomputed here for a ragged M, three N tiles and two
    K splits (5 and 5 chunks: one wave with two chunks)."""
    M, N, K, tm, tn, S = 40, 96, 640, 32, 32, 2
    KS, mb, nb = K // 32, tm // 16, tn // 16
    mtiles, ntiles = (M + tm - 1) // tm, N // tn
    rng = np.random.default_rng(47)
    a_words = rng.integers(0, 2**32, ((M + 15) // 16) * KS * 256, dtype=np.uint64).astype(np.uint32)
    w_words = rng.integers(0, 2**32, (N // 16) * KS * 256, dtype=np.uint64).astype(np.uint32)
    A = torch.from_numpy(a_words.view(np.int32)).to(dev())
    W = torch.from_numpy(w_words.view(np.int32)).to(dev())
    nwords = _lib.lib().fc_gemm_walk_probe_words(M, N, tm, tn, S)
    out = torch.zeros(nwords, dtype=torch.int32, device=dev())
    check(_lib.lib().fc_gemm_walk_probe(A.data_ptr(), W.data_ptr(), M, N, K, tm, tn, S, reg_loads, out.data_ptr(),
                                        stream()), "fc_gemm_walk_probe")
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint32).reshape(-1, 4)
    blk_xor = lambda words, i: np.bitwise_xor.reduce(words[i * 256:(i + 1) * 256])  # noqa: E731
    tiles = mtiles * ntiles * S
    per_xcd = (tiles + 7) // 8
    want = np.zeros((8 * per_xcd, 4), np.uint32)
    last_blk = (M - 1) // 16
    for g in range(8 * per_xcd):
        t = (g % 8) * per_xcd + g // 8
        if g // 8 >= per_xcd or t >= tiles:
            continue
        mt, rest = t % mtiles, t // mtiles
        sp, nt = rest % S, rest // S
        C = KS // 2
        c0, c1 = sp * C // S, (sp + 1) * C // S
        for w in range(4):
            seq = []
            for c in range(c0 + w, c1, 4):
                for b in range(nb + mb):
                    for h in range(2):
                        ks = 2 * c + h
                        if b < nb:
                            seq.append(blk_xor(w_words, (nt * nb + b) * KS + ks))
                        else:
                            seq.append(blk_xor(a_words, min(mt * mb + b - nb, last_blk) * KS + ks))
            x = np.uint32(0)
            for v in (seq if reg_loads else seq[-16:]):
                x ^= v
            want[g, w] = x
    assert np.array_equal(got, want)


def test_l2_read_probe_reads_its_region():
    """fc_l2_read_probe (the L2-to-CU ceiling bench.py reports): workgroup w
    walks 4 KB steps through the region of XCD w % 8 from offset
    (w / 8) * 64 KB, wave v loading the 1 KB at 1 KB v of each step into LDS
    slot (step % 16); its output word is the XOR over lanes of slot 0, the
    last step whose index is a multiple of 16. A host recomputation of those
    addresses checks the walk stays in its region."""
    region, wgs, per_wg = 64 << 10, 16, 256 << 10  # 64 steps per workgroup
    rng = np.random.default_rng(41)
    words = rng.integers(0, 2**32, 8 * region // 4, dtype=np.uint64).astype(np.uint32)
    src = torch.from_numpy(words.view(np.int32)).to(dev())
    out = torch.zeros(4 * wgs, dtype=torch.int32, device=dev())
    check(_lib.lib().fc_l2_read_probe(src.data_ptr(), region, per_wg * wgs, out.data_ptr(), wgs, stream()),
          "fc_l2_read_probe")
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint32).reshape(wgs, 4)
    steps = per_wg // 4096
    want = np.zeros((wgs, 4), np.uint32)
    for w in range(wgs):
        off = ((w // 8) * 65536 + 4096 * 16 * ((steps - 1) // 16)) % region
        base = (w % 8) * region + off
        for v in range(4):
            blk = words[(base + 1024 * v) // 4:(base + 1024 * v + 1024) // 4]
            want[w, v] = np.bitwise_xor.reduce(blk)
    assert np.array_equal(got, want)
    assert _lib.lib().fc_l2_read_probe(src.data_ptr(), 1000, per_wg * wgs, out.data_ptr(), wgs, stream()) != 0


def test_read_probe_reads_each_share():
    """fc_read_probe (the HBM read ceiling bench.py reports): workgroup b
    streams the 16-byte entries [b per, (b + 1) per) of the buffer, thread
    t the entries t, t + 256, ...; wave v's output word is the XOR of its
    threads' entries, recomputed here (including a ragged last share)."""
    n16, wgs = 10000, 7
    rng = np.random.default_rng(43)
    words = rng.integers(0, 2**32, n16 * 4, dtype=np.uint64).astype(np.uint32)
    src = torch.from_numpy(words.view(np.int32)).to(dev())
    out = torch.zeros(4 * wgs, dtype=torch.int32, device=dev())
    check(_lib.lib().fc_read_probe(src.data_ptr(), n16 * 16, out.data_ptr(), wgs, stream()), "fc_read_probe")
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint32).reshape(wgs, 4)
    e = np.bitwise_xor.reduce(words.reshape(n16, 4), axis=1)  # each entry's 4 words
    per = (n16 + wgs - 1) // wgs
    want = np.zeros((wgs, 4), np.uint32)
    for b in range(wgs):
        j = np.arange(b * per, min((b + 1) * per, n16))
        wave = ((j - b * per) % 256) // 64
        for v in range(4):
            want[b, v] = np.bitwise_xor.reduce(e[j[wave == v]]) if (wave == v).any() else 0
    assert np.array_equal(got, want)
