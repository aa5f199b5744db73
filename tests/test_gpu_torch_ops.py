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


# ---------------------------------------------------------------- engine entry points as operators
def _spec_args(s):
    from flaxchat_amd.torch_ops import SPEC_BUFFERS
    st = s.state
    return ([s.bufs[n] for n in SPEC_BUFFERS], st.batch, st.k, st.max_tokens, st.gen_cap, st.vocab, st.temperature,
            st.top_k, st.seed)


@pytest.mark.parametrize("T,top_k", [(0.8, None), (0.0, 40), (1.0, 5)])
def test_spec_round_op_matches_c_abi(T, top_k, tiny_pair):
    """Speculative rounds through torch.ops.flaxchat_mi355x.spec_round equal
    the engine's own C-ABI calls bit for bit: every device buffer of the
    state, the caches and the token streams after each round (fp32 and
    bf16 models of the cfg1 width)."""
    import ctypes
    from flaxchat_amd.engine import SpecSession, as_device_model
    from tests.golden.make_golden import cfg1_models
    tgt, draft = cfg1_models()
    for dtype in ("fp32", "bf16"):
        _say(f"spec_round op T={T} top_k={top_k} {dtype}")
        t, d = as_device_model(tgt, dtype), as_device_model(draft, dtype)
        rng = np.random.default_rng(3)
        rows = [rng.integers(0, 8192, n).tolist() for n in (9, 30, 17)]
        a = SpecSession(t, d, rows, 24, T, top_k, 11, 4, use_graph=False)
        b = SpecSession(t, d, rows, 24, T, top_k, 11, 4, use_graph=False)
        a.prefill()
        b.prefill()
        torch.cuda.synchronize()
        for r in range(6):
            with torch.cuda.stream(a.stream):
                a._round_call()
            bufs, *scal = _spec_args(b)
            with torch.cuda.stream(b.stream):
                OPS.spec_round(ctypes.addressof(t.desc), ctypes.addressof(d.desc), b.tcache.k, b.tcache.v,
                               b.tcache.hist, b.dcache.k, b.dcache.v, b.dcache.hist, bufs, *scal, b.ws.buf)
            torch.cuda.synchronize()
            for n in a.bufs:
                if n == "part":
                    continue
                assert torch.equal(a.bufs[n], b.bufs[n]), f"round {r}: buffer {n} differs"
            for x, y in ((a.tcache.k, b.tcache.k), (a.tcache.v, b.tcache.v), (a.dcache.hist, b.dcache.hist)):
                assert torch.equal(x, y), f"round {r}: caches differ"
        a.close()
        b.close()


def test_forward_and_row_stats_ops(cfg1_pair):
    """forward (one packed chunk, logits of the last token per row) and
    row_stats through torch.ops against fc_forward via the runtime and
    fc_row_stats: identical results."""
    import ctypes
    from flaxchat_amd import _lib
    from flaxchat_amd.engine import as_device_model
    from flaxchat_amd.runtime import DeviceCache, Workspace, forward_rows, pack_rows
    tgt = cfg1_pair[0]
    dm = as_device_model(tgt, "bf16")
    rng = np.random.default_rng(4)
    rows = [rng.integers(0, 8192, n).tolist() for n in (7, 3, 12)]
    B = len(rows)
    ca, cb = DeviceCache(dm, B, 64), DeviceCache(dm, B, 64)
    la = torch.zeros(B, 1, dm.V, device=dev())
    lb = torch.zeros(B, 1, dm.V, device=dev())
    forward_rows(dm, ca, rows, [0] * B, 1, la, Workspace(dev()))
    tok, off, mpr = pack_rows(rows)
    ws = torch.zeros(_lib.lib().fc_forward_workspace_bytes(ctypes.byref(dm.desc), B, len(tok), mpr, 0),
                     dtype=torch.uint8, device=dev())
    t = lambda a: torch.from_numpy(np.asarray(a, np.int32)).to(dev())  # noqa: E731
    OPS.forward(ctypes.addressof(dm.desc), cb.k, cb.v, cb.hist, t(tok), t(off), t([0] * B), mpr, 1, lb, ws)
    torch.cuda.synchronize()
    assert torch.equal(la, lb) and torch.equal(ca.k, cb.k) and torch.equal(ca.v, cb.v)
    mx, sm, tau, tie, am = OPS.row_stats(lb[:, 0].contiguous(), 0.8, 40)
    raw = torch.zeros(B * 32, dtype=torch.uint8, device=dev())
    _lib.check(_lib.lib().fc_row_stats(lb.data_ptr(), B, dm.V, 0.8, 40, raw.data_ptr(),
                                       torch.cuda.current_stream().cuda_stream), "row stats")
    torch.cuda.synchronize()
    ref = raw.view(torch.int32).view(B, 8)
    assert torch.equal(mx.view(torch.int32), ref[:, 0]) and torch.equal(sm.view(torch.int32), ref[:, 1])
    assert torch.equal(tie, ref[:, 3]) and torch.equal(am, ref[:, 4])
    assert torch.equal(am.long().cpu(), lb[:, 0].argmax(-1).cpu())


def test_attn_ops_match_c_abi():
    """attn_qkv (fused epilogue at 160 rows) and attn_prologue through
    torch.ops equal the C-ABI entries on the same inputs."""
    import ctypes
    from flaxchat_amd import _lib
    from flaxchat_amd.config import GPTConfig
    from flaxchat_amd.gpt import GPT
    from flaxchat_amd.runtime import DeviceCache, DeviceModel, pack_operand
    cfg = GPTConfig(sequence_len=256, vocab_size=1024, n_layer=2, n_head=4, n_kv_head=2, n_embd=512,
                    window_pattern="SL", short_window=64)
    dm = DeviceModel.from_host(GPT.init_normal(cfg, seed=2, std=0.05), dtype="bf16", device=dev())
    M, B, cap = 160, 2, 128
    rng = np.random.default_rng(1)
    slots = rng.permutation(B * cap)[:M]
    t = lambda a: torch.from_numpy(np.asarray(a, np.int32)).to(dev())  # noqa: E731
    tok, row, pos = t(rng.integers(0, 1024, M)), t(slots // cap), t(slots % cap)
    h = pack_operand(torch.from_numpy(rng.standard_normal((M, 512)).astype(np.float32)).to(dev(), torch.bfloat16))
    L = _lib.lib()
    for layer in (0, 1):
        ca, cb = DeviceCache(dm, B, cap), DeviceCache(dm, B, cap)
        qa = torch.zeros(M, 4, 128, dtype=torch.bfloat16, device=dev())
        _lib.check(L.fc_attn_qkv(ctypes.byref(dm.desc), layer, ctypes.byref(ca.desc), h.data_ptr(), tok.data_ptr(),
                                 row.data_ptr(), pos.data_ptr(), M, 0, qa.data_ptr(), None, 0,
                                 torch.cuda.current_stream().cuda_stream), "attn_qkv")
        qb = OPS.attn_qkv(ctypes.addressof(dm.desc), layer, cb.k, cb.v, h, tok, row, pos, 0)
        torch.cuda.synchronize()
        assert torch.equal(qa, qb) and torch.equal(ca.k, cb.k) and torch.equal(ca.v, cb.v)
        qkv = torch.from_numpy(rng.standard_normal((M, 1024)).astype(np.float32)).to(dev())
        cc, cd = DeviceCache(dm, B, cap), DeviceCache(dm, B, cap)
        qc = torch.zeros(M, 4, 128, dtype=torch.bfloat16, device=dev())
        _lib.check(L.fc_attn_prologue(ctypes.byref(dm.desc), layer, ctypes.byref(cc.desc), qkv.data_ptr(),
                                      h.data_ptr(), tok.data_ptr(), row.data_ptr(), pos.data_ptr(), M, qc.data_ptr(),
                                      torch.cuda.current_stream().cuda_stream), "prologue")
        qd = OPS.attn_prologue(ctypes.addressof(dm.desc), layer, cd.k, cd.v, qkv, h, tok, row, pos)
        torch.cuda.synchronize()
        assert torch.equal(qc, qd) and torch.equal(cc.k, cd.k) and torch.equal(cc.v, cd.v)


def test_engine_delegates(tiny_pair):
    """Engine.generate_speculative / Engine.generate_fast (flaxchat/engine.py:
    877-908) equal the module-level functions they delegate to, with the
    reference's defaults."""
    from flaxchat_amd.engine import Engine, generate_fast, generate_speculative
    tgt, draft = tiny_pair
    eng = Engine(tgt, dtype="fp32")
    prompt = [3, 1, 4, 1, 5]
    a = eng.generate_speculative(draft, prompt, max_tokens=20, draft_steps=3)
    b = generate_speculative(tgt, draft, prompt, max_tokens=20, draft_steps=3, dtype="fp32")
    assert a == b and len(a) == len(prompt) + 20
    c = eng.generate_fast(prompt, max_tokens=20, temperature=0.0, eos_token=-1)
    d = generate_fast(tgt, prompt, max_tokens=20, temperature=0.0, eos_token=-1, dtype="fp32")
    assert c == d
    from oracle.spec import spec_literal, generate_fast as ofast
    assert a == spec_literal(tgt, draft, prompt, max_tokens=20, temperature=1.0, top_k=40, seed=42, draft_steps=3)
    assert c == ofast(tgt, prompt, max_tokens=20, temperature=0.0, top_k=40, seed=42, eos_token=-1)
