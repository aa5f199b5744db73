"""fc_attention_noalloc, the allocation-free variant of fc_attention: its
split-KV partials live in the library's static device scratch instead of a
caller-supplied workspace. Checked through the C-ABI against fc_attention
on the same inputs (same kernels, so bit-identical output), on two calls in
a row where the second is smaller, and a size beyond the scratch is refused
before anything is launched."""

import ctypes
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from flaxchat_amd import _lib  # noqa: E402
from flaxchat_amd._lib import check, lib  # noqa: E402

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _fn():
    return lib().fc_attention_noalloc


def _case(seed, B, W, H, G, window, lmax, dtype):
    """Random q / K / V in the cache layouts (any bf16 bit patterns of
    N(0,1) values; the layout does not matter for an output comparison)."""
    rng = np.random.default_rng(seed)
    d = 128
    cap = ((lmax + W + 31) // 32) * 32 + 32
    L = rng.integers(max(1, W), lmax, size=B)
    nvalid = np.minimum(rng.integers(1, W + 1, size=B), L).astype(np.int32)
    start = (L - nvalid).astype(np.int32)
    off = np.zeros(B + 1, np.int32)
    off[1:] = np.cumsum(nvalid)
    tot = int(off[-1])
    tdt = torch.bfloat16 if dtype == _lib.FC_BF16 else torch.float32
    dev = torch.device("cuda", 0)
    q = torch.from_numpy(rng.standard_normal((tot, H, d)).astype(np.float32)).to(dev, tdt)
    K = torch.from_numpy(rng.standard_normal((B, G, cap, d)).astype(np.float32)).to(dev, tdt)
    V = torch.from_numpy(rng.standard_normal((B, G, cap, d)).astype(np.float32)).to(dev, tdt)
    rows = (tot + 15) // 16 * 16
    max_keys = min(cap, window + W) if window > 0 else cap
    return dict(q=q, K=K, V=V, B=B, W=W, H=H, G=G, d=d, cap=cap, tot=tot, rows=rows, window=window,
                max_keys=max_keys, code=dtype, tdt=tdt, ro=torch.from_numpy(off).to(dev),
                st=torch.from_numpy(start).to(dev))


def _run(c, noalloc):
    dev = torch.device("cuda", 0)
    y = torch.full((c["rows"], c["H"] * c["d"]), 3.0, device=dev, dtype=c["tdt"])
    s = torch.cuda.current_stream().cuda_stream
    args = (c["q"].data_ptr(), c["K"].data_ptr(), c["V"].data_ptr(), y.data_ptr(), c["B"], c["tot"], c["W"], c["H"],
            c["G"], c["d"], c["cap"], c["ro"].data_ptr(), c["st"].data_ptr(), c["window"], c["max_keys"], c["code"])
    if noalloc:
        check(_fn()(*args, s), "fc_attention_noalloc")
    else:
        nb = lib().fc_attention_workspace_bytes(c["B"], c["W"], c["H"], c["G"], c["d"], c["max_keys"])
        ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=dev)
        check(lib().fc_attention(*args, ws.data_ptr(), ws.numel(), s), "fc_attention")
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("dtype", [_lib.FC_BF16, _lib.FC_F32])
def test_noalloc_matches_workspace_entry_point(dtype):
    # first call: several key splits (few row x group units); second: smaller
    # batch, fewer keys, a window; third: one split per unit (nothing in scratch)
    for i, shape in enumerate([(3, 9, 12, 4, 0, 1500), (2, 5, 6, 6, 256, 700), (32, 2, 8, 8, 0, 300)]):
        _say(f"noalloc attention dtype={dtype} call {i} shape={shape}")
        c = _case(100 + i, *shape, dtype)
        ref = _run(c, noalloc=False)
        got = _run(c, noalloc=True)
        assert torch.equal(got, ref), f"call {i}: differs from fc_attention"


def test_noalloc_prefill_width_needs_no_scratch():
    """bf16 chunks of >= 128 query columns per row and KV group take the
    prefill kernel, which writes no partials: the allocation-free entry point
    runs them whatever their size and matches fc_attention bit for bit, and a
    smaller decode-width call after it still matches."""
    L = lib()
    # 4 rows x 1024 tokens x 12 heads: fc_attention_workspace_bytes reports
    # the decode kernel's partials (far above the scratch), none are needed
    need = L.fc_attention_workspace_bytes(4, 1024, 12, 12, 128, 2048)
    assert need > L.fc_attention_noalloc_max_bytes()
    for i, shape in enumerate([(4, 1024, 12, 12, 0, 1100), (3, 7, 12, 4, 256, 900)]):
        _say(f"noalloc attention prefill-width call {i} shape={shape}")
        c = _case(300 + i, *shape, _lib.FC_BF16)
        ref = _run(c, noalloc=False)
        got = _run(c, noalloc=True)
        assert torch.equal(got, ref), f"call {i}: differs from fc_attention"


def test_noalloc_under_graph_capture():
    """fc_attention_noalloc recorded into a graph between fc_graph_begin and
    fc_graph_end (which looks the scratch address up before the capture),
    replayed three times with eager work and synchronisations between the
    replays: every replay equals the eager fc_attention output."""
    L = lib()
    c = _case(400, 6, 7, 12, 4, 0, 1300, _lib.FC_BF16)
    ref = _run(c, noalloc=False)
    dev = torch.device("cuda", 0)
    side = torch.cuda.Stream(device=dev)
    y = torch.full((c["rows"], c["H"] * c["d"]), 3.0, device=dev, dtype=c["tdt"])
    args = (c["q"].data_ptr(), c["K"].data_ptr(), c["V"].data_ptr(), y.data_ptr(), c["B"], c["tot"], c["W"], c["H"],
            c["G"], c["d"], c["cap"], c["ro"].data_ptr(), c["st"].data_ptr(), c["window"], c["max_keys"], c["code"])
    torch.cuda.synchronize()
    _say("noalloc attention: capture")
    ex = ctypes.c_void_p()
    check(L.fc_graph_begin(side.cuda_stream), "fc_graph_begin")
    rc = L.fc_attention_noalloc(*args, side.cuda_stream)
    check(L.fc_graph_end(side.cuda_stream, ctypes.byref(ex)), "fc_graph_end")
    check(rc, "fc_attention_noalloc (captured)")
    try:
        for rep in range(3):
            _say(f"noalloc attention: replay {rep}")
            y.fill_(3.0)  # the value fc_attention's output buffer started from (padding rows keep it)
            torch.cuda.synchronize()
            check(L.fc_graph_launch(ex, side.cuda_stream), "fc_graph_launch")
            side.synchronize()
            assert torch.equal(y, ref), f"replay {rep} differs from fc_attention"
            _run(_case(500 + rep, 2, 3, 6, 6, 0, 400, _lib.FC_BF16), noalloc=False)  # eager work in between
    finally:
        L.fc_graph_destroy(ex)
