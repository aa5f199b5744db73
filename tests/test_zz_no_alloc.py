"""fc_attention_noalloc, the allocation-free variant of fc_attention: its
split-KV partials live in the library's static device scratch instead of a
caller-supplied workspace. Checked through the C-ABI against fc_attention
on the same inputs (same kernels, so bit-identical output), on two calls in
a row where the second is smaller, and a size beyond the scratch is refused
before anything is launched."""

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


def test_noalloc_refuses_sizes_beyond_scratch():
    f = _fn()
    cap_bytes = lib().fc_attention_noalloc_max_bytes()
    assert cap_bytes > 0
    # 4096 rows x 16 KV groups x 64-token chunks needs far more partials
    need = lib().fc_attention_workspace_bytes(4096, 64, 16, 16, 128, 8192)
    assert need > cap_bytes
    dummy = torch.zeros(16, dtype=torch.int32, device="cuda")
    p = dummy.data_ptr()
    rc = f(p, p, p, p, 4096, 4096 * 64, 64, 16, 16, 128, 8192, p, p, 0, 8192, _lib.FC_BF16,
           torch.cuda.current_stream().cuda_stream)
    assert rc == -4 and b"scratch" in lib().fc_last_error()
