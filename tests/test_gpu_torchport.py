"""The HIP engine against logits of the reference's own PyTorch port.

tests/golden/torchport_forward.npz holds logits that the reference's
`GELU_GPT(mlp="relu2")` (flaxchat/torch_port/torch_gpt.py:268-375) computed;
tests/test_torchport_pin.py shows the CPU restatement reproduces them within
1e-5. Here the device paths are held to them directly:

* `gpt_forward` (GPT.__call__, flaxchat/gpt.py:407-454) in fp32 within 1e-3
  max-abs for every case;
* the decode path (`fc_forward` over packed chunks, the per-token forward of
  flaxchat/engine.py:51-177) in fp32 within 1e-3 at every position of the
  smear-free cases, fed in uneven chunks so cache reads cross chunk
  boundaries;
* bf16 on the head_dim-128 cases within a bound set from the measured error;
* the converter-written checkpoint (tests/golden/torchport_tiny.pt) loaded by
  `load_torch_port` and run through the engine: logits, and greedy
  speculative / fast streams equal to the oracle's on the same weights.
"""
import os
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from flaxchat_amd.checkpoint import load_torch_port  # noqa: E402
from flaxchat_amd.engine import as_device_model, generate_fast, generate_speculative, gpt_forward  # noqa: E402
from flaxchat_amd.runtime import DeviceCache, Workspace, forward_rows  # noqa: E402
from tests.golden.torchport_cases import CASES, build_model  # noqa: E402

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
FIX = os.path.join(HERE, "golden", "torchport_forward.npz")
PT = os.path.join(HERE, "golden", "torchport_tiny.pt")
# bf16 weights and activations against fp32 logits whose |z| reaches ~3-4:
# measured 1.1e-2 - 1.6e-2 on these cases; the bound leaves 2x headroom.
BF16_TOL = 3e-2


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def fixtures():
    return np.load(FIX, allow_pickle=False)


@pytest.mark.parametrize("name", list(CASES))
def test_gpt_forward_fp32_vs_port(name, fixtures):
    _say(f"gpt_forward fp32 vs port: {name}")
    m = build_model(CASES[name])
    ids, ref = fixtures[f"{name}/ids"], fixtures[f"{name}/logits"]
    got = gpt_forward(m, ids, dtype="fp32").cpu().numpy()
    err = float(np.abs(got - ref).max())
    _say(f"  max-abs {err:.3e}")
    assert err < 1e-3


@pytest.mark.parametrize("name", ["nosmear", "d128_nosmear"])
def test_decode_fp32_vs_port(name, fixtures):
    """Every position's logits from the cached decode path."""
    _say(f"decode fp32 vs port: {name}")
    m = build_model(CASES[name])
    ids, ref = fixtures[f"{name}/ids"], fixtures[f"{name}/logits"]
    dm = as_device_model(m, "fp32")
    B, T = ids.shape
    cache = DeviceCache(dm, B, T + 8)
    ws = Workspace(dm.device)
    chunks = [1, 6, 2, 13, 1]
    chunks.append(T - sum(chunks))
    pos, outs = 0, []
    for w in chunks:
        lg = torch.zeros(B, w, dm.V, device=dm.device)
        forward_rows(dm, cache, [ids[b, pos:pos + w].tolist() for b in range(B)], [pos] * B, w, lg, ws)
        outs.append(lg.cpu().numpy())
        pos += w
    torch.cuda.synchronize()
    got = np.concatenate(outs, axis=1)
    err = float(np.abs(got - ref).max())
    _say(f"  max-abs {err:.3e}")
    assert err < 1e-3


@pytest.mark.parametrize("name", ["d128_smear", "d128_nosmear"])
def test_gpt_forward_bf16_vs_port(name, fixtures):
    _say(f"gpt_forward bf16 vs port: {name}")
    m = build_model(CASES[name])
    ids, ref = fixtures[f"{name}/ids"], fixtures[f"{name}/logits"]
    got = gpt_forward(m, ids, dtype="bf16").cpu().numpy()
    err = float(np.abs(got - ref).max())
    _say(f"  max-abs {err:.3e} (|z| max {np.abs(ref).max():.2f})")
    assert err < BF16_TOL


def test_loaded_checkpoint_runs_on_device(fixtures):
    """load_torch_port on the converter's file, then the engine."""
    from oracle.spec import generate_fast as o_fast
    from oracle.spec import spec_literal
    _say("torch-port checkpoint on the engine")
    m = load_torch_port(PT)
    ids, ref = fixtures["tiny_pt/ids"], fixtures["tiny_pt/logits"]
    got = gpt_forward(m, ids, dtype="fp32").cpu().numpy()
    assert float(np.abs(got - ref).max()) < 1e-3
    draft = m.make_draft(1)
    prompt = ids[0, :12].tolist()
    toks = generate_speculative(m, draft, prompt, max_tokens=24, temperature=0.0, top_k=40, draft_steps=3,
                                dtype="fp32")
    assert toks == spec_literal(m, draft, prompt, max_tokens=24, temperature=0.0, top_k=40, draft_steps=3)
    toks = generate_fast(m, prompt, max_tokens=16, temperature=0.0, top_k=40, dtype="fp32")
    assert toks == o_fast(m, prompt, max_tokens=16, temperature=0.0, top_k=40)
