"""Engine.generate on the HIP engine (flaxchat/engine.py:686-874) against
the oracle's restatement (oracle/engine_stream.py): in fp32 every yielded
column and mask must be identical, including tool blocks whose output is
forced into the stream and rows that complete at different steps."""

import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from flaxchat_amd.engine import Engine, generate_with_cache  # noqa: E402
from oracle import engine_stream  # noqa: E402
from tests.tooltok import ToolTokenizer  # noqa: E402
from tests.test_tools import _block  # noqa: E402

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _no_tools(V):
    return ToolTokenizer(V, V + 1, V + 2, V + 3, V + 4, V + 5, V + 6)


def _compare(tgt, prompt, tok, **kw):
    got = list(Engine(tgt, tok, dtype="fp32").generate(prompt, **kw))
    ref = engine_stream.engine_generate(tgt, prompt, tok, **kw)
    assert len(got) == len(ref)
    for s, (a, b) in enumerate(zip(got, ref)):
        assert a == b, f"step {s}: {a} vs {b}"
    return ref


@pytest.mark.parametrize("num_samples", [1, 3])
def test_stream_greedy_tool_block(num_samples, tiny_pair):
    _say(f"stream greedy tool block n={num_samples}")
    tgt = tiny_pair[0]
    V = tgt.config.vocab_size
    prompt = [3, 1, 4, 1, 5]
    g = [c[0] for c, _ in engine_stream.engine_generate(tgt, prompt, _no_tools(V), max_tokens=12, temperature=0.0)]
    i, j = _block(g)
    tok = ToolTokenizer(V, g[i], g[j], V - 1, V - 2, V + 5, V + 6)
    ref = _compare(tgt, prompt, tok, num_samples=num_samples, max_tokens=24, temperature=0.0)
    assert any(m == 0 for _, ms in ref for m in ms), "the tool block produced no forced tokens"


@pytest.mark.parametrize("T,top_k", [(1.0, 5), (0.8, None), (1.0, 0)])
def test_stream_sampling_tool_block(T, top_k, tiny_pair):
    _say(f"stream sampling T={T} top_k={top_k}")
    tgt = tiny_pair[0]
    V = tgt.config.vocab_size
    prompt = [7, 2, 9]
    kw = dict(num_samples=3, max_tokens=24, temperature=T, top_k=top_k, seed=11)
    g = [c[0] for c, _ in engine_stream.engine_generate(tgt, prompt, _no_tools(V), **kw)]
    i, j = _block(g)
    tok = ToolTokenizer(V, g[i], g[j], V - 1, V - 2, V + 5, V + 6)
    ref = _compare(tgt, prompt, tok, **kw)
    assert any(m == 0 for _, ms in ref for m in ms)
    rows = [[c[r] for c, _ in ref] for r in range(3)]
    assert rows[0] != rows[1] or rows[1] != rows[2], "independent rows drew identical streams"


def test_stream_completion_and_batch(tiny_pair):
    _say("stream completion / generate_batch")
    tgt = tiny_pair[0]
    V = tgt.config.vocab_size
    prompt = [3, 1, 4, 1, 5]
    g = [c[0] for c, _ in engine_stream.engine_generate(tgt, prompt, _no_tools(V), max_tokens=8, temperature=0.0)]
    stop = next(s for s in range(2, 8) if g[s] not in g[:s])
    tok = ToolTokenizer(V, V + 1, V + 2, V + 3, V + 4, g[stop], V + 6)
    cols = _compare(tgt, prompt, tok, num_samples=2, max_tokens=8, temperature=0.0)
    assert len(cols) == stop + 1
    eng = Engine(tgt, tok, dtype="fp32")
    res, masks = eng.generate_batch(prompt, num_samples=2, max_tokens=8, temperature=0.0)
    assert res == [prompt + g[:stop]] * 2
    assert masks == [[0] * len(prompt) + [1] * stop] * 2
    # sampling: rows complete at different steps; completed rows keep sampling
    tok2 = ToolTokenizer(V, V + 1, V + 2, V + 3, V + 4, g[0], V + 6)
    _compare(tgt, prompt, tok2, num_samples=4, max_tokens=30, temperature=1.5, top_k=3, seed=3)


def test_stream_default_length(tiny_pair):
    _say("stream max_tokens=None")
    tgt = tiny_pair[0]
    V = tgt.config.vocab_size
    cols = list(Engine(tgt, _no_tools(V), dtype="fp32").generate([5, 6], max_tokens=None, temperature=0.0))
    assert len(cols) == 256
    ref = generate_with_cache(tgt, [5, 6], max_tokens=256, temperature=0.0, top_k=40, dtype="fp32")
    assert [c[0] for c, _ in cols] == ref[2:]


def test_stream_bf16_matches_cached(cfg1_pair):
    """bf16: the streaming session runs the same kernels as
    generate_with_cache at one row, so greedy streams are identical."""
    _say("stream bf16 vs cached")
    tgt = cfg1_pair[0]
    V = tgt.config.vocab_size
    prompt = np.random.default_rng(2).integers(0, V, 40).tolist()
    cols = list(Engine(tgt, _no_tools(V), dtype="bf16").generate(prompt, max_tokens=32, temperature=0.0))
    ref = generate_with_cache(tgt, prompt, max_tokens=32, temperature=0.0, top_k=40, dtype="bf16")
    assert [c[0] for c, _ in cols] == ref[len(prompt):]


def test_generate_text(tiny_pair):
    tgt = tiny_pair[0]
    V = tgt.config.vocab_size
    tok = _no_tools(V)
    tok.bos = 0
    text = Engine(tgt, tok, dtype="fp32").generate_text("hi", max_tokens=6, temperature=0.0)
    ref = engine_stream.engine_generate(tgt, tok("hi", prepend="<|bos|>"), tok, max_tokens=6, temperature=0.0)
    ids = []
    for c, _ in ref:
        if c[0] in (tok.bos, V + 5):
            break
        ids.append(c[0])
    assert text == tok.decode(tok("hi", prepend="<|bos|>") + ids)
