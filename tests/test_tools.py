"""Engine.generate's host side (flaxchat/engine.py:614-838): the calculator
tool and the per-row tool state machine, checked against the reference's
own calculator tests and hand-worked token sequences; the oracle's
streaming loop against generate_with_cache greedy."""

import os
import sys
from collections import namedtuple

import pytest

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

from flaxchat_amd.engine import RowState, ToolUse, use_calculator  # noqa: E402
from oracle import engine_stream  # noqa: E402
from tests.tooltok import ToolTokenizer  # noqa: E402

CALCS = [use_calculator, engine_stream.use_calculator]


@pytest.mark.parametrize("calc", CALCS)
def test_calculator_reference_cases(calc):
    """The reference's tests/test_engine.py:153-171."""
    assert calc("2 + 3") == 5
    assert calc("10 * 5") == 50
    assert calc("100 / 4") == 25.0
    assert calc("'hello'.count('l')") == 2
    assert calc("'strawberry'.count('r')") == 3
    assert calc("__import__('os')") is None
    assert calc("exec('bad')") is None
    assert calc("2**100") is None
    assert calc("1,000 + 2,000") == 3000


EXPRS = ["7 // 2", "-3 * (4 - 10)", "1 / 0", "2 ** 3", "+5", "", "3 -", "1.5 * 4", "(1+2)*(3+4)/7", "...",
         "()", "10 % 3", "'a b a'.count('a')", "'x'.count('x', 1)", "\"ab\".count(\"b\")", "12 12",
         "((((((((1))))))))", "5 - - 3", "1e3", "0.1 + 0.2"]


@pytest.mark.parametrize("expr", EXPRS)
def test_calculator_matches_restatement(expr):
    a, b = use_calculator(expr), engine_stream.use_calculator(expr)
    assert a == b and type(a) is type(b), (expr, a, b)


def test_calculator_hand_worked():
    assert use_calculator("7 // 2") == 3
    assert use_calculator("-3 * (4 - 10)") == 18
    assert use_calculator("1 / 0") is None
    assert use_calculator("+5") is None          # unary plus is not in the allowed node set
    assert use_calculator("10 % 3") is None      # '%' is not an allowed character
    assert use_calculator("'a b a'.count('a')") == 2
    assert use_calculator("1e3") is None


Result = namedtuple("Result", "success stdout")


def _tool(executor=None):
    tok = ToolTokenizer(256, python_start=10, python_end=11, output_start=12, output_end=13, assistant_end=14,
                        bos=1)
    return tok, ToolUse(tok, executor)


def _run(tool, st, sampled):
    return [tool.next_token(st, s) for s in sampled]


def test_state_machine_python_block():
    tok, tool = _tool()
    st = RowState([1, 2])
    # sampled: 5, <python_start>, 20, 33, <python_end>, then whatever is sampled is ignored while forcing
    sampled = [5, 10, 20, 33, 11, 99, 99, 99, 99, 98, 7]
    out = _run(tool, st, sampled)
    forced = [12] + tok.encode(str(20 + 33)) + [13]       # decode -> "20+33" -> 53
    assert len(forced) == 4
    assert [t for t, _ in out] == [5, 10, 20, 33, 11] + forced + [98, 7]
    assert [m for _, m in out] == [1] * 5 + [0] * 4 + [1, 1]
    assert st.current_tokens == [1, 2] + [t for t, _ in out]
    assert not st.in_python_block and not st.completed


def test_state_machine_edge_cases():
    tok, tool = _tool()
    st = RowState([])
    out = _run(tool, st, [11, 10, 11, 3])             # stray python_end; empty block forces nothing
    assert out == [(11, 1), (10, 1), (11, 1), (3, 1)]
    assert not st.forced_tokens
    st = RowState([])
    _run(tool, st, [10, 60, 11])                      # decode([60]) = "10"
    assert list(st.forced_tokens) == [12] + tok.encode("10") + [13]
    st = RowState([])
    _run(tool, st, [3, 14])
    assert st.completed
    st = RowState([])
    _run(tool, st, [1])
    assert st.completed                                # bos also completes


def test_state_machine_executor_and_error():
    class Tok(ToolTokenizer):
        def decode(self, ids):
            return "print(%d)" % len(ids)
    tok = Tok(256, 10, 11, 12, 13, 14, 1)
    calls = []

    def ex(code):
        calls.append(code)
        return Result(True, "42\n")
    tool = ToolUse(tok, ex)
    st = RowState([])
    _run(tool, st, [10, 5, 6, 11])
    assert calls == ["print(2)"]
    assert list(st.forced_tokens) == [12] + tok.encode("42") + [13]
    tool = ToolUse(tok, None)
    st = RowState([])
    _run(tool, st, [10, 5, 11])
    assert list(st.forced_tokens) == [12] + tok.encode("Error") + [13]
    tool = ToolUse(tok, lambda c: Result(False, ""))
    st = RowState([])
    _run(tool, st, [10, 5, 11])
    assert list(st.forced_tokens) == [12] + tok.encode("Error") + [13]


def test_oracle_stream_greedy_equals_cached(tiny_pair):
    """Without tool tokens in play, greedy streaming is generate_with_cache."""
    from oracle.spec import generate_with_cache
    tgt = tiny_pair[0]
    V = tgt.config.vocab_size
    tok = ToolTokenizer(V, V + 1, V + 2, V + 3, V + 4, V + 5, V + 6)
    prompt = [3, 1, 4, 1, 5]
    cols = engine_stream.engine_generate(tgt, prompt, tok, num_samples=2, max_tokens=10, temperature=0.0)
    ref = generate_with_cache(tgt, prompt, max_tokens=10, temperature=0.0, top_k=40)[len(prompt):]
    assert len(cols) == 10
    for i in range(2):
        assert [c[i] for c, _ in cols] == ref
    assert all(m == [1, 1] for _, m in cols)


def test_oracle_stream_forcing(tiny_pair):
    """Tool tokens chosen from the greedy stream: the block's output is
    forced, and greedy continues from the sequence that includes it."""
    from oracle.spec import generate_with_cache
    tgt = tiny_pair[0]
    V = tgt.config.vocab_size
    prompt = [3, 1, 4, 1, 5]
    g = generate_with_cache(tgt, prompt, max_tokens=12, temperature=0.0, top_k=40)[len(prompt):]
    i, j = _block(g)
    tok = ToolTokenizer(V, g[i], g[j], V - 1, V - 2, V + 5, V + 6)
    cols = engine_stream.engine_generate(tgt, prompt, tok, num_samples=1, max_tokens=20, temperature=0.0)
    seq = [c[0] for c, _ in cols]
    forced = [V - 1] + tok.encode(str(use_calculator(tok.decode(g[i + 1:j])))) + [V - 2]
    assert seq[:j + 1] == g[:j + 1]
    assert seq[j + 1:j + 1 + len(forced)] == forced
    assert [m[0] for _, m in cols][j + 1:j + 1 + len(forced)] == [0] * len(forced)
    k = j + 1 + len(forced)
    cont = generate_with_cache(tgt, prompt + seq[:k], max_tokens=len(seq) - k, temperature=0.0, top_k=40)
    assert seq[k:] == cont[len(prompt) + k:]


def _block(g):
    """First (i, j), j >= i + 2, with g[i] and g[j] distinct tokens whose
    first occurrences are at i and j."""
    for i in range(len(g)):
        if g[i] in g[:i]:
            continue
        for j in range(i + 2, len(g)):
            if g[j] not in g[:j] and g[j] != g[i]:
                return i, j
    raise AssertionError(f"no python block can be placed in {g}")
