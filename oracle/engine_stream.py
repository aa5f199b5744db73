"""Engine.generate restated on the numpy forward — TEST INFRASTRUCTURE
(parity oracle; see oracle/__init__.py for who may import it).

Follows flaxchat/engine.py:686-838 statement by statement: the prompt is
prefilled (once per row here; the reference prefills once and copies the
cache, which is the same state), then each step samples every row
(`_sample_next_token`, engine.py:666-683: argmax at temperature 0, else a
categorical over the top-k values, or over everything when top_k is None or
0), takes the head of the row's forced queue instead when there is one,
applies the tool protocol, yields the column, and feeds it.

Draws use the engine's Philox stream: row b, round = step index, slot 0
(the same ids as generate_fast), so the HIP engine's columns must equal
these exactly in fp32.
"""

from __future__ import annotations

import ast
import re
from collections import deque

from .spec import _as_oracle
from .sampling import fast_sample

_ALLOWED = (ast.Expression, ast.BinOp, ast.UnaryOp, ast.Constant, ast.Add, ast.Sub, ast.Mult, ast.Div,
            ast.FloorDiv, ast.Mod, ast.USub)


def use_calculator(expr):
    """flaxchat/engine.py:614-643: drop commas; arithmetic over the
    characters 0-9 * + - / . ( ) and space, no '**', syntax tree limited to
    numbers, unary minus and + - * / // %; or 'text'.count('word');
    anything else (or an error while evaluating) is None."""
    expr = expr.replace(",", "")
    if set(expr) <= set("0123456789*+-/.() "):
        if "**" in expr:
            return None
        try:
            tree = ast.parse(expr, mode="eval")
            if not all(isinstance(n, _ALLOWED) for n in ast.walk(tree)):
                return None
            return eval(compile(tree, "<calc>", "eval"), {"__builtins__": {}}, {})
        except Exception:
            return None
    m = re.fullmatch(r"""['"]([\w\s]+)['"]\s*\.\s*count\s*\(\s*['"](\w+)['"]\s*\)""", expr)
    return m.group(1).count(m.group(2)) if m else None


def engine_generate(model, tokens, tokenizer, num_samples=1, max_tokens=None, temperature=1.0, top_k=40,
                    seed=42, code_executor=None):
    """List of (token_column, token_masks) as Engine.generate yields them
    (flaxchat/engine.py:686-838). max_tokens=None runs 256 steps at most."""
    M = _as_oracle(model)
    enc = tokenizer.encode_special
    py_s, py_e = enc("<|python_start|>"), enc("<|python_end|>")
    out_s, out_e = enc("<|output_start|>"), enc("<|output_end|>")
    a_end, bos = enc("<|assistant_end|>"), tokenizer.get_bos_token_id()
    steps = 256 if max_tokens is None else max_tokens
    P = len(tokens)
    sts, logits = [], []
    for _ in range(num_samples):
        st = M.new_state(P + steps + 1)
        logits.append(M.prefill(tokens, st))
        sts.append(st)
    forced = [deque() for _ in range(num_samples)]
    in_py = [False] * num_samples
    expr = [[] for _ in range(num_samples)]
    done = [False] * num_samples
    cols = []
    for s in range(steps):
        if all(done):
            break
        col, masks = [], []
        for i in range(num_samples):
            sampled = fast_sample(logits[i], temperature, top_k if top_k is not None else 0, seed, i, s)
            if forced[i]:
                t, m = forced[i].popleft(), 0
            else:
                t, m = sampled, 1
            col.append(t)
            masks.append(m)
            if t == a_end or t == bos:
                done[i] = True
            if t == py_s:
                in_py[i], expr[i] = True, []
            elif t == py_e and in_py[i]:
                in_py[i] = False
                if expr[i]:
                    text = tokenizer.decode(expr[i])
                    res = use_calculator(text)
                    if res is None:
                        r = code_executor(text) if code_executor is not None else None
                        res = r.stdout.rstrip("\n") if r is not None and r.success else "Error"
                    forced[i].extend([out_s] + list(tokenizer.encode(str(res))) + [out_e])
                expr[i] = []
            elif in_py[i]:
                expr[i].append(t)
        cols.append((col, masks))
        for i in range(num_samples):
            logits[i] = M.step(col[i], P + s, sts[i])
    return cols
