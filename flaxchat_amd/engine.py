"""Speculative and fast decoding on the HIP engine, with the reference's call
surface (flaxchat/engine.py:259-260, 410-411, 877-908).

    generate_speculative(model, draft_model, tokens, max_tokens=256,
                         temperature=1.0, top_k=40, seed=42, draft_steps=4)
    generate_fast(model, tokens, max_tokens=256, temperature=1.0, top_k=40,
                  seed=42, eos_token=0)
    generate_with_cache(model, tokens, max_tokens=256, temperature=1.0,
                        top_k=40, seed=42)
    Engine(model, tokenizer).generate(tokens, num_samples=1, max_tokens=None,
                                      temperature=1.0, top_k=40, seed=42)
        (streaming, with the calculator tool's forced output tokens;
        also generate_batch / generate_text)

`model` / `draft_model` are host GPT containers (flaxchat_amd.gpt.GPT, the
reference's parameter tree) or DeviceModel instances. `tokens` is a list of
ints (returns a list of ints, like the reference) or a batch: a list of
lists or a [B, P] integer array/tensor (returns a list of lists).

Differences from the reference, by design:
  * the random stream is Philox4x32-10 (counter = element, row, round,
    slot), not jax.random; distributions are the same;
  * verification is one (pending + k)-token chunk per round and rejection
    rolls the cache length pointer back instead of re-prefilling; the
    emitted tokens are the same, including the last-index-rejection quirk
    (flaxchat/engine.py:573), whose stale cache entry is reproduced and
    later repaired exactly when the reference's re-prefill would repair it;
  * cache overflow raises instead of clamping (engine.py:121-126);
  * temperature < 0 behaves as greedy;
  * Engine.generate with max_tokens=None stops after 256 steps (the
    reference's cache ends there and later writes are clamped); a Python
    block the calculator cannot evaluate goes to the Engine's
    code_executor (the reference calls its sandbox, flaxchat/execution.py;
    pass flaxchat.execution.execute_code to get the same behaviour), and
    without one its result is "Error".
"""

from __future__ import annotations

import ast
import ctypes
import operator
import re
import weakref
from collections import deque
from dataclasses import dataclass, field
from typing import Callable, Iterator, List, Optional, Sequence, Tuple, Union

import numpy as np
import torch

from . import _lib
from ._lib import FcSpecState, FcRowstat, PMAX, RES_STRIDE, check, lib
from .runtime import DeviceCache, DeviceModel, Workspace, default_device, forward_packed, prefill_rows

_BIG_POS = 0x3FFFFFFF
_DEVICE_MODELS: "weakref.WeakKeyDictionary" = weakref.WeakKeyDictionary()


class VocabMismatchError(AssertionError, ValueError):
    """Main and draft vocabularies differ (flaxchat/engine.py:438-439 asserts)."""


def _env_dtype() -> str:
    import os
    env = os.environ.get("FLAXCHAT_DTYPE")  # same knob as flaxchat/common.py:24-26
    return {"bfloat16": "bf16", "float32": "fp32"}.get(env, env) if env else "bf16"


def as_device_model(model, dtype=None, device=None) -> DeviceModel:
    """DeviceModel for `model` (uploaded once per (model, dtype, device))."""
    if isinstance(model, DeviceModel):
        return model
    dtype = dtype or _env_dtype()
    device = device or default_device()
    per = _DEVICE_MODELS.setdefault(model, {})
    key = (str(dtype), str(device))
    if key not in per:
        per[key] = DeviceModel.from_host(model, dtype=dtype, device=device)
    return per[key]


def _batch(tokens):
    """(rows, single) from the accepted token argument forms."""
    if isinstance(tokens, torch.Tensor):
        tokens = tokens.detach().cpu().numpy()
    if isinstance(tokens, np.ndarray):
        if tokens.ndim == 1:
            return [tokens.astype(np.int64).tolist()], True
        return [r.astype(np.int64).tolist() for r in tokens], False
    tokens = list(tokens)
    if len(tokens) and isinstance(tokens[0], (list, tuple, np.ndarray)):
        return [list(map(int, r)) for r in tokens], False
    return [list(map(int, tokens))], True


def _check_rows(rows, V):
    for r in rows:
        if len(r) == 0:
            raise ValueError("empty prompt")
        if min(r) < 0 or max(r) >= V:
            raise ValueError(f"token id outside [0, {V})")


class SpecSession:
    """Device state of one batched speculative-decoding call.

    Every round has the same launch shapes (chunks are packed and sized for
    their capacities), so the first eager round is followed by one captured
    graph that every later round replays. The host keeps `depth` rounds in
    flight: each round's result record is copied to its own pinned slot, and
    round r is read while round r + 1 runs. A row whose rollback needs more
    than FC_PMAX re-fed tokens stalls on the device: it drafts nothing and
    re-feeds FC_PMAX tokens of its backlog per round (its round counter does
    not move) until both caches have caught up; the host is not involved.
    """

    def __init__(self, target: DeviceModel, draft: DeviceModel, rows: List[List[int]], max_tokens: int,
                 temperature: float, top_k: Optional[int], seed: int, draft_steps: int,
                 use_graph: bool = True, stream: Optional[torch.cuda.Stream] = None, depth: int = 2):
        if target.V != draft.V:
            raise VocabMismatchError("Main and draft models must share the same vocabulary size")
        if draft_steps < 1 or draft_steps > 16:
            raise ValueError("draft_steps must be in 1..16")
        if target.dtype != draft.dtype:
            raise ValueError("main and draft models must use the same dtype")
        _check_rows(rows, target.V)
        self.T, self.Dm = target, draft
        self.rows = rows
        self.B = B = len(rows)
        self.k = k = int(draft_steps)
        self.max_tokens = int(max_tokens)
        self.temperature = float(temperature)
        self.top_k = int(top_k) if top_k is not None and top_k > 0 else 0
        self.seed = int(seed) & 0xFFFFFFFFFFFFFFFF
        self.use_graph = use_graph
        self.depth = max(1, int(depth))
        self.dev = dev = target.device
        self.stream = stream or torch.cuda.Stream(device=dev)
        P = max(len(r) for r in rows)
        self.cap = P + self.max_tokens + 2 * k + 8
        self.gen_cap = self.cap
        for dm in (target, draft):
            rope = dm.t["rope_cos"].shape[0]
            if self.cap > rope:
                raise ValueError(f"sequence of {self.cap} positions exceeds the RoPE table ({rope})")
        V = target.V
        i32 = dict(dtype=torch.int32, device=dev)
        with torch.cuda.stream(self.stream):
            self.tcache = DeviceCache(target, B, self.cap)
            self.dcache = DeviceCache(draft, B, self.cap)
            z = lambda *s: torch.zeros(*s, **i32)
            self.bufs = dict(
                t_len=z(B), d_len=z(B), t_pend=z(B, PMAX), d_pend=z(B, PMAX), t_pend_n=z(B), d_pend_n=z(B),
                t_dirty=torch.full((B,), _BIG_POS, **i32), d_dirty=torch.full((B,), _BIG_POS, **i32),
                gen=z(B, self.gen_cap), gen_n=z(B), prompt_len=z(B), round=z(B), stall=z(B),
                result=z(B, RES_STRIDE),
                tok_d0=z(B * PMAX), off_d0=z(B + 1), start_d=z(k, B), tok_ds=z(k, B), off_ds=z(B + 1),
                tok_v=z(B * (PMAX + k)), off_v=z(B + 1), start_v=z(B), drafts=z(B, k),
                q_logits=torch.zeros(B, k, V, dtype=torch.float32, device=dev),
                p_logits=torch.zeros(B, k + 1, V, dtype=torch.float32, device=dev),
                q_stats=torch.zeros(B * k * ctypes.sizeof(FcRowstat), dtype=torch.uint8, device=dev),
                p_stats=torch.zeros(B * (k + 1) * ctypes.sizeof(FcRowstat), dtype=torch.uint8, device=dev),
                part=torch.zeros(lib().fc_spec_part_bytes(B, k, V), dtype=torch.uint8, device=dev))
        self.state = FcSpecState(B, k, self.max_tokens, self.gen_cap, V, self.temperature, self.top_k, self.seed,
                                 *[self.bufs[n].data_ptr() for n in _lib._SPEC_PTRS],
                                 self.bufs["part"].data_ptr(), self.bufs["part"].numel())
        self.ws = Workspace(dev)          # captured by the round graph: never reallocated after capture
        self.ws_prefill = Workspace(dev)
        nb = lib().fc_spec_workspace_bytes(ctypes.byref(target.desc), ctypes.byref(draft.desc), B, k)
        if nb < 0:
            raise RuntimeError("fc_spec_workspace_bytes failed")
        with torch.cuda.stream(self.stream):
            self.ws.get(nb)
        self.graph = None
        self.launched = 0
        self.res_h = [torch.empty(B, RES_STRIDE, dtype=torch.int32, pin_memory=True) for _ in range(self.depth)]
        self.rounds = 0
        self.accept_hist = []
        self.stalls = 0         # rollbacks longer than FC_PMAX (row stalled to re-feed)
        self.refeed_rounds = 0  # row-rounds spent re-feeding such a backlog

    # ------------------------------------------------------------ phases
    def prefill(self):
        b = self.bufs
        with torch.cuda.stream(self.stream):
            for dm, cache in ((self.T, self.tcache), (self.Dm, self.dcache)):
                prefill_rows(dm, cache, [r[:-1] for r in self.rows], [0] * self.B, self.ws_prefill)
            P = np.array([len(r) for r in self.rows], np.int32)
            last = np.array([r[-1] for r in self.rows], np.int32)
            gen = np.zeros((self.B, self.gen_cap), np.int32)
            for i, r in enumerate(self.rows):
                gen[i, :len(r)] = r
            pend = np.zeros((self.B, PMAX), np.int32)
            pend[:, 0] = last
            b["t_len"].copy_(torch.from_numpy(P - 1))
            b["d_len"].copy_(torch.from_numpy(P - 1))
            b["t_pend"].copy_(torch.from_numpy(pend))
            b["d_pend"].copy_(torch.from_numpy(pend))
            b["t_pend_n"].fill_(1)
            b["d_pend_n"].fill_(1)
            b["gen"].copy_(torch.from_numpy(gen))
            b["gen_n"].copy_(torch.from_numpy(P))
            b["prompt_len"].copy_(torch.from_numpy(P))

    def _round_call(self):
        buf = self.ws.buf
        check(lib().fc_spec_round(ctypes.byref(self.T.desc), ctypes.byref(self.tcache.desc),
                                  ctypes.byref(self.Dm.desc), ctypes.byref(self.dcache.desc),
                                  ctypes.byref(self.state), buf.data_ptr(), buf.numel(),
                                  self.stream.cuda_stream), "fc_spec_round")

    def launch_round(self):
        """Enqueue one round: replay the graph, capture it on the second
        round, or run the first round eagerly."""
        s = self.stream.cuda_stream
        if self.graph is not None:
            check(lib().fc_graph_launch(self.graph, s), "fc_graph_launch")
        elif self.use_graph and self.launched >= 1:
            check(lib().fc_graph_begin(s), "fc_graph_begin")
            try:
                self._round_call()
            finally:
                ex = ctypes.c_void_p()
                rc = lib().fc_graph_end(s, ctypes.byref(ex))
            check(rc, "fc_graph_end")
            self.graph = ex
            check(lib().fc_graph_launch(self.graph, s), "fc_graph_launch")
        else:
            self._round_call()
        self.launched += 1

    def _record(self, res) -> int:
        active = res[:, 4] > 0
        if active.any():
            self.rounds += 1
            self.accept_hist.append(res[active, 1].copy())
        self.stalls += int(((res[:, 3] & 1) != 0).sum())
        self.refeed_rounds += int(((res[:, 3] & 8) != 0).sum())
        return int(np.bitwise_or.reduce(res[:, 3]))

    def run(self, max_rounds: Optional[int] = None):
        """Run rounds until every row has max_tokens (or max_rounds rounds)."""
        inflight = deque()
        n = 0
        stop = False
        while True:
            while not stop and len(inflight) < self.depth:
                slot = self.launched % self.depth
                with torch.cuda.stream(self.stream):
                    self.launch_round()
                    self.res_h[slot].copy_(self.bufs["result"], non_blocking=True)
                    ev = torch.cuda.Event()
                    ev.record(self.stream)
                inflight.append((ev, slot))
                n += 1
                if max_rounds is not None and n >= max_rounds:
                    stop = True
            if not inflight:
                break
            ev, slot = inflight.popleft()
            ev.synchronize()
            res = self.res_h[slot].numpy().copy()
            self._record(res)
            if ((res[:, 3] & 4) != 0).all():
                stop = True

    def outputs(self) -> List[List[int]]:
        self.stream.synchronize()
        gen = self.bufs["gen"].cpu().numpy()
        return [gen[i, :len(r) + self.max_tokens].tolist() for i, r in enumerate(self.rows)]

    def emitted_tokens(self) -> int:
        self.stream.synchronize()
        gen_n = self.bufs["gen_n"].cpu().numpy()
        P = np.array([len(r) for r in self.rows])
        return int(np.minimum(gen_n - P, self.max_tokens).sum())

    def close(self):
        if self.graph is not None:
            lib().fc_graph_destroy(self.graph)
            self.graph = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def generate_speculative(model, draft_model, tokens, max_tokens=256, temperature=1.0, top_k=40, seed=42,
                         draft_steps=4, *, dtype=None, device=None, use_graph=True):
    """Speculative decoding (flaxchat/engine.py:410-608) on the HIP engine.

    Returns prompt + generated tokens, truncated to len(prompt) + max_tokens,
    per row; a single prompt returns a single list like the reference.
    """
    target = as_device_model(model, dtype, device)
    draft = as_device_model(draft_model, dtype or ("bf16" if target.dtype else "fp32"), target.device)
    if target.V != draft.V:
        raise VocabMismatchError("Main and draft models must share the same vocabulary size")
    rows, single = _batch(tokens)
    if max_tokens <= 0:
        out = [list(r) for r in rows]
        return out[0] if single else out
    s = SpecSession(target, draft, rows, max_tokens, temperature, top_k, seed, draft_steps, use_graph=use_graph)
    try:
        s.prefill()
        s.run()
        out = s.outputs()
    finally:
        s.close()
    return out[0] if single else out


class FastSession:
    """Device state of one batched generate_fast call (flaxchat/engine.py:259-376)."""

    def __init__(self, dm: DeviceModel, rows, max_tokens, temperature, top_k, seed, eos_token,
                 use_graph=True, stream=None):
        _check_rows(rows, dm.V)
        self.dm, self.rows = dm, rows
        self.B = B = len(rows)
        self.max_tokens = int(max_tokens)
        self.temperature, self.top_k = float(temperature), int(top_k)
        self.seed = int(seed) & 0xFFFFFFFFFFFFFFFF
        self.eos = int(eos_token)
        self.use_graph = use_graph
        dev = dm.device
        self.stream = stream or torch.cuda.Stream(device=dev)
        P = max(len(r) for r in rows)
        self.cap = P + self.max_tokens + 8
        if self.cap > dm.t["rope_cos"].shape[0]:
            raise ValueError("sequence exceeds the RoPE table")
        i32 = dict(dtype=torch.int32, device=dev)
        with torch.cuda.stream(self.stream):
            self.cache = DeviceCache(dm, B, self.cap)
            self.gen = torch.zeros(B, self.cap, **i32)
            self.pos = torch.zeros(B, **i32)
            self.done = torch.zeros(B, **i32)
            self.step = torch.zeros(B, **i32)
            self.max_pos = torch.zeros(B, **i32)
            self.tok = torch.zeros(B, **i32)
            self.row_off = torch.arange(B + 1, **i32)
            self.logits = torch.zeros(B, dm.V, dtype=torch.float32, device=dev)
            self.stats = torch.zeros(B * ctypes.sizeof(FcRowstat), dtype=torch.uint8, device=dev)
        self.ws = Workspace(dev)
        self.ws_pre = Workspace(dev)
        nb = lib().fc_forward_workspace_bytes(ctypes.byref(dm.desc), B, B, 1, B)
        with torch.cuda.stream(self.stream):
            self.ws.get(nb)
        self.graph = None
        self.steps_run = 0

    def prefill(self):
        with torch.cuda.stream(self.stream):
            prefill_rows(self.dm, self.cache, [r[:-1] for r in self.rows], [0] * self.B, self.ws_pre)
            P = np.array([len(r) for r in self.rows], np.int32)
            gen = np.zeros((self.B, self.cap), np.int32)
            for i, r in enumerate(self.rows):
                gen[i, :len(r)] = r
            self.gen.copy_(torch.from_numpy(gen))
            self.pos.copy_(torch.from_numpy(P - 1))
            self.tok.copy_(torch.from_numpy(np.array([r[-1] for r in self.rows], np.int32)))
            self.max_pos.copy_(torch.from_numpy(P + self.max_tokens - 1))

    def _step_call(self):
        s = self.stream.cuda_stream
        forward_packed(self.dm, self.cache, self.tok, self.row_off, self.pos, 1, 1, self.logits, self.ws, s)
        check(lib().fc_fast_sample(self.logits.data_ptr(), self.B, self.dm.V, self.temperature, self.top_k,
                                   self.seed, self.eos, self.gen.data_ptr(), self.cap, self.pos.data_ptr(),
                                   self.done.data_ptr(), self.step.data_ptr(), self.max_pos.data_ptr(),
                                   self.tok.data_ptr(), self.stats.data_ptr(), s), "fc_fast_sample")

    def launch_step(self):
        s = self.stream.cuda_stream
        if self.graph is not None:
            check(lib().fc_graph_launch(self.graph, s), "fc_graph_launch")
        elif self.use_graph and self.steps_run >= 1:
            check(lib().fc_graph_begin(s), "fc_graph_begin")
            try:
                self._step_call()
            finally:
                ex = ctypes.c_void_p()
                rc = lib().fc_graph_end(s, ctypes.byref(ex))
            check(rc, "fc_graph_end")
            self.graph = ex
            check(lib().fc_graph_launch(self.graph, s), "fc_graph_launch")
        else:
            self._step_call()
        self.steps_run += 1

    def run(self, check_every: int = 16):
        left = self.max_tokens
        while left > 0:
            n = min(check_every, left)
            with torch.cuda.stream(self.stream):
                for _ in range(n):
                    self.launch_step()
            left -= n
            self.stream.synchronize()
            done = self.done.cpu().numpy()
            pos = self.pos.cpu().numpy()
            if np.all((done != 0) | (pos >= self.max_pos.cpu().numpy())):
                break

    def outputs(self, truncate_eos: bool = True):
        self.stream.synchronize()
        gen = self.gen.cpu().numpy()
        pos = self.pos.cpu().numpy()
        out = []
        for i, r in enumerate(self.rows):
            n = min(int(pos[i]) + 1, len(r) + self.max_tokens) if truncate_eos else len(r) + self.max_tokens
            out.append(gen[i, :n].tolist())
        return out

    def close(self):
        if self.graph is not None:
            lib().fc_graph_destroy(self.graph)
            self.graph = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def generate_fast(model, tokens, max_tokens=256, temperature=1.0, top_k=40, seed=42, eos_token=0, *,
                  dtype=None, device=None, use_graph=True):
    """generate_fast (flaxchat/engine.py:259-376): top-k sampling (greedy when
    temperature <= 0) until eos_token or max_tokens; the EOS token is kept."""
    if top_k is None:
        raise TypeError("generate_fast requires an integer top_k (flaxchat/engine.py:310)")
    dm = as_device_model(model, dtype, device)
    rows, single = _batch(tokens)
    if max_tokens <= 0:
        out = [list(r) for r in rows]
        return out[0] if single else out
    s = FastSession(dm, rows, max_tokens, temperature, min(int(top_k), dm.V), seed, eos_token, use_graph)
    try:
        s.prefill()
        s.run()
        out = s.outputs()
    finally:
        s.close()
    return out[0] if single else out


def generate_with_cache(model, tokens, max_tokens=256, temperature=1.0, top_k=40, seed=42, *, dtype=None,
                        device=None):
    """generate_with_cache (flaxchat/engine.py:209-253): max_tokens top-k
    samples (argmax when temperature <= 0), no EOS stop."""
    if top_k is None:
        raise TypeError("generate_with_cache requires an integer top_k (flaxchat/engine.py:237)")
    dm = as_device_model(model, dtype, device)
    rows, single = _batch(tokens)
    s = FastSession(dm, rows, max_tokens, temperature, min(int(top_k), dm.V), seed, -1)
    try:
        s.prefill()
        s.run()
        out = s.outputs(truncate_eos=False)
    finally:
        s.close()
    return out[0] if single else out


# ---------------------------------------------------------------------------
# Calculator tool and per-row tool-use state (flaxchat/engine.py:614-658)
# ---------------------------------------------------------------------------
_CALC_CHARS = frozenset("0123456789*+-/.() ")
_CALC_OPS = {ast.Add: operator.add, ast.Sub: operator.sub, ast.Mult: operator.mul, ast.Div: operator.truediv,
             ast.FloorDiv: operator.floordiv, ast.Mod: operator.mod}
# 'literal'.count('literal'): letters/digits/underscore/space in the string,
# one word in the argument (the form flaxchat/engine.py:636-640 accepts)
_COUNT_FORM = re.compile(r"""['"]([\w\s]+)['"]\s*\.\s*count\s*\(\s*['"](\w+)['"]\s*\)""")


def _calc_node(node):
    if isinstance(node, ast.Expression):
        return _calc_node(node.body)
    if isinstance(node, ast.Constant):
        return node.value
    if isinstance(node, ast.UnaryOp) and isinstance(node.op, ast.USub):
        return -_calc_node(node.operand)
    if isinstance(node, ast.BinOp) and type(node.op) in _CALC_OPS:
        return _CALC_OPS[type(node.op)](_calc_node(node.left), _calc_node(node.right))
    raise ValueError("not a calculator expression")


def use_calculator(expr: str):
    """The reference's calculator tool (flaxchat/engine.py:614-643): commas
    are dropped; an expression of digits, + - * / // ( ) . and spaces (no
    ``**``) is evaluated by walking its syntax tree (numbers, unary minus and
    the binary operators only; nothing is compiled or executed), or
    ``'text'.count('word')`` is counted. Anything else, or an arithmetic
    error, gives None."""
    expr = expr.replace(",", "")
    if all(ch in _CALC_CHARS for ch in expr):
        if "**" in expr:
            return None
        try:
            return _calc_node(ast.parse(expr, mode="eval"))
        except Exception:
            return None
    m = _COUNT_FORM.fullmatch(expr)
    if m:
        return m.group(1).count(m.group(2))
    return None


@dataclass
class RowState:
    """Per-row state of Engine.generate (flaxchat/engine.py:649-658)."""
    current_tokens: List[int] = field(default_factory=list)
    forced_tokens: deque = field(default_factory=deque)
    in_python_block: bool = False
    python_expr_tokens: List[int] = field(default_factory=list)
    completed: bool = False


class ToolUse:
    """Host side of Engine.generate's tool protocol
    (flaxchat/engine.py:742-749, 786-822): the special token ids, and the
    transition of one row on its next token: completion on assistant_end or
    bos; tokens between python_start and python_end are decoded and
    evaluated (calculator, then `code_executor`), and the result is queued
    as output_start + tokens + output_end."""

    def __init__(self, tokenizer, code_executor: Optional[Callable] = None):
        sp = tokenizer.encode_special
        self.tokenizer = tokenizer
        self.python_start, self.python_end = sp("<|python_start|>"), sp("<|python_end|>")
        self.output_start, self.output_end = sp("<|output_start|>"), sp("<|output_end|>")
        self.assistant_end = sp("<|assistant_end|>")
        self.bos = tokenizer.get_bos_token_id()
        self.code_executor = code_executor

    def evaluate(self, expr: str) -> str:
        result = use_calculator(expr)
        if result is not None:
            return str(result)
        if self.code_executor is not None:
            r = self.code_executor(expr)
            if r.success:
                return r.stdout.rstrip("\n")
        return "Error"

    def next_token(self, state: RowState, sampled: int) -> Tuple[int, int]:
        """The row's token for this step (the head of its forced queue, else
        `sampled`) and its mask (0 forced, 1 sampled); updates the state."""
        forced = len(state.forced_tokens) > 0
        tok = state.forced_tokens.popleft() if forced else int(sampled)
        state.current_tokens.append(tok)
        if tok == self.assistant_end or tok == self.bos:
            state.completed = True
        if tok == self.python_start:
            state.in_python_block = True
            state.python_expr_tokens = []
        elif tok == self.python_end and state.in_python_block:
            state.in_python_block = False
            if state.python_expr_tokens:
                out = self.tokenizer.encode(self.evaluate(self.tokenizer.decode(state.python_expr_tokens)))
                state.forced_tokens.append(self.output_start)
                state.forced_tokens.extend(int(t) for t in out)
                state.forced_tokens.append(self.output_end)
            state.python_expr_tokens = []
        elif state.in_python_block:
            state.python_expr_tokens.append(tok)
        return tok, 0 if forced else 1


class StreamSession:
    """Device state of Engine.generate (flaxchat/engine.py:686-838): the
    prompt is prefilled once and copied into `num_samples` rows; each step
    picks a forced or sampled token per row on the device (fc_engine_sample),
    copies the column to the host, and feeds it, so the next forward runs
    while the host applies the tool protocol to this column."""

    def __init__(self, dm: DeviceModel, tokens: List[int], num_samples: int, steps: int, temperature: float,
                 top_k: Optional[int], seed: int, use_graph: bool = True, stream=None):
        _check_rows([tokens], dm.V)
        if num_samples < 1:
            raise ValueError("num_samples must be >= 1")
        self.dm, self.tokens = dm, list(tokens)
        self.B = B = int(num_samples)
        self.temperature = float(temperature)
        self.top_k = min(int(top_k), dm.V) if top_k is not None and top_k > 0 else 0
        self.seed = int(seed) & 0xFFFFFFFFFFFFFFFF
        self.use_graph = use_graph
        dev = dm.device
        self.stream = stream or torch.cuda.Stream(device=dev)
        P = len(tokens)
        self.cap = P + int(steps) + 8
        if self.cap > dm.t["rope_cos"].shape[0]:
            raise ValueError("sequence exceeds the RoPE table")
        i32 = dict(dtype=torch.int32, device=dev)
        with torch.cuda.stream(self.stream):
            self.cache = DeviceCache(dm, B, self.cap)
            self.gen = torch.zeros(B, self.cap, **i32)
            self.pos = torch.full((B,), P - 1, **i32)
            self.step = torch.zeros(B, **i32)
            self.tok = torch.full((B,), int(tokens[-1]), **i32)
            self.forced = torch.full((B,), -1, **i32)
            self.row_off = torch.arange(B + 1, **i32)
            self.logits = torch.zeros(B, dm.V, dtype=torch.float32, device=dev)
            self.stats = torch.zeros(B * ctypes.sizeof(FcRowstat), dtype=torch.uint8, device=dev)
        self.forced_host = torch.full((B,), -1, dtype=torch.int32).pin_memory()
        self.tok_host = torch.zeros(B, dtype=torch.int32).pin_memory()
        self.event = torch.cuda.Event()
        self.ws = Workspace(dev)
        self.ws_pre = Workspace(dev)
        nb = lib().fc_forward_workspace_bytes(ctypes.byref(dm.desc), B, B, 1, B)
        with torch.cuda.stream(self.stream):
            self.ws.get(nb)
        self.graph = None
        self.forwards = 0

    def _forward(self):
        forward_packed(self.dm, self.cache, self.tok, self.row_off, self.pos, 1, 1, self.logits, self.ws,
                       self.stream.cuda_stream)

    def _launch_forward(self):
        s = self.stream.cuda_stream
        if self.graph is not None:
            check(lib().fc_graph_launch(self.graph, s), "fc_graph_launch")
        elif self.use_graph and self.forwards >= 1:
            check(lib().fc_graph_begin(s), "fc_graph_begin")
            try:
                self._forward()
            finally:
                ex = ctypes.c_void_p()
                rc = lib().fc_graph_end(s, ctypes.byref(ex))
            check(rc, "fc_graph_end")
            self.graph = ex
            check(lib().fc_graph_launch(self.graph, s), "fc_graph_launch")
        else:
            self._forward()
        self.forwards += 1

    def prefill(self):
        """Prefill row 0 with the prompt, copy its cache into every row, and
        compute the logits after the last prompt token."""
        with torch.cuda.stream(self.stream):
            prefill_rows(self.dm, self.cache, [self.tokens[:-1]] + [[]] * (self.B - 1), [0] * self.B, self.ws_pre)
            c = self.cache
            if self.B > 1:
                c.k[:, 1:] = c.k[:, :1]
                c.v[:, 1:] = c.v[:, :1]
                c.hist[1:] = c.hist[:1]
            self.gen[:, :len(self.tokens)] = torch.tensor(self.tokens, dtype=torch.int32, device=self.gen.device)
            self._launch_forward()

    def next_column(self, forced: Sequence[int]) -> List[int]:
        """One column: row b takes forced[b] when >= 0, else a sample; the
        forward of the chosen column is queued before this returns."""
        self.forced_host.numpy()[:] = forced
        s = self.stream.cuda_stream
        with torch.cuda.stream(self.stream):
            self.forced.copy_(self.forced_host, non_blocking=True)
            check(lib().fc_engine_sample(self.logits.data_ptr(), self.B, self.dm.V, self.temperature, self.top_k,
                                         self.seed, self.forced.data_ptr(), self.gen.data_ptr(), self.cap,
                                         self.pos.data_ptr(), self.step.data_ptr(), self.tok.data_ptr(),
                                         self.stats.data_ptr(), s), "fc_engine_sample")
            self.tok_host.copy_(self.tok, non_blocking=True)
            self.event.record(self.stream)
            self._launch_forward()
        self.event.synchronize()
        return self.tok_host.numpy().tolist()

    def close(self):
        if self.graph is not None:
            lib().fc_graph_destroy(self.graph)
            self.graph = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---------------------------------------------------------------------------
# Full-sequence forward: GPT.__call__ (flaxchat/gpt.py:407-454)
# ---------------------------------------------------------------------------
_FULL_CHUNK = 1024  # tokens per row per forward chunk (the embed kernel's limit)


def gpt_forward(model, idx, targets=None, *, dtype=None, device=None, chunk: int = _FULL_CHUNK):
    """GPT.__call__(idx, targets=None) on the HIP engine (flaxchat/gpt.py:407-454).

    idx: [B, T] token ids (list of lists, array or tensor). Returns the
    softcapped fp32 logits [B, T, vocab] as a device tensor or, with
    targets [B, T] (entries < 0 are masked), the mean cross-entropy over the
    unmasked positions as a 0-d device tensor. The forward is the engine's
    packed-chunk forward over all positions (chunks of up to `chunk` tokens
    per row, each position's logits kept), with the full-sequence smear
    (gate_t * n_{t-1}, FC_CHUNK_FULL_SMEAR) instead of the decode one."""
    dm = as_device_model(model, dtype, device)
    dev = dm.device
    ids = torch.as_tensor(np.asarray(idx.cpu() if torch.is_tensor(idx) else idx), dtype=torch.int32)
    if ids.dim() != 2 or ids.shape[1] == 0:
        raise ValueError("idx must be [B, T] with T >= 1")
    B, T = ids.shape
    if int(ids.min()) < 0 or int(ids.max()) >= dm.V:
        raise ValueError(f"token ids must be in [0, {dm.V})")
    if T > dm.t["rope_cos"].shape[0]:
        raise ValueError("sequence exceeds the RoPE table")
    chunk = max(1, min(int(chunk), _FULL_CHUNK))
    cache = DeviceCache(dm, B, T)
    ws = Workspace(dev)
    logits = torch.empty(B, T, dm.V, dtype=torch.float32, device=dev)
    ids_dev = ids.to(dev)
    for c0 in range(0, T, chunk):
        n = min(chunk, T - c0)
        tok = ids_dev[:, c0:c0 + n].contiguous().view(-1)
        off = torch.arange(0, B * n + 1, n, dtype=torch.int32, device=dev)
        start = torch.full((B,), c0, dtype=torch.int32, device=dev)
        forward_packed(dm, cache, tok, off, start, n, n, logits[:, c0:], ws, logits_stride=T * dm.V,
                       flags=_lib.FC_CHUNK_FULL_SMEAR)
    if targets is None:
        return logits
    tgt = torch.as_tensor(np.asarray(targets.cpu() if torch.is_tensor(targets) else targets), dtype=torch.int32)
    if tuple(tgt.shape) != (B, T):
        raise ValueError("targets must have the shape of idx")
    if int(tgt.max()) >= dm.V:
        raise ValueError(f"targets must be < {dm.V} (negative entries are masked)")
    tgt_dev = tgt.to(dev).contiguous().view(-1)
    loss = torch.empty(B * T, dtype=torch.float32, device=dev)
    s = torch.cuda.current_stream(dev).cuda_stream
    check(lib().fc_cross_entropy(logits.data_ptr(), dm.V, tgt_dev.data_ptr(), B * T, dm.V, loss.data_ptr(), s),
          "fc_cross_entropy")
    mask = (tgt_dev >= 0).float()
    return loss.sum() / torch.clamp(mask.sum(), min=1.0)


class Engine:
    """The reference Engine (flaxchat/engine.py:661-908): streaming
    generation with tool use, and the fast / speculative decode entry points.
    `code_executor(code) -> result with .success and .stdout` runs Python
    blocks the calculator cannot (the reference's sandboxed execute_code,
    flaxchat/execution.py:190)."""

    def __init__(self, model, tokenizer=None, *, dtype=None, device=None, code_executor=None):
        self.model = model
        self.tokenizer = tokenizer
        self.dtype, self.device = dtype, device
        self.code_executor = code_executor

    def generate(self, tokens, num_samples=1, max_tokens=None, temperature=1.0, top_k=40,
                 seed=42) -> Iterator[Tuple[List[int], List[int]]]:
        """Yields (token_column, token_masks) per step, one entry per sample
        (flaxchat/engine.py:686-838): 1 = sampled, 0 = forced tool output.
        Stops after max_tokens steps (256 when None) or when every row has
        emitted assistant_end or bos; completed rows keep sampling until
        then, as in the reference."""
        assert isinstance(tokens, list) and isinstance(tokens[0], int), "expecting list of ints"
        assert temperature >= 0.0, "temperature must be non-negative"
        if self.tokenizer is None:
            raise ValueError("Engine.generate needs a tokenizer (special tokens of the tool protocol)")
        tool = ToolUse(self.tokenizer, self.code_executor)
        dm = as_device_model(self.model, self.dtype, self.device)
        steps = 256 if max_tokens is None else int(max_tokens)
        if steps <= 0:
            return
        sess = StreamSession(dm, tokens, num_samples, steps, temperature, top_k, seed)
        rows = [RowState(list(tokens)) for _ in range(num_samples)]
        try:
            sess.prefill()
            for _ in range(steps):
                if all(r.completed for r in rows):
                    break
                forced = [r.forced_tokens[0] if r.forced_tokens else -1 for r in rows]
                for f in forced:
                    if f >= dm.V:
                        raise ValueError(f"tool output token {f} is outside the vocabulary ({dm.V})")
                sampled = sess.next_column(forced)
                column, masks = [], []
                for r, t in zip(rows, sampled):
                    tok, mask = tool.next_token(r, t)
                    column.append(tok)
                    masks.append(mask)
                yield column, masks
        finally:
            sess.close()

    def generate_batch(self, tokens, num_samples=1, **kwargs):
        """Final sequences and masks (flaxchat/engine.py:840-864): prompt
        plus generated tokens up to, not including, assistant_end / bos;
        mask 0 for prompt and forced tokens, 1 for sampled ones."""
        tool_end = self.tokenizer.encode_special("<|assistant_end|>")
        bos = self.tokenizer.get_bos_token_id()
        results = [list(tokens) for _ in range(num_samples)]
        masks = [[0] * len(tokens) for _ in range(num_samples)]
        completed = [False] * num_samples
        for column, cmask in self.generate(tokens, num_samples, **kwargs):
            for i, (tok, m) in enumerate(zip(column, cmask)):
                if completed[i]:
                    continue
                if tok == tool_end or tok == bos:
                    completed[i] = True
                else:
                    results[i].append(tok)
                    masks[i].append(m)
            if all(completed):
                break
        return results, masks

    def generate_text(self, prompt, max_tokens=256, temperature=1.0, top_k=40, seed=42):
        """Decoded text of one streamed sample (flaxchat/engine.py:866-874)."""
        tokens = self.tokenizer(prompt, prepend="<|bos|>")
        results, _ = self.generate_batch(tokens, num_samples=1, max_tokens=max_tokens, temperature=temperature,
                                         top_k=top_k, seed=seed)
        return self.tokenizer.decode(results[0])

    def generate_fast(self, tokens, max_tokens=256, temperature=1.0, top_k=40, seed=42, eos_token=0):
        return generate_fast(self.model, tokens, max_tokens=max_tokens, temperature=temperature, top_k=top_k,
                             seed=seed, eos_token=eos_token, dtype=self.dtype, device=self.device)

    def generate_speculative(self, draft_model, tokens, max_tokens=256, temperature=1.0, top_k=40, seed=42,
                             draft_steps=4):
        return generate_speculative(self.model, draft_model, tokens, max_tokens=max_tokens,
                                    temperature=temperature, top_k=top_k, seed=seed, draft_steps=draft_steps,
                                    dtype=self.dtype, device=self.device)
