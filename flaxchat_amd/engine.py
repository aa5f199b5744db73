"""Speculative and fast decoding on the HIP engine, with the reference's call
surface (flaxchat/engine.py:259-260, 410-411, 877-908).

    generate_speculative(model, draft_model, tokens, max_tokens=256,
                         temperature=1.0, top_k=40, seed=42, draft_steps=4)
    generate_fast(model, tokens, max_tokens=256, temperature=1.0, top_k=40,
                  seed=42, eos_token=0)
    generate_with_cache(model, tokens, max_tokens=256, temperature=1.0,
                        top_k=40, seed=42)

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
  * temperature < 0 behaves as greedy.
"""

from __future__ import annotations

import ctypes
import weakref
from collections import deque
from typing import List, Optional, Sequence, Union

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


class Engine:
    """The reference Engine's decode entry points (flaxchat/engine.py:877-908)."""

    def __init__(self, model, tokenizer=None, *, dtype=None, device=None):
        self.model = model
        self.tokenizer = tokenizer
        self.dtype, self.device = dtype, device

    def generate_fast(self, tokens, max_tokens=256, temperature=1.0, top_k=40, seed=42, eos_token=0):
        return generate_fast(self.model, tokens, max_tokens=max_tokens, temperature=temperature, top_k=top_k,
                             seed=seed, eos_token=eos_token, dtype=self.dtype, device=self.device)

    def generate_speculative(self, draft_model, tokens, max_tokens=256, temperature=1.0, top_k=40, seed=42,
                             draft_steps=4):
        return generate_speculative(self.model, draft_model, tokens, max_tokens=max_tokens,
                                    temperature=temperature, top_k=top_k, seed=seed, draft_steps=draft_steps,
                                    dtype=self.dtype, device=self.device)
