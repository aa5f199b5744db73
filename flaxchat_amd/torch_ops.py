"""The C-ABI kernels as PyTorch operators: ``torch.ops.flaxchat_mi355x.*``.

Importing this module registers the namespace (``torch.library.custom_op``),
so code that composes torch tensors can call the hot kernels directly, and
shape propagation (meta / fake tensors) works without a GPU. Each operator
is a thin call of one C-ABI entry point on the current stream of the input's
device; the engine itself (``SpecSession``, ``Engine``) calls the C-ABI
directly and does not go through here.

Operators:
  pack_operand(src)                  bf16 [R][K] row-major -> fragment order [round16(R)][K]
  linear(x, w, softcap=False)        fp32 x @ w^T (nnx.Linear, flaxchat/gpt.py:93-99); softcap applies
                                     15 tanh(z / 15) (flaxchat/engine.py:173-174)
  attention(q, k_cache, v_cache, row_off, start, max_per_row, window)
                                     decode / verify attention over one cache layer
                                     (flaxchat/engine.py:128-156)
  cross_entropy(logits, targets)     per-row logsumexp(z) - z[t], 0 where t < 0
                                     (flaxchat/gpt.py:446-452)

The engine entry points take a model as the address of its fc_model
descriptor (`DeviceModel.desc`, read-only weights that stay alive with the
DeviceModel) and everything they write as tensors, declared mutated:
  forward(model, k_cache, v_cache, hist, tokens, row_off, start, max_per_row, n_out, logits,
          workspace, typ_tokens=0, flags=0)
                                     one packed chunk through the model (fc_forward;
                                     flaxchat/engine.py:51-177, 396-407)
  attn_prologue(model, layer, k_cache, v_cache, qkv, h, tokens, tok_row, tok_pos) -> q
                                     RoPE, QK-norm, VE gate, cache append (engine.py:96-126)
  attn_qkv(model, layer, k_cache, v_cache, h, tokens, tok_row, tok_pos, typ_tokens=0) -> q
                                     the QKV projection with that prologue fused
  row_stats(logits, temperature, top_k) -> (mx, sum, tau, tie_idx, argmax)
                                     top-k keep set and softmax statistics (engine.py:461-476)
  spec_accept(buffers, batch, k, max_tokens, gen_cap, vocab, temperature, top_k, seed)
                                     accept / reject / bonus and the rollback bookkeeping
                                     (engine.py:525-606) on a round's logits
  spec_round(target, draft, t_k, t_v, t_hist, d_k, d_v, d_hist, buffers, batch, k, max_tokens,
             gen_cap, vocab, temperature, top_k, seed, workspace)
                                     one whole speculative round (engine.py:484-606)
`buffers` is the speculative state's device arrays in fc_spec_state order
(`SPEC_BUFFERS`: t_len .. p_stats, then the partials buffer `part`).
"""

from __future__ import annotations

import torch

from . import _lib
from ._lib import check, lib

__all__ = ["pack_operand", "linear", "attention", "cross_entropy", "frag_to_rows", "forward", "attn_prologue",
           "attn_qkv", "row_stats", "spec_accept", "spec_round", "SPEC_BUFFERS"]

NS = "flaxchat_mi355x"


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return _lib.FC_BF16
    if t.dtype == torch.float32:
        return _lib.FC_F32
    raise ValueError(f"flaxchat_mi355x operators take bf16 or fp32 tensors (got {t.dtype})")


def frag_to_rows(t: torch.Tensor, rows: int) -> torch.Tensor:
    """Row-major [rows][K] view of a fragment-order [round16(rows)][K]
    tensor: 16-row x 32-column blocks of 512 elements, element (r, k) of a
    block at ((k % 32) // 8 * 16 + r) * 8 + k % 8."""
    R, K = t.shape
    blk = t.reshape(R // 16, K // 32, 4, 16, 8)          # [row block][k block][k group][row][k % 8]
    return blk.permute(0, 3, 1, 2, 4).reshape(R, K)[:rows]


# ---------------------------------------------------------------- pack_operand
@torch.library.custom_op(f"{NS}::pack_operand", mutates_args=())
def pack_operand(src: torch.Tensor) -> torch.Tensor:
    if src.dtype != torch.bfloat16 or src.dim() != 2 or src.shape[1] % 64 != 0:
        raise ValueError("pack_operand takes a bf16 [R][K] matrix with K % 64 == 0")
    src = src.contiguous()
    R, K = src.shape
    out = torch.empty(((R + 15) // 16 * 16, K), dtype=src.dtype, device=src.device)
    check(lib().fc_pack_operand(src.data_ptr(), out.data_ptr(), R, K, _stream(src)), "fc_pack_operand")
    return out


@pack_operand.register_fake
def _(src):
    return src.new_empty(((src.shape[0] + 15) // 16 * 16, src.shape[1]))


# ---------------------------------------------------------------- linear
@torch.library.custom_op(f"{NS}::linear", mutates_args=())
def linear(x: torch.Tensor, w: torch.Tensor, softcap: bool = False) -> torch.Tensor:
    if x.dim() != 2 or w.dim() != 2 or x.shape[1] != w.shape[1] or x.dtype != w.dtype:
        raise ValueError("linear takes x [M][K] and w [N][K] of one dtype")
    code = _dtype_code(x)
    M, K = x.shape
    N = w.shape[0]
    if code == _lib.FC_BF16:
        if K % 64 != 0 or N % 32 != 0:
            raise ValueError(f"bf16 linear needs K % 64 == 0 and N % 32 == 0 (got K={K}, N={N})")
        a, b = pack_operand(x), pack_operand(w)
    else:
        a, b = x.contiguous(), w.contiguous()
    out = torch.empty((M, N), dtype=torch.float32, device=x.device)
    check(lib().fc_gemm(a.data_ptr(), b.data_ptr(), out.data_ptr(), M, N, K, code, 4 if softcap else 0,
                        _stream(x)), "fc_gemm")
    return out


@linear.register_fake
def _(x, w, softcap=False):
    return x.new_empty((x.shape[0], w.shape[0]), dtype=torch.float32)


# ---------------------------------------------------------------- attention
@torch.library.custom_op(f"{NS}::attention", mutates_args=())
def attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, row_off: torch.Tensor,
              start: torch.Tensor, max_per_row: int, window: int) -> torch.Tensor:
    """q [tokens][H][128] packed by row (row b's queries at row_off[b] ..
    row_off[b+1], at positions start[b] ..); k_cache / v_cache one layer of
    the engine's cache in its layout: k_cache shaped [B][G][cap][128] (bf16:
    32-key blocks in S^T fragment order; fp32: row-major), v_cache with as
    many elements, [B][G][cap / 32][128][32] (any shape of that size);
    window 0 = full causal, else keys with pos - j <= window. Returns
    [tokens][H * 128] in q's dtype, row-major."""
    code = _dtype_code(q)
    if q.dim() != 3 or k_cache.dim() != 4 or v_cache.numel() != k_cache.numel():
        raise ValueError("attention takes q [T][H][hd], k_cache [B][G][cap][hd] and a v_cache of the same size")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("attention: the caches must be contiguous")
    tot, H, hd = q.shape
    B, G, cap, hd2 = k_cache.shape
    if hd != hd2 or H % G != 0 or row_off.numel() != B + 1 or start.numel() != B:
        raise ValueError("attention: head_dim, GQA grouping or row_off / start sizes do not match")
    if k_cache.dtype != q.dtype or v_cache.dtype != q.dtype:
        raise ValueError("attention: q and the caches share one dtype")
    if row_off.dtype != torch.int32 or start.dtype != torch.int32:
        raise ValueError("attention: row_off and start are int32")
    max_keys = min(cap, window + max_per_row) if window > 0 else cap
    nb = lib().fc_attention_workspace_bytes(B, max_per_row, H, G, hd, max_keys)
    ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=q.device)
    rows = (tot + 15) // 16 * 16 if code == _lib.FC_BF16 else tot
    y = torch.empty((max(rows, 1), H * hd), dtype=q.dtype, device=q.device)
    qc = q.contiguous()
    check(lib().fc_attention(qc.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), y.data_ptr(), B, tot,
                             max_per_row, H, G, hd, cap, row_off.data_ptr(), start.data_ptr(), window, max_keys,
                             code, ws.data_ptr(), ws.numel(), _stream(q)), "fc_attention")
    if code == _lib.FC_BF16:
        return frag_to_rows(y, tot).contiguous()
    return y[:tot]


@attention.register_fake
def _(q, k_cache, v_cache, row_off, start, max_per_row, window):
    return q.new_empty((q.shape[0], q.shape[1] * q.shape[2]))


# ---------------------------------------------------------------- cross_entropy
@torch.library.custom_op(f"{NS}::cross_entropy", mutates_args=())
def cross_entropy(logits: torch.Tensor, targets: torch.Tensor) -> torch.Tensor:
    if logits.dtype != torch.float32 or logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("cross_entropy takes fp32 logits [rows][V] with unit column stride")
    rows, V = logits.shape
    t = targets.to(torch.int32).contiguous()
    if t.numel() != rows:
        raise ValueError("cross_entropy: one target per logits row")
    if rows and int(t.max()) >= V:
        raise ValueError("cross_entropy: target id >= vocabulary size")
    loss = torch.empty(rows, dtype=torch.float32, device=logits.device)
    check(lib().fc_cross_entropy(logits.data_ptr(), logits.stride(0), t.data_ptr(), rows, V, loss.data_ptr(),
                                 _stream(logits)), "fc_cross_entropy")
    return loss


@cross_entropy.register_fake
def _(logits, targets):
    return logits.new_empty((logits.shape[0],))


# ---------------------------------------------------------------- engine entry points
import ctypes  # noqa: E402
from typing import List, Tuple  # noqa: E402

SPEC_BUFFERS = list(_lib._SPEC_PTRS) + ["part"]


def _model(addr: int):
    """(descriptor pointer, DeviceModel) of the live DeviceModel whose
    fc_model descriptor sits at host address `addr`. Any other integer (a
    stale address of a collected model, a hand-built descriptor) is refused:
    the kernels would dereference its weight pointers."""
    from .runtime import live_model
    dm = live_model(addr) if addr else None
    if dm is None:
        raise ValueError("model: the descriptor address of a live DeviceModel (ctypes.addressof(DeviceModel.desc))")
    return ctypes.pointer(dm.desc), dm


def _tdt(dm) -> torch.dtype:
    return torch.bfloat16 if dm.dtype == _lib.FC_BF16 else torch.float32


def _same_device(dm, *ts):
    """Every tensor on the model's device (meta / fake tensors carry no
    memory and are checked for shape only)."""
    for t in ts:
        if t is not None and t.device.type != "meta" and t.device != dm.device:
            raise ValueError(f"tensor on {t.device}, the model's weights are on {dm.device}")


def _cache(dm, k_cache: torch.Tensor, v_cache: torch.Tensor, hist: torch.Tensor = None) -> _lib.FcCache:
    """fc_cache over one model's cache tensors, checked against the model:
    k [n_layer][batch][n_kv_head][cap][head_dim] in the model dtype, v of as
    many elements, hist [batch][cap][n_embd] fp32 (or absent)."""
    if k_cache.dim() != 5 or (k_cache.shape[0], k_cache.shape[2], k_cache.shape[4]) != (dm.L, dm.G, dm.hd):
        raise ValueError(f"k_cache [n_layer={dm.L}][batch][n_kv_head={dm.G}][cap][head_dim={dm.hd}] "
                         f"(got {tuple(k_cache.shape)})")
    if v_cache.numel() != k_cache.numel():
        raise ValueError("v_cache must hold as many elements as k_cache")
    if k_cache.dtype != _tdt(dm) or v_cache.dtype != _tdt(dm):
        raise ValueError(f"the caches are {_tdt(dm)} like the model (got {k_cache.dtype} / {v_cache.dtype})")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("the caches must be contiguous")
    B, cap = k_cache.shape[1], k_cache.shape[3]
    if B < 1 or cap % 32 != 0:
        raise ValueError("cache capacity must be a multiple of 32")
    if hist is not None and (hist.dtype != torch.float32 or tuple(hist.shape) != (B, cap, dm.D)
                             or not hist.is_contiguous()):
        raise ValueError(f"hist: contiguous fp32 [batch={B}][cap={cap}][n_embd={dm.D}]")
    _same_device(dm, k_cache, v_cache, hist)
    return _lib.FcCache(k_cache.data_ptr(), v_cache.data_ptr(), hist.data_ptr() if hist is not None else 0, B, cap)


def _i32(*ts):
    for t in ts:
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise ValueError("index arrays are contiguous int32 tensors")


def _gemm_input(dm, h: torch.Tensor, M: int, name: str):
    """h: the RMS-normed GEMM input of M tokens: bf16 in fragment order
    ([round16(M)][n_embd], as the forward writes it) or fp32 row-major."""
    rows = (M + 15) // 16 * 16 if dm.dtype == _lib.FC_BF16 else M
    if h.dtype != _tdt(dm) or h.numel() < rows * dm.D or not h.is_contiguous():
        raise ValueError(f"{name}: h is contiguous {_tdt(dm)} with at least {rows} x {dm.D} elements")


@torch.library.custom_op(f"{NS}::forward", mutates_args=("k_cache", "v_cache", "hist", "logits", "workspace"))
def forward(model: int, k_cache: torch.Tensor, v_cache: torch.Tensor, hist: torch.Tensor, tokens: torch.Tensor,
            row_off: torch.Tensor, start: torch.Tensor, max_per_row: int, n_out: int, logits: torch.Tensor,
            workspace: torch.Tensor, typ_tokens: int = 0, flags: int = 0) -> None:
    m, dm = _model(model)
    c = _cache(dm, k_cache, v_cache, hist)
    _i32(tokens, row_off, start)
    _same_device(dm, tokens, row_off, start, logits, workspace)
    B = c.batch
    if row_off.numel() != B + 1 or start.numel() != B:
        raise ValueError("forward: row_off has batch + 1 entries and start batch")
    V = dm.V
    if n_out > 0 and (logits.dtype != torch.float32 or logits.numel() < B * n_out * V or not logits.is_contiguous()):
        raise ValueError("forward: logits is contiguous fp32 with at least batch * n_out * vocab elements")
    need = lib().fc_forward_workspace_bytes(m, B, tokens.numel(), max_per_row, typ_tokens)
    if need < 0 or workspace.numel() < need:
        raise ValueError(f"forward: workspace of {workspace.numel()} bytes, {need} needed")
    ch = _lib.FcChunk(tokens.numel(), max_per_row, typ_tokens, tokens.data_ptr(), row_off.data_ptr(),
                      start.data_ptr(), n_out, logits.data_ptr() if n_out > 0 else 0, n_out * V, flags)
    check(lib().fc_forward(m, ctypes.byref(c), ctypes.byref(ch), workspace.data_ptr(), workspace.numel(),
                           _stream(tokens)), "fc_forward")


@forward.register_fake
def _(model, k_cache, v_cache, hist, tokens, row_off, start, max_per_row, n_out, logits, workspace, typ_tokens=0,
      flags=0):
    return None


def _q_out(dm, M: int, like: torch.Tensor) -> torch.Tensor:
    return torch.empty((M, dm.H, dm.hd), dtype=_tdt(dm), device=like.device)


@torch.library.custom_op(f"{NS}::attn_prologue", mutates_args=("k_cache", "v_cache"))
def attn_prologue(model: int, layer: int, k_cache: torch.Tensor, v_cache: torch.Tensor, qkv: torch.Tensor,
                  h: torch.Tensor, tokens: torch.Tensor, tok_row: torch.Tensor, tok_pos: torch.Tensor) -> torch.Tensor:
    _i32(tokens, tok_row, tok_pos)
    m, dm = _model(model)
    M = tokens.numel()
    if not 0 <= layer < dm.L:
        raise ValueError(f"attn_prologue: layer {layer} outside [0, {dm.L})")
    nqkv = (dm.H + 2 * dm.G) * dm.hd
    if (qkv.dtype != torch.float32 or qkv.dim() != 2 or qkv.shape[0] < M or qkv.shape[1] != nqkv
            or not qkv.is_contiguous()):
        raise ValueError(f"attn_prologue: qkv is contiguous fp32 [M][{nqkv}]")
    if tok_row.numel() < M or tok_pos.numel() < M:
        raise ValueError("attn_prologue: tok_row / tok_pos hold one entry per token")
    _gemm_input(dm, h, M, "attn_prologue")
    c = _cache(dm, k_cache, v_cache)
    _same_device(dm, qkv, h, tokens, tok_row, tok_pos)
    q = _q_out(dm, M, qkv)
    check(lib().fc_attn_prologue(m, layer, ctypes.byref(c), qkv.data_ptr(), h.data_ptr(),
                                 tokens.data_ptr(), tok_row.data_ptr(), tok_pos.data_ptr(), M, q.data_ptr(),
                                 _stream(qkv)), "fc_attn_prologue")
    return q


def _q_fake(model: int, M, like: torch.Tensor, cache: torch.Tensor) -> torch.Tensor:
    _, dm = _model(model)  # the descriptor is host memory: readable while tracing
    return like.new_empty((M, dm.H, dm.hd), dtype=cache.dtype)


@attn_prologue.register_fake
def _(model, layer, k_cache, v_cache, qkv, h, tokens, tok_row, tok_pos):
    return _q_fake(model, tokens.shape[0], qkv, k_cache)


@torch.library.custom_op(f"{NS}::attn_qkv", mutates_args=("k_cache", "v_cache"))
def attn_qkv(model: int, layer: int, k_cache: torch.Tensor, v_cache: torch.Tensor, h: torch.Tensor,
             tokens: torch.Tensor, tok_row: torch.Tensor, tok_pos: torch.Tensor, typ_tokens: int = 0) -> torch.Tensor:
    _i32(tokens, tok_row, tok_pos)
    M = tokens.numel()
    m, dm = _model(model)
    if not 0 <= layer < dm.L:
        raise ValueError(f"attn_qkv: layer {layer} outside [0, {dm.L})")
    if tok_row.numel() < M or tok_pos.numel() < M:
        raise ValueError("attn_qkv: tok_row / tok_pos hold one entry per token")
    _gemm_input(dm, h, M, "attn_qkv")
    c = _cache(dm, k_cache, v_cache)
    _same_device(dm, h, tokens, tok_row, tok_pos)
    q = _q_out(dm, M, h)
    need = lib().fc_attn_qkv_workspace_bytes(m, M, typ_tokens)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=h.device)
    check(lib().fc_attn_qkv(m, layer, ctypes.byref(c), h.data_ptr(), tokens.data_ptr(), tok_row.data_ptr(),
                            tok_pos.data_ptr(), M, typ_tokens, q.data_ptr(), ws.data_ptr(), ws.numel(), _stream(h)),
          "fc_attn_qkv")
    return q


@attn_qkv.register_fake
def _(model, layer, k_cache, v_cache, h, tokens, tok_row, tok_pos, typ_tokens=0):
    return _q_fake(model, tokens.shape[0], h, k_cache)


@torch.library.custom_op(f"{NS}::row_stats", mutates_args=())
def row_stats(logits: torch.Tensor, temperature: float, top_k: int) -> Tuple[torch.Tensor, torch.Tensor,
                                                                             torch.Tensor, torch.Tensor,
                                                                             torch.Tensor]:
    if logits.dtype != torch.float32 or logits.dim() != 2 or not logits.is_contiguous():
        raise ValueError("row_stats takes contiguous fp32 logits [rows][V]")
    rows, V = logits.shape
    raw = torch.empty((rows, 8), dtype=torch.int32, device=logits.device)
    check(lib().fc_row_stats(logits.data_ptr(), rows, V, temperature, top_k, raw.data_ptr(), _stream(logits)),
          "fc_row_stats")
    f = raw.view(torch.float32)
    return f[:, 0].clone(), f[:, 1].clone(), f[:, 2].clone(), raw[:, 3].clone(), raw[:, 4].clone()


@row_stats.register_fake
def _(logits, temperature, top_k):
    r = logits.shape[0]
    f = lambda: logits.new_empty((r,))  # noqa: E731
    i = lambda: logits.new_empty((r,), dtype=torch.int32)  # noqa: E731
    return f(), f(), f(), i(), i()


_PMAX, _RES_STRIDE, _ROWSTAT = 16, 40, ctypes.sizeof(_lib.FcRowstat)


def _spec_bytes(batch: int, k: int, gen_cap: int, vocab: int) -> dict:
    """Bytes each fc_spec_state array needs (include/flaxchat_amd.h)."""
    B = batch
    n = dict(t_len=B, d_len=B, t_pend=B * _PMAX, d_pend=B * _PMAX, t_pend_n=B, d_pend_n=B, t_dirty=B, d_dirty=B,
             gen=B * gen_cap, gen_n=B, prompt_len=B, round=B, stall=B, result=B * _RES_STRIDE, tok_d0=B * _PMAX,
             off_d0=B + 1, start_d=k * B, tok_ds=k * B, off_ds=B + 1, tok_v=B * (_PMAX + k), off_v=B + 1,
             start_v=B, drafts=B * k, q_logits=B * k * vocab, p_logits=B * (k + 1) * vocab)
    out = {name: 4 * v for name, v in n.items()}
    out["q_stats"] = B * k * _ROWSTAT
    out["p_stats"] = B * (k + 1) * _ROWSTAT
    out["part"] = int(lib().fc_spec_part_bytes(B, k, vocab))
    return out


def _spec_state(buffers: List[torch.Tensor], batch, k, max_tokens, gen_cap, vocab, temperature, top_k, seed,
                device=None):
    if len(buffers) != len(SPEC_BUFFERS):
        raise ValueError(f"buffers: the {len(SPEC_BUFFERS)} arrays of SPEC_BUFFERS in order")
    if batch < 1 or k < 1 or vocab < 1 or gen_cap < 1:
        raise ValueError("batch, k, gen_cap and vocab must be positive")
    need = _spec_bytes(batch, k, gen_cap, vocab)
    dev = device if device is not None else buffers[0].device
    for name, t in zip(SPEC_BUFFERS, buffers):
        if not t.is_contiguous():
            raise ValueError(f"buffer {name} must be contiguous")
        if t.numel() * t.element_size() < need[name]:
            raise ValueError(f"buffer {name}: {t.numel() * t.element_size()} bytes, {need[name]} needed "
                             f"for batch {batch}, k {k}, gen_cap {gen_cap}, vocab {vocab}")
        if t.device != dev:
            raise ValueError(f"buffer {name} is on {t.device}, not {dev}")
    part = buffers[-1]
    return _lib.FcSpecState(batch, k, max_tokens, gen_cap, vocab, temperature, top_k, seed,
                            *[t.data_ptr() for t in buffers[:-1]], part.data_ptr(), part.numel())


@torch.library.custom_op(f"{NS}::spec_accept", mutates_args=("buffers",))
def spec_accept(buffers: List[torch.Tensor], batch: int, k: int, max_tokens: int, gen_cap: int, vocab: int,
                temperature: float, top_k: int, seed: int) -> None:
    if buffers and buffers[0].device.type != "cuda":
        raise ValueError("spec_accept: the state buffers live on a CUDA device")
    st = _spec_state(buffers, batch, k, max_tokens, gen_cap, vocab, temperature, top_k, seed)
    check(lib().fc_spec_accept(ctypes.byref(st), _stream(buffers[0])), "fc_spec_accept")


@spec_accept.register_fake
def _(buffers, batch, k, max_tokens, gen_cap, vocab, temperature, top_k, seed):
    return None


@torch.library.custom_op(f"{NS}::spec_round",
                         mutates_args=("t_k", "t_v", "t_hist", "d_k", "d_v", "d_hist", "buffers", "workspace"))
def spec_round(target: int, draft: int, t_k: torch.Tensor, t_v: torch.Tensor, t_hist: torch.Tensor,
               d_k: torch.Tensor, d_v: torch.Tensor, d_hist: torch.Tensor, buffers: List[torch.Tensor], batch: int,
               k: int, max_tokens: int, gen_cap: int, vocab: int, temperature: float, top_k: int, seed: int,
               workspace: torch.Tensor) -> None:
    (mt, tdm), (md, ddm) = _model(target), _model(draft)
    if tdm.V != vocab or ddm.V != vocab:
        raise ValueError(f"spec_round: vocab {vocab}, the models have {tdm.V} / {ddm.V}")
    if tdm.device != ddm.device:
        raise ValueError("spec_round: target and draft on different devices")
    tc, dc = _cache(tdm, t_k, t_v, t_hist), _cache(ddm, d_k, d_v, d_hist)
    if tc.batch != batch or dc.batch != batch:
        raise ValueError(f"spec_round: the caches hold {tc.batch} / {dc.batch} rows, batch is {batch}")
    _same_device(tdm, workspace)
    st = _spec_state(buffers, batch, k, max_tokens, gen_cap, vocab, temperature, top_k, seed, device=tdm.device)
    need = lib().fc_spec_workspace_bytes(mt, md, batch, k)
    if need < 0 or workspace.numel() < need:
        raise ValueError(f"spec_round: workspace of {workspace.numel()} bytes, {need} needed")
    check(lib().fc_spec_round(mt, ctypes.byref(tc), md, ctypes.byref(dc), ctypes.byref(st), workspace.data_ptr(),
                              workspace.numel(), _stream(workspace)), "fc_spec_round")


@spec_round.register_fake
def _(target, draft, t_k, t_v, t_hist, d_k, d_v, d_hist, buffers, batch, k, max_tokens, gen_cap, vocab, temperature,
      top_k, seed, workspace):
    return None
