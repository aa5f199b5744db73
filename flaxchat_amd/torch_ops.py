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
"""

from __future__ import annotations

import torch

from . import _lib
from ._lib import check, lib

__all__ = ["pack_operand", "linear", "attention", "cross_entropy", "frag_to_rows"]

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
