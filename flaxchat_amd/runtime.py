"""Device-resident weights, KV caches and the chunked forward.

PyTorch is used only to own device memory and the stream; every kernel is in
libflaxchat_amd.so and is called through the C-ABI.
"""

from __future__ import annotations

import ctypes
import math
import weakref
from typing import List, Optional

import numpy as np
import torch

from . import _lib
from ._lib import FcCache, FcChunk, FcLayer, FcModel, check, lib
from .config import GPTConfig, compute_window_sizes, has_ve, padded_vocab
from .gpt import precompute_rotary_embeddings, reference_lambdas

_TORCH_DT = {_lib.FC_F32: torch.float32, _lib.FC_BF16: torch.bfloat16}


def dtype_code(dtype) -> int:
    if dtype in ("bf16", "bfloat16", torch.bfloat16, _lib.FC_BF16):
        return _lib.FC_BF16
    if dtype in ("fp32", "float32", torch.float32, _lib.FC_F32, None):
        return _lib.FC_F32
    raise ValueError(f"unsupported dtype {dtype!r}")


def _ptr(t: Optional[torch.Tensor]) -> int:
    return 0 if t is None else t.data_ptr()


def frag_pack(a: np.ndarray) -> np.ndarray:
    """Fragment order (include/flaxchat_amd.h) of a [R][K] matrix as a
    [round16(R)][K] array whose memory is in fragment order (zero padding)."""
    R, K = a.shape
    assert K % 32 == 0, "fragment order needs K % 32 == 0"
    R16 = (R + 15) // 16 * 16
    pad = np.zeros((R16, K), a.dtype)
    pad[:R] = a
    return np.ascontiguousarray(pad.reshape(R16 // 16, 16, K // 32, 4, 8).transpose(0, 2, 3, 1, 4)).reshape(R16, K)


def frag_unpack(p: np.ndarray, R: int) -> np.ndarray:
    """Inverse of frag_pack: the first R rows of the row-major matrix."""
    R16, K = p.shape
    return np.ascontiguousarray(p.reshape(R16 // 16, K // 32, 4, 16, 8).transpose(0, 3, 1, 2, 4)).reshape(R16, K)[:R]


def pack_operand(t: torch.Tensor) -> torch.Tensor:
    """Device copy of a row-major bf16 [R][K] matrix in fragment order
    ([round16(R)][K]), through fc_pack_operand on the current stream."""
    R, K = t.shape
    if K % 64 != 0 or R % 32 != 0:
        raise ValueError(f"bf16 weights need rows % 32 == 0 and K % 64 == 0 (got {R} x {K})")
    out = torch.empty(((R + 15) // 16 * 16, K), dtype=t.dtype, device=t.device)
    check(lib().fc_pack_operand(t.data_ptr(), out.data_ptr(), R, K, torch.cuda.current_stream().cuda_stream),
          "fc_pack_operand")
    return out


def default_device() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("flaxchat_amd needs a ROCm GPU (torch.cuda.is_available() is False)")
    return torch.device("cuda", torch.cuda.current_device())


_MATS = ("wqkv", "wo", "wfc", "wproj")

# Live DeviceModels by the host address of their fc_model descriptor: callers
# that hand a model across an integer boundary (the torch operators) resolve
# it here, so a stale or foreign address is refused instead of dereferenced.
_LIVE_MODELS: "weakref.WeakValueDictionary[int, DeviceModel]" = weakref.WeakValueDictionary()


def live_model(addr: int) -> Optional["DeviceModel"]:
    """The live DeviceModel whose descriptor is at host address `addr`, or
    None (never built, or already garbage-collected)."""
    dm = _LIVE_MODELS.get(int(addr))
    return dm if dm is not None and ctypes.addressof(dm.desc) == int(addr) else None


class DeviceModel:
    """A model's parameters in the engine's HBM layout plus the fc_model
    descriptor the kernels read (include/flaxchat_amd.h: fc_model/fc_layer).
    In bf16 the linear weights and lm_head are in fragment order; wte and
    the value-embedding tables stay row-major (they are gathered by token)."""

    def __init__(self, config: GPTConfig, dtype: int, device, tensors: dict, scalars: dict):
        self.config = config
        self.dtype = dtype
        self.device = device
        self.t = tensors
        self.s = scalars
        c = config
        self.L, self.D, self.H, self.G = c.n_layer, c.n_embd, c.n_head, c.n_kv_head
        self.hd = self.D // self.H
        self.V, self.Vp = c.vocab_size, padded_vocab(c)
        self.windows = [w for (w, _) in compute_window_sizes(c)]
        self._build_desc()

    # ---------------------------------------------------------------- build
    def _build_desc(self):
        L = self.L
        self._layers = (FcLayer * L)()
        for i in range(L):
            lt = self.t["layers"][i]
            self._layers[i] = FcLayer(_ptr(lt["wqkv"]), _ptr(lt["wo"]), _ptr(lt["wfc"]), _ptr(lt["wproj"]),
                                      _ptr(lt.get("ve")), _ptr(lt.get("ve_gate")), int(self.windows[i]),
                                      float(self.s["resid"][i]), float(self.s["x0"][i]))
        self.desc = FcModel(L, self.D, self.H, self.G, self.hd, self.V, self.Vp, self.dtype,
                            _ptr(self.t["wte"]), _ptr(self.t["lm_head"]), _ptr(self.t["smear_gate"]),
                            float(self.s["smear_lambda"]), float(self.s["backout_lambda"]),
                            _ptr(self.t["rope_cos"]), _ptr(self.t["rope_sin"]), int(self.t["rope_cos"].shape[0]),
                            ctypes.cast(self._layers, ctypes.POINTER(FcLayer)))
        _LIVE_MODELS[ctypes.addressof(self.desc)] = self

    @staticmethod
    def _rope(config: GPTConfig, device, rope_len: Optional[int] = None):
        n = rope_len or config.sequence_len * 10
        cos, sin = precompute_rotary_embeddings(n, config.n_embd // config.n_head)
        return torch.from_numpy(cos).to(device), torch.from_numpy(sin).to(device)

    @classmethod
    def from_host(cls, model, dtype="fp32", device=None) -> "DeviceModel":
        """Upload a host GPT container (flaxchat_amd.gpt.GPT). Flax (in, out)
        kernels are transposed once to the [out][in] layout."""
        device = device or default_device()
        code = dtype_code(dtype)
        tdt = _TORCH_DT[code]
        c = model.config

        def up(a, dt=tdt):
            return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device=device, dtype=dt)

        def mat(a):  # a linear weight [out][in] in the GEMM layout of this dtype
            t = up(a)
            return pack_operand(t) if code == _lib.FC_BF16 else t

        layers = []
        for i, blk in enumerate(model.blocks):
            a = blk.attn
            wqkv = np.concatenate([a.c_q.kernel.T, a.c_k.kernel.T, a.c_v.kernel.T], axis=0)
            lt = dict(wqkv=mat(wqkv), wo=mat(a.c_proj.kernel.T), wfc=mat(blk.mlp.c_fc.kernel.T),
                      wproj=mat(blk.mlp.c_proj.kernel.T))
            if str(i) in model.value_embeds:
                lt["ve"] = up(model.value_embeds[str(i)].embedding)
                lt["ve_gate"] = up(a.ve_gate.kernel.T, torch.float32)
            layers.append(lt)
        wte = up(model.wte.embedding)
        if code == _lib.FC_BF16:
            lm = pack_operand(wte) if model._tie_embeddings else mat(model.lm_head.kernel.T)
        else:
            lm = wte if model._tie_embeddings else up(model.lm_head.kernel.T)
        cos, sin = cls._rope(c, device)
        tensors = dict(wte=wte, lm_head=lm, layers=layers, rope_cos=cos, rope_sin=sin,
                       smear_gate=up(model.smear_gate.kernel.reshape(-1), torch.float32))
        scalars = dict(resid=model.resid_lambdas.tolist(), x0=model.x0_lambdas.tolist(),
                       smear_lambda=float(model.smear_lambda[0]), backout_lambda=float(model.backout_lambda[0]))
        if torch.device(device).type == "cuda":
            torch.cuda.synchronize(device)  # engine streams do not order after the default stream
        return cls(c, code, torch.device(device), tensors, scalars)

    @classmethod
    def random_init(cls, config: GPTConfig, seed: int = 0, dtype="bf16", device=None, std: float = 0.02,
                    rope_len: Optional[int] = None) -> "DeviceModel":
        """Random-init weights drawn on the device: every matrix and embedding
        ~ N(0, std) from a seeded torch generator; scalars at the reference's
        init values (flaxchat/gpt.py:242, 245, 300-303)."""
        device = device or default_device()
        code = dtype_code(dtype)
        tdt = _TORCH_DT[code]
        gen = torch.Generator(device=device)
        gen.manual_seed(int(seed))
        c = config
        D, H, G, L = c.n_embd, c.n_head, c.n_kv_head, c.n_layer
        d = D // H
        Vp = padded_vocab(c)

        def nrm(*shape, dt=tdt):
            out = torch.empty(*shape, device=device, dtype=dt)
            flat = out.view(-1)
            step = 1 << 26
            for s in range(0, flat.numel(), step):
                n = min(step, flat.numel() - s)
                flat[s:s + n] = (torch.randn(n, device=device, generator=gen) * std).to(dt)
            return out

        bf16 = code == _lib.FC_BF16

        def mat(*shape):
            t = nrm(*shape)
            return pack_operand(t) if bf16 else t

        wte = nrm(Vp, D)
        if c.tie_embeddings:
            lm = pack_operand(wte) if bf16 else wte
        else:
            lm = mat(Vp, D)
        layers = []
        for i in range(L):
            lt = dict(wqkv=mat((H + 2 * G) * d, D), wo=mat(D, D), wfc=mat(4 * D, D), wproj=mat(D, 4 * D))
            if has_ve(i, L):
                lt["ve_gate"] = nrm(G, 12, dt=torch.float32)
            layers.append(lt)
        for i in range(L):
            if has_ve(i, L):
                layers[i]["ve"] = nrm(Vp, G * d)
        cos, sin = cls._rope(c, device, rope_len)
        resid, x0 = reference_lambdas(L)
        tensors = dict(wte=wte, lm_head=lm, layers=layers, rope_cos=cos, rope_sin=sin,
                       smear_gate=nrm(24, dt=torch.float32))
        scalars = dict(resid=resid.tolist(), x0=x0.tolist(), smear_lambda=0.0, backout_lambda=0.2)
        torch.cuda.synchronize(device)  # engine streams do not order after the default stream
        return cls(c, code, device, tensors, scalars)

    def make_draft(self, n_layer: int) -> "DeviceModel":
        """Draft whose layers are this model's layers 0..n_layer-1 (shared
        tensors), sharing wte / lm_head and the RoPE tables."""
        c = self.config.with_(n_layer=n_layer)
        layers = []
        for i in range(n_layer):
            lt = dict(self.t["layers"][i])
            if has_ve(i, n_layer) and "ve" not in lt:
                lt["ve"] = torch.zeros(self.Vp, self.G * self.hd, device=self.device, dtype=_TORCH_DT[self.dtype])
                lt["ve_gate"] = torch.zeros(self.G, 12, device=self.device, dtype=torch.float32)
            if not has_ve(i, n_layer):
                lt.pop("ve", None)
                lt.pop("ve_gate", None)
            layers.append(lt)
        tensors = dict(self.t)
        tensors["layers"] = layers
        scalars = dict(self.s)
        scalars["resid"] = list(self.s["resid"][:n_layer])
        scalars["x0"] = list(self.s["x0"][:n_layer])
        return DeviceModel(c, self.dtype, self.device, tensors, scalars)

    def weight_bytes(self, with_head: bool = True) -> int:
        """Bytes of the matrices one forward step streams (excluding embedding
        row gathers)."""
        es = 2 if self.dtype == _lib.FC_BF16 else 4
        per = sum(self.t["layers"][0][k].numel() for k in ("wqkv", "wo", "wfc", "wproj"))
        n = per * self.L + (self.Vp * self.D if with_head else 0)
        return n * es


class DeviceCache:
    """Preallocated KV cache + smear history for `batch` rows of `cap` positions
    (include/flaxchat_amd.h layouts). Zero-filled so unused slots are finite."""

    def __init__(self, dm: DeviceModel, batch: int, cap: int):
        cap = int(math.ceil(cap / 32) * 32)
        tdt = _TORCH_DT[dm.dtype]
        self.batch, self.cap = batch, cap
        self.k = torch.zeros(dm.L, batch, dm.G, cap, dm.hd, device=dm.device, dtype=tdt)
        self.v = torch.zeros(dm.L, batch, dm.G, cap // 32, dm.hd, 32, device=dm.device, dtype=tdt)
        self.hist = torch.zeros(batch, cap, dm.D, device=dm.device, dtype=torch.float32)
        self.desc = FcCache(self.k.data_ptr(), self.v.data_ptr(), self.hist.data_ptr(), batch, cap)

    def k_at(self, layer, b, g, pos):
        return self.k[layer, b, g, pos]

    def v_at(self, layer, b, g, pos):
        return self.v[layer, b, g, pos // 32, :, pos % 32]


class Workspace:
    """Growable, zero-filled device scratch (the library keeps the split-K
    counters it holds at zero between calls)."""

    def __init__(self, device):
        self.device = device
        self.buf = None

    def get(self, nbytes: int) -> torch.Tensor:
        if self.buf is None or self.buf.numel() < nbytes:
            self.buf = torch.zeros(int(nbytes), dtype=torch.uint8, device=self.device)
        return self.buf


def forward_packed(dm: DeviceModel, cache: DeviceCache, tokens: torch.Tensor, row_off: torch.Tensor,
                   start: torch.Tensor, max_per_row: int, n_out: int, logits: Optional[torch.Tensor],
                   ws: Workspace, stream=None, logits_stride: Optional[int] = None, typ_tokens: int = 0,
                   flags: int = 0):
    """Feed a packed chunk (include/flaxchat_amd.h, fc_chunk): row b's tokens
    are tokens[row_off[b]:row_off[b+1]] at positions start[b].. (device int32
    arrays; tokens has the chunk's capacity). Writes softcapped logits of the
    last n_out tokens of each row into logits[B][n_out][V]."""
    B = cache.batch
    max_tokens = int(tokens.numel())
    assert tokens.dtype == torch.int32 and row_off.numel() == B + 1 and start.numel() == B
    nbytes = lib().fc_forward_workspace_bytes(ctypes.byref(dm.desc), B, max_tokens, max_per_row, typ_tokens)
    if nbytes < 0:
        raise RuntimeError("fc_forward_workspace_bytes failed")
    buf = ws.get(nbytes)
    stride = logits_stride if logits_stride is not None else n_out * dm.V
    ch = FcChunk(max_tokens, max_per_row, typ_tokens, tokens.data_ptr(), row_off.data_ptr(), start.data_ptr(),
                 n_out, _ptr(logits) if n_out > 0 else 0, stride, flags)
    s = stream if stream is not None else torch.cuda.current_stream().cuda_stream
    check(lib().fc_forward(ctypes.byref(dm.desc), ctypes.byref(cache.desc), ctypes.byref(ch),
                           buf.data_ptr(), buf.numel(), s), "fc_forward")


def pack_rows(rows: List[List[int]]):
    """(tokens, row_off, max_per_row) of host token lists in the packed layout."""
    n = np.array([len(r) for r in rows], np.int64)
    off = np.zeros(len(rows) + 1, np.int32)
    off[1:] = np.cumsum(n)
    tok = np.zeros(max(1, int(off[-1])), np.int32)
    for b, r in enumerate(rows):
        tok[off[b]:off[b + 1]] = r
    return tok, off, max(1, int(n.max()) if len(rows) else 1)


def forward_rows(dm: DeviceModel, cache: DeviceCache, rows: List[List[int]], starts: List[int], n_out: int,
                 logits: Optional[torch.Tensor], ws: Workspace, stream=None):
    """Feed host token lists rows[b] at positions starts[b].. in one chunk."""
    dev = dm.device
    tok, off, mpr = pack_rows(rows)
    forward_packed(dm, cache, torch.from_numpy(tok).to(dev), torch.from_numpy(off).to(dev),
                   torch.from_numpy(np.asarray(starts, np.int32)).to(dev), mpr, n_out, logits, ws, stream)


def prefill_rows(dm: DeviceModel, cache: DeviceCache, rows: List[List[int]], starts: List[int], ws: Workspace,
                 chunk: int = 256, stream=None):
    """Feed rows[b] at positions starts[b].. (no logits), in chunks of up to
    `chunk` tokens per row; rows may have different lengths (a row with
    nothing left feeds nothing)."""
    n_max = max((len(r) for r in rows), default=0)
    for c0 in range(0, n_max, chunk):
        pieces = [r[c0:c0 + chunk] for r in rows]
        st = [starts[b] + c0 for b in range(len(rows))]
        forward_rows(dm, cache, pieces, st, 0, None, ws, stream)


def to_host(dm: DeviceModel):
    """Download a DeviceModel into a host GPT container (fp32 numpy, Flax
    (in, out) kernel orientation). Shared tensors stay shared."""
    from .gpt import GPT, Attention, Block, Embed, Linear, MLP
    memo = {}
    packed = dm.dtype == _lib.FC_BF16

    def get(t, transpose=False, frag=False):
        key = (t.data_ptr(), transpose, frag)
        if key not in memo:
            a = t.float().cpu().numpy()
            if frag and packed:
                a = frag_unpack(a, a.shape[0])
            memo[key] = a.T if transpose else a
        return memo[key]

    c = dm.config
    H, G, d = dm.H, dm.G, dm.hd
    blocks, ves = [], {}
    for i, lt in enumerate(dm.t["layers"]):
        wqkv = get(lt["wqkv"], frag=True)
        attn = Attention(Linear(wqkv[:H * d].T), Linear(wqkv[H * d:(H + G) * d].T), Linear(wqkv[(H + G) * d:].T),
                         Linear(get(lt["wo"], True, True)))
        if "ve" in lt:
            attn.ve_gate = Linear(get(lt["ve_gate"], True))
            ves[str(i)] = Embed(get(lt["ve"]))
        blocks.append(Block(attn, MLP(Linear(get(lt["wfc"], True, True)), Linear(get(lt["wproj"], True, True)))))
    wte = Embed(get(dm.t["wte"]))
    lm = None if c.tie_embeddings else Linear(get(dm.t["lm_head"], True, True))
    return GPT(c, wte, blocks, lm, np.array(dm.s["resid"], np.float32), np.array(dm.s["x0"], np.float32),
               Linear(get(dm.t["smear_gate"]).reshape(24, 1)), np.float32(dm.s["smear_lambda"]),
               np.float32(dm.s["backout_lambda"]), ves)
