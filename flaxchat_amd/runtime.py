"""Device-resident weights, KV caches and the chunked forward.

PyTorch is used only to own device memory and the stream; every kernel is in
libflaxchat_amd.so and is called through the C-ABI.
"""

from __future__ import annotations

import ctypes
import math
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


def default_device() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("flaxchat_amd needs a ROCm GPU (torch.cuda.is_available() is False)")
    return torch.device("cuda", torch.cuda.current_device())


class DeviceModel:
    """A model's parameters in the engine's HBM layout plus the fc_model
    descriptor the kernels read (include/flaxchat_amd.h: fc_model/fc_layer)."""

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

        layers = []
        for i, blk in enumerate(model.blocks):
            a = blk.attn
            wqkv = np.concatenate([a.c_q.kernel.T, a.c_k.kernel.T, a.c_v.kernel.T], axis=0)
            lt = dict(wqkv=up(wqkv), wo=up(a.c_proj.kernel.T), wfc=up(blk.mlp.c_fc.kernel.T),
                      wproj=up(blk.mlp.c_proj.kernel.T))
            if str(i) in model.value_embeds:
                lt["ve"] = up(model.value_embeds[str(i)].embedding)
                lt["ve_gate"] = up(a.ve_gate.kernel.T, torch.float32)
            layers.append(lt)
        wte = up(model.wte.embedding)
        lm = wte if model._tie_embeddings else up(model.lm_head.kernel.T)
        cos, sin = cls._rope(c, device)
        tensors = dict(wte=wte, lm_head=lm, layers=layers, rope_cos=cos, rope_sin=sin,
                       smear_gate=up(model.smear_gate.kernel.reshape(-1), torch.float32))
        scalars = dict(resid=model.resid_lambdas.tolist(), x0=model.x0_lambdas.tolist(),
                       smear_lambda=float(model.smear_lambda[0]), backout_lambda=float(model.backout_lambda[0]))
        torch.cuda.synchronize(device)  # engine streams do not order after the default stream
        return cls(c, code, device, tensors, scalars)

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

        wte = nrm(Vp, D)
        lm = wte if c.tie_embeddings else nrm(Vp, D)
        layers = []
        for i in range(L):
            lt = dict(wqkv=nrm((H + 2 * G) * d, D), wo=nrm(D, D), wfc=nrm(4 * D, D), wproj=nrm(D, 4 * D))
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


def forward_chunk(dm: DeviceModel, cache: DeviceCache, tokens: torch.Tensor, start: torch.Tensor,
                  nvalid: torch.Tensor, n_out: int, logits: Optional[torch.Tensor], ws: Workspace,
                  stream=None, logits_stride: Optional[int] = None):
    """Feed tokens[B][W] (valid slots right-aligned) at positions start[b]..;
    write softcapped logits of the last n_out slots into logits[B][n_out][V]."""
    B, W = tokens.shape
    assert B == cache.batch and tokens.dtype == torch.int32
    nbytes = lib().fc_forward_workspace_bytes(ctypes.byref(dm.desc), B, W, n_out)
    if nbytes < 0:
        raise RuntimeError("fc_forward_workspace_bytes failed")
    buf = ws.get(nbytes)
    stride = logits_stride if logits_stride is not None else n_out * dm.V
    ch = FcChunk(W, tokens.data_ptr(), start.data_ptr(), nvalid.data_ptr(), n_out,
                 _ptr(logits) if n_out > 0 else 0, stride)
    s = stream if stream is not None else torch.cuda.current_stream().cuda_stream
    check(lib().fc_forward(ctypes.byref(dm.desc), ctypes.byref(cache.desc), ctypes.byref(ch),
                           buf.data_ptr(), buf.numel(), s), "fc_forward")


def prefill_rows(dm: DeviceModel, cache: DeviceCache, rows: List[List[int]], starts: List[int], ws: Workspace,
                 chunk: int = 256, stream=None):
    """Feed rows[b] at positions starts[b].. (no logits), in chunks of `chunk`
    slots; rows may have different lengths (empty rows are skipped)."""
    B = cache.batch
    dev = dm.device
    n_max = max((len(r) for r in rows), default=0)
    for c0 in range(0, n_max, chunk):
        W = min(chunk, n_max - c0)
        tok = np.zeros((B, W), np.int32)
        st = np.zeros(B, np.int32)
        nv = np.zeros(B, np.int32)
        for b, r in enumerate(rows):
            piece = r[c0:c0 + W]
            n = len(piece)
            if n:
                tok[b, W - n:] = piece
            st[b] = starts[b] + c0
            nv[b] = n
        forward_chunk(dm, cache, torch.from_numpy(tok).to(dev), torch.from_numpy(st).to(dev),
                      torch.from_numpy(nv).to(dev), 0, None, ws, stream)


def to_host(dm: DeviceModel):
    """Download a DeviceModel into a host GPT container (fp32 numpy, Flax
    (in, out) kernel orientation). Shared tensors stay shared."""
    from .gpt import GPT, Attention, Block, Embed, Linear, MLP
    memo = {}

    def get(t, transpose=False):
        key = (t.data_ptr(), transpose)
        if key not in memo:
            a = t.float().cpu().numpy()
            memo[key] = a.T if transpose else a
        return memo[key]

    c = dm.config
    H, G, d = dm.H, dm.G, dm.hd
    blocks, ves = [], {}
    for i, lt in enumerate(dm.t["layers"]):
        wqkv = get(lt["wqkv"])
        attn = Attention(Linear(wqkv[:H * d].T), Linear(wqkv[H * d:(H + G) * d].T), Linear(wqkv[(H + G) * d:].T),
                         Linear(get(lt["wo"], True)))
        if "ve" in lt:
            attn.ve_gate = Linear(get(lt["ve_gate"], True))
            ves[str(i)] = Embed(get(lt["ve"]))
        blocks.append(Block(attn, MLP(Linear(get(lt["wfc"], True)), Linear(get(lt["wproj"], True)))))
    wte = Embed(get(dm.t["wte"]))
    lm = None if c.tie_embeddings else Linear(get(dm.t["lm_head"], True))
    return GPT(c, wte, blocks, lm, np.array(dm.s["resid"], np.float32), np.array(dm.s["x0"], np.float32),
               Linear(get(dm.t["smear_gate"]).reshape(24, 1)), np.float32(dm.s["smear_lambda"]),
               np.float32(dm.s["backout_lambda"]), ves)
