"""Host-side weight container with the reference's parameter tree.

The engine reads the same fields the reference's per-token forward reads
(flaxchat/engine.py:69-175): `wte.embedding`, `blocks[i].attn.{c_q,c_k,c_v,
c_proj,ve_gate}.kernel`, `blocks[i].mlp.{c_fc,c_proj}.kernel`,
`value_embeds[str(i)].embedding`, `resid_lambdas`, `x0_lambdas`,
`smear_gate.kernel`, `smear_lambda`, `backout_lambda`, `lm_head.kernel`.
Kernels keep Flax's (in, out) orientation (flaxchat/gpt.py:93-99, 154-163);
the device loader transposes them once into the [out][in] layout the HIP
GEMMs stream. Arrays are numpy float32 on the host.
"""

from __future__ import annotations

import os

import numpy as np
from typing import Dict, List, Optional

from .config import GPTConfig, compute_window_sizes, has_ve, padded_vocab


class Linear:
    """nnx.Linear without bias: y = x @ kernel, kernel shape (in, out)."""
    __slots__ = ("kernel",)

    def __init__(self, kernel: np.ndarray):
        self.kernel = kernel


class Embed:
    """nnx.Embed: rows of `embedding` (V, dim)."""
    __slots__ = ("embedding",)

    def __init__(self, embedding: np.ndarray):
        self.embedding = embedding


class Attention:
    def __init__(self, c_q, c_k, c_v, c_proj, ve_gate=None):
        self.c_q, self.c_k, self.c_v, self.c_proj = c_q, c_k, c_v, c_proj
        self.ve_gate = ve_gate


class MLP:
    def __init__(self, c_fc, c_proj):
        self.c_fc, self.c_proj = c_fc, c_proj


class Block:
    def __init__(self, attn: Attention, mlp: MLP):
        self.attn, self.mlp = attn, mlp


def precompute_rotary_embeddings(seq_len: int, head_dim: int, base: float = 100000.0):
    """cos/sin tables of shape (seq_len, head_dim // 2), float32
    (flaxchat/gpt.py:52-62: fp32 inv_freq, fp32 outer product)."""
    channel_range = np.arange(0, head_dim, 2, dtype=np.float32)
    inv_freq = (np.float32(1.0) / (np.float32(base) ** (channel_range / np.float32(head_dim)))).astype(np.float32)
    t = np.arange(seq_len, dtype=np.float32)
    freqs = np.outer(t, inv_freq).astype(np.float32)
    return np.cos(freqs).astype(np.float32), np.sin(freqs).astype(np.float32)


class GPT:
    """Parameter tree of flaxchat's GPT (flaxchat/gpt.py:202-261)."""

    def __init__(self, config: GPTConfig, wte: Embed, blocks: List[Block],
                 lm_head: Optional[Linear], resid_lambdas, x0_lambdas,
                 smear_gate: Linear, smear_lambda, backout_lambda,
                 value_embeds: Dict[str, Embed]):
        self.config = config
        self.wte = wte
        self.blocks = blocks
        self.lm_head = lm_head
        self._tie_embeddings = bool(config.tie_embeddings)
        self.resid_lambdas = np.asarray(resid_lambdas, dtype=np.float32)
        self.x0_lambdas = np.asarray(x0_lambdas, dtype=np.float32)
        self.smear_gate = smear_gate
        self.smear_lambda = np.asarray(smear_lambda, dtype=np.float32).reshape(1)
        self.backout_lambda = np.asarray(backout_lambda, dtype=np.float32).reshape(1)
        self.value_embeds = value_embeds
        self.window_sizes = compute_window_sizes(config)
        self.padded_vocab_size = padded_vocab(config)
        self._check()

    def _check(self):
        c = self.config
        D, H, G = c.n_embd, c.n_head, c.n_kv_head
        d = D // H
        if D % H or H % G:
            raise ValueError("n_embd must divide by n_head and n_head by n_kv_head")
        if len(self.blocks) != c.n_layer:
            raise ValueError("block count differs from n_layer")
        for i, b in enumerate(self.blocks):
            assert b.attn.c_q.kernel.shape == (D, H * d)
            assert b.attn.c_k.kernel.shape == (D, G * d)
            assert b.attn.c_v.kernel.shape == (D, G * d)
            assert b.attn.c_proj.kernel.shape == (D, D)
            assert b.mlp.c_fc.kernel.shape == (D, 4 * D)
            assert b.mlp.c_proj.kernel.shape == (4 * D, D)
            if has_ve(i, c.n_layer):
                assert b.attn.ve_gate is not None and b.attn.ve_gate.kernel.shape == (12, G)
                assert self.value_embeds[str(i)].embedding.shape[1] == G * d

    @property
    def head_dim(self) -> int:
        return self.config.n_embd // self.config.n_head

    def lm_head_kernel(self) -> np.ndarray:
        """(D, V_pad) matrix the head multiplies by (tied: wte^T)."""
        if self._tie_embeddings:
            return self.wte.embedding.T
        return self.lm_head.kernel

    def __call__(self, idx, targets=None, *, dtype=None, device=None):
        """GPT.__call__(idx, targets=None) (flaxchat/gpt.py:407-454) on the
        HIP engine: softcapped fp32 logits [B, T, vocab], or with targets
        the mean cross-entropy over targets >= 0 (device tensors)."""
        from .engine import gpt_forward
        return gpt_forward(self, idx, targets, dtype=dtype, device=device)

    # ------------------------------------------------------------------
    # Initialisation recipes
    # ------------------------------------------------------------------
    @classmethod
    def init_normal(cls, config: GPTConfig, seed: int = 0, std: float = 0.02) -> "GPT":
        """Every matrix and embedding ~ N(0, std), seeded; scalars at the
        reference's init values (flaxchat/gpt.py:242, 245, 300-303).

        This is the benchmark recipe: a random-init model of the named
        architecture. Draw order: wte, lm_head, then per block c_q, c_k,
        c_v, c_proj, c_fc, mlp.c_proj, ve_gate, then value embeddings in
        layer order, then smear_gate.
        """
        rng = np.random.default_rng(seed)
        D, H, G, L = config.n_embd, config.n_head, config.n_kv_head, config.n_layer
        d = D // H
        Vp = padded_vocab(config)

        def nrm(*shape):
            return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)

        wte = Embed(nrm(Vp, D))
        lm_head = None if config.tie_embeddings else Linear(nrm(D, Vp))
        blocks = []
        for i in range(L):
            attn = Attention(Linear(nrm(D, H * d)), Linear(nrm(D, G * d)), Linear(nrm(D, G * d)),
                             Linear(nrm(D, D)))
            mlp = MLP(Linear(nrm(D, 4 * D)), Linear(nrm(4 * D, D)))
            if has_ve(i, L):
                attn.ve_gate = Linear(nrm(12, G))
            blocks.append(Block(attn, mlp))
        value_embeds = {str(i): Embed(nrm(Vp, G * d)) for i in range(L) if has_ve(i, L)}
        smear_gate = Linear(nrm(24, 1))
        resid, x0 = reference_lambdas(L)
        return cls(config, wte, blocks, lm_head, resid, x0, smear_gate,
                   np.zeros(1, np.float32), np.full(1, 0.2, np.float32), value_embeds)

    @classmethod
    def init_normal_parallel(cls, config: GPTConfig, seed: int = 0, std: float = 0.02,
                             threads: Optional[int] = None) -> "GPT":
        """init_normal's recipe (same tensors, same draw order, N(0, std),
        reference scalars) with each tensor drawn from its own stream, so
        the draws run in threads: tensor i of the draw order takes child i
        of SeedSequence(seed), split into row blocks of about 4M elements
        that take that child's children in order. Same distribution as
        init_normal, different values; for the large configurations (a d24
        model at vocabulary 65536 holds about 2.1e9 parameters)."""
        from concurrent.futures import ThreadPoolExecutor
        D, H, G, L = config.n_embd, config.n_head, config.n_kv_head, config.n_layer
        d = D // H
        Vp = padded_vocab(config)
        shapes = [(Vp, D)]
        if not config.tie_embeddings:
            shapes.append((D, Vp))
        for i in range(L):
            shapes += [(D, H * d), (D, G * d), (D, G * d), (D, D), (D, 4 * D), (4 * D, D)]
            if has_ve(i, L):
                shapes.append((12, G))
        shapes += [(Vp, G * d) for i in range(L) if has_ve(i, L)]
        shapes.append((24, 1))
        out = [np.empty(s, np.float32) for s in shapes]
        jobs = []
        for t, child in enumerate(np.random.SeedSequence(seed).spawn(len(shapes))):
            rows, cols = shapes[t]
            per = max(1, (1 << 22) // cols)
            nblk = (rows + per - 1) // per
            for j, ss in enumerate(child.spawn(nblk)):
                jobs.append((t, j * per, min(rows, (j + 1) * per), ss))

        def draw(job):
            t, r0, r1, ss = job
            blk = out[t][r0:r1]
            np.random.Generator(np.random.PCG64(ss)).standard_normal(blk.shape, dtype=np.float32, out=blk)
            blk *= np.float32(std)

        with ThreadPoolExecutor(max_workers=threads or min(16, os.cpu_count() or 1)) as ex:
            list(ex.map(draw, jobs))
        it = iter(out)
        wte = Embed(next(it))
        lm_head = None if config.tie_embeddings else Linear(next(it))
        blocks = []
        for i in range(L):
            attn = Attention(Linear(next(it)), Linear(next(it)), Linear(next(it)), Linear(next(it)))
            mlp = MLP(Linear(next(it)), Linear(next(it)))
            if has_ve(i, L):
                attn.ve_gate = Linear(next(it))
            blocks.append(Block(attn, mlp))
        value_embeds = {str(i): Embed(next(it)) for i in range(L) if has_ve(i, L)}
        smear_gate = Linear(next(it))
        resid, x0 = reference_lambdas(L)
        return cls(config, wte, blocks, lm_head, resid, x0, smear_gate,
                   np.zeros(1, np.float32), np.full(1, 0.2, np.float32), value_embeds)

    def make_draft(self, n_layer: int, window_pattern: Optional[str] = None) -> "GPT":
        """Draft model whose layers are copies of this model's layers
        0..n_layer-1, sharing wte and lm_head (the same arrays).

        Per-layer scalars are copied from the same layers; smear and backout
        parameters are copied. Value embeddings are shared where the draft
        layer index carries VE in both models.
        """
        c = self.config
        dc = c.with_(n_layer=n_layer, window_pattern=window_pattern or c.window_pattern)
        blocks, ves = [], {}
        for i in range(n_layer):
            sb = self.blocks[i]
            attn = Attention(sb.attn.c_q, sb.attn.c_k, sb.attn.c_v, sb.attn.c_proj)
            if has_ve(i, n_layer):
                if sb.attn.ve_gate is not None:
                    attn.ve_gate = sb.attn.ve_gate
                    ves[str(i)] = self.value_embeds[str(i)]
                else:  # target layer without VE: give the draft its own zero gate/table
                    G, d = c.n_kv_head, self.head_dim
                    attn.ve_gate = Linear(np.zeros((12, G), np.float32))
                    ves[str(i)] = Embed(np.zeros((self.padded_vocab_size, G * d), np.float32))
            blocks.append(Block(attn, MLP(sb.mlp.c_fc, sb.mlp.c_proj)))
        return GPT(dc, self.wte, blocks, self.lm_head,
                   self.resid_lambdas[:n_layer].copy(), self.x0_lambdas[:n_layer].copy(),
                   self.smear_gate, self.smear_lambda.copy(), self.backout_lambda.copy(), ves)

    def perturb_scalars(self, seed: int = 1, smear: float = 0.7) -> "GPT":
        """Set a non-zero smear_lambda and jitter the per-layer lambdas so the
        smear chain and the lambda mixes are exercised by parity tests."""
        rng = np.random.default_rng(seed)
        self.smear_lambda = np.full(1, smear, np.float32)
        L = self.config.n_layer
        self.resid_lambdas = (self.resid_lambdas + rng.uniform(-0.1, 0.1, L)).astype(np.float32)
        self.x0_lambdas = (self.x0_lambdas + rng.uniform(-0.05, 0.05, L)).astype(np.float32)
        self.backout_lambda = np.full(1, 0.35, np.float32)
        return self


def reference_lambdas(n_layer: int):
    """resid_lambdas / x0_lambdas init (flaxchat/gpt.py:300-303)."""
    den = max(n_layer - 1, 1)
    resid = np.array([1.15 - (0.10 * i / den) for i in range(n_layer)], dtype=np.float32)
    x0 = np.array([0.20 - (0.15 * i / den) for i in range(n_layer)], dtype=np.float32)
    return resid, x0


# ----------------------------------------------------------------------
# Loading the reference's parameter tree
# ----------------------------------------------------------------------
def _get(d, *keys):
    for k in keys:
        if isinstance(d, dict):
            if k in d:
                d = d[k]
            elif str(k) in d:
                d = d[str(k)]
            elif isinstance(k, str) and k.isdigit() and int(k) in d:
                d = d[int(k)]
            else:
                raise KeyError(f"missing parameter {'/'.join(map(str, keys))}")
        else:
            d = d[int(k)]
    return np.asarray(d, dtype=np.float32)


def from_pure_dict(config: GPTConfig, params: dict) -> GPT:
    """Build the host container from the nested dict the reference exports
    with `nnx.to_pure_dict(nnx.state(model, nnx.Param))`
    (flaxchat/scripts/run_tinystories.py:328-345, flaxchat/checkpoint.py:47-66).
    Block indices may be ints or strings."""
    L = config.n_layer
    blocks = []
    for i in range(L):
        a = Attention(Linear(_get(params, "blocks", i, "attn", "c_q", "kernel")),
                      Linear(_get(params, "blocks", i, "attn", "c_k", "kernel")),
                      Linear(_get(params, "blocks", i, "attn", "c_v", "kernel")),
                      Linear(_get(params, "blocks", i, "attn", "c_proj", "kernel")))
        if has_ve(i, L):
            a.ve_gate = Linear(_get(params, "blocks", i, "attn", "ve_gate", "kernel"))
        m = MLP(Linear(_get(params, "blocks", i, "mlp", "c_fc", "kernel")),
                Linear(_get(params, "blocks", i, "mlp", "c_proj", "kernel")))
        blocks.append(Block(a, m))
    ves = {str(i): Embed(_get(params, "value_embeds", str(i), "embedding")) for i in range(L) if has_ve(i, L)}
    lm = None if config.tie_embeddings else Linear(_get(params, "lm_head", "kernel"))
    return GPT(config, Embed(_get(params, "wte", "embedding")), blocks, lm, _get(params, "resid_lambdas"),
               _get(params, "x0_lambdas"), Linear(_get(params, "smear_gate", "kernel")),
               _get(params, "smear_lambda"), _get(params, "backout_lambda"), ves)


def to_pure_dict(model: GPT) -> dict:
    """The inverse of from_pure_dict (reference parameter tree, numpy)."""
    d = {"wte": {"embedding": model.wte.embedding}, "blocks": {},
         "resid_lambdas": model.resid_lambdas, "x0_lambdas": model.x0_lambdas,
         "smear_gate": {"kernel": model.smear_gate.kernel}, "smear_lambda": model.smear_lambda,
         "backout_lambda": model.backout_lambda,
         "value_embeds": {k: {"embedding": v.embedding} for k, v in model.value_embeds.items()}}
    if model.lm_head is not None:
        d["lm_head"] = {"kernel": model.lm_head.kernel}
    for i, b in enumerate(model.blocks):
        attn = {"c_q": {"kernel": b.attn.c_q.kernel}, "c_k": {"kernel": b.attn.c_k.kernel},
                "c_v": {"kernel": b.attn.c_v.kernel}, "c_proj": {"kernel": b.attn.c_proj.kernel}}
        if b.attn.ve_gate is not None:
            attn["ve_gate"] = {"kernel": b.attn.ve_gate.kernel}
        d["blocks"][i] = {"attn": attn, "mlp": {"c_fc": {"kernel": b.mlp.c_fc.kernel},
                                                "c_proj": {"kernel": b.mlp.c_proj.kernel}}}
    return d


def save_npz(model: GPT, path: str) -> None:
    """Flatten the parameter tree to 'a/b/c' keys in an .npz (no pickle)."""
    flat = {}

    def walk(prefix, node):
        if isinstance(node, dict):
            for k, v in node.items():
                walk(f"{prefix}/{k}" if prefix else str(k), v)
        else:
            flat[prefix] = np.asarray(node)
    walk("", to_pure_dict(model))
    cfg = model.config
    flat["__config__"] = np.array([cfg.sequence_len, cfg.vocab_size, cfg.n_layer, cfg.n_head, cfg.n_kv_head,
                                   cfg.n_embd, int(cfg.tie_embeddings), cfg.short_window or 0], np.int64)
    flat["__window_pattern__"] = np.frombuffer(cfg.window_pattern.encode(), dtype=np.uint8)
    np.savez(path, **flat)


def load_npz(path: str) -> GPT:
    """Load a model saved by save_npz (numpy.load without pickle)."""
    z = np.load(path, allow_pickle=False)
    c = z["__config__"].tolist()
    cfg = GPTConfig(sequence_len=c[0], vocab_size=c[1], n_layer=c[2], n_head=c[3], n_kv_head=c[4], n_embd=c[5],
                    tie_embeddings=bool(c[6]), short_window=(c[7] or None),
                    window_pattern=bytes(z["__window_pattern__"]).decode())
    tree: dict = {}
    for key in z.files:
        if key.startswith("__"):
            continue
        node = tree
        parts = key.split("/")
        for p in parts[:-1]:
            node = node.setdefault(p, {})
        node[parts[-1]] = z[key]
    return from_pure_dict(cfg, tree)
