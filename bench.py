#!/usr/bin/env python3
"""Speculative-decoding throughput on one MI355X.

Workload (default `--config cfg4`, BASELINE configs[3], the metric's
"d24+d4, bs32"): target d24 (D 1536, 12 heads of 128, 12 KV heads, vocab
65536, max_seq_len 2048, SSSL with short window 1024), draft = 4 layers
sharing the target's layers 0-3 and wte / lm_head; random-init N(0, 0.02)
weights drawn on the device (seed 2), bf16 weights / KV cache with fp32
accumulation; batch 32, prompts of 1024 uniform random ids, 512 new tokens,
draft_steps 6, temperature 0.8 rejection sampling, Philox seed 2, no top-k.

A "step" is one speculative round for the whole batch (k draft steps,
the (k+1)-token verify, accept/reject, bookkeeping, one host sync). Prompt
prefill and `--warmup` rounds are untimed; then `--steps` rounds (0 = until
every row has its max_tokens) are timed between two synchronisations.
value = tokens emitted in the timed rounds (accepted drafts + corrections +
bonus tokens, counted up to max_tokens per row) / timed seconds.

roofline: the verify-pass attention (flash-decode, the dominant HBM
consumer) timed with HIP events on the engine's stream, at the state the
timed run ends in, walking every layer's cache in turn (so the 256 MB
Infinity Cache holds no layer between calls, as in a real round); S
(window 1024) and L (full) layers are timed apart and weighted 18:6 like the
d24 SSSL stack. Algorithmic bytes per launch = the distinct visible K and V
bytes of every row (read once) + Q + O.

cpu_baseline: the CPU restatement of the reference algorithm (oracle/,
literal mode: token-by-token verify and full re-prefill on rejection) on
the same architecture with the same weights, batch 1, on a bounded sample.
"""

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

CONFIGS = {
    # name: (target cfg kwargs, draft layers, batch, prompt, new, k, temperature, seed)
    "cfg2": (dict(sequence_len=2048, vocab_size=65536, n_layer=12, n_head=6, n_kv_head=6, n_embd=768,
                  window_pattern="SSSL", short_window=1024), 2, 1, 512, 256, 4, 0.0, 0),
    "cfg4": (dict(sequence_len=2048, vocab_size=65536, n_layer=24, n_head=12, n_kv_head=12, n_embd=1536,
                  window_pattern="SSSL", short_window=1024), 4, 32, 1024, 512, 6, 0.8, 2),
    "cfg5": (dict(sequence_len=8192, vocab_size=65536, n_layer=24, n_head=12, n_kv_head=4, n_embd=1536,
                  window_pattern="SSSL", short_window=2048), 4, 128, 6144, 1024, 8, 0.0, 3),
}
HBM_PEAK_GBS = 8000.0
# HBM bytes / algorithmic bytes of the verify attention (k_attn_mfma, one key
# split, no combine), from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE passes
# over `bench.py --roofline-only`, each scaled by the counter's reading for a
# 256 MiB copy (FETCH_SIZE x2.0, WRITE_SIZE x1.0); see profiles/.
ATTN_TRAFFIC_RATIO = 1.02


def attention_roofline(sess, n_rep=3):
    """Time the verify attention at the session's current lengths: every row
    feeds k+1 queries (one pending token and k drafts) at its cache length.
    Each timed pass walks all layers in order (7.4 GB of K/V at cfg4), so no
    layer is served from the 256 MB Infinity Cache, as in a real round."""
    import torch
    from flaxchat_amd import _lib
    T = sess.T
    B, k = sess.B, sess.k
    W = k + 1
    dev = T.device
    s = sess.stream
    t_len = sess.bufs["t_len"].cpu().numpy().astype(np.int64)
    q = torch.randn(B * W, T.H, T.hd, device=dev).to(torch.bfloat16)
    y = torch.empty(((B * W + 15) // 16 * 16, T.H * T.hd), device=dev, dtype=torch.bfloat16)
    start = sess.bufs["t_len"].clone()
    row_off = torch.arange(0, B * W + 1, W, dtype=torch.int32, device=dev)
    cap = sess.tcache.cap
    es = 2
    layer_elems = B * T.G * cap * T.hd
    launches = []
    for layer in range(T.L):
        win = T.windows[layer]
        max_keys = min(cap, win + W) if win > 0 else cap
        nb = _lib.lib().fc_attention_workspace_bytes(B, W, T.H, T.G, T.hd, max_keys)
        launches.append((layer, win, max_keys, torch.empty(max(nb, 1), dtype=torch.uint8, device=dev)))

    def run_all(sel):
        for layer, win, max_keys, ws in launches:
            if not sel(win):
                continue
            kp = sess.tcache.k.data_ptr() + layer * layer_elems * es
            vp = sess.tcache.v.data_ptr() + layer * layer_elems * es
            _lib.check(_lib.lib().fc_attention(q.data_ptr(), kp, vp, y.data_ptr(), B, B * W, W, T.H, T.G, T.hd, cap,
                                               row_off.data_ptr(), start.data_ptr(), win, max_keys, 1,
                                               ws.data_ptr(), ws.numel(), s.cuda_stream), "attention")

    torch.cuda.synchronize()  # inputs above were made on the default stream; the launches use the engine's
    res = {}
    short = lambda w: 0 < w < T.config.sequence_len
    for name, sel in (("S", short), ("L", lambda w: not short(w))):
        n_layers = sum(1 for _, w, _, _ in launches if sel(w))
        with torch.cuda.stream(s):
            run_all(sel)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            for _ in range(n_rep):
                run_all(sel)
            e1.record(s)
        e1.synchronize()
        ms = e0.elapsed_time(e1) / (n_rep * n_layers)
        win = next(w for _, w, _, _ in launches if sel(w))
        # distinct visible keys per row: full layer 0..pos_last; window layer
        # from max(0, pos_first - window) to pos_last
        pos_last = t_len + W - 1
        lo = np.maximum(0, t_len - win) if short(win) else np.zeros_like(t_len)
        keys = (pos_last - lo + 1).sum()
        kv_bytes = keys * T.G * T.hd * 2 * es
        qo_bytes = 2 * B * W * T.H * T.hd * es
        res[name] = dict(ms=ms, bytes=int(kv_bytes + qo_bytes), layers=n_layers)
    nS, nL = res["S"]["layers"], res["L"]["layers"]
    tot_b = nS * res["S"]["bytes"] + nL * res["L"]["bytes"]
    tot_s = (nS * res["S"]["ms"] + nL * res["L"]["ms"]) / 1e3
    return dict(achieved=tot_b / tot_s / 1e9, per_launch_bytes=tot_b / T.L, per_launch_us=tot_s / T.L * 1e6,
                S=res["S"], L=res["L"], nS=nS, nL=nL)


def lm_head_gemv(dev, M=32, N=65536, K=1536, n_copies=3, n_rep=4):
    """The draft lm_head as the engine runs it (fc_gemm at the draft step's row
    count: the kernel and tiles the engine's plan picks for it, non-temporal
    weight loads, softcap epilogue into fp32 logits; cfg4: 32 rows on the
    LDS-shared 32 x 64 tiles), weights cycled over `n_copies` copies so
    every launch reads them from HBM. GB/s of algorithmic bytes (weights +
    activations + logits) and us per launch."""
    import torch
    from flaxchat_amd import _lib
    w = torch.ones((n_copies, N, K), dtype=torch.bfloat16, device=dev)
    a = torch.ones((M, K), dtype=torch.bfloat16, device=dev)
    out = torch.empty((M, N), dtype=torch.float32, device=dev)
    s = torch.cuda.current_stream(dev)
    run = lambda i: _lib.check(_lib.lib().fc_gemm(a.data_ptr(), w[i % n_copies].data_ptr(), out.data_ptr(),  # noqa: E731
                                                  M, N, K, _lib.FC_BF16, _lib.EPI_SOFTCAP, s.cuda_stream), "fc_gemm")
    for i in range(n_copies):
        run(i)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for i in range(n_rep * n_copies):
        run(i)
    e1.record(s)
    e1.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (n_rep * n_copies)
    nbytes = N * K * 2 + M * K * 2 + M * N * 4
    del w, a, out
    return {"kernel": f"draft lm_head ({M} x {N} x {K}, softcap)", "us": round(us, 2),
            "achieved": round(nbytes / us / 1e3, 1), "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}


def copy_ceiling(dev, n_bytes=1 << 30, n_rep=5):
    """Measured streaming ceiling: a device-to-device copy of `n_bytes`
    (the runtime's copy kernel), rated by the bytes it reads plus writes."""
    import torch
    src = torch.empty(n_bytes, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(n_rep):
        dst.copy_(src)
    e1.record()
    e1.synchronize()
    gbs = 2 * n_bytes * n_rep / (e0.elapsed_time(e1) / 1e3) / 1e9
    del src, dst
    return gbs


def read_ceiling(dev, n_bytes=1 << 30, n_rep=5, n_buf=1, grids=(1024, 2048, 4096, 8192, 16384)):
    """Measured HBM read ceiling: fc_read_probe (each workgroup streams a
    contiguous share with 16-byte non-temporal loads, nothing written) over
    `n_bytes`, the best of a few grid sizes, rated by the bytes it reads.
    Below the 256 MB Infinity Cache, `n_buf` buffers are read in turn so no
    launch finds its bytes cached."""
    import torch
    from flaxchat_amd import _lib
    n_bytes -= n_bytes % 4096
    srcs = [torch.empty(n_bytes, dtype=torch.uint8, device=dev) for _ in range(n_buf)]
    out = torch.empty(4 * 16384, dtype=torch.int32, device=dev)
    s = torch.cuda.current_stream(dev)
    best = 0.0
    for wgs in grids:
        run = lambda i: _lib.check(_lib.lib().fc_read_probe(srcs[i % n_buf].data_ptr(), n_bytes,  # noqa: E731
                                                            out.data_ptr(), wgs, s.cuda_stream), "fc_read_probe")
        for i in range(n_buf):
            run(i)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for i in range(n_rep * n_buf):
            run(i)
        e1.record(s)
        e1.synchronize()
        best = max(best, n_bytes * n_rep * n_buf / (e0.elapsed_time(e1) / 1e3) / 1e9)
    del srcs, out
    return best


def walk_ceiling(dev, units, n_bytes, n_rep=5, n_buf=3):
    """The verify attention's own load walk without its compute
    (fc_walk_probe): `units` workgroups (rows x KV groups), each reading its
    share of `n_bytes` as 16 KB tiles, four waves taking every fourth tile
    with sixteen 1 KB non-temporal loads each; `n_buf` buffers read in turn
    so no launch finds its bytes in the Infinity Cache. GB/s."""
    import torch
    from flaxchat_amd import _lib
    tiles = max(1, int(round(n_bytes / (units * 16384))))
    nb = units * tiles * 16384
    srcs = [torch.ones(nb, dtype=torch.uint8, device=dev) for _ in range(n_buf)]
    out = torch.empty(256 * units, dtype=torch.int32, device=dev)
    s = torch.cuda.current_stream(dev)
    run = lambda i: _lib.check(_lib.lib().fc_walk_probe(srcs[i % n_buf].data_ptr(), units, tiles,  # noqa: E731
                                                        out.data_ptr(), s.cuda_stream), "fc_walk_probe")
    for i in range(n_buf):
        run(i)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for i in range(n_rep * n_buf):
        run(i)
    e1.record(s)
    e1.synchronize()
    res = nb * n_rep * n_buf / (e0.elapsed_time(e1) / 1e3) / 1e9
    del srcs, out
    return res


# The cfg4 verify GEMMs (224 packed tokens) and draft-step GEMMs (32 rows)
# at the tilings the engine's plan gives them: (name, M, N, K, tile_m,
# tile_n, K splits)
GEMM_TILINGS = [("verify_qkv_32x128", 224, 4608, 1536, 32, 128, 1),
                ("verify_attn_cproj_32x32", 224, 1536, 1536, 32, 32, 1),
                ("verify_c_fc_64x64", 224, 6144, 1536, 64, 64, 1),
                ("verify_mlp_cproj_64x96_split4", 224, 1536, 6144, 64, 96, 4),
                ("draft_qkv_32x32", 32, 4608, 1536, 32, 32, 1),
                ("draft_attn_cproj_32x16", 32, 1536, 1536, 32, 16, 1),
                ("draft_c_fc_32x32", 32, 6144, 1536, 32, 32, 1),
                ("draft_mlp_cproj_32x16_split8", 32, 1536, 6144, 32, 16, 8),
                ("draft_lm_head_32x64", 32, 65536, 1536, 32, 64, 1)]


def gemm_walks(dev, n_rep=4, pool_bytes=640 << 20):
    """The cfg4 GEMMs' operand walks without their arithmetic
    (fc_gemm_walk_probe) at the engine's tilings, with direct-to-LDS loads
    and with register loads: the activation operand L2-resident (one buffer,
    as its producer just wrote it), the weights cycled over copies filling
    `pool_bytes` so every launch reads them from HBM, as in a round.
    {name: {"lds_us", "reg_us": per launch, "l2_to_cu_mb": the bytes the
    CUs read}}."""
    import torch
    from flaxchat_amd import _lib
    pool = torch.ones(pool_bytes, dtype=torch.uint8, device=dev)
    s = torch.cuda.current_stream(dev)
    res = {}
    for name, M, N, K, tm, tn, S in GEMM_TILINGS:
        a = torch.ones((M + 15) // 16 * 16 * K * 2, dtype=torch.uint8, device=dev)
        wb = N * K * 2
        n_copies = pool_bytes // wb
        out = torch.empty(_lib.lib().fc_gemm_walk_probe_words(M, N, tm, tn, S), dtype=torch.int32, device=dev)
        mt = (M + tm - 1) // tm
        res[name] = {"l2_to_cu_mb": round(mt * (N // tn) * K * 2 * (tm + tn) / 1e6, 1)}
        for key, reg in (("lds_us", 0), ("reg_us", 1)):
            run = lambda i: _lib.check(_lib.lib().fc_gemm_walk_probe(  # noqa: E731
                a.data_ptr(), pool.data_ptr() + (i % n_copies) * wb, M, N, K, tm, tn, S, reg, out.data_ptr(),
                s.cuda_stream), "fc_gemm_walk_probe")
            for i in range(n_copies):
                run(i)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            for i in range(n_rep * n_copies):
                run(i)
            e1.record(s)
            e1.synchronize()
            res[name][key] = round(e0.elapsed_time(e1) * 1e3 / (n_rep * n_copies), 2)
        del a, out
    del pool
    return res


def l2_ceiling(dev, region=1 << 20, n_bytes=1 << 30, n_rep=5, grids=(256, 512, 1024)):
    """Measured L2-to-CU read ceiling: fc_l2_read_probe (each XCD's workgroups
    read a 1 MB region that stays in that XCD's L2, direct-to-LDS loads)
    over `n_bytes`, per grid size (256 = one workgroup per CU, the occupancy
    of the verify GEMMs): {workgroups: GB/s}."""
    import torch
    from flaxchat_amd import _lib
    src = torch.ones(8 * region, dtype=torch.uint8, device=dev)
    out = torch.empty(4 * max(grids), dtype=torch.int32, device=dev)
    s = torch.cuda.current_stream(dev)
    res = {}
    for wgs in grids:
        per = n_bytes // wgs // 65536 * 65536
        run = lambda: _lib.check(_lib.lib().fc_l2_read_probe(src.data_ptr(), region, n_bytes, out.data_ptr(),  # noqa: E731
                                                             wgs, s.cuda_stream), "fc_l2_read_probe")
        run()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(n_rep):
            run()
        e1.record(s)
        e1.synchronize()
        res[wgs] = round(per * wgs * n_rep / (e0.elapsed_time(e1) / 1e3) / 1e9, 1)
    del src, out
    return res


def gemm_calibration(n_iter=20, n_copies=4):
    """fc_gemm (fragment-order operands, store epilogue) against torch.matmul
    (hipBLASLt) on the cfg4 engine's GEMM shapes; `n_copies` weight copies are
    cycled so no launch finds its weights in the Infinity Cache."""
    import torch
    from flaxchat_amd import _lib
    from flaxchat_amd.runtime import pack_operand
    dev = torch.device("cuda", torch.cuda.current_device())
    s = torch.cuda.current_stream()
    out = []
    for (label, M, N, K) in [("draft c_q|c_k|c_v", 32, 4608, 1536), ("draft c_fc", 32, 6144, 1536),
                             ("draft c_proj (mlp)", 32, 1536, 6144), ("draft lm_head", 32, 65536, 1536),
                             ("verify c_q|c_k|c_v", 224, 4608, 1536), ("verify c_fc", 224, 6144, 1536),
                             ("verify c_proj (mlp)", 224, 1536, 6144), ("verify lm_head", 224, 65536, 1536)]:
        A = torch.randn(M, K, device=dev).to(torch.bfloat16)
        Ws = [torch.randn(N, K, device=dev).mul_(0.02).to(torch.bfloat16) for _ in range(n_copies)]
        Ap = pack_operand(A) if M % 32 == 0 else None
        Wps = [pack_operand(w) for w in Ws]
        C = torch.empty(M, N, device=dev)
        torch.cuda.synchronize()

        def t_of(fn):
            for i in range(n_copies):
                fn(i)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            for i in range(n_iter):
                fn(i % n_copies)
            e1.record(s)
            e1.synchronize()
            return e0.elapsed_time(e1) / n_iter * 1e3

        ours = t_of(lambda i: _lib.check(_lib.lib().fc_gemm(Ap.data_ptr(), Wps[i].data_ptr(), C.data_ptr(), M, N, K,
                                                            _lib.FC_BF16, 0, s.cuda_stream), "fc_gemm"))
        blas = t_of(lambda i: torch.matmul(A, Ws[i].t()))
        out.append(dict(gemm=label, M=M, N=N, K=K, weight_mb=round(N * K * 2 / 1e6, 1), fc_gemm_us=round(ours, 1),
                        hipblaslt_us=round(blas, 1)))
        del Ws, Wps
    return out


def cpu_baseline(dm_t, dm_d, cfg_name, seed, k, temperature, budget_s=25.0, at_position=None, p_reject=None,
                 accepted=None):
    """The oracle's literal-mode generate_speculative on host cores."""
    from flaxchat_amd.runtime import to_host
    from oracle.spec import spec_literal
    try:
        from threadpoolctl import threadpool_info
        cores = max([i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"] or [1])
    except Exception:
        cores = 1
    ht = to_host(dm_t)
    hd = to_host(dm_d)
    V = dm_t.V
    prompt = np.random.default_rng(seed).integers(0, V, 64).tolist()
    new = 48
    t0 = time.perf_counter()
    out = spec_literal(ht, hd, prompt, max_tokens=new, temperature=temperature, top_k=None, seed=seed,
                       draft_steps=k)
    dt = time.perf_counter() - t0
    res = {"value": round((len(out) - len(prompt)) / dt, 4), "unit": "tokens/s", "cores": int(cores),
           "kind": "port",
           "sample": f"oracle spec_literal (restatement of flaxchat/engine.py:410-608, fp32 numpy) on the "
                     f"{cfg_name} architecture and weights, batch 1, prompt 64 ids (not the full prompt), "
                     f"{new} new tokens, k={k}, T={temperature}, including prefill; {dt:.1f} s"}
    if at_position and p_reject is not None and accepted is not None:
        # one per-token forward of each model at the workload's context length
        # (the cache holds zeros: the cost does not depend on the values)
        from oracle.model import OracleModel
        cost = {}
        for name, m in (("target", ht), ("draft", hd)):
            om = OracleModel(m)
            st = om.new_state(at_position + 8)
            om.step(1, at_position - 1, st)
            t1 = time.perf_counter()
            for i in range(3):
                om.step(2 + i, at_position + i, st)
            cost[name] = (time.perf_counter() - t1) / 3
        # the literal loop per round: k draft steps, k target steps, and on a
        # mid-round rejection a re-prefill of both models over the whole
        # sequence (flaxchat/engine.py:492-523, 593-606)
        round_s = k * (cost["draft"] + cost["target"]) + p_reject * at_position * (cost["draft"] + cost["target"])
        res["per_token_forward_ms_at_context"] = {"context": at_position, "target": round(cost["target"] * 1e3, 1),
                                                  "draft": round(cost["draft"] * 1e3, 1)}
        res["estimate_at_context"] = {
            "tokens_per_s": round(accepted / round_s, 5),
            "how": f"extrapolated, not measured: per round {k} draft + {k} target forwards plus, with the "
                   f"GPU run's mid-round rejection rate {p_reject:.2f}, a re-prefill of both models over "
                   f"{at_position} positions; {accepted:.2f} tokens per round (the GPU run's mean)"}
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=0, help="timed rounds (0 = until every row is done)")
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", default="cfg4", choices=sorted(CONFIGS))
    ap.add_argument("--top-k", type=int, default=0)
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-roofline", action="store_true")
    ap.add_argument("--no-full-run", action="store_true",
                    help="stop after the timed rounds (profiling passes); full_run is then null")
    ap.add_argument("--no-topk-line", action="store_true",
                    help="skip the second measurement with the drop-in default top_k=40")
    ap.add_argument("--gemm-calibration", action="store_true",
                    help="time fc_gemm against torch.matmul (hipBLASLt) on the cfg4 GEMM shapes and exit")
    ap.add_argument("--roofline-only", action="store_true",
                    help="prefill + warmup rounds, then only the verify-attention timing and a 256 MiB copy "
                         "(the counter-calibration kernel); for rocprofv3 --pmc passes")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only; the speculative engine shards over the batch "
              "(one full replica per GPU, no collective in the decode loop), which is not built here.",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from flaxchat_amd.config import GPTConfig
    from flaxchat_amd.engine import SpecSession
    from flaxchat_amd.runtime import DeviceModel

    if args.gemm_calibration:
        for row in gemm_calibration():
            print(json.dumps(row), flush=True)
        return

    tk, n_draft, B, P, new, k, temp, seed = CONFIGS[args.config]
    cfg = GPTConfig(**tk)
    t_init = time.perf_counter()
    target = DeviceModel.random_init(cfg, seed=seed, dtype="bf16")
    draft = target.make_draft(n_draft)
    prompts = np.random.default_rng(seed).integers(0, cfg.vocab_size, (B, P)).tolist()
    sess = SpecSession(target, draft, prompts, new, temp, args.top_k or None, seed, k, use_graph=not args.no_graph)
    torch.cuda.synchronize()
    t_pre = time.perf_counter()
    sess.prefill()
    sess.stream.synchronize()
    prefill_s = time.perf_counter() - t_pre
    print(f"[bench] init {t_pre - t_init:.1f}s prefill {prefill_s:.2f}s ({B}x{P} tokens)", file=sys.stderr, flush=True)
    if args.warmup:
        sess.run(max_rounds=args.warmup)
    if args.roofline_only:
        r = attention_roofline(sess)
        src = torch.empty(1 << 28, dtype=torch.uint8, device=target.device)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"verify_attention": r, "copy_bytes": 1 << 28}))
        return
    done_before = sess.emitted_tokens()
    rounds_before = sess.rounds
    sess.stream.synchronize()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    sess.run(max_rounds=args.steps or None)
    sess.stream.synchronize()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    steps = sess.rounds - rounds_before
    toks = sess.emitted_tokens() - done_before
    acc = np.concatenate(sess.accept_hist) if sess.accept_hist else np.zeros(1)
    print(f"[bench] {steps} rounds {toks} tokens {el:.3f}s mean accepted/round {acc.mean():.2f}",
          file=sys.stderr, flush=True)
    # the rest of the run (to every row's max_tokens) and the whole timed + rest
    # figure: tail rounds still pay for finished rows
    full_run = None
    if not args.no_full_run:
        t1 = time.perf_counter()
        sess.run()
        sess.stream.synchronize()
        el_all = el + (time.perf_counter() - t1)
        steps_all = sess.rounds - rounds_before
        toks_all = sess.emitted_tokens() - done_before
        full_run = {"rounds": int(steps_all), "tokens": int(toks_all),
                    "ms_per_round": round(el_all / max(steps_all, 1) * 1e3, 3),
                    "tokens_per_s": round(toks_all / el_all, 2),
                    "what": "timed window plus the remaining rounds until every row has max_tokens"}
        print(f"[bench] full run: {steps_all} rounds {toks_all} tokens {el_all:.3f}s", file=sys.stderr, flush=True)
    acc_all = np.concatenate(sess.accept_hist) if sess.accept_hist else np.zeros(1)
    p_reject = float(np.mean(acc_all < k)) if sess.accept_hist else None

    roof = None
    if not args.no_roofline:
        r = attention_roofline(sess)
        ceil = copy_ceiling(target.device)
        rceil = read_ceiling(target.device)
        # the same probe over one attention launch's bytes: its launch ramp and drain weigh as much
        rceil_l = read_ceiling(target.device, n_bytes=int(r["per_launch_bytes"]), n_buf=3,
                               grids=(256, 512, 1024, 2048, 4096))
        l2c = l2_ceiling(target.device)
        # the attention's own grid and tile walk without its compute
        wceil = walk_ceiling(target.device, sess.B * sess.T.G, int(r["per_launch_bytes"]))
        # the GEMMs' operand walks at their tilings (cfg4 shapes)
        gwalks = gemm_walks(target.device) if args.config == "cfg4" else None
        # the largest GEMV of a draft step, against the same HBM peak
        gemv = lm_head_gemv(target.device, M=sess.B, K=sess.T.D) if sess.B <= 32 else None
        roof = {"bound": "hbm", "achieved": round(r["achieved"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(r["achieved"] / HBM_PEAK_GBS, 4),
                "traffic": int(r["per_launch_bytes"] * ATTN_TRAFFIC_RATIO),
                "kernel": "k_attn_mfma (verify, k+1 queries per row, one key split)",
                "per_launch_bytes": int(r["per_launch_bytes"]), "per_launch_us": round(r["per_launch_us"], 2),
                "S_layer": r["S"], "L_layer": r["L"],
                "copy_ceiling": round(ceil, 1), "frac_of_copy_ceiling": round(r["achieved"] / ceil, 4),
                "read_ceiling": round(rceil, 1), "frac_of_read_ceiling": round(r["achieved"] / rceil, 4),
                "read_ceiling_launch_bytes": round(rceil_l, 1),
                "frac_of_read_ceiling_launch_bytes": round(r["achieved"] / rceil_l, 4),
                "walk_ceiling": round(wceil, 1), "frac_of_walk_ceiling": round(r["achieved"] / wceil, 4),
                "l2_read_ceiling_by_workgroups": l2c,
                "gemm_walks": gwalks,
                "draft_lm_head_gemv": gemv}
        print(f"[bench] verify attention {r['achieved']:.0f} GB/s (1 GiB copy: {ceil:.0f} GB/s, "
              f"1 GiB streaming read: {rceil:.0f} GB/s, streaming read of one launch's "
              f"{r['per_launch_bytes'] / 1e6:.0f} MB: {rceil_l:.0f} GB/s; its own load walk: {wceil:.0f} GB/s; "
              f"L2-resident read by workgroups: {l2c})",
              file=sys.stderr, flush=True)
    topk_line = None
    prefill_warm_s = None
    if not args.no_topk_line and not args.top_k and temp > 0:
        # the same workload with generate_speculative's default top_k=40
        # (flaxchat/engine.py:411): same prompts, steps and warm-up
        s2 = SpecSession(target, draft, prompts, new, temp, 40, seed, k, use_graph=not args.no_graph)
        torch.cuda.synchronize()
        t_p2 = time.perf_counter()
        s2.prefill()
        s2.stream.synchronize()
        # the same prefill again, its kernels loaded and the GPU out of idle
        prefill_warm_s = time.perf_counter() - t_p2
        if args.warmup:
            s2.run(max_rounds=args.warmup)
        b2, r2 = s2.emitted_tokens(), s2.rounds
        s2.stream.synchronize()
        t2 = time.perf_counter()
        s2.run(max_rounds=args.steps or None)
        s2.stream.synchronize()
        e2 = time.perf_counter() - t2
        n2, k2 = s2.rounds - r2, s2.emitted_tokens() - b2
        a2 = np.concatenate(s2.accept_hist) if s2.accept_hist else np.zeros(1)
        topk_line = {"top_k": 40, "rounds": int(n2), "ms_per_round": round(e2 / max(n2, 1) * 1e3, 3),
                     "tokens_per_s": round(k2 / e2, 2), "mean_accepted_per_round": round(float(a2.mean()), 3)}
        s2.close()
        del s2
        torch.cuda.empty_cache()
        print(f"[bench] top_k=40: {n2} rounds {k2} tokens {e2:.3f}s", file=sys.stderr, flush=True)
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(target, draft, args.config, seed, k, temp, at_position=P, p_reject=p_reject,
                           accepted=float(acc_all.mean()))
    out = {
        "metric": "spec-decode accepted tokens/s (d24+d4, bs32); verify-attn % HBM peak",
        "value": round(toks / el, 2), "unit": "tokens/s", "n_gpus": 1, "steps": int(steps),
        "warmup": int(args.warmup), "ms_per_step": round(el / max(steps, 1) * 1e3, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (uniform random prompt ids, random-init N(0,0.02) weights)",
        "config": {"workload": f"{args.config}: d{cfg.n_layer}+d{n_draft} D{cfg.n_embd} H{cfg.n_head} "
                               f"G{cfg.n_kv_head} V{cfg.vocab_size}, batch {B}, prompt {P}, {new} new, "
                               f"k={k}, T={temp}, top_k={args.top_k or None}, Philox seed {seed}",
                   "global_batch": B, "seq_len": P + new, "parallelism": "single GPU",
                   "graph": not args.no_graph},
        "mean_accepted_per_round": round(float(acc.mean()), 3),
        "full_run": full_run,
        "top_k_default": topk_line,
        "prefill_s": round(prefill_s, 3),
        "prefill_warm_s": None if prefill_warm_s is None else round(prefill_warm_s, 3),
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
