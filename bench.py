#!/usr/bin/env python3
"""Trie-attention fwd+bwd throughput on one MI355X (BASELINE.json metric).

One step = one forward (agpt_attn_fwd) and one backward (agpt_attn_bwd) over
every node-token of the synthetic trie of the chosen config (default C2:
1.1M-char order-5 Markov corpus, 65 symbols, Zipf 1.1, depth 32,
d_model 128 = 8 heads x 16, fp32). Inputs are resident in HBM before timing.
Prints one JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import platform
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = ("trie-attn fwd+bwd node-tokens/sec (1 GPU, depth 32); % of HBM/MFMA roofline")
HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, published
MFMA_PEAK_TFLOPS = {"f32": 157.3, "bf16": 2500.0}  # MI355X dense matrix peaks


def log(msg: str) -> None:
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


class HipEvents:
    """hipEvent_t handles via the HIP runtime (timed on the launch stream)."""

    def __init__(self):
        import torch  # noqa: F401  (loads libamdhip64 into the process)
        self.lib = C.CDLL("libamdhip64.so")
        self.lib.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.lib.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        self.lib.hipEventSynchronize.argtypes = [C.c_void_p]
        self.lib.hipEventDestroy.argtypes = [C.c_void_p]
        self.lib.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]

    def create(self, n: int) -> list[int]:
        out = []
        for _ in range(n):
            e = C.c_void_p()
            assert self.lib.hipEventCreate(C.byref(e)) == 0
            out.append(e.value)
        return out

    def record(self, e: int, stream: int) -> None:
        assert self.lib.hipEventRecord(C.c_void_p(e), C.c_void_p(stream)) == 0

    def ms(self, a: int, b: int) -> float:
        assert self.lib.hipEventSynchronize(C.c_void_p(b)) == 0
        f = C.c_float()
        assert self.lib.hipEventElapsedTime(C.byref(f), C.c_void_p(a), C.c_void_p(b)) == 0
        return f.value

    def destroy(self, evs: list[int]) -> None:
        for e in evs:
            self.lib.hipEventDestroy(C.c_void_p(e))


def bytes_per_token(D: int, H: int, b_in: int) -> dict:
    """HBM bytes per node-token, one layer. "step" is the compulsory
    (flash-standard) total: fwd reads Q,K,V and writes O, lse; bwd reads
    Q,K,V,O,dO,lse and writes dQ,dK,dV (fp32). The per-kernel figures are
    each kernel's own minimal I/O."""
    fwd = 4 * D * b_in + 4 * H
    bwd = 5 * D * b_in + 4 * H + 3 * D * 4
    return {"step": fwd + bwd, "trie_fwd": fwd, "trie_bwd": bwd,
            # split backward: the query half reads Q,K,V,O,dO,lse and writes
            # dQ and δ; the key half reads Q,K,V,dO,lse,δ and writes dK,dV
            "trie_bwd_q": 5 * D * b_in + 4 * H + D * 4 + 4 * H,
            "trie_bwd_kv": 4 * D * b_in + 8 * H + 2 * D * 4}


def make_inputs(tr, D, H, hd, dtype, seed, dev):
    """Q, K, V from node embeddings X = tok_emb[token] + pos_emb[depth-1]
    projected by N(0, 0.02^2) weights (the config's stated init); dO ~ N(0,1)."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    T = tr.n_nodes
    vocab = int(tr.token.max()) + 1
    tok_emb = torch.randn(vocab, D, generator=g, device=dev)
    pos_emb = torch.randn(tr.max_depth, D, generator=g, device=dev)
    tok = torch.from_numpy(tr.token.astype(np.int64)).to(dev)
    dep = torch.from_numpy((tr.depth - 1).astype(np.int64)).to(dev)
    outs = []
    for _ in range(3):
        w = torch.randn(D, D, generator=g, device=dev) * 0.02
        y = torch.empty(T, D, device=dev, dtype=dtype)
        step = 1 << 22
        for s in range(0, T, step):
            x = tok_emb[tok[s:s + step]] + pos_emb[dep[s:s + step]]
            y[s:s + step] = (x @ w).to(dtype)
        outs.append(y)
    d_o = torch.empty(T, D, device=dev, dtype=dtype)
    for s in range(0, T, 1 << 22):
        d_o[s:s + (1 << 22)] = torch.randn(min(1 << 22, T - s), D, generator=g, device=dev).to(dtype)
    del tok, dep
    return outs[0], outs[1], outs[2], d_o


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), else the platform's."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(tr, q, k, v, d_o, H, hd, rows: int, reps: int = 5) -> dict:
    """The oracle (single-threaded C restatement of the Crystal CPU loops)
    over the first `rows` DFS rows of the same trie and tensors: the median
    of `reps` repetitions."""
    from oracle import oracle as ORC
    M = min(rows, tr.n_nodes)
    par = tr.parent[:M]
    dep = tr.depth[:M]
    Q, K, V, G = (x[:M].float().cpu().numpy() for x in (q, k, v, d_o))
    scale = float(np.float32(1.0 / np.sqrt(hd)))
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        O, W, _ = ORC.fwd(par, Q, K, V, H, hd, scale, depth=dep)
        ORC.bwd(par, Q, K, V, W, G, H, hd, scale, depth=dep)
        times.append(time.perf_counter() - t0)
        del O, W
    dt = float(np.median(times))
    return {"value": M / dt, "unit": "node-tokens/s", "cores": 1, "kind": "port",
            "sample": (f"first {M} DFS rows of the same trie (a closed sub-forest, "
                       f"{int(dep.astype(np.int64).sum())} keys attended), same Q/K/V/dO, "
                       f"oracle fwd+bwd (C restatement of cpu_grouped_attention + "
                       f"optimized_attention_backward_head + accumulators), 1 thread, "
                       f"median of {reps} reps ({min(times):.2f}-{max(times):.2f} s each) on "
                       f"{cpu_model()}, nproc {os.cpu_count()}")}


LOSS_METRIC = "AGPT per-query loss (softmax + targets + d_logits) queries/sec (1 GPU)"


def loss_inputs(tr, V: int, seed: int):
    """The radix query layout of the trie (one query per node-token, radix
    nodes in DFS order) with its tokens as the intermediate targets, and as
    each endpoint's next-token counts its child edges' first tokens with
    seeded counts 1..40 (the trie builder keeps no corpus counts)."""
    rng = np.random.default_rng(seed)
    heads = np.flatnonzero(tr.radix_head)
    R = heads.shape[0]
    q2n = (np.cumsum(tr.radix_head) - 1).astype(np.int32)
    qoff = np.append(heads, tr.n_nodes).astype(np.int32)
    rpar = q2n[tr.parent[heads]]
    rpar[tr.parent[heads] < 0] = -1
    kids = np.flatnonzero(rpar >= 0)  # child radix nodes, grouped by parent (DFS order keeps them sorted)
    order = kids[np.argsort(rpar[kids], kind="stable")]
    cnt = np.bincount(rpar[kids], minlength=R)
    coff = np.zeros(R + 1, np.int64)
    np.cumsum(cnt, out=coff[1:])
    ctok = tr.token[heads[order]].astype(np.int32) % V
    cval = rng.integers(1, 41, ctok.shape[0]).astype(np.int32)
    return dict(query_to_node=q2n, query_offsets=qoff, radix_ids=np.arange(R, dtype=np.int32),
                token_ids=(tr.token % V).astype(np.int32), counts_offset=coff.astype(np.int32),
                counts_tok=ctok, counts_val=cval)


def bench_loss(args, tr, V: int) -> int:
    """One step = agpt_loss_per_query over every query of the trie (T_q =
    node-tokens) with logits [T_q, V] resident; algorithmic bytes per query:
    logits read + d_logits write (8V) + loss write, query_to_node and the
    next token read (12)."""
    import torch
    from agpt_amd import loss as L

    dev = torch.device("cuda:0")
    b = loss_inputs(tr, V, seed=77)
    T_q = tr.n_nodes
    idx = [torch.from_numpy(b[k]).to(dev) for k in ("query_to_node", "query_offsets", "radix_ids",
                                                     "token_ids", "counts_offset", "counts_tok",
                                                     "counts_val")]
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    logits = torch.randn(T_q, V, generator=g, device=dev) * 2.0
    d_logits = torch.empty_like(logits)
    loss_out = torch.empty(T_q, device=dev)
    torch.cuda.synchronize()
    log(f"loss inputs resident: T_q {T_q}, V {V}, {torch.cuda.memory_allocated() / 2**30:.1f} GiB")

    def step():
        L.loss_per_query(logits, *idx, d_logits=d_logits, loss_out=loss_out)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    hev = HipEvents()
    evs = [hev.create(2) for _ in range(args.steps)]
    stream = torch.cuda.current_stream(dev).cuda_stream
    t0 = time.perf_counter()
    for e in evs:
        hev.record(e[0], stream)
        step()
        hev.record(e[1], stream)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    k_ms = float(np.mean([hev.ms(a, c) for a, c in evs]))
    for e in evs:
        hev.destroy(e)
    per_q = 8 * V + 12
    achieved = per_q * T_q / (k_ms * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu:
        from oracle import oracle as ORC
        M = min(args.cpu_rows, T_q)
        end = int(np.searchsorted(b["query_offsets"], M, side="right")) - 1  # whole radix nodes
        M = int(b["query_offsets"][end])
        lg = logits[:M].cpu().numpy()
        sub = dict(b, query_to_node=b["query_to_node"][:M], token_ids=b["token_ids"][:M])
        t0c = time.perf_counter()
        ORC.loss_per_query(lg, sub["query_to_node"], sub["query_offsets"], sub["radix_ids"],
                           sub["token_ids"], sub["counts_offset"], sub["counts_tok"], sub["counts_val"])
        dt = time.perf_counter() - t0c
        cpu = {"value": M / dt, "unit": "queries/s", "cores": 1, "kind": "port",
               "sample": f"first {M} queries (whole radix nodes) of the same batch, oracle "
                         f"(C restatement of agpt_loss_per_query_kernel), 1 thread, {dt:.1f} s"}
    out = {
        "metric": LOSS_METRIC, "value": T_q * args.steps / elapsed, "unit": "queries/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": elapsed / args.steps * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded Markov corpus -> radix trie queries; random logits and counts)",
        "config": {"workload": f"{args.workload}: per-query AGPT loss over every node-token",
                   "queries": T_q, "radix_nodes": int(b["radix_ids"].shape[0]), "vocab": V,
                   "count_entries": int(b["counts_tok"].shape[0])},
        "roofline": {"bound": "hbm", "kernel": "agpt_loss", "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "traffic": load_traffic(f"agpt_loss_{args.workload}"),
                     "algorithmic_bytes_per_launch": per_q * T_q, "avg_launch_ms": k_ms},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


VARLEN_METRIC = ("packed varlen drop-ins (agpt_varlen_attention + _backward) fwd+bwd node-tokens/sec "
                 "(1 GPU, the reference's packed layout)")


def pack_paths(parent: np.ndarray, depth: np.ndarray, nodes: np.ndarray | None = None):
    """The reference's packed layout (batched_depth_forward.cr:668-742): node
    n's rows are its root-to-node path, depth[n] of them, nodes in order (all
    nodes, or the given ones). Returns (kv_offsets, kv_lengths, rows)."""
    if nodes is None:
        nodes = np.arange(parent.shape[0], dtype=np.int64)
    nodes = np.asarray(nodes, np.int64)
    T = nodes.shape[0]
    depth = depth[nodes]
    maxd = int(depth.max())
    anc = np.full((T, maxd), -1, np.int64)
    cur = nodes.copy()
    pos = depth.astype(np.int64) - 1
    for _ in range(maxd):
        ok = pos >= 0
        if not ok.any():
            break
        anc[np.flatnonzero(ok), pos[ok]] = cur[ok]
        cur = np.where(ok, parent[np.maximum(cur, 0)], cur)
        pos = pos - 1
    rows = anc[anc >= 0]  # row-major: node by node, root first
    lens = depth.astype(np.int32)
    offs = np.zeros(T, np.int64)
    offs[1:] = np.cumsum(lens.astype(np.int64))[:-1]
    return offs, lens, rows


def bench_varlen(args, tr) -> int:
    """One step = agpt_varlen_attention then agpt_varlen_attention_backward
    over every node of the trie in the reference's packed layout (each node
    carries its own copy of its path's K/V rows: L = Σ depth packed rows).
    Algorithmic bytes per step, fp32: forward q, packed K, V read, O and the
    saved weights written; backward q, dO, packed K, V and the weights read,
    dQ and the packed dK, dV written: 20·T·D + 24·L·D + 8·L·H."""
    import torch
    from agpt_amd import attention as A

    dev = torch.device("cuda:0")
    from agpt_amd import trie as trie_mod
    cfg = trie_mod.CONFIGS[args.workload]
    H, hd = cfg["H"], cfg["hd"]
    D = H * hd
    T = tr.n_nodes
    radix = args.varlen_layout == "radix"
    if radix:
        # the chunk packer's layout (agpt_train.cu:4456-4479): the queries of
        # radix node r are its edge rows; its packed rows are the path to its
        # last row, shared by its queries
        heads = np.flatnonzero(tr.radix_head)
        qoff = np.append(heads, T).astype(np.int32)
        elen = np.diff(qoff)
        q2n = np.repeat(np.arange(heads.shape[0], dtype=np.int32), elen)
        offs, lens, rows = pack_paths(tr.parent, tr.depth, qoff[1:] - 1)
        # visible keys of query t of node r: len - L + j + 1
        vis = (lens[q2n] - elen[q2n] + (np.arange(T) - qoff[q2n]) + 1).astype(np.int64)
    else:
        offs, lens, rows = pack_paths(tr.parent, tr.depth)
        vis = lens.astype(np.int64)
    if offs[-1] + lens[-1] >= 2**31:
        print("bench.py: --path varlen: packed rows exceed the int32 offsets of the drop-in API; "
              "use a smaller --scale", file=sys.stderr)
        return 2
    L = int(rows.shape[0])
    max_len = int(lens.max())
    q, k, v, d_o = make_inputs(tr, D, H, hd, torch.float32, seed=1234, dev=dev)
    ridx = torch.from_numpy(rows).to(dev)
    kp = k.index_select(0, ridx)
    vp = v.index_select(0, ridx)
    del k, v, ridx
    offs_d = torch.from_numpy(offs.astype(np.int32)).to(dev)
    lens_d = torch.from_numpy(lens).to(dev)
    out = torch.empty(T * D, device=dev)
    w = torch.zeros(T * H * max_len, device=dev)
    dq = torch.empty(T * D, device=dev)
    dk = torch.empty(L * D, device=dev)
    dv = torch.empty(L * D, device=dev)
    scale = A.default_scale(hd)
    torch.cuda.synchronize()
    log(f"varlen inputs resident: T {T}, packed rows {L}, max_len {max_len}, "
        f"{torch.cuda.memory_allocated() / 2**30:.1f} GiB")
    stream = torch.cuda.current_stream(dev).cuda_stream

    if radix:
        q2n_d = torch.from_numpy(q2n).to(dev)
        qoff_d = torch.from_numpy(qoff).to(dev)

    def step(e=None):
        if e is not None:
            hev.record(e[0], stream)
        if radix:
            A.batched_varlen_attention_L_queries(q, kp, vp, q2n_d, qoff_d, offs_d, lens_d, out, w, T, H, hd,
                                                 max_len, scale)
        else:
            A.batched_varlen_attention(q, kp, vp, offs_d, lens_d, out, w, T, H, hd, max_len, scale)
        if e is not None:
            hev.record(e[1], stream)
        if radix:  # accumulates into dk, dv
            A.batched_varlen_attention_L_queries_backward(q, kp, vp, w, d_o, q2n_d, qoff_d, offs_d, lens_d,
                                                          dq, dk, dv, T, H, hd, max_len, scale)
        else:
            A.batched_varlen_attention_backward(q, kp, vp, w, d_o, offs_d, lens_d, dq, dk, dv, T, H, hd,
                                                max_len, scale)
        if e is not None:
            hev.record(e[2], stream)

    hev = HipEvents()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    evs = [hev.create(3) for _ in range(args.steps)]
    t0 = time.perf_counter()
    for e in evs:
        step(e)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    f_ms = float(np.mean([hev.ms(e[0], e[1]) for e in evs]))
    b_ms = float(np.mean([hev.ms(e[1], e[2]) for e in evs]))
    for e in evs:
        hev.destroy(e)
    W = int(vis.sum())  # weights written by the forward, read by the backward
    fwd_bytes = 4 * (2 * T * D + 2 * L * D + W * H)
    bwd_bytes = 4 * (3 * T * D + (6 if radix else 4) * L * D + W * H)  # radix: dK, dV read and added to
    dom, dom_ms, dom_bytes = ("varlen_bwd", b_ms, bwd_bytes) if b_ms >= f_ms else ("varlen_fwd", f_ms, fwd_bytes)
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9
    step_ms = elapsed / args.steps * 1e3
    cpu = None
    if not args.no_cpu and radix:
        from oracle import oracle as ORC
        R = int(np.searchsorted(qoff, min(args.cpu_rows // 8, T), side="right")) - 1  # whole radix nodes
        R = max(R, 1)
        Tm = int(qoff[R])
        Lm = int(offs[R - 1] + lens[R - 1])
        qm, gm = q[:Tm].cpu().numpy(), d_o[:Tm].cpu().numpy()
        km, vm = kp[:Lm].cpu().numpy(), vp[:Lm].cpu().numpy()
        om = offs[:R].astype(np.int32)
        reps = 0
        t0c = time.perf_counter()
        while True:  # repeat the bounded sample to about 10 s of CPU work
            o_r, w_r = ORC.varlen_L_fwd(qm, km, vm, q2n[:Tm], qoff[:R + 1], om, lens[:R], Tm, H, hd, max_len, scale)
            ORC.varlen_L_bwd(qm, km, vm, w_r, gm, q2n[:Tm], qoff[:R + 1], om, lens[:R], Tm, H, hd, max_len, scale,
                             Lm)
            reps += 1
            dt = time.perf_counter() - t0c
            if dt >= 10.0:
                break
        cpu = {"value": Tm * reps / dt, "unit": "node-tokens/s", "cores": 1, "kind": "port",
               "sample": f"first {R} radix nodes ({Tm} queries, {Lm} packed rows) of the same layout, oracle "
                         f"L-query forward + backward (C restatement of the packed path), {reps} passes, "
                         f"1 thread, {dt:.1f} s",
               "cpu_model": cpu_model()}
    if not args.no_cpu and not radix:
        from oracle import oracle as ORC
        M = min(args.cpu_rows // 8, T)
        Lm = int(offs[M - 1] + lens[M - 1]) if M < T else L
        qm = q[:M].cpu().numpy()
        km = kp[:Lm].cpu().numpy()
        vm = vp[:Lm].cpu().numpy()
        gm = d_o[:M].cpu().numpy()
        om = offs[:M].astype(np.int32)
        reps = 0
        t0c = time.perf_counter()
        while True:  # repeat the bounded sample to about 10 s of CPU work
            o_r, w_r = ORC.varlen_fwd(qm, km, vm, om, lens[:M], M, H, hd, max_len, scale)
            ORC.varlen_bwd(qm, km, vm, w_r, gm, om, lens[:M], M, H, hd, max_len, scale, Lm)
            reps += 1
            dt = time.perf_counter() - t0c
            if dt >= 10.0:
                break
        cpu = {"value": M * reps / dt, "unit": "node-tokens/s", "cores": 1, "kind": "port",
               "sample": f"first {M} nodes ({Lm} packed rows) of the same layout, oracle varlen "
                         f"forward + backward (C restatement of the packed path), {reps} passes, "
                         f"1 thread, {dt:.1f} s",
               "cpu_model": cpu_model()}
    res = {
        "metric": VARLEN_METRIC, "value": T * args.steps / elapsed, "unit": "node-tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": step_ms, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded Markov corpus -> radix trie, packed per node; random-init projections)",
        "config": {"workload": f"{args.workload} packed varlen drop-ins, "
                               f"{'radix-node queries (L-query API)' if radix else 'one query per node'}",
                   "node_tokens": T,
                   "packed_rows": L, "max_len": max_len, "d_model": D, "heads": H, "head_dim": hd,
                   "corpus_scale": args.scale},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": achieved, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS, "traffic": None,
                     "algorithmic_bytes_per_launch": dom_bytes, "avg_launch_ms": dom_ms},
        "step_roofline": {"bytes_per_step": fwd_bytes + bwd_bytes,
                          "achieved_GBps": (fwd_bytes + bwd_bytes) / (step_ms * 1e-3) / 1e9,
                          "frac": (fwd_bytes + bwd_bytes) / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBS},
        "kernel_avg_ms": {"varlen_fwd": f_ms, "varlen_bwd": b_ms},
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)
    return 0


C3_METRIC = "C3 training step node-tokens/sec (4-layer µGPT over the C1 trie: fwd+bwd+RMSProp, 1 GPU)"


def bench_c3(args) -> int:
    """One step = forward and backward of the 4-layer model over every
    batch of whole root-child subtrees of the C1 trie (<= 1M rows each),
    then one RMSProp update (agpt_amd.model). HIP events around every
    trie-attention call give the attention share of the step."""
    import torch
    from agpt_amd import model, trie as trie_mod

    dev = torch.device("cuda:0")
    log(f"building C1 trie with counts (scale {args.scale})")
    tr = trie_mod.config_trie("C1", args.scale, counts=True)
    cfg = model.ModelConfig(vocab=65, d_model=128, n_heads=8, n_layers=4, d_ff=512, max_depth=32, norm="rms")
    m = model.TrieGPT(cfg, device=dev, seed=1)
    m.plan(tr, max_rows=1 << 20)
    log(f"C3: {tr.n_nodes} node-tokens in {len(m.groups)} batches; {m.flat.numel()} parameters")
    hev = HipEvents()
    pool: list[int] = []
    stream = torch.cuda.current_stream(dev).cuda_stream

    def hook():
        e = hev.create(1)[0]
        hev.record(e, stream)
        pool.append(e)

    for _ in range(args.warmup):
        m.step()
    torch.cuda.synchronize()
    m.attn_hook = hook
    step_ms, attn_ms, losses = [], [], []
    for _ in range(args.steps):
        pool.clear()
        t0 = time.perf_counter()
        lv = m.step()
        torch.cuda.synchronize()
        step_ms.append((time.perf_counter() - t0) * 1e3)
        attn_ms.append(sum(hev.ms(pool[i], pool[i + 1]) for i in range(0, len(pool), 2)))
        hev.destroy(pool)
        losses.append(float(lv))
    m.attn_hook = None
    ms = float(np.mean(step_ms))
    am = float(np.mean(attn_ms))
    log(f"C3 step {ms:.2f} ms, trie attention {am:.2f} ms ({am / ms:.1%}); loss {losses[0]:.4g} -> {losses[-1]:.4g}")
    out = {
        "metric": C3_METRIC, "value": tr.n_nodes * 1e3 / ms, "unit": "node-tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded order-3 Markov corpus -> C1 trie with counts; random-init weights)",
        "config": {"workload": "C3: 4-layer training step on the C1 trie", "node_tokens": tr.n_nodes,
                   "batches": len(m.groups), "d_model": 128, "heads": 8, "layers": 4, "d_ff": 512,
                   "vocab": 65, "norm": "rms", "optimizer": "rmsprop(beta=0.999, lr=3e-4)",
                   "loss": "per-query AGPT loss, linear mass weights"},
        "attention_ms_per_step": am, "attention_share": am / ms,
        "loss_first_last": [losses[0], losses[-1]],
        "cpu_baseline": None,
    }
    print(json.dumps(out), flush=True)
    m.close()
    return 0


FULL_METRIC = ("trie-attn fwd+bwd node-tokens/sec over a whole corpus's trie, batch by batch "
               "(1 GPU, exact range batches)")


def bench_full(args) -> int:
    """A corpus whose trie does not fit one GPU (full-size C4: ~6e8
    node-tokens, 0.6 TB per bf16 [T, 512] tensor), processed batch by batch
    on one GPU. The trie is built one root-child subtree at a time
    (agpt_trie_build_radix_part, on host threads ahead of the GPU); each
    subtree is cut at its bigram partitions into batches of at most
    --batch-rows rows, each planned alone with its context rows (the
    ancestors before it) packed in front (agpt_attn_plan_range, packed: the
    batch returns the context rows' dK/dV share, for their owner batch to
    add). Per batch: its inputs are made on the GPU, then W untimed and K
    timed fwd+bwd steps with HIP events; the job's time is the sum over the
    batches of their mean step, and value = node-tokens / that time."""
    import gc
    from concurrent.futures import ThreadPoolExecutor

    import torch
    from agpt_amd import trie as trie_mod
    from agpt_amd.attention import TrieAttention, partition_starts, range_batches

    dev = torch.device("cuda:0")
    cfg = trie_mod.CONFIGS[args.workload]
    H, hd = cfg["H"], cfg["hd"]
    D = H * hd
    dtype = torch.float32 if cfg["dtype"] == "f32" else torch.bfloat16
    b_in = 4 if cfg["dtype"] == "f32" else 2
    batch_rows = args.batch_rows or (12 << 20)
    n = max(2, int(cfg["n"] * args.scale))
    log(f"{args.workload} full: corpus of {n} tokens")
    t0 = time.time()
    tok = trie_mod.markov_corpus(n, cfg["order"], cfg["vocab"], cfg["zipf"], cfg["seed"])
    log(f"corpus in {time.time() - t0:.1f}s; building {cfg['vocab']} root-child subtrees on host threads")
    g = torch.Generator(device=dev)
    g.manual_seed(1234)
    tok_emb = torch.randn(cfg["vocab"], D, generator=g, device=dev)
    pos_emb = torch.randn(cfg["depth"], D, generator=g, device=dev)
    ws = [torch.randn(D, D, generator=g, device=dev) * 0.02 for _ in range(3)]
    hev = HipEvents()
    stream = torch.cuda.current_stream(dev).cuda_stream
    total_rows, total_ms, n_batches, sum_depth, max_rows = 0, 0.0, 0, 0, 0
    k_sum = {}
    desc = ""
    pool = ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1))
    futs = [pool.submit(trie_mod.build_radix_part, tok, cfg["depth"], x) for x in range(cfg["vocab"])]
    t_job = time.time()
    for x, fut in enumerate(futs):
        tr = fut.result()
        futs[x] = None
        if tr.n_nodes == 0:
            continue
        ranges = range_batches(tr.n_nodes, batch_rows, partition_starts(tr.radix_head, tr.depth))
        tk = torch.from_numpy(tr.token.astype(np.int64))
        dp = torch.from_numpy((tr.depth - 1).astype(np.int64))
        for a, b in ranges:
            att = TrieAttention(H, hd, max_depth=cfg["depth"], dtype=dtype)
            att.plan_range(tr.parent, a, b, packed=True)
            ctx = []
            r = int(tr.parent[a])
            while r >= 0:
                ctx.append(r)
                r = int(tr.parent[r])
            rows = torch.cat([torch.tensor(ctx[::-1], dtype=torch.int64), torch.arange(a, b)])
            T = int(rows.shape[0])
            ti, di = tk[rows].to(dev), dp[rows].to(dev)
            qkv = []
            for w in ws:
                y = torch.empty(T, D, device=dev, dtype=dtype)
                for s0 in range(0, T, 1 << 22):
                    xe = tok_emb[ti[s0:s0 + (1 << 22)]] + pos_emb[di[s0:s0 + (1 << 22)]]
                    y[s0:s0 + (1 << 22)] = (xe @ w).to(dtype)
                qkv.append(y)
            d_o = torch.empty(T, D, device=dev, dtype=dtype)
            for s0 in range(0, T, 1 << 22):
                d_o[s0:s0 + (1 << 22)] = torch.randn(min(1 << 22, T - s0), D, generator=g, device=dev).to(dtype)
            o = torch.empty(T, D, device=dev, dtype=dtype)
            lse = torch.empty(T, H, device=dev, dtype=torch.float32)
            grads = tuple(torch.empty(T, D, device=dev, dtype=torch.float32) for _ in range(3))
            q, k, v = qkv
            for _ in range(args.warmup):
                att.forward(q, k, v, out=o, lse=lse)
                att.backward(q, k, v, o, lse, d_o, out=grads)
            evs = [(hev.create(2), hev.create(5)) for _ in range(args.steps)]
            steps = []
            for fe, be in evs:
                e0, e1 = hev.create(2)
                hev.record(e0, stream)
                att.forward(q, k, v, out=o, lse=lse, events=fe)
                att.backward(q, k, v, o, lse, d_o, out=grads, events=be)
                hev.record(e1, stream)
                steps.append((e0, e1))
            torch.cuda.synchronize()
            ms = float(np.mean([hev.ms(e0, e1) for e0, e1 in steps]))
            desc = att.describe()
            for fe, be in evs:
                for name, (i, j) in (("trie_fwd", (fe[0], fe[1])), ("trie_bwd_q", (be[0], be[1])),
                                     ("trie_bwd_kv", (be[1], be[2])), ("trie_bwd_tail", (be[2], be[4]))):
                    k_sum[name] = k_sum.get(name, 0.0) + hev.ms(i, j) / args.steps
                hev.destroy(fe + be)
            for e0, e1 in steps:
                hev.destroy([e0, e1])
            nb = b - a
            total_rows += nb
            total_ms += ms
            sum_depth += int(tr.depth[a:b].astype(np.int64).sum())
            max_rows = max(max_rows, nb)
            n_batches += 1
            att.close()
            del q, k, v, d_o, o, lse, grads, qkv, ti, di, att
            gc.collect()
            torch.cuda.empty_cache()
            if n_batches % 8 == 0:
                log(f"{n_batches} batches, {total_rows} node-tokens, {total_ms:.0f} ms of steps")
        del tr, tk, dp
    pool.shutdown()
    log(f"{n_batches} batches over {total_rows} node-tokens in {time.time() - t_job:.0f}s of job time")
    bpt = bytes_per_token(D, H, b_in)
    value = total_rows / (total_ms * 1e-3)
    gbs = bpt["step"] * total_rows / (total_ms * 1e-3) / 1e9
    out = {
        "metric": FULL_METRIC, "value": value, "unit": "node-tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": total_ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": cfg["dtype"],
        "data": "synthetic (seeded Markov corpus -> radix trie built per root child; random-init projections)",
        "config": {"workload": f"{args.workload} at corpus scale {args.scale}, batch by batch",
                   "node_tokens": total_rows, "sum_depth": sum_depth, "batches": n_batches,
                   "largest_batch_rows": max_rows, "batch_rows": batch_rows, "d_model": D, "heads": H,
                   "head_dim": hd, "kernel": desc,
                   "timing": "per batch: inputs made on the GPU, then warmup and timed steps; "
                             "ms_per_step = sum over batches of the mean step"},
        "step_roofline": {"bytes_per_node_token": bpt["step"], "achieved_GBps": gbs, "frac": gbs / HBM_PEAK_GBS},
        "kernel_ms_per_pass": k_sum,
        "cpu_baseline": None,
    }
    print(json.dumps(out), flush=True)
    return 0


def load_traffic(name: str):
    """HBM bytes per launch of the dominant kernel from the committed
    rocprofv3 PMC summary (FETCH_SIZE + WRITE_SIZE, copy-kernel scaled)."""
    p = ROOT / "profiles" / f"traffic_{name}.json"
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text()).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def load_counters(workload: str, kernel: str) -> dict | None:
    """The committed rocprofv3 counters of one kernel on one workload
    (profiles/counters_<workload>.json: MfmaUtil, VALUBusy, occupancy,
    FETCH_SIZE / WRITE_SIZE scaled to HBM bytes, and the commit measured)."""
    p = ROOT / "profiles" / f"counters_{workload}.json"
    if not p.exists():
        return None
    try:
        d = json.loads(p.read_text())
    except (OSError, ValueError):
        return None
    k = d.get("kernels", {}).get(kernel)
    if k is None:
        return None
    return {"commit": d.get("commit"), **k}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="C2", choices=["C1", "C2", "C4", "C5"])
    ap.add_argument("--path", default="attn", choices=["attn", "loss", "c3", "varlen"],
                    help="attn: trie attention fwd+bwd (the headline); loss: per-query AGPT loss; "
                         "c3: the 4-layer training step of config C3 (C1 trie); varlen: the packed "
                         "varlen drop-ins a renaming caller gets (fp32 workloads)")
    ap.add_argument("--vocab", type=int, default=65, help="loss path: vocabulary size V")
    ap.add_argument("--varlen-layout", default="node", choices=["node", "radix"],
                    help="varlen path: one query per node (agpt_varlen_attention) or the queries of "
                         "each radix node over its shared prefix (agpt_varlen_attention_L_queries)")
    ap.add_argument("--scale", type=float, default=None,
                    help="corpus scale (1 = BASELINE size; default: 1, or the largest share "
                         "one GPU holds)")
    ap.add_argument("--batch-streams", type=int, default=3,
                    help="with --batch-rows: streams the batches are dealt over (1 = one after another)")
    ap.add_argument("--batch-rows", type=int, default=None,
                    help="attn path: batches of whole bigram partitions of at most this many rows, "
                         "one plan each, run in row order (default 0: every partition in one plan)")
    ap.add_argument("--full", action="store_true",
                    help="attn path: build the trie one root-child subtree at a time and run it batch "
                         "by batch (for a corpus whose trie does not fit one GPU, e.g. C4 at --scale 1)")
    ap.add_argument("--events-after", action="store_true",
                    help="attn path: time the steps without the per-kernel HIP events and take the "
                         "kernel times from as many steps again (default with one batch: the events "
                         "ride along in the timed steps)")
    ap.add_argument("--cpu-rows", type=int, default=250_000)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="only run a plain device copy of this many MiB (PMC byte-counter "
                         "calibration) and exit")
    args = ap.parse_args()
    if args.copy_probe_mib:
        import torch
        n = args.copy_probe_mib * (1 << 20) // 4
        src = torch.ones(n, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy probe: 3 copies of {args.copy_probe_mib} MiB "
            f"(read {args.copy_probe_mib} MiB + write {args.copy_probe_mib} MiB each)")
        return 0
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this build runs on one GPU "
              "(sharding the trie by subtree needs no exchange beyond the shared top "
              "rows, but multi-GPU runs are not part of this build)",
              file=sys.stderr)
        return 2

    import torch
    from agpt_amd import trie as trie_mod
    from agpt_amd.attention import RangedTrieAttention, TrieAttention, partition_starts, range_batches

    if args.path == "c3":
        if args.scale is None:
            args.scale = 1.0
        return bench_c3(args)
    cfg = trie_mod.CONFIGS[args.workload]
    if args.full:
        if args.scale is None:
            args.scale = 1.0
        if "chains" in cfg:
            print("bench.py: --full needs a corpus workload (C1, C2, C4)", file=sys.stderr)
            return 2
        return bench_full(args)
    if args.scale is None:
        # the packed layout repeats every path row per node (C2 in full: 0.3 TB per tensor)
        args.scale = 0.05 if args.path == "varlen" else cfg.get("one_gpu_scale", 1.0)
    H, hd = cfg["H"], cfg["hd"]
    D = H * hd
    dtype = torch.float32 if cfg["dtype"] == "f32" else torch.bfloat16
    b_in = 4 if cfg["dtype"] == "f32" else 2
    log(f"building {args.workload} trie (scale {args.scale})")
    t0 = time.time()
    tr = trie_mod.config_trie(args.workload, args.scale)
    T = tr.n_nodes
    log(f"trie: {T} node-tokens, {tr.n_radix} radix nodes, sum depth {tr.sum_depth}, "
        f"max depth {tr.max_depth} ({time.time() - t0:.1f}s)")
    if args.path == "loss":
        return bench_loss(args, tr, args.vocab)
    if args.path == "varlen":
        return bench_varlen(args, tr)
    dev = torch.device("cuda:0")
    # One plan per batch: the whole trie, or contiguous runs of whole bigram
    # partitions of at most --batch-rows rows (each reads its context rows,
    # the ancestors before it, as keys and adds their dK/dV share in place).
    batch_rows = args.batch_rows if args.batch_rows is not None else 0
    starts = partition_starts(tr.radix_head, tr.depth)
    ranges = range_batches(T, batch_rows, starts) if batch_rows > 0 else [(0, T)]
    ratt = None
    if len(ranges) == 1:
        att = TrieAttention(H, hd, max_depth=max(tr.max_depth, 1), dtype=dtype)
        att.plan(tr.parent)
        parts = [att]
    else:
        ratt = RangedTrieAttention(H, hd, tr.parent, ranges, max_depth=max(tr.max_depth, 1), dtype=dtype)
        parts = ratt.parts
    infos = [p.plan_info() for p in parts]
    info = {"n_nodes": T, "n_tiles": sum(i["n_tiles"] for i in infos), "batches": len(parts)}
    batching = (f"one batch: all {starts.shape[0]} bigram partitions in one plan" if len(parts) == 1 else
                f"{len(parts)} batches of whole bigram partitions ({starts.shape[0]} partitions), "
                f"<= {batch_rows} rows each, dealt over {args.batch_streams} stream(s)")
    log(f"plan: {info}; {batching}; kernel: {parts[0].describe()}")
    q, k, v, d_o = make_inputs(tr, D, H, hd, dtype, seed=1234, dev=dev)
    o = torch.empty(T, D, device=dev, dtype=dtype)
    lse = torch.empty(T, H, device=dev, dtype=torch.float32)
    grads = tuple(torch.empty(T, D, device=dev, dtype=torch.float32) for _ in range(3))
    torch.cuda.synchronize()
    log(f"inputs resident: {torch.cuda.memory_allocated() / 2**30:.1f} GiB")

    def step(evs=None):
        # per batch: forward, then backward (the per-subtree trainer's order);
        # batches dealt over --batch-streams streams
        if ratt is not None:
            ratt.fwd_bwd(q, k, v, d_o, out=o, lse=lse, grads=grads, n_streams=args.batch_streams, events=evs)
            return
        for j, att in enumerate(parts):
            att.forward(q, k, v, out=o, lse=lse, events=None if evs is None else evs[j][0])
            att.backward(q, k, v, o, lse, d_o, out=grads, events=None if evs is None else evs[j][1])

    for i in range(args.warmup):
        step()
        torch.cuda.synchronize()
        log(f"warmup step {i + 1}/{args.warmup} done")

    hev = HipEvents()
    # One batch: the per-kernel events ride along in the timed steps, on the
    # library's stream. Many batches, or --events-after: the timed steps run
    # without them (7 event records per batch are work of their own on the
    # stream, ~20 us per step, which a sub-millisecond C5 step shows) and
    # the per-kernel times come from as many steps again with the events,
    # outside the timed region.
    events_in_timed = len(parts) == 1 and not args.events_after
    ev_steps = args.steps
    evs = [[(hev.create(2), hev.create(5)) for _ in parts] for _ in range(ev_steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(evs[i] if events_in_timed else None)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    log(f"timed {args.steps} steps: {elapsed:.3f}s")
    if not events_in_timed:
        for i in range(ev_steps):
            step(evs[i])
        torch.cuda.synchronize()
    desc = parts[0].describe()
    split = "split backward" in desc
    carry = "path-carry" in desc  # one reduction kernel (chunk partials) instead of chunk + reduce
    by_range = "subtree range" in desc or "nothing to reduce" in desc  # no reduction kernel
    names = (["trie_fwd", "trie_bwd_q", "trie_bwd_kv"] if split else ["trie_fwd", "trie_bwd"])
    tail = [] if by_range else ["trie_bwd_carry"] if carry else ["trie_bwd_chunk", "trie_bwd_reduce"]
    k_ms = {n: [] for n in names + tail}
    for step_evs in evs:
        acc = {n: 0.0 for n in k_ms}  # per step: summed over the batches
        for fe, be in step_evs:
            acc["trie_fwd"] += hev.ms(fe[0], fe[1])
            if split:
                acc["trie_bwd_q"] += hev.ms(be[0], be[1])
                acc["trie_bwd_kv"] += hev.ms(be[1], be[2])
            else:
                acc["trie_bwd"] += hev.ms(be[0], be[2])
            if by_range:
                pass
            elif carry:
                acc["trie_bwd_carry"] += hev.ms(be[3], be[4])
            else:
                acc["trie_bwd_chunk"] += hev.ms(be[2], be[3])
                acc["trie_bwd_reduce"] += hev.ms(be[3], be[4])
            hev.destroy(fe + be)
        for n, x in acc.items():
            k_ms[n].append(x)
    avg = {n: float(np.mean(x)) for n, x in k_ms.items()}
    log("kernel avg ms per step: " + ", ".join(f"{n} {m:.3f}" for n, m in avg.items()))

    bpt = bytes_per_token(D, H, b_in)
    kern_bytes = {n: bpt[n] * T for n in names}
    dominant = max(kern_bytes, key=lambda n: avg[n])
    achieved = kern_bytes[dominant] / (avg[dominant] * 1e-3) / 1e9
    ms_step = elapsed / args.steps * 1e3
    value = T * args.steps / elapsed
    step_gbs = bpt["step"] * T / (ms_step * 1e-3) / 1e9

    cpu = None
    if not args.no_cpu:
        log(f"cpu baseline: oracle on the first {args.cpu_rows} rows")
        cpu = cpu_baseline(tr, q, k, v, d_o, H, hd, args.cpu_rows)
        log(f"cpu baseline: {cpu['value']:.0f} node-tokens/s")

    flops = 12.0 * tr.sum_depth * D
    ctr = load_counters(args.workload, dominant) if args.scale == cfg.get("one_gpu_scale", 1.0) else None
    out = {
        "metric": METRIC,
        "value": value,
        "unit": "node-tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg["dtype"],
        "data": "synthetic (seeded Markov corpus -> leveled trie; random-init projections)",
        "config": {
            "workload": f"{args.workload}: single-layer trie attention fwd+bwd",
            "node_tokens": T, "radix_nodes": tr.n_radix, "sum_depth": tr.sum_depth,
            "max_depth": tr.max_depth, "d_model": D, "heads": H, "head_dim": hd,
            "corpus_scale": args.scale, "tiles": info["n_tiles"], "batching": batching,
            "kernel": desc,
            "kernel_events": ("HIP events around each kernel in the timed steps" if events_in_timed else
                              "HIP events around each kernel in as many steps after the timed ones"),
        },
        "roofline": {
            "bound": "hbm", "kernel": dominant, "achieved": achieved, "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
            "traffic": (ctr or {}).get("traffic_bytes"),
            "algorithmic_bytes_per_launch": kern_bytes[dominant],
            "avg_launch_ms": avg[dominant],
            "mfma_util": (ctr or {}).get("mfma_util"),
            "counters": None if ctr is None else {
                "source": f"profiles/counters_{args.workload}.md", "commit": ctr["commit"],
                "mfma_util": ctr["mfma_util"], "valu_busy": ctr["valu_busy"],
                "occupancy": ctr["occupancy"], "lds_bank_conflict": ctr["lds_bank_conflict"],
                "mfma_tflop_executed": (ctr["mfma_flop_f32"] + ctr["mfma_flop_bf16"]) / 1e12},
        },
        "step_roofline": {"bytes_per_node_token": bpt["step"], "achieved_GBps": step_gbs,
                          "frac": step_gbs / HBM_PEAK_GBS,
                          "tflops_algorithmic": flops / (ms_step * 1e-3) / 1e12,
                          # the same useful flops against the dense matrix peak of
                          # the step's input type (plain causal attention's roofline)
                          "mfma_peak_tflops": MFMA_PEAK_TFLOPS[cfg["dtype"]],
                          "mfma_frac": flops / (ms_step * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS[cfg["dtype"]]},
        "kernel_avg_ms": avg,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    for att in parts:
        att.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
