"""The headline C2 workload at full size (the bench's configuration: 31.5M
node-tokens, radix trie at depth 32, 8 heads x 16, fp32), through the C ABI.

The CPU oracle cannot run at this size in a test, so parity here rests on
what the mathematics fixes, each checked against a float64 evaluation on
the GPU:
  * exact rows: 4,096 sampled queries (O, lse, dQ from a float64 softmax
    over their own paths) and 512 sampled keys with small subtrees (dK, dV
    summed over every query of the subtree in float64);
  * sum over all rows of dV = sum over all rows of dO, per column (each
    query's weights sum to 1);
  * sum over all rows of dK = 0 without RoPE (each query's dS sums to 0);
  * a second fwd+bwd gives identical bytes (fixed-order reductions).
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import ATOL_F32, RTOL_F32, assert_close, scale_of

pytestmark = pytest.mark.gpu


def _paths(parent: np.ndarray, depth: np.ndarray, rows: np.ndarray, P: int) -> np.ndarray:
    """[len(rows), P] ancestor rows of each row, root first, -1 padded."""
    out = np.full((rows.shape[0], P), -1, np.int64)
    cur = rows.astype(np.int64)
    d = depth[rows].astype(np.int64)
    for step in range(P):
        live = cur >= 0
        col = d - 1 - step
        ok = live & (col >= 0)
        out[np.flatnonzero(ok), col[ok]] = cur[ok]
        cur = np.where(live, parent[np.maximum(cur, 0)], -1)
    return out


def _f64_rows(torch, q, k, v, g, path_idx, H, hd, scale):
    """float64 softmax attention of queries over their paths (last path
    entry = the query row). Returns o, lse, dq [N, H, hd] / [N, H] and the
    weights w and dS [N, H, P] for key-side sums."""
    dev = q.device
    pi = torch.from_numpy(path_idx).to(dev)
    N, P = pi.shape
    valid = pi >= 0
    safe = pi.clamp(min=0)
    qrow = pi.gather(1, (valid.sum(1, keepdim=True) - 1))[:, 0]
    Qn = q[qrow].double().view(N, H, hd)
    Kp = k[safe.view(-1)].double().view(N, P, H, hd)
    Vp = v[safe.view(-1)].double().view(N, P, H, hd)
    Gn = g[qrow].double().view(N, H, hd)
    # elementwise products and sums (no batched BLAS calls)
    s = (Qn[:, None] * Kp).sum(-1).transpose(1, 2) * scale          # [N, H, P]
    s = s.masked_fill(~valid[:, None, :], float("-inf"))
    lse = torch.logsumexp(s, -1)
    w = torch.exp(s - lse[..., None])
    o = (w.transpose(1, 2)[..., None] * Vp).sum(1)                 # [N, H, hd]
    dw = (Gn[:, None] * Vp).sum(-1).transpose(1, 2)
    delta = (w * dw).sum(-1, keepdim=True)
    ds = w * (dw - delta) * scale
    dq = (ds.transpose(1, 2)[..., None] * Kp).sum(1)
    return o, lse, dq, w, ds, Qn, Gn


def test_c2_full_size(gpu):
    import torch

    from agpt_amd import trie
    from agpt_amd.attention import TrieAttention

    print("building the C2 trie", flush=True)
    tr = trie.config_trie("C2")
    T, H, hd = tr.n_nodes, 8, 16
    D = H * hd
    assert T > 30_000_000 and tr.max_depth == 32
    att = TrieAttention(H, hd, max_depth=32)
    att.plan(tr.parent)
    print("planned:", att.describe(), flush=True)
    gen = torch.Generator(device=gpu).manual_seed(2)
    q, k, v, g = (torch.randn(T, D, device=gpu, generator=gen) for _ in range(4))
    o, lse = att.forward(q, k, v)
    dq, dk, dv = att.backward(q, k, v, o, lse, g)
    torch.cuda.synchronize()
    print("fwd+bwd done", flush=True)
    scale = scale_of(hd)

    # exact rows: sampled queries
    rng = np.random.default_rng(0)
    rows = np.sort(rng.choice(T, 4096, replace=False))
    pidx = _paths(tr.parent, tr.depth, rows, 32)
    o64, lse64, dq64, *_ = _f64_rows(torch, q, k, v, g, pidx, H, hd, scale)
    rt = torch.from_numpy(rows).to(gpu)
    assert_close(o[rt].cpu().numpy(), o64.reshape(-1, D).cpu().numpy(), what="O rows")
    assert_close(lse[rt].cpu().numpy(), lse64.cpu().numpy(), what="lse rows")
    assert_close(dq[rt].cpu().numpy(), dq64.reshape(-1, D).cpu().numpy(), what="dQ rows")

    # exact rows: sampled keys with subtrees of at most 256 rows, summed over
    # every query of the subtree
    size = tr.subtree_end.astype(np.int64) - np.arange(T)
    cand = np.flatnonzero((size >= 2) & (size <= 256))
    keys = np.sort(rng.choice(cand, 512, replace=False))
    qs = np.concatenate([np.arange(a, tr.subtree_end[a]) for a in keys])
    own = np.repeat(np.arange(keys.shape[0]), size[keys])  # which sampled key each query serves
    pidx = _paths(tr.parent, tr.depth, qs, 32)
    _, _, _, w, ds, Qn, Gn = _f64_rows(torch, q, k, v, g, pidx, H, hd, scale)
    col = torch.from_numpy(tr.depth[keys].astype(np.int64) - 1).to(gpu)[torch.from_numpy(own).to(gpu)]
    wa = w.gather(2, col.view(-1, 1, 1).expand(-1, H, 1))[..., 0]    # [Nq, H] weight of the key
    dsa = ds.gather(2, col.view(-1, 1, 1).expand(-1, H, 1))[..., 0]
    ot = torch.from_numpy(own).to(gpu)
    dk64 = torch.zeros(keys.shape[0], H, hd, dtype=torch.float64, device=gpu).index_add_(0, ot, dsa[..., None] * Qn)
    dv64 = torch.zeros(keys.shape[0], H, hd, dtype=torch.float64, device=gpu).index_add_(0, ot, wa[..., None] * Gn)
    kt = torch.from_numpy(keys).to(gpu)
    assert_close(dv[kt].cpu().numpy(), dv64.reshape(-1, D).cpu().numpy(), what="dV rows")
    assert_close(dk[kt].cpu().numpy(), dk64.reshape(-1, D).cpu().numpy(), RTOL_F32, ATOL_F32, what="dK rows",
                 row_scale=hd)
    print("sampled rows match", flush=True)

    # whole-trie identities, summed in float64 over row slices
    def colsum(x):
        acc = torch.zeros(D, dtype=torch.float64, device=gpu)
        mag = torch.zeros(D, dtype=torch.float64, device=gpu)
        for a in range(0, T, 1 << 22):
            blk = x[a:a + (1 << 22)].double()
            acc += blk.sum(0)
            mag += blk.abs().sum(0)
        return acc, mag

    sdv, _ = colsum(dv)
    sg, mg = colsum(g)
    assert torch.all((sdv - sg).abs() <= 1e-6 * mg + 1e-3), float((sdv - sg).abs().max())
    sdk, mk = colsum(dk)
    assert torch.all(sdk.abs() <= 1e-6 * mk + 1e-3), float(sdk.abs().max())

    # bitwise-equal rerun
    o2, lse2 = att.forward(q, k, v)
    assert torch.equal(o, o2) and torch.equal(lse, lse2)
    del o2, lse2
    dq2, dk2, dv2 = att.backward(q, k, v, o, lse, g)
    assert torch.equal(dq, dq2) and torch.equal(dk, dk2) and torch.equal(dv, dv2)
    att.close()
