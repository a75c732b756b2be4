"""The packed varlen drop-ins (agpt_varlen_attention{,_backward,_L_queries,
_L_queries_backward}) against the oracle's packed restatement and the trie
oracle, through the C ABI, over head counts (odd ones leave lanes idle) and
head dims (32 and 64 split a head slice over lanes).

Bar: fp32 within 1e-4 relative / 1e-5 absolute.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import assert_close, scale_of, small_trie, tensors
from oracle import oracle as ORC

pytestmark = pytest.mark.gpu


def _pack_nodes(parent, Q, K, V, H, hd):
    """Reference packing (batched_depth_forward.cr:668-742): node i's packed
    prefix = its ancestors' rows then its own, duplicated per node."""
    depth = ORC.depths(parent)
    T = parent.shape[0]
    offs = np.zeros(T, np.int32)
    lens = depth.astype(np.int32)
    offs[1:] = np.cumsum(lens)[:-1]
    rows = []
    for n in range(T):
        path = []
        a = n
        while a >= 0:
            path.append(a)
            a = parent[a]
        rows.extend(path[::-1])
    rows = np.array(rows, np.int64)
    return offs, lens, rows, K[rows], V[rows]


@pytest.mark.parametrize("H,hd", [(4, 8), (1, 4), (3, 16), (8, 16), (2, 32), (5, 32), (16, 64)])
def test_varlen_matches_trie(gpu, H, hd):
    import torch

    from agpt_amd import attention as A
    tr = small_trie(n_tokens=300, depth=9, seed=31)
    T = tr.n_nodes
    D = H * hd
    Q, K, V, G = tensors(T, D, 13)
    scale = scale_of(hd)
    offs, lens, rows, Kp, Vp = _pack_nodes(tr.parent, Q, K, V, H, hd)
    max_len = int(lens.max())
    cu = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    out = torch.zeros(T * D, device="cuda")
    w = torch.zeros(T * H * max_len, device="cuda")
    A.batched_varlen_attention(cu(Q), cu(Kp), cu(Vp), cu(offs), cu(lens), out, w, T, H, hd,
                               max_len, scale)
    o_ref, w_ref = ORC.varlen_fwd(Q, Kp, Vp, offs, lens, T, H, hd, max_len, scale)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), o_ref, what="varlen O")
    assert_close(w.cpu().numpy(), w_ref, what="varlen W")
    unp = torch.empty(T, D, device="cuda")
    A.unpack_batched_attn_output(out, unp, T, H, hd)
    dq = torch.zeros(T * D, device="cuda")
    dk = torch.full((rows.size * D,), 7.0, device="cuda")  # overwritten, not accumulated
    dv = torch.full((rows.size * D,), 7.0, device="cuda")
    A.batched_varlen_attention_backward(cu(Q), cu(Kp), cu(Vp), w, cu(G), cu(offs), cu(lens), dq,
                                        dk, dv, T, H, hd, max_len, scale)
    dq_r, dk_r, dv_r = ORC.varlen_bwd(Q, Kp, Vp, w_ref, G, offs, lens, T, H, hd, max_len, scale,
                                      rows.size)
    torch.cuda.synchronize()
    assert_close(unp.cpu().numpy().ravel(), o_ref, what="unpack")
    assert_close(dq.cpu().numpy(), dq_r, what="varlen dQ")
    assert_close(dk.cpu().numpy(), dk_r, what="varlen dK")
    assert_close(dv.cpu().numpy(), dv_r, what="varlen dV")


@pytest.mark.parametrize("H,hd,kind", [(2, 16, "small"), (3, 8, "small"), (8, 32, "small"), (4, 64, "small"),
                                       (8, 16, "c2"), (2, 16, "chains"), (32, 4, "deep")])
def test_varlen_L_queries(gpu, H, hd, kind):
    """small: a depth-12 trie; c2: a C2-shaped sample (depth 32, 8 x 16);
    chains: radix nodes of 1..300 queries (blocks of 64 queries cut inside
    a node, more (query, head) pairs than lanes); deep: max_len x H past the
    radix-node kernel's δ table (the per-(node, head) fallback)."""
    import torch

    from agpt_amd import attention as A
    from agpt_amd import trie as T_
    if kind == "small":
        tr = small_trie(n_tokens=500, depth=12, seed=41)
    elif kind == "c2":
        tr = T_.config_trie("C2", scale=0.001)
    elif kind == "chains":
        tok = np.concatenate([T_.uniform_tokens(300, 5, 1), T_.uniform_tokens(40, 5, 2)]).astype(np.int32)
        tr = T_.build_radix_trie(tok, 300)
    else:
        tr = small_trie(n_tokens=400, depth=40, seed=43)
    rpar, elen = tr.radix()
    R = rpar.shape[0]
    D = H * hd
    T = tr.n_nodes
    Q, K, V, G = tensors(T, D, 17)
    scale = scale_of(hd)
    # chunk-packer layout (agpt_train.cu:4456-4479): queries of radix node i
    # are its edge rows; its packed prefix = ancestor rows then edge rows.
    heads = np.flatnonzero(tr.radix_head)
    qoff = np.append(heads, T).astype(np.int32)
    q2n = np.repeat(np.arange(R, dtype=np.int32), elen)
    kv_rows = []
    kv_off = np.zeros(R, np.int32)
    kv_len = np.zeros(R, np.int32)
    for r in range(R):
        last = qoff[r + 1] - 1
        path = []
        a = last
        while a >= 0:
            path.append(a)
            a = tr.parent[a]
        kv_off[r] = len(kv_rows)
        kv_len[r] = len(path)
        kv_rows.extend(path[::-1])
    kv_rows = np.array(kv_rows, np.int64)
    Kp, Vp = K[kv_rows], V[kv_rows]
    max_kv = int(kv_len.max())
    cu = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    out = torch.zeros(T * D, device="cuda")
    w = torch.zeros(T * H * max_kv, device="cuda")
    A.batched_varlen_attention_L_queries(cu(Q), cu(Kp), cu(Vp), cu(q2n), cu(qoff), cu(kv_off),
                                         cu(kv_len), out, w, T, H, hd, max_kv, scale)
    o_ref, w_ref = ORC.varlen_L_fwd(Q, Kp, Vp, q2n, qoff, kv_off, kv_len, T, H, hd, max_kv, scale)
    # the radix layout is the trie semantics: same outputs as the trie oracle
    O_trie, _, _ = ORC.fwd(tr.parent, Q, K, V, H, hd, scale)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), o_ref, what="L O")
    # the saved weights: every visible entry (query t of node r sees
    # kv_len[r] - L_r + j + 1 rows)
    vis = kv_len[q2n] - elen[q2n] + (np.arange(T) - qoff[q2n]) + 1
    mask = (np.arange(max_kv)[None, None, :] < vis[:, None, None]) & np.ones((T, H, 1), bool)
    wg = w.cpu().numpy().reshape(T, H, max_kv)
    assert_close(wg[mask], w_ref.reshape(T, H, max_kv)[mask], what="L weights")
    assert_close(o_ref.reshape(T, D), O_trie, what="L oracle vs trie oracle")
    dq = torch.zeros(T * D, device="cuda")
    seed_k = np.random.default_rng(3).standard_normal(kv_rows.size * D).astype(np.float32)
    dk = cu(seed_k.copy())
    dv = cu(seed_k.copy())
    A.batched_varlen_attention_L_queries_backward(cu(Q), cu(Kp), cu(Vp), w, cu(G), cu(q2n),
                                                  cu(qoff), cu(kv_off), cu(kv_len), dq, dk, dv, T,
                                                  H, hd, max_kv, scale)
    dq_r, dk_r, dv_r = ORC.varlen_L_bwd(Q, Kp, Vp, w_ref, G, q2n, qoff, kv_off, kv_len, T, H, hd,
                                        max_kv, scale, kv_rows.size, dk=seed_k, dv=seed_k)
    torch.cuda.synchronize()
    assert_close(dq.cpu().numpy(), dq_r, what="L dQ")
    assert_close(dk.cpu().numpy(), dk_r, what="L dK")
    assert_close(dv.cpu().numpy(), dv_r, what="L dV")
