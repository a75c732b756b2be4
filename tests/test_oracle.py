"""Pins the CPU oracle (oracle/trie_attn_oracle.c) — CPU only.

Each check is chosen so that a plausible mistake (a dropped ancestor term, a
transposed operand, a missing scale, a wrong rotation direction, a wrong
sign) fails at least one of them:
  1. the spec's own two-formulation agreement on its closed-form model
     (spec/agpt_backward_attention_spec.cr:299-538, tolerance 1e-5);
  2. brute force: masked dense attention softmax(QKᵀ·s + log M)·V in torch
     float64 with autograd through RoPE (a library routine, not reference
     code) — pins forward, lse and all gradients incl. the subtree sums;
  3. a chain trie equals dense causal attention (torch SDPA, is_causal);
  4. central finite differences of L = Σ O·G;
  5. closed forms and invariants (p = 1, Σw = 1, constant keys, sibling
     order, packed-varlen layout == trie layout);
  6. planted mistakes: variants with one of the mistakes above must fail 2.
"""
from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import assert_close, scale_of, small_trie, tensors
from oracle import oracle as ORC

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import spec_model as SM  # noqa: E402


# ---------------------------------------------------------------- brute force

def _rope_t(x, pos, H, hd, inverse=False):
    T = x.shape[0]
    xr = x.view(T, H, hd // 2, 2)
    i = torch.arange(hd // 2, dtype=torch.float64)
    th = pos[:, None].double() / torch.pow(torch.tensor(10000.0, dtype=torch.float64), 2 * i / hd)
    c = torch.cos(th)[:, None, :]
    s = torch.sin(th)[:, None, :]
    x0, x1 = xr[..., 0], xr[..., 1]
    if inverse:
        return torch.stack([x0 * c + x1 * s, -x0 * s + x1 * c], -1).view(T, H * hd)
    return torch.stack([x0 * c - x1 * s, x0 * s + x1 * c], -1).view(T, H * hd)


def brute_force(parent, Q, K, V, G, H, hd, scale, rope=False, acc=None):
    """float64 masked-dense attention + autograd. Q, K are post-RoPE inputs;
    with rope=True the gradients are taken w.r.t. the pre-RoPE values (the
    inverse rotation the reference applies, as a true VJP)."""
    T = parent.shape[0]
    D = H * hd
    depth = ORC.depths(parent)
    M = np.zeros((T, T), bool)
    for n in range(T):
        a = n
        while a >= 0:
            M[n, a] = True
            a = parent[a]
    pos = torch.tensor(depth - 1)
    q0 = torch.tensor(Q, dtype=torch.float64)
    k0 = torch.tensor(K, dtype=torch.float64)
    if rope:
        q0 = _rope_t(q0, pos, H, hd, inverse=True)
        k0 = _rope_t(k0, pos, H, hd, inverse=True)
    qpre = q0.clone().requires_grad_()
    kpre = k0.clone().requires_grad_()
    v = torch.tensor(V, dtype=torch.float64, requires_grad=True)
    q = _rope_t(qpre, pos, H, hd) if rope else qpre
    k = _rope_t(kpre, pos, H, hd) if rope else kpre
    qh = q.view(T, H, hd).transpose(0, 1)
    kh = k.view(T, H, hd).transpose(0, 1)
    s = (qh @ kh.transpose(1, 2).contiguous()) * scale
    s = s.masked_fill(~torch.tensor(M)[None], -math.inf)
    lse = torch.logsumexp(s, -1).T
    p = torch.softmax(s, -1)
    o = (p @ v.view(T, H, hd).transpose(0, 1).contiguous()).transpose(0, 1).reshape(T, D)
    (o * torch.tensor(G, dtype=torch.float64)).sum().backward()
    dq, dk, dv = qpre.grad.numpy(), kpre.grad.numpy(), v.grad.numpy()
    if acc is not None:  # seeds enter dK before the inverse rotation
        ak = torch.tensor(acc[0], dtype=torch.float64)
        dk = dk + (_rope_t(ak, pos, H, hd, inverse=True).numpy() if rope else acc[0])
        dv = dv + acc[1]
    return o.detach().numpy(), lse.detach().numpy(), dq, dk, dv


CASES = [(2, 8, False, False, 1.0), (3, 4, True, False, 1.0), (4, 16, True, True, 1.0),
         (2, 8, True, True, 6.0)]


@pytest.mark.parametrize("H,hd,rope,acc,sharp", CASES)
def test_oracle_vs_bruteforce(H, hd, rope, acc, sharp):
    tr = small_trie(n_tokens=150, depth=9, seed=H * 7 + hd)
    T, D = tr.n_nodes, H * hd
    Q, K, V, G = tensors(T, D, seed=H + hd, sharp=sharp)
    accs = None
    if acc:
        rng = np.random.default_rng(1)
        accs = [rng.standard_normal((T, D)).astype(np.float32) for _ in range(2)]
    sc = scale_of(hd)
    rt = ORC.rope_table(16, hd) if rope else None
    O, W, lse = ORC.fwd(tr.parent, Q, K, V, H, hd, sc)
    dQ, dK, dV = ORC.bwd(tr.parent, Q, K, V, W, G, H, hd, sc, acc_dk=None if accs is None else accs[0],
                         acc_dv=None if accs is None else accs[1], rope=rt)
    o, l, dq, dk, dv = brute_force(tr.parent, Q, K, V, G, H, hd, sc, rope=rope, acc=accs)
    rs = hd if sharp > 1 else None
    assert_close(O, o, what="O", row_scale=rs)
    assert_close(lse, l, what="lse", rtol=1e-5)
    assert_close(dQ, dq, what="dQ", row_scale=rs)
    assert_close(dK, dk, what="dK", row_scale=rs)
    assert_close(dV, dv, what="dV", row_scale=rs)


def test_chain_is_causal_attention():
    from agpt_amd import trie as trie_mod
    tr = trie_mod.build_chains(trie_mod.uniform_tokens(3 * 24, 65, 9), 3, 24)
    H, hd = 2, 16
    T, D = tr.n_nodes, H * hd
    Q, K, V, G = tensors(T, D, seed=4)
    sc = scale_of(hd)
    O, W, lse = ORC.fwd(tr.parent, Q, K, V, H, hd, sc)
    dQ, dK, dV = ORC.bwd(tr.parent, Q, K, V, W, G, H, hd, sc)
    f = lambda x: torch.tensor(x, dtype=torch.float64).view(3, 24, H, hd).transpose(1, 2)
    q, k, v = (f(x).requires_grad_() for x in (Q, K, V))
    o = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True, scale=sc)
    (o * f(G)).sum().backward()
    back = lambda x: x.detach().transpose(1, 2).reshape(T, D).numpy()
    assert_close(O, back(o), what="O")
    assert_close(dQ, back(q.grad), what="dQ")
    assert_close(dK, back(k.grad), what="dK")
    assert_close(dV, back(v.grad), what="dV")


def test_finite_differences():
    tr = small_trie(n_tokens=40, depth=5, seed=2)
    H, hd = 1, 4
    T, D = tr.n_nodes, H * hd
    Q, K, V, G = tensors(T, D, seed=3)
    sc = scale_of(hd)
    O, W, _ = ORC.fwd(tr.parent, Q, K, V, H, hd, sc)
    dQ, dK, dV = ORC.bwd(tr.parent, Q, K, V, W, G, H, hd, sc)
    rng = np.random.default_rng(0)
    eps = 1e-2
    loss = lambda q, k, v: float((ORC.fwd(tr.parent, q, k, v, H, hd, sc)[0].astype(np.float64) * G).sum())
    for name, grad, which in (("dQ", dQ, 0), ("dK", dK, 1), ("dV", dV, 2)):
        for _ in range(12):
            i, j = int(rng.integers(T)), int(rng.integers(D))
            args = [Q.copy(), K.copy(), V.copy()]
            args[which][i, j] += eps
            lp = loss(*args)
            args[which][i, j] -= 2 * eps
            lm = loss(*args)
            fd = (lp - lm) / (2 * eps)
            assert abs(fd - grad[i, j]) <= 2e-3 + 2e-2 * abs(fd), (name, i, j, fd, grad[i, j])


def test_closed_forms():
    tr = small_trie(n_tokens=200, depth=8, seed=5)
    H, hd = 2, 8
    T, D = tr.n_nodes, H * hd
    Q, K, V, G = tensors(T, D, seed=6)
    sc = scale_of(hd)
    O, W, lse = ORC.fwd(tr.parent, Q, K, V, H, hd, sc)
    dQ, dK, dV = ORC.bwd(tr.parent, Q, K, V, W, G, H, hd, sc)
    depth = ORC.depths(tr.parent)
    roots = depth == 1
    # p = 1: w = 1, o = v_self, ds = 0 => dq = 0 (incl. the self term)
    assert_close(O[roots], V[roots], rtol=1e-6, atol=1e-7, what="o = v at p=1")
    assert np.all(dQ[roots] == 0)
    assert np.allclose(W[roots][:, :, 0], 1.0)
    # Σ_j w_j = 1 over each path
    for n in range(T):
        assert abs(W[n, :, :depth[n]].sum(-1) - 1).max() < 1e-5
    # Σ_j ds_j = 0 per (query, head) => column sums of dK (no RoPE, no seeds) vanish
    colsum = dK.astype(np.float64).sum(0)
    assert np.abs(colsum).max() < 1e-3 * np.abs(dK).sum(0).max()
    # Σ_a dV[a] = Σ_n dO_n (every query's weights sum to one)
    assert_close(dV.astype(np.float64).sum(0), G.astype(np.float64).sum(0), rtol=1e-4, atol=1e-3)
    # constant keys => uniform weights
    Kc = np.tile(K[:1], (T, 1))
    _, Wc, _ = ORC.fwd(tr.parent, Q, Kc, V, H, hd, sc)
    for n in range(T):
        assert np.allclose(Wc[n, :, :depth[n]], 1.0 / depth[n], atol=1e-6)


def test_sibling_order_invariance():
    """Reordering siblings (a different DFS preorder) permutes the results."""
    from agpt_amd._native import attn_lib
    import ctypes as C
    tr = small_trie(n_tokens=120, depth=6, seed=8)
    T, H, hd = tr.n_nodes, 2, 4
    Q, K, V, G = tensors(T, H * hd, seed=9)
    # reverse every node's child order, then re-linearise in preorder
    par = tr.parent.copy()
    rev = np.arange(T)[::-1].copy()  # rows visited in reverse as the "original order"
    par_rev = np.array([-1 if par[r] < 0 else int(np.flatnonzero(rev == par[r])[0]) for r in rev],
                       np.int32)
    perm = np.empty(T, np.int32)
    assert attn_lib().agpt_attn_dfs_order(par_rev.ctypes.data_as(C.POINTER(C.c_int32)), T,
                                          perm.ctypes.data_as(C.POINTER(C.c_int32))) == 0
    rows = rev[perm]  # original row of each new position
    inv = np.empty(T, np.int64)
    inv[rows] = np.arange(T)
    new_par = np.array([-1 if par[r] < 0 else inv[par[r]] for r in rows], np.int32)
    assert not np.array_equal(rows, np.arange(T))
    sc = scale_of(hd)
    O, W, _ = ORC.fwd(tr.parent, Q, K, V, H, hd, sc)
    dQ, dK, dV = ORC.bwd(tr.parent, Q, K, V, W, G, H, hd, sc)
    O2, W2, _ = ORC.fwd(new_par, Q[rows], K[rows], V[rows], H, hd, sc)
    dQ2, dK2, dV2 = ORC.bwd(new_par, Q[rows], K[rows], V[rows], W2, G[rows], H, hd, sc)
    for a, b, n in ((O, O2, "O"), (dQ, dQ2, "dQ"), (dK, dK2, "dK"), (dV, dV2, "dV")):
        assert_close(b, a[rows], rtol=1e-5, atol=1e-6, what=n)


def test_varlen_layout_equals_trie():
    """Packing every node's path (batched_depth_forward.cr:668-742) and
    scatter-adding the packed dK/dV rows back to their owners reproduces the
    trie results."""
    tr = small_trie(n_tokens=100, depth=7, seed=12)
    T, H, hd = tr.n_nodes, 2, 8
    D = H * hd
    Q, K, V, G = tensors(T, D, seed=13)
    sc = scale_of(hd)
    depth = ORC.depths(tr.parent)
    offs = np.concatenate([[0], np.cumsum(depth)[:-1]]).astype(np.int32)
    rows = []
    for n in range(T):
        path, a = [], n
        while a >= 0:
            path.append(a)
            a = tr.parent[a]
        rows.extend(path[::-1])
    rows = np.array(rows)
    maxd = int(depth.max())
    o, w = ORC.varlen_fwd(Q, K[rows], V[rows], offs, depth, T, H, hd, maxd, sc)
    O, W, _ = ORC.fwd(tr.parent, Q, K, V, H, hd, sc)
    assert_close(o.reshape(T, D), O, rtol=1e-5, atol=1e-6, what="varlen O")
    dq, dk, dv = ORC.varlen_bwd(Q, K[rows], V[rows], w, G, offs, depth, T, H, hd, maxd, sc, rows.size)
    dQ, dK, dV = ORC.bwd(tr.parent, Q, K, V, W, G, H, hd, sc)
    dk_s = np.zeros((T, D))
    dv_s = np.zeros((T, D))
    np.add.at(dk_s, rows, dk.reshape(-1, D))
    np.add.at(dv_s, rows, dv.reshape(-1, D))
    assert_close(dq.reshape(T, D), dQ, rtol=1e-5, atol=1e-6, what="varlen dQ")
    assert_close(dk_s, dK, what="scatter dK")
    assert_close(dv_s, dV, what="scatter dV")


@pytest.mark.parametrize("rope,acc", [(False, False), (True, True)])
def test_f64_key_grads_equals_bruteforce(rope, acc):
    """The float64 subtree sums the GPU parity tests fall back to for
    cancelling dK/dV rows (helpers.f64_key_grads) equal the masked-dense
    float64 autograd, with RoPE and accumulator seeds."""
    from helpers import f64_key_grads
    tr = small_trie(n_tokens=150, depth=9, seed=31)
    T, H, hd = tr.n_nodes, 2, 8
    Q, K, V, G = tensors(T, H * hd, seed=32)
    sc = scale_of(hd)
    accs = None
    if acc:
        rng = np.random.default_rng(3)
        accs = [rng.standard_normal((T, H * hd)).astype(np.float32) for _ in range(2)]
    _, _, _, bdk, bdv = brute_force(tr.parent, Q, K, V, G, H, hd, sc, rope=rope, acc=accs)
    keys = np.arange(T)
    rt = ORC.rope_table(64, hd) if rope else None
    dk, dv = f64_key_grads(tr.parent, Q, K, V, G, H, hd, sc, keys, rope=rt, acc=accs)
    assert np.abs(dk - bdk).max() <= 1e-5 * max(np.abs(bdk).max(), 1.0)
    assert np.abs(dv - bdv).max() <= 1e-9 * max(np.abs(bdv).max(), 1.0)


def test_varlen_L_layout_equals_bruteforce():
    """The radix chunk-packer layout (agpt_train.cu:4456-4479): the queries
    of radix node i are its edge rows, its packed prefix is its ancestor
    rows then its edge rows, query j of the edge sees the first
    kv_len - L + j + 1 of them (agpt_train.cu:3106-3117). Scatter-adding the
    packed dK/dV rows of oracle_varlen_L_bwd back to their owner rows, and
    reading dQ by query, reproduces the float64 masked-dense autograd (and
    the trie oracle); seeded packed accumulators pass through unchanged
    (the backward accumulates)."""
    tr = small_trie(n_tokens=140, depth=8, seed=21)
    T, H, hd = tr.n_nodes, 2, 8
    D = H * hd
    Q, K, V, G = tensors(T, D, seed=22)
    sc = scale_of(hd)
    heads = np.flatnonzero(tr.radix_head)
    R = heads.shape[0]
    assert R < T  # some edges hold several rows, so L > 1 queries share a prefix
    qoff = np.append(heads, T).astype(np.int32)
    q2n = np.repeat(np.arange(R, dtype=np.int32), np.diff(qoff))
    kv_rows, kv_off, kv_len = [], np.zeros(R, np.int32), np.zeros(R, np.int32)
    for r in range(R):
        path, a = [], int(qoff[r + 1]) - 1
        while a >= 0:
            path.append(a)
            a = int(tr.parent[a])
        kv_off[r], kv_len[r] = len(kv_rows), len(path)
        kv_rows.extend(path[::-1])
    kv_rows = np.array(kv_rows)
    Kp, Vp = K[kv_rows], V[kv_rows]
    max_kv = int(kv_len.max())
    o, w = ORC.varlen_L_fwd(Q, Kp, Vp, q2n, qoff, kv_off, kv_len, T, H, hd, max_kv, sc)
    seed = np.random.default_rng(5).standard_normal(kv_rows.size * D).astype(np.float32)
    dq, dk, dv = ORC.varlen_L_bwd(Q, Kp, Vp, w, G, q2n, qoff, kv_off, kv_len, T, H, hd, max_kv, sc,
                                  kv_rows.size, dk=seed, dv=seed)
    dk_s = np.zeros((T, D))
    dv_s = np.zeros((T, D))
    np.add.at(dk_s, kv_rows, (dk - seed).reshape(-1, D))
    np.add.at(dv_s, kv_rows, (dv - seed).reshape(-1, D))
    bo, blse, bdq, bdk, bdv = brute_force(tr.parent, Q, K, V, G, H, hd, sc)
    assert_close(o.reshape(T, D), bo, what="L O vs brute force")
    assert_close(dq.reshape(T, D), bdq, what="L dQ vs brute force")
    assert_close(dk_s, bdk, what="L scattered dK vs brute force")
    assert_close(dv_s, bdv, what="L scattered dV vs brute force")
    O, W, _ = ORC.fwd(tr.parent, Q, K, V, H, hd, sc)
    dQ, dK, dV = ORC.bwd(tr.parent, Q, K, V, W, G, H, hd, sc)
    assert_close(dk_s, dK, what="L scattered dK vs trie oracle")
    assert_close(dv_s, dV, what="L scattered dV vs trie oracle")
    # weights: query t's visible prefix only, and they sum to 1 per (t, h)
    wv = w.reshape(T, H, max_kv)
    vis = (kv_len[q2n] - np.diff(qoff)[q2n] + (np.arange(T) - qoff[q2n]) + 1)
    assert np.allclose(wv.sum(-1), 1.0, atol=1e-6)
    assert all(np.all(wv[t, :, vis[t]:] == 0) for t in range(T))


# ------------------------------------------------- the spec's own agreement

def _spec_chain_inputs():
    from agpt_amd import trie as trie_mod
    tr = trie_mod.build_trie(np.arange(8, dtype=np.int32), 6, max_starts=1)
    cos_t, sin_t = ORC.rope_table(SM.SEQ_LEN, SM.HEAD_DIM)
    Q, K, V = SM.qkv(tr.token, tr.depth, cos_t, sin_t)
    return tr, Q, K, V, (cos_t, sin_t)


def test_spec_chain_trie_shape():
    """from_token_ids([0..7], max_depth 6, max_starts 1): one path of 6 nodes."""
    tr, *_ = _spec_chain_inputs()
    assert tr.n_nodes == 6
    assert list(tr.parent) == [-1, 0, 1, 2, 3, 4]
    assert list(tr.token) == [0, 1, 2, 3, 4, 5]


@pytest.mark.parametrize("prefix_len", [1, 2, 3, 4])
def test_spec_two_formulations_chain(prefix_len):
    """spec:299-429 at tolerance 1e-5: forward = W·V (matrix) = direct loop =
    grouped output; backward loop form = matrix form, incl. ancestors."""
    tr, Q, K, V, rope = _spec_chain_inputs()
    H, hd = SM.N_HEADS, SM.HEAD_DIM
    sc = scale_of(hd)
    O, W, _ = ORC.fwd(tr.parent, Q, K, V, H, hd, sc)
    O2, W2, _ = ORC.fwd(tr.parent, Q, K, V, H, hd, sc, per_node=True)
    n = prefix_len - 1
    for h in range(H):
        w = W[n, h, :prefix_len]
        vv = V[:prefix_len, h * hd:(h + 1) * hd]
        direct = (w[:, None].astype(np.float32) * vv).sum(0)
        assert np.abs(direct - O[n, h * hd:(h + 1) * hd]).max() <= 1e-5
        assert np.abs(O2[n, h * hd:(h + 1) * hd] - O[n, h * hd:(h + 1) * hd]).max() <= 1e-5
    T = tr.n_nodes
    dO = np.zeros((T, SM.D_MODEL), np.float32)
    dO[n] = SM.d_head_out(SM.chain_d_attn_proj(prefix_len))
    ak = np.zeros_like(dO)
    av = np.zeros_like(dO)
    ak[n], av[n] = SM.current_accum(prefix_len)
    loop = ORC.bwd(tr.parent, Q, K, V, W, dO, H, hd, sc, acc_dk=ak, acc_dv=av, rope=rope)
    mat = ORC.bwd(tr.parent, Q, K, V, W, dO, H, hd, sc, acc_dk=ak, acc_dv=av, rope=rope,
                  matrix_form=True)
    for a, b in zip(loop, mat):
        assert np.abs(a - b).max() <= 1e-5
    # only the query row and its ancestors receive gradient
    dQ, dK, dV = loop
    assert np.all(dQ[prefix_len:] == 0) and np.all(dK[prefix_len:] == 0)
    # prefix_len 1: ds = 0, so dq = 0 and dk = the seeded accumulator (rotated back)
    if prefix_len == 1:
        assert np.all(dQ[0] == 0)
        seed = ak[0].copy()
        for h in range(H):
            sl = slice(h * hd, (h + 1) * hd)
            x = seed[sl].copy()
            ORC.lib()  # tables from the oracle
            c, s = rope[0][0], rope[1][0]
            y = np.empty_like(x)
            for i in range(hd // 2):
                y[2 * i] = x[2 * i] * c[2 * i] + x[2 * i + 1] * s[2 * i]
                y[2 * i + 1] = -x[2 * i] * s[2 * i] + x[2 * i + 1] * c[2 * i]
            assert np.abs(dK[0, sl] - y).max() <= 1e-7


def test_spec_branching_batch():
    """spec:432-538: the first depth level with more than one node."""
    from agpt_amd import trie as trie_mod
    tok = np.array([0, 1, 2, 7, 0, 1, 3, 7, 0, 4, 2, 7, 0, 4, 3, 7], np.int32)
    tr = trie_mod.build_trie(tok, 4)
    roots = np.flatnonzero(tr.depth == 1)
    assert sorted(tr.token[roots]) == [0, 1, 2, 3, 4, 7]
    cos_t, sin_t = ORC.rope_table(SM.SEQ_LEN, SM.HEAD_DIM)
    Q, K, V = SM.qkv(tr.token, tr.depth, cos_t, sin_t)
    H, hd = SM.N_HEADS, SM.HEAD_DIM
    sc = scale_of(hd)
    O, W, _ = ORC.fwd(tr.parent, Q, K, V, H, hd, sc)
    T = tr.n_nodes
    dO = np.zeros((T, SM.D_MODEL), np.float32)
    for i, r in enumerate(roots):
        dO[r] = SM.d_head_out(SM.branch_d_attn_proj(i))
    loop = ORC.bwd(tr.parent, Q, K, V, W, dO, H, hd, sc, rope=(cos_t, sin_t))
    mat = ORC.bwd(tr.parent, Q, K, V, W, dO, H, hd, sc, rope=(cos_t, sin_t), matrix_form=True)
    for a, b in zip(loop, mat):
        assert np.abs(a - b).max() <= 1e-5
    assert np.all(loop[0][roots] == 0)  # p = 1 everywhere in the batch
    assert_close(loop[2][roots], dO[roots], rtol=0, atol=0, what="dv = w dO = dO at p=1")


# ------------------------------------------------------- planted mistakes

def test_planted_mistakes_are_caught():
    """Oracle variants with one plausible mistake each fail the brute force."""
    tr = small_trie(n_tokens=100, depth=7, seed=21)
    H, hd = 2, 8
    T, D = tr.n_nodes, H * hd
    Q, K, V, G = tensors(T, D, seed=22)
    sc = scale_of(hd)
    rt = ORC.rope_table(16, hd)
    o, l, dq, dk, dv = brute_force(tr.parent, Q, K, V, G, H, hd, sc, rope=True)

    def run(parent=tr.parent, q=Q, k=K, v=V, scale=sc, rope=rt):
        O, W, _ = ORC.fwd(parent, q, k, v, H, hd, scale)
        return (O,) + ORC.bwd(parent, q, k, v, W, G, H, hd, scale, rope=rope)

    def fails(res):
        try:
            for got, want in zip(res, (o, dq, dk, dv)):
                assert_close(got, want)
        except AssertionError:
            return True
        return False

    assert not fails(run())                                 # the oracle itself passes
    assert fails(run(k=V, v=K))                             # transposed operands
    assert fails(run(scale=1.0))                            # dropped scale
    assert fails(run(rope=None))                            # no inverse rotation
    assert fails(run(rope=(rt[0], -rt[1])))                 # rotation the wrong way
    assert fails(run(parent=np.full(T, -1, np.int32)))      # ancestors dropped
    Qh = Q.reshape(T, H, hd)[:, ::-1].reshape(T, D).copy()  # heads swapped
    assert fails(run(q=Qh))


def test_abs_terms_bound_the_oracle():
    """The bf16 bar's term magnitudes (helpers.abs_terms): every oracle
    element is at most its sum of |terms| (triangle inequality), with
    equality where all terms are non-negative (V >= 0 for O, dO >= 0 for
    dV), with RoPE and accumulators."""
    from helpers import abs_terms, scale_of, small_trie, tensors
    tr = small_trie(n_tokens=300, depth=9, seed=5)
    T, H, hd = tr.n_nodes, 2, 8
    Q, K, V, G = tensors(T, H * hd, 3)
    acc = tensors(T, H * hd, 4, n=2)
    scale = scale_of(hd)
    rope = ORC.rope_table(16, hd)
    rows = np.arange(T)
    for pos in (False, True):
        Vx, Gx = (np.abs(V), np.abs(G)) if pos else (V, G)
        O, W, _ = ORC.fwd(tr.parent, Q, K, Vx, H, hd, scale)
        dQ, dK, dV = ORC.bwd(tr.parent, Q, K, Vx, W, Gx, H, hd, scale, acc_dk=acc[0],
                             acc_dv=np.abs(acc[1]) if pos else acc[1], rope=rope)
        for kind, x in (("O", O), ("dQ", dQ), ("dK", dK), ("dV", dV)):
            t = abs_terms(kind, tr.parent, Q, K, Vx, Gx, W, H, hd, scale, rows, rope=rope,
                          acc=(acc[0], np.abs(acc[1]) if pos else acc[1]))
            assert (np.abs(x) <= t * (1 + 1e-5) + 1e-6).all(), kind
            if pos and kind in ("O", "dV"):
                np.testing.assert_allclose(t, x, rtol=1e-5, atol=1e-6)
