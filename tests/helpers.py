"""Shared test helpers: seeded tries and tensors, tolerance checks."""
from __future__ import annotations

import math

import numpy as np

from agpt_amd import trie as trie_mod
from oracle import oracle as ORC

# fp32 parity bar: 1e-4 relative / 1e-5 absolute.
RTOL_F32, ATOL_F32 = 1e-4, 1e-5
# bf16-input variants: 2e-2 relative (absolute floor for values near zero).
RTOL_BF16, ATOL_BF16 = 2e-2, 2e-3


def assert_close(got, want, rtol=RTOL_F32, atol=ATOL_F32, what="", row_scale=None):
    """|got - want| <= atol + rtol * |want| elementwise.

    row_scale=hd switches the relative term to the largest |want| of the
    element's (row, head) slice: a normwise bound for sums whose terms are
    much larger than the result (sharp softmax gradients), where two float32
    summation orders legitimately differ by more than 1e-4 of the element."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    err = np.abs(got - want)
    mag = np.abs(want)
    if row_scale:
        m = mag.reshape(mag.shape[0], -1, row_scale).max(axis=2, keepdims=True)
        mag = np.broadcast_to(m, mag.shape[:1] + (mag.size // mag.shape[0] // row_scale, row_scale)
                              ).reshape(mag.shape)
    bound = atol + rtol * mag
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.size} outside |d| <= {atol} + {rtol}|ref|; "
            f"worst at {i}: got {got[i]!r} want {want[i]!r} (max abs err {err.max():.3e})")


def scale_of(hd: int) -> float:
    return float(np.float32(1.0 / math.sqrt(hd)))


def small_trie(n_tokens=400, order=2, vocab=6, depth=10, seed=3):
    tok = trie_mod.markov_corpus(n_tokens, order, vocab, 1.1, seed)
    return trie_mod.build_trie(tok, depth)


def tensors(T, D, seed, sharp=1.0, n=4):
    rng = np.random.default_rng(seed)
    out = [rng.standard_normal((T, D)).astype(np.float32) for _ in range(n)]
    out[0] *= np.float32(sharp)
    return out


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even to bfloat16, returned as float32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def loss_batch(n_nodes, V, seed, max_edge=4, max_entries=6, dup=False, empty_frac=0.1,
               logit_scale=2.0):
    """Seeded radix query batch for the per-query loss: n_nodes radix nodes
    with 1..max_edge queries each, global radix ids spread over 2*n_nodes,
    next-token counts CSR by global id (distinct tokens unless dup; a share
    of endpoints without counts), random targets and logits.
    Returns a dict of numpy arrays keyed like agpt_loss_per_query's arguments."""
    rng = np.random.default_rng(seed)
    edge = rng.integers(1, max_edge + 1, n_nodes)
    off = np.zeros(n_nodes + 1, np.int64)
    np.cumsum(edge, out=off[1:])
    T_q = int(off[-1])
    q2n = np.repeat(np.arange(n_nodes, dtype=np.int32), edge)
    R = 2 * n_nodes + 1
    radix_ids = rng.permutation(R)[:n_nodes].astype(np.int32)
    ne = rng.integers(1, max_entries + 1, R)
    ne[rng.random(R) < empty_frac] = 0
    ne = np.minimum(ne, V)
    coff = np.zeros(R + 1, np.int64)
    np.cumsum(ne, out=coff[1:])
    n_ent = int(coff[-1])
    if dup:
        ctok = rng.integers(0, V, n_ent)
    else:  # distinct per node: base_r + j (mod V) with a random stride coprime to V
        j = np.arange(n_ent) - np.repeat(coff[:-1], ne)
        base = np.repeat(rng.integers(0, V, R), ne)
        strides = [s for s in range(1, V + 1) if math.gcd(s, V) == 1]
        step = np.repeat(rng.choice(strides, R), ne)
        ctok = (base + j * step) % V
    ctok = ctok.astype(np.int32)
    cval = rng.integers(1, 40, n_ent).astype(np.int32)
    return dict(
        logits=(rng.standard_normal((T_q, V)) * logit_scale).astype(np.float32),
        query_to_node=q2n, query_offsets=off.astype(np.int32), radix_ids=radix_ids,
        token_ids=rng.integers(0, V, T_q).astype(np.int32), counts_offset=coff.astype(np.int32),
        counts_tok=ctok, counts_val=cval,
        edge_mass=rng.integers(1, 1000, R).astype(np.int32), edge_len_by_id=np.zeros(R, np.int32))


def f64_key_grads(parent, Q, K, V, G, H, hd, scale, keys, rope=None, acc=None):
    """float64 dK, dV of the given key rows: each key's sums over every query
    of its subtree (dK[a] = R(pos_a)^T (sum ds_{n,a} q_n + acc_k[a]),
    dV[a] = sum w_{n,a} dO_n + acc_v[a]), from each query's softmax over its
    own path. parent in DFS preorder; rope = (cos, sin) tables or None."""
    T = parent.shape[0]
    depth = np.zeros(T, np.int64)
    end = np.arange(1, T + 1)
    for i in range(T):
        depth[i] = 1 if parent[i] < 0 else depth[parent[i]] + 1
    for i in range(T - 1, -1, -1):
        if parent[i] >= 0:
            end[parent[i]] = max(end[parent[i]], end[i])
    D = H * hd
    out_k = np.zeros((len(keys), D))
    out_v = np.zeros((len(keys), D))
    for x, a in enumerate(keys):
        qs = np.arange(a, end[a])
        da = int(depth[a])
        # path of every query, root first; column da-1 is the key a
        P = int(depth[qs].max())
        path = np.full((qs.size, P), -1, np.int64)
        cur = qs.copy()
        for step in range(P):
            col = depth[qs] - 1 - step
            ok = (cur >= 0) & (col >= 0)
            path[np.flatnonzero(ok), col[ok]] = cur[ok]
            cur = np.where(cur >= 0, parent[np.maximum(cur, 0)], -1)
        valid = path >= 0
        safe = np.maximum(path, 0)
        for h in range(H):
            sl = slice(h * hd, (h + 1) * hd)
            q = Q[qs, sl].astype(np.float64)
            kp = K[safe, sl].astype(np.float64)
            vp = V[safe, sl].astype(np.float64)
            g = G[qs, sl].astype(np.float64)
            s = np.einsum("nd,npd->np", q, kp) * scale
            s = np.where(valid, s, -np.inf)
            s -= s.max(1, keepdims=True)
            w = np.exp(s)
            w /= w.sum(1, keepdims=True)
            dw = np.einsum("nd,npd->np", g, vp)
            ds = w * (dw - (w * dw).sum(1, keepdims=True)) * scale
            dk = (ds[:, da - 1, None] * q).sum(0)
            dv = (w[:, da - 1, None] * g).sum(0)
            if acc is not None:
                dk += acc[0][a, sl]
                dv += acc[1][a, sl]
            if rope is not None:
                pos = min(da - 1, rope[0].shape[0] - 1)
                c = rope[0][pos].astype(np.float64)
                sn = rope[1][pos].astype(np.float64)
                d0, d1 = dk[0::2].copy(), dk[1::2].copy()
                dk[0::2] = d0 * c[0::2] + d1 * sn[0::2]
                dk[1::2] = -d0 * sn[0::2] + d1 * c[0::2]
            out_k[x, sl] = dk
            out_v[x, sl] = dv
    return out_k, out_v


def assert_close_or_f64(got, want, f64_rows, rtol=RTOL_F32, atol=ATOL_F32, what=""):
    """assert_close elementwise against `want` (the float32 oracle); rows that
    fail it must pass the same bar against their float64 value,
    f64_rows(rows) -> [len(rows), D]. For sums over a key's whole subtree
    (dK, dV), whose terms can be far larger than the result: two float32
    summation orders then differ by more than 1e-4 of the result, and the
    bar is held against the true value."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    bad = (np.abs(got - want) > atol + rtol * np.abs(want)).any(1)
    rows = np.flatnonzero(bad)
    assert rows.size <= 64, f"{what}: {rows.size} rows outside the bar against the oracle"
    if rows.size:
        assert_close(got[rows], f64_rows(rows), rtol, atol, f"{what} (rows {rows[:8].tolist()} vs float64)")


def run_gpu(tr_parent, Q, K, V, G, H, hd, dtype, rope=None, acc=None, max_depth=None):
    import torch

    from agpt_amd.attention import TrieAttention

    dev = torch.device("cuda:0")
    tdt = torch.float32 if dtype == "f32" else torch.bfloat16
    md = max_depth or max(1, int(ORC.depths(tr_parent).max()))
    att = TrieAttention(H, hd, max_depth=md, dtype=tdt)
    att.plan(tr_parent)
    print("kernel:", att.describe())
    q, k, v, g = (torch.from_numpy(x).to(dev).to(tdt).contiguous() for x in (Q, K, V, G))
    o, lse = att.forward(q, k, v)
    rt = None
    if rope is not None:
        rt = tuple(torch.from_numpy(x).to(dev).contiguous() for x in rope)
    acc_t = [None, None]
    if acc is not None:
        acc_t = [torch.from_numpy(x).to(dev).contiguous() for x in acc]
    dq, dk, dv = att.backward(q, k, v, o, lse, g, acc_dk=acc_t[0], acc_dv=acc_t[1], rope=rt)
    torch.cuda.synchronize()
    res = [x.float().cpu().numpy() for x in (o, lse, dq, dk, dv)]
    att.close()
    return res


def run_gpu_ranges(tr_parent, Q, K, V, G, H, hd, dtype, ranges, packed, rope=None, acc=None, max_depth=None):
    """The trie as contiguous row ranges, one plan each, in ascending order.
    Whole-trie tensors (packed=False), or per range a packed copy [context
    rows, range rows] whose context dK/dV share is added to the owner rows
    here, in range order."""
    import torch

    from agpt_amd.attention import RangedTrieAttention, TrieAttention

    dev = torch.device("cuda:0")
    tdt = torch.float32 if dtype == "f32" else torch.bfloat16
    md = max_depth or max(1, int(ORC.depths(tr_parent).max()))
    T, D = tr_parent.shape[0], H * hd
    cu = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    rt = None if rope is None else tuple(cu(x) for x in rope)
    if not packed:
        ratt = RangedTrieAttention(H, hd, tr_parent, ranges, max_depth=md, dtype=tdt)
        print("kernel:", ratt.parts[-1].describe())
        q, k, v, g = (cu(x).to(tdt).contiguous() for x in (Q, K, V, G))
        o, lse = ratt.forward(q, k, v)
        ak = None if acc is None else cu(acc[0])
        av = None if acc is None else cu(acc[1])
        dq, dk, dv = ratt.backward(q, k, v, o, lse, g, acc_dk=ak, acc_dv=av, rope=rt)
        torch.cuda.synchronize()
        res = [x.float().cpu().numpy() for x in (o, lse, dq, dk, dv)]
        ratt.close()
        return res
    out = [np.zeros((T, D), np.float32), np.zeros((T, H), np.float32)] + [np.zeros((T, D), np.float64)
                                                                         for _ in range(3)]
    for a, b in ranges:
        ctx = []
        x = int(tr_parent[a])
        while x >= 0:
            ctx.append(x)
            x = int(tr_parent[x])
        rows = np.concatenate([np.array(ctx[::-1], np.int64), np.arange(a, b)])
        nc = len(ctx)
        att = TrieAttention(H, hd, max_depth=md, dtype=tdt)
        att.plan_range(tr_parent, a, b, packed=True)
        assert att.n_ctx == nc
        q, k, v, g = (cu(x[rows]).to(tdt).contiguous() for x in (Q, K, V, G))
        g[:nc] = 0  # context rows are not queries: their dO is unused
        o, lse = att.forward(q, k, v)
        ak = av = None
        if acc is not None:  # the owner batch adds a row's seeds, context rows get none
            ak, av = (cu(np.concatenate([np.zeros((nc, D), np.float32), s[a:b]])) for s in acc)
        dq, dk, dv = att.backward(q, k, v, o, lse, g, acc_dk=ak, acc_dv=av, rope=rt)
        torch.cuda.synchronize()
        o, lse, dq, dk, dv = (x.float().cpu().numpy() for x in (o, lse, dq, dk, dv))
        out[0][a:b], out[1][a:b], out[2][a:b] = o[nc:], lse[nc:], dq[nc:]
        out[3][a:b] += dk[nc:]
        out[4][a:b] += dv[nc:]
        out[3][rows[:nc]] += dk[:nc]  # the range's share of its context rows, to their owners
        out[4][rows[:nc]] += dv[:nc]
        att.close()
    return out


def _path_table(parent, depth, rows, P):
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


def _rope_abs(t, rows_pos, rope):
    """Magnitude bound after the inverse rotation of pairs (2i, 2i+1):
    |c a + s b| and |-s a + c b| are both <= |a| + |b|."""
    if rope is None:
        return t
    pair = t[..., 0::2] + t[..., 1::2]
    out = np.empty_like(t)
    out[..., 0::2] = pair
    out[..., 1::2] = pair
    return out


def abs_terms(kind, parent, Q, K, V, G, W, H, hd, scale, rows, rope=None, acc=None):
    """float64 sum of the absolute values of the terms that make each element
    of the given rows (the scale a rounding of the terms is relative to):
      O[n]  = sum_j w_nj v_j            -> sum_j w_nj |v_j|
      dQ[n] = sum_j ds_nj k_j           -> sum_j |ds_nj| |k_j|
      dK[a] = sum_{n in sub(a)} ds_na q_n (+ acc) -> sum |ds_na| |q_n| (+ |acc|)
      dV[a] = sum_{n in sub(a)} w_na dO_n (+ acc) -> sum w_na |dO_n| (+ |acc|)
    with w the oracle's saved weights W [T, H, P] (root first) and
    ds = w (dO.v - sum w dO.v) scale. With RoPE the pair bound of _rope_abs."""
    parent = np.asarray(parent)
    T = parent.shape[0]
    depth = ORC.depths(parent).astype(np.int64)
    D = H * hd
    rows = np.asarray(rows, np.int64)
    out = np.zeros((rows.shape[0], D))
    if kind in ("O", "dQ"):
        P = int(depth[rows].max())
        path = _path_table(parent, depth, rows, P)
        valid = path >= 0
        safe = np.maximum(path, 0)
        for h in range(H):
            sl = slice(h * hd, (h + 1) * hd)
            w = W[rows, h, :P].astype(np.float64) * valid
            vp = V[safe, sl].astype(np.float64)
            if kind == "O":
                out[:, sl] = np.einsum("np,npd->nd", w, np.abs(vp))
            else:
                dw = np.einsum("nd,npd->np", G[rows, sl].astype(np.float64), vp)
                ds = w * (dw - (w * dw).sum(1, keepdims=True)) * scale
                out[:, sl] = np.einsum("np,npd->nd", np.abs(ds), np.abs(K[safe, sl].astype(np.float64)))
        return _rope_abs(out, None, rope) if kind == "dQ" else out
    end = np.arange(1, T + 1)
    for i in range(T - 1, -1, -1):
        if parent[i] >= 0:
            end[parent[i]] = max(end[parent[i]], end[i])
    for x, a in enumerate(rows):
        qs = np.arange(a, end[a])
        da = int(depth[a])
        for h in range(H):
            sl = slice(h * hd, (h + 1) * hd)
            w = W[qs, h, da - 1].astype(np.float64)
            if kind == "dV":
                out[x, sl] = w @ np.abs(G[qs, sl].astype(np.float64))
                continue
            P = int(depth[qs].max())
            path = _path_table(parent, depth, qs, P)
            valid = path >= 0
            wq = W[qs, h, :P].astype(np.float64) * valid
            vp = V[np.maximum(path, 0), sl].astype(np.float64)
            dw = np.einsum("nd,npd->np", G[qs, sl].astype(np.float64), vp)
            ds = w * (dw[:, da - 1] - (wq * dw).sum(1)) * scale
            out[x, sl] = np.abs(ds) @ np.abs(Q[qs, sl].astype(np.float64))
        if acc is not None:
            out[x] += np.abs(acc[0 if kind == "dK" else 1][a])
    return _rope_abs(out, None, rope) if kind == "dK" else out


def assert_close_terms(got, want, terms_rows, rtol=RTOL_BF16, atol=ATOL_BF16, what="", max_frac=1e-3):
    """The bf16 bar: |got - want| <= atol + rtol |want| elementwise. An
    element outside it passes only if its error is within the same bar
    relative to the sum of its terms' magnitudes, terms_rows(rows) ->
    [len(rows), D] (abs_terms): the inputs of the second products (P, dS)
    are rounded to bf16, a relative change of at most 2^-9 per term, so an
    element whose terms cancel carries that error relative to the terms, not
    to the result. Such exceptions may be at most max_frac of the elements,
    or 8 on tensors too small for that fraction to admit a handful (a 17-row
    chain at 2 x 64 has 2,176 elements: its 4 exceptions, the same from the
    chain kernels and the general ones, sit at 0.09 of the bar against their
    terms); their number and their worst ratio to that bar are printed."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    err = np.abs(got - want)
    bad = err > atol + rtol * np.abs(want)
    n_bad = int(bad.sum())
    print(f"{what}: {bad.size - n_bad} of {bad.size} elements within {rtol}|ref| + {atol} "
          f"({n_bad} exceptions)", flush=True)
    if not n_bad:
        return
    rows = np.flatnonzero(bad.any(1))
    terms = terms_rows(rows)
    e, b = err[rows], bad[rows]
    ok = e <= atol + rtol * terms
    if not ok[b].all():
        r, c = np.argwhere(b & ~ok)[0]
        raise AssertionError(f"{what}: row {rows[r]} col {c}: got {got[rows[r], c]!r} want {want[rows[r], c]!r}, "
                             f"error {e[r, c]:.3e} > {atol} + {rtol} x terms {terms[r, c]:.3e}")
    worst = float(np.max(e[b] / (atol + rtol * terms[b])))
    print(f"{what}: every exception within the bar against its terms (worst at {worst:.2f} of it)", flush=True)
    assert n_bad <= max(max_frac * bad.size, 8), f"{what}: {n_bad} of {bad.size} elements outside the elementwise bar"
