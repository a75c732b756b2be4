"""Pins the C restatement of the per-query AGPT loss (oracle/loss_oracle.c,
agpt_train.cu:2069-2194) and its mass weights (agpt_train.cu:4608-4637)
before it is trusted as the GPU kernel's checker: an independent float64
formulation (log-sum-exp), central finite differences of the loss against the
gradient, closed forms at uniform logits, the entropy weight of two equal
counts, row sums, and the weights' normalisation. CPU only."""
from __future__ import annotations

import math

import numpy as np
import pytest

from helpers import loss_batch
from oracle import oracle as ORC

ARGS = ("logits", "query_to_node", "query_offsets", "radix_ids", "token_ids", "counts_offset",
        "counts_tok", "counts_val")


def _oracle(b, **kw):
    return ORC.loss_per_query(*(b[k] for k in ARGS), **kw)


def _f64(b, mass=None, lam=0.0, iw=1.0, ce_only=False):
    """The loss written from its definition in float64: log p by log-sum-exp,
    the target distribution t (one-hot or counts / total), loss = -t.log(p +
    1e-10), grad = p - t, both times the weight."""
    lg = b["logits"].astype(np.float64)
    T_q, V = lg.shape
    lp = lg - lg.max(1, keepdims=True)
    lp -= np.log(np.exp(lp).sum(1, keepdims=True))
    p = np.exp(lp)
    g = p.copy()
    loss = np.zeros(T_q)
    for q in range(T_q):
        n = b["query_to_node"][q]
        end = b["query_offsets"][n + 1]
        t = np.zeros(V)
        if q + 1 == end and not (ce_only and q + 1 < T_q):
            r = b["radix_ids"][n]
            s, e = b["counts_offset"][r], b["counts_offset"][r + 1]
            if s == e:
                continue
            c = b["counts_val"][s:e].astype(np.float64)
            np.add.at(t, b["counts_tok"][s:e], c / c.sum())
            w = 1.0
            if lam > 0 and e - s > 1:
                qe = c / c.sum()
                w = 1.0 + lam * (-(qe * np.log(qe)).sum() / math.log(V))
        else:
            t[b["token_ids"][q + 1]] = 1.0
            w = iw
        if mass is not None:
            w *= mass[q]
        loss[q] = -w * (t * np.log(p[q] + 1e-10)).sum()
        g[q] = w * (p[q] - t)
    return g, loss


@pytest.mark.parametrize("V", [3, 16, 65, 256])
@pytest.mark.parametrize("opts", [{}, {"lam": 0.5}, {"iw": 0.3}, {"ce_only": True}, {"mass": True}])
def test_oracle_matches_float64_definition(V, opts):
    b = loss_batch(60, V, seed=V)
    mass = np.random.default_rng(1).uniform(0.2, 3.0, b["logits"].shape[0]).astype(np.float32) \
        if opts.get("mass") else None
    g, lo = _oracle(b, mass_weights=mass, entropy_lambda=opts.get("lam", 0.0),
                    intermediate_weight=opts.get("iw", 1.0), ce_only=opts.get("ce_only", False))
    g64, lo64 = _f64(b, mass=mass, lam=opts.get("lam", 0.0), iw=opts.get("iw", 1.0),
                     ce_only=opts.get("ce_only", False))
    np.testing.assert_allclose(g, g64, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(lo, lo64, rtol=1e-5, atol=1e-6)


def test_oracle_repeated_tokens_accumulate():
    """A token listed twice: the gradient takes both shares; the second
    entry's loss term reads the already-reduced row value, as the
    reference's in-place loop does (agpt_train.cu:2170-2175)."""
    b = loss_batch(40, 7, seed=3, dup=True, max_entries=6)
    g, _ = _oracle(b)
    g64, _ = _f64(b)
    np.testing.assert_allclose(g, g64, rtol=1e-5, atol=1e-6)
    one = dict(logits=np.zeros((1, 2), np.float32), query_to_node=np.zeros(1, np.int32),
               query_offsets=np.array([0, 1], np.int32), radix_ids=np.zeros(1, np.int32),
               token_ids=np.zeros(1, np.int32), counts_offset=np.array([0, 2], np.int32),
               counts_tok=np.array([1, 1], np.int32), counts_val=np.array([1, 3], np.int32))
    g1, lo1 = _oracle(one)
    np.testing.assert_allclose(lo1[0], -0.25 * math.log(0.5) - 0.75 * math.log(0.25 + 1e-10), rtol=1e-6)
    np.testing.assert_allclose(g1[0], [0.5, -0.5], rtol=1e-6)


def test_gradient_is_the_derivative_of_the_loss():
    b = loss_batch(12, 9, seed=5, logit_scale=1.0)
    mass = np.random.default_rng(2).uniform(0.5, 2.0, b["logits"].shape[0]).astype(np.float32)
    kw = dict(mass_weights=mass, entropy_lambda=0.7, intermediate_weight=0.6)
    g, lo = _oracle(b, **kw)
    eps = 1e-2
    T_q, V = b["logits"].shape
    for q in range(T_q):
        for j in range(V):
            bp, bm = dict(b), dict(b)
            bp["logits"] = b["logits"].copy()
            bm["logits"] = b["logits"].copy()
            bp["logits"][q, j] += eps
            bm["logits"][q, j] -= eps
            fd = (float(_oracle(bp, **kw)[1][q]) - float(_oracle(bm, **kw)[1][q])) / (2 * eps)
            assert abs(fd - g[q, j]) < 2e-3 * max(1.0, abs(g[q, j])), (q, j, fd, g[q, j])


def test_closed_forms_at_uniform_logits():
    V = 10
    # node 0: queries 0,1,2 (two intermediates + endpoint with counts {4: 3});
    # node 1: query 3 (endpoint with two equal counts); node 2: query 4 (no counts)
    b = dict(logits=np.zeros((5, V), np.float32), query_to_node=np.array([0, 0, 0, 1, 2], np.int32),
             query_offsets=np.array([0, 3, 4, 5], np.int32), radix_ids=np.array([0, 1, 2], np.int32),
             token_ids=np.array([1, 2, 3, 4, 5], np.int32), counts_offset=np.array([0, 1, 3, 3], np.int32),
             counts_tok=np.array([4, 6, 7], np.int32), counts_val=np.array([3, 2, 2], np.int32))
    g, lo = _oracle(b, entropy_lambda=0.5)
    lv = -math.log(0.1 + 1e-10)
    np.testing.assert_allclose(lo[:3], [lv, lv, lv], rtol=1e-6)
    assert abs(g[0, 2] - (0.1 - 1.0)) < 1e-6 and abs(g[1, 3] - (0.1 - 1.0)) < 1e-6  # target = token_ids[q+1]
    assert abs(g[2, 4] - (0.1 - 1.0)) < 1e-6
    w = 1.0 + 0.5 * math.log(2.0) / math.log(V)  # H of {1/2, 1/2}
    np.testing.assert_allclose(lo[3], w * lv, rtol=1e-6)
    np.testing.assert_allclose(g[3, [6, 7]], w * (0.1 - 0.5), rtol=1e-6)
    np.testing.assert_allclose(g[3, 0], w * 0.1, rtol=1e-6)
    assert lo[4] == 0.0 and np.allclose(g[4], 0.1)  # no counts: loss 0, grad = p


def test_row_sums_and_ce_only():
    b = loss_batch(80, 33, seed=9)
    g, lo = _oracle(b, intermediate_weight=0.4, entropy_lambda=0.3)
    s = g.astype(np.float64).sum(1)
    T_q = g.shape[0]
    ends = b["query_offsets"][b["query_to_node"] + 1] == np.arange(T_q) + 1
    empty = np.array([b["counts_offset"][b["radix_ids"][n]] == b["counts_offset"][b["radix_ids"][n] + 1]
                      for n in b["query_to_node"]]) & ends
    np.testing.assert_allclose(s[~empty], 0.0, atol=2e-6)
    np.testing.assert_allclose(s[empty], 1.0, atol=2e-6)
    assert (lo[empty] == 0).all() and (lo[~empty] > 0).all()
    g2, lo2 = _oracle(b, ce_only=True)
    last = T_q - 1
    inner_ends = ends & (np.arange(T_q) < last)
    q = int(np.flatnonzero(inner_ends)[0])
    t = b["token_ids"][q + 1]
    p = np.exp(b["logits"][q].astype(np.float64) - b["logits"][q].max())
    p /= p.sum()
    np.testing.assert_allclose(lo2[q], -math.log(p[t] + 1e-10), rtol=1e-5)


@pytest.mark.parametrize("mode", [0, 1, 2, 3])
def test_mass_weights_normalised(mode):
    rng = np.random.default_rng(mode)
    n, R = 50, 120
    rid = rng.permutation(R)[:n].astype(np.int32)
    mass = rng.integers(1, 500, R).astype(np.int32)
    elen = rng.integers(1, 6, R).astype(np.int32)
    off = np.zeros(n + 1, np.int32)
    np.cumsum(elen[rid], out=off[1:])
    T_q = int(off[-1])
    w = ORC.loss_mass_weights(rid, mass, elen, off, T_q, mode)
    assert abs(w.astype(np.float64).mean() - 1.0) < 1e-5  # mean over queries is 1
    f = {0: lambda m: np.ones_like(m), 1: np.log1p, 2: np.sqrt, 3: lambda m: m}[mode]
    fm = f(mass[rid].astype(np.float64))
    for i in range(n):  # constant over a node's queries, proportional to f(mass)
        assert np.allclose(w[off[i]:off[i + 1]], w[off[0]] * fm[i] / fm[0], rtol=1e-5)
