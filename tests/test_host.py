"""Host logic (CPU only): trie construction, tree validation, DFS ordering,
and the C ABI of both libraries (loads, exports every declared symbol; no
device calls)."""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

from agpt_amd import _native, trie

ROOT = Path(__file__).resolve().parent.parent


def _declared(header: str) -> list[str]:
    text = (ROOT / "include" / header).read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(agpt_[A-Za-z0-9_]+)\s*\(", text)))


@pytest.mark.parametrize("header,loader,table,n_min", [
    ("agpt_attn.h", _native.attn_lib, _native.ATTN_SYMBOLS, 8),
    ("agpt_loss.h", _native.attn_lib, _native.LOSS_SYMBOLS, 2),
    ("agpt_block.h", _native.attn_lib, _native.BLOCK_SYMBOLS, 6),
    ("agpt_trie.h", _native.trie_lib, _native.TRIE_SYMBOLS, 8)])
def test_abi_exports_every_declared_symbol(header, loader, table, n_min):
    lib = loader()
    names = _declared(header)
    assert len(names) >= n_min
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(table) == set(names)  # the ctypes table binds exactly the header


def _brute_prefixes(tokens, max_depth, starts):
    nodes = set()
    n = len(tokens)
    for s in starts:
        L = min(max_depth, n - 1 - s)
        for d in range(1, L + 1):
            nodes.add(tuple(tokens[s:s + d]))
    return nodes


@pytest.mark.parametrize("n,order,vocab,depth,max_starts", [(300, 2, 5, 8, 0), (500, 3, 9, 12, 0),
                                                            (400, 1, 4, 6, 37)])
def test_trie_matches_ingest_semantics(n, order, vocab, depth, max_starts):
    tok = trie.markov_corpus(n, order, vocab, 1.1, seed=n)
    tr = trie.build_trie(tok, depth, max_starts=max_starts)
    total = n - 1
    if max_starts:
        starts = [(i * total // max_starts) % total for i in range(max_starts)]
    else:
        starts = range(total)
    want = _brute_prefixes(list(tok), depth, starts)
    # reconstruct each node's path string from the parent links
    paths = []
    for i in range(tr.n_nodes):
        p = tr.parent[i]
        paths.append((paths[p] if p >= 0 else ()) + (int(tr.token[i]),))
        assert tr.depth[i] == len(paths[i])
    assert len(set(paths)) == tr.n_nodes  # no duplicate nodes
    assert set(paths) == want
    # DFS preorder with ascending child tokens = lexicographic order of paths
    assert paths == sorted(paths)
    # subtree ranges contiguous and exact
    for i in range(0, tr.n_nodes, max(1, tr.n_nodes // 50)):
        e = tr.subtree_end[i]
        assert all(paths[j][:len(paths[i])] == paths[i] for j in range(i, e))
        assert e == tr.n_nodes or paths[e][:len(paths[i])] != paths[i]


def test_trie_stats_radix_and_partitions():
    tok = trie.markov_corpus(2000, 3, 7, 1.1, seed=4)
    tr = trie.build_trie(tok, 16)
    nchild = np.bincount(tr.parent[tr.parent >= 0], minlength=tr.n_nodes)
    heads = (tr.parent < 0) | (nchild[np.maximum(tr.parent, 0)] != 1)
    assert tr.n_radix == int(heads.sum()) == int(tr.radix_head.sum())
    rpar, elen = tr.radix()
    assert elen.sum() == tr.n_nodes and rpar.shape[0] == tr.n_radix
    assert np.all(rpar < np.arange(tr.n_radix))
    # bigram key: (first token << 8) | second token (255 at depth 1)
    for i in range(0, tr.n_nodes, 97):
        a, path = i, []
        while a >= 0:
            path.append(int(tr.token[a]))
            a = tr.parent[a]
        path = path[::-1]
        second = path[1] if len(path) > 1 else 255
        assert tr.partition[i] == (path[0] << 8) | second


def test_markov_corpus_is_seeded_and_zipf_like():
    a = trie.markov_corpus(50_000, 3, 65, 1.1, seed=7)
    b = trie.markov_corpus(50_000, 3, 65, 1.1, seed=7)
    c = trie.markov_corpus(50_000, 3, 65, 1.1, seed=8)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    assert a.min() >= 0 and a.max() < 65
    counts = np.bincount(a, minlength=65)
    assert counts[:5].sum() > counts[-20:].sum()  # low ranks dominate


def test_chain_trie():
    tok = trie.uniform_tokens(5 * 7, 65, seed=1)
    tr = trie.build_chains(tok, 5, 7)
    assert tr.n_nodes == 35 and tr.max_depth == 7 and tr.n_radix == 5
    assert np.array_equal(tr.parent[:8], [-1, 0, 1, 2, 3, 4, 5, -1])


def _check_tree(parent):
    lib = _native.attn_lib()
    par = np.ascontiguousarray(parent, np.int32)
    d = np.zeros(par.shape[0], np.int32)
    e = np.zeros(par.shape[0], np.int32)
    rc = lib.agpt_attn_check_tree(par.ctypes.data_as(C.POINTER(C.c_int32)), par.shape[0],
                                  d.ctypes.data_as(C.POINTER(C.c_int32)),
                                  e.ctypes.data_as(C.POINTER(C.c_int32)))
    return rc, d, e


def test_check_tree():
    tok = trie.markov_corpus(300, 2, 5, 1.1, seed=3)
    tr = trie.build_trie(tok, 9)
    rc, d, e = _check_tree(tr.parent)
    assert rc == _native.AGPT_OK
    assert np.array_equal(d, tr.depth) and np.array_equal(e, tr.subtree_end)
    assert _check_tree([-1, 0, -1, 1])[0] == _native.AGPT_ERR_NOT_DFS  # closed subtree
    assert _check_tree([0])[0] == _native.AGPT_ERR_NOT_DFS             # self parent
    assert _check_tree([-1, 2, 0])[0] == _native.AGPT_ERR_NOT_DFS      # forward parent
    assert _check_tree([-2])[0] == _native.AGPT_ERR_NOT_DFS
    rc, d, e = _check_tree([-1, -1, 1, 2, 1])
    assert rc == 0 and list(d) == [1, 1, 2, 3, 2] and list(e) == [1, 5, 4, 4, 5]
    msg = _native.attn_lib().agpt_last_error()
    assert isinstance(msg, bytes)


def test_dfs_order_of_arbitrary_forest():
    rng = np.random.default_rng(0)
    n = 500
    # random forest in BFS-like order, then shuffled labels
    parent = np.array([-1 if i < 5 or rng.random() < 0.05 else int(rng.integers(0, i))
                       for i in range(n)], np.int32)
    lab = rng.permutation(n)
    inv = np.argsort(lab)
    shuffled = np.array([-1 if parent[inv[j]] < 0 else lab[parent[inv[j]]] for j in range(n)],
                        np.int32)
    perm = np.empty(n, np.int32)
    lib = _native.attn_lib()
    assert lib.agpt_attn_dfs_order(shuffled.ctypes.data_as(C.POINTER(C.c_int32)), n,
                                   perm.ctypes.data_as(C.POINTER(C.c_int32))) == 0
    assert sorted(perm) == list(range(n))
    pos = np.empty(n, np.int64)
    pos[perm] = np.arange(n)
    new_parent = np.array([-1 if shuffled[r] < 0 else pos[shuffled[r]] for r in perm], np.int32)
    assert _check_tree(new_parent)[0] == 0
    cyc = np.array([1, 0], np.int32)
    assert lib.agpt_attn_dfs_order(cyc.ctypes.data_as(C.POINTER(C.c_int32)), 2,
                                   perm.ctypes.data_as(C.POINTER(C.c_int32))) != 0


def test_create_fails_loudly_without_device():
    """No silent CPU path: without a GPU the handle cannot be created."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    from agpt_amd.attention import TrieAttention
    with pytest.raises(_native.AgptError):
        TrieAttention(2, 8)


@pytest.mark.parametrize("n,order,vocab,depth", [(300, 2, 5, 6), (500, 3, 7, 9)])
def test_trie_next_counts_match_corpus_scan(n, order, vocab, depth):
    """visits and next-token counts against a direct scan of the corpus with
    TrieCorpus#ingest's loop (trie_corpus.cr:210-219): every step of every
    start observes the token after its prefix."""
    tok = trie.markov_corpus(n, order, vocab, 1.1, seed=4)
    tr = trie.build_trie(tok, depth, counts=True)
    hist, visits = {}, {}
    for s in range(n - 1):
        for d in range(1, min(depth, n - 1 - s) + 1):
            key = tuple(tok[s:s + d])
            visits[key] = visits.get(key, 0) + 1
            h = hist.setdefault(key, {})
            h[int(tok[s + d])] = h.get(int(tok[s + d]), 0) + 1
    paths = []
    for i in range(tr.n_nodes):
        p = tr.parent[i]
        paths.append((paths[p] if p >= 0 else ()) + (int(tr.token[i]),))
    assert len(paths) == len(visits)
    for i, key in enumerate(paths):
        assert tr.visits[i] == visits[key]
        a, b = tr.next_offsets[i], tr.next_offsets[i + 1]
        got = dict(zip(tr.next_tok[a:b].tolist(), tr.next_val[a:b].tolist()))
        assert got == hist[key]
        assert list(tr.next_tok[a:b]) == sorted(got)


def test_new_entry_points_reject_bad_arguments_without_a_device():
    """The loss, epilogue, norm and RMSProp entry points check their
    arguments before any device call: bad sizes and null pointers come back
    as AGPT_ERR_INVALID_ARG / AGPT_ERR_UNSUPPORTED with a message."""
    lib = _native.attn_lib()
    nul = [None] * 11

    def msg():
        return lib.agpt_last_error().decode()

    assert lib.agpt_loss_per_query(*nul, -1, 65, 0.0, 1.0, 0, None) == _native.AGPT_ERR_INVALID_ARG
    assert lib.agpt_loss_per_query(*nul, 5, 0, 0.0, 1.0, 0, None) == _native.AGPT_ERR_INVALID_ARG
    assert lib.agpt_loss_per_query(*nul, 5, 65, 0.0, 1.0, 0, None) == _native.AGPT_ERR_INVALID_ARG
    assert "null pointer" in msg()
    assert lib.agpt_loss_per_query(*nul, 0, 65, 0.0, 1.0, 0, None) == _native.AGPT_OK  # empty batch
    assert lib.agpt_bias_rope(None, None, None, None, None, 0, 4, 2, 6, None) == _native.AGPT_ERR_INVALID_ARG
    assert "multiple of 4" in msg()
    assert lib.agpt_bias_rope(None, None, None, None, None, 0, 4, 2, 8, None) == _native.AGPT_ERR_INVALID_ARG
    assert lib.agpt_rmsprop(None, None, None, 1e-3, 0.9, 1e-8, 10, None) == _native.AGPT_ERR_INVALID_ARG
    assert lib.agpt_rmsprop(None, None, None, 1e-3, 0.9, 1e-8, 0, None) == _native.AGPT_OK
    assert lib.agpt_norm_fwd(None, None, None, None, None, None, 3, 128, 1e-5, None) == _native.AGPT_ERR_INVALID_ARG
    assert lib.agpt_norm_workspace_floats(128) == 2 * 1024 * 128
    assert lib.agpt_norm_bwd(*[None] * 10, 0, 3, 128, None) == _native.AGPT_ERR_INVALID_ARG
    assert lib.agpt_relu_bwd(*[None] * 5, 0, 3, 512, None) == _native.AGPT_ERR_INVALID_ARG
    mass = np.zeros(3, np.float32)
    i = lambda *v: np.array(v, np.int32).ctypes.data_as(C.POINTER(C.c_int32))
    assert lib.agpt_loss_mass_weights(i(0), i(5), i(2), i(0, 2), 1, 2, 9,
                                      mass.ctypes.data_as(C.POINTER(C.c_float))) == _native.AGPT_ERR_INVALID_ARG


def test_bench_one_gpu_contract():
    """bench.py refuses --gpus N > 1 with a message (one GPU per box), and
    has a dense matrix peak for every input type a workload computes in."""
    import subprocess
    import sys

    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       cwd=ROOT, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    sys.path.insert(0, str(ROOT))
    import bench

    assert {c["dtype"] for c in trie.CONFIGS.values()} <= set(bench.MFMA_PEAK_TFLOPS)
