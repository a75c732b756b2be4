"""Root-child subtrees built one at a time (agpt_trie_build_radix_part)
equal the whole radix trie's rows in order: what lets a corpus whose trie
does not fit on one GPU (full-size C4) be built and batched subtree by
subtree."""
from __future__ import annotations

import numpy as np

from agpt_amd import trie


def _concat(parts):
    off, cols = 0, {k: [] for k in ("parent", "depth", "token", "radix_head", "subtree_end")}
    for p in parts:
        cols["parent"].append(np.where(p.parent < 0, -1, p.parent + off))
        cols["subtree_end"].append(p.subtree_end + off)
        for k in ("depth", "token", "radix_head"):
            cols[k].append(getattr(p, k))
        off += p.n_nodes
    return {k: np.concatenate(v) for k, v in cols.items()}


def test_parts_concatenate_to_whole_trie():
    c = trie.CONFIGS["C4"]
    tok = trie.markov_corpus(4000, c["order"], c["vocab"], c["zipf"], c["seed"])
    whole = trie.build_radix_trie(tok, 128)
    parts = [trie.build_radix_part(tok, 128, x) for x in range(c["vocab"])]
    assert sum(p.n_nodes for p in parts) == whole.n_nodes
    assert all(p.n_root_children <= 1 for p in parts)
    got = _concat(p for p in parts if p.n_nodes)
    for k, v in got.items():
        assert np.array_equal(v, getattr(whole, k)), k


def test_part_of_absent_token_is_empty():
    tok = np.array([0, 1, 0, 1, 2, 0], np.int32)
    assert trie.build_radix_part(tok, 8, 7).n_nodes == 0
