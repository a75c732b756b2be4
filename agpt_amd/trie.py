"""Synthetic corpora and tries (the inputs of the trie-attention path).

Thin numpy wrappers over libagpt_trie.so (include/agpt_trie.h).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from ._native import trie_lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_int32))


def markov_corpus(n: int, order: int, vocab: int, zipf_s: float, seed: int,
                  sigma: float = 2.0) -> np.ndarray:
    """Order-k Markov tokens with Zipf marginal ranks (see include/agpt_trie.h)."""
    out = np.empty(n, dtype=np.int32)
    rc = trie_lib().agpt_markov_corpus(seed, order, vocab, zipf_s, sigma, n, _ptr(out))
    if rc:
        raise ValueError("agpt_markov_corpus: bad arguments")
    return out


def uniform_tokens(n: int, vocab: int, seed: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    if trie_lib().agpt_uniform_tokens(seed, vocab, n, _ptr(out)):
        raise ValueError("agpt_uniform_tokens: bad arguments")
    return out


@dataclass
class Trie:
    """Node-token tables in DFS preorder (one row = one query position)."""
    parent: np.ndarray       # int32 [T], -1 for depth-1 nodes
    depth: np.ndarray        # int32 [T], 1-based = keys attended
    token: np.ndarray        # int32 [T]
    subtree_end: np.ndarray  # int32 [T], exclusive
    radix_head: np.ndarray   # int32 [T]
    partition: np.ndarray    # int32 [T], bigram key
    n_radix: int
    n_root_children: int
    n_bigram_parts: int
    # Corpus observations (build_trie(..., counts=True) only): visits per
    # node and its next-token counts, CSR (offsets [T+1], tok, val).
    visits: np.ndarray | None = None
    next_offsets: np.ndarray | None = None
    next_tok: np.ndarray | None = None
    next_val: np.ndarray | None = None

    @property
    def n_nodes(self) -> int:
        return int(self.parent.shape[0])

    @property
    def sum_depth(self) -> int:
        return int(self.depth.astype(np.int64).sum())

    @property
    def max_depth(self) -> int:
        return int(self.depth.max()) if self.n_nodes else 0

    def radix(self) -> tuple[np.ndarray, np.ndarray]:
        """(radix_parent, edge_len) of the radix view, DFS preorder."""
        heads = np.flatnonzero(self.radix_head)
        edge_len = np.diff(np.append(heads, self.n_nodes)).astype(np.int32)
        radix_of = np.cumsum(self.radix_head) - 1
        par = self.parent[heads]
        radix_parent = np.where(par < 0, -1, radix_of[np.maximum(par, 0)]).astype(np.int32)
        return radix_parent, edge_len


def _export(h, counts: bool = False) -> Trie:
    lib = trie_lib()
    n = C.c_int64()
    nr = C.c_int64()
    sd = C.c_int64()
    md = C.c_int32()
    nrc = C.c_int64()
    nbp = C.c_int64()
    lib.agpt_trie_stats(h, C.byref(n), C.byref(nr), C.byref(sd), C.byref(md), C.byref(nrc),
                        C.byref(nbp))
    T = n.value
    arrs = [np.empty(T, dtype=np.int32) for _ in range(6)]
    lib.agpt_trie_export(h, *[_ptr(a) for a in arrs])
    extra = {}
    if counts:
        ne = C.c_int64()
        vis = np.empty(T, np.int32)
        if lib.agpt_trie_next_counts(h, _ptr(vis), C.byref(ne), None, None, None):
            lib.agpt_trie_free(h)
            raise ValueError("agpt_trie_next_counts: this trie has no corpus")
        off = np.empty(T + 1, np.int32)
        tk = np.empty(ne.value, np.int32)
        vl = np.empty(ne.value, np.int32)
        lib.agpt_trie_next_counts(h, None, C.byref(ne), _ptr(off), _ptr(tk), _ptr(vl))
        extra = dict(visits=vis, next_offsets=off, next_tok=tk, next_val=vl)
    lib.agpt_trie_free(h)
    return Trie(*arrs, n_radix=nr.value, n_root_children=nrc.value, n_bigram_parts=nbp.value, **extra)


def build_trie(tokens: np.ndarray, max_depth: int, max_starts: int = 0, counts: bool = False) -> Trie:
    """Leveled trie with TrieCorpus#ingest semantics (trie_corpus.cr:200-228);
    counts=True also exports the corpus observations (visits, next-token counts)."""
    tok = np.ascontiguousarray(tokens, dtype=np.int32)
    h = C.c_void_p()
    if trie_lib().agpt_trie_build(_ptr(tok), tok.shape[0], max_depth, max_starts, C.byref(h)):
        raise ValueError("agpt_trie_build: bad arguments")
    return _export(h, counts)


def build_radix_trie(tokens: np.ndarray, max_depth: int, counts: bool = False) -> Trie:
    """The node-tokens the reference's on-disk radix pipeline trains on
    (StreamingLeveledBuilder + StreamingRadixBuilder: paths run onto the
    corpus' last token, edges are cut on next-token entries, edges ending at
    the end-of-corpus leaf are dropped; see include/agpt_trie.h)."""
    tok = np.ascontiguousarray(tokens, dtype=np.int32)
    h = C.c_void_p()
    if trie_lib().agpt_trie_build_radix(_ptr(tok), tok.shape[0], max_depth, C.byref(h)):
        raise ValueError("agpt_trie_build_radix: bad arguments")
    return _export(h, counts)


def build_radix_part(tokens: np.ndarray, max_depth: int, first_token: int) -> Trie:
    """build_radix_trie's subtree of one root child (the starts whose first
    token is first_token): the whole trie is these subtrees in token order."""
    tok = np.ascontiguousarray(tokens, dtype=np.int32)
    h = C.c_void_p()
    if trie_lib().agpt_trie_build_radix_part(_ptr(tok), tok.shape[0], max_depth, int(first_token), C.byref(h)):
        raise ValueError("agpt_trie_build_radix_part: bad arguments")
    return _export(h)


def build_chains(tokens: np.ndarray, n_chains: int, chain_len: int) -> Trie:
    tok = np.ascontiguousarray(tokens, dtype=np.int32)
    assert tok.shape[0] >= n_chains * chain_len
    h = C.c_void_p()
    if trie_lib().agpt_trie_build_chains(_ptr(tok), n_chains, chain_len, C.byref(h)):
        raise ValueError("agpt_trie_build_chains: bad arguments")
    return _export(h)


def write_radix_files(tokens: np.ndarray, max_depth: int, out_dir: str, vocab: int,
                      pipeline: str = "radix") -> None:
    """Builds the trie of `tokens` and writes the reference's radix files
    (subtrees/radix_subtree_%06d.bin, manifest.bin, meta.bin, format v2).
    pipeline "radix": the reference's on-disk builders (build_radix_trie);
    "ingest": the in-memory TrieCorpus trie (build_trie)."""
    import os
    os.makedirs(os.path.join(out_dir, "subtrees"), exist_ok=True)
    tok = np.ascontiguousarray(tokens, dtype=np.int32)
    h = C.c_void_p()
    lib = trie_lib()
    if pipeline == "radix":
        rc = lib.agpt_trie_build_radix(_ptr(tok), tok.shape[0], max_depth, C.byref(h))
    elif pipeline == "ingest":
        rc = lib.agpt_trie_build(_ptr(tok), tok.shape[0], max_depth, 0, C.byref(h))
    else:
        raise ValueError(f"pipeline {pipeline!r}: 'radix' or 'ingest'")
    if rc:
        raise ValueError("trie build: bad arguments")
    rc = lib.agpt_radix_write_subtrees(h, out_dir.encode(), vocab)
    lib.agpt_trie_free(h)
    if rc:
        raise OSError(f"agpt_radix_write_subtrees failed ({rc})")


@dataclass
class RadixSubtree:
    """One radix_subtree_%06d.bin, radix nodes in DFS preorder."""
    root_child_id: int
    max_endpoint_depth: int
    radix_id: np.ndarray          # [R] global ids
    radix_parent: np.ndarray      # [R] local, -1 for the root child
    first_char_depth: np.ndarray  # [R]
    edge_len: np.ndarray          # [R]
    edge_mass: np.ndarray         # [R]
    edge_tokens: np.ndarray       # [node-tokens], row order
    counts_offset: np.ndarray     # [R+1]
    counts_tok: np.ndarray
    counts_val: np.ndarray

    def rows(self) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
        """Node-token rows (one per edge char, DFS order): (parent, token,
        depth), the input of TrieAttention.plan."""
        qoff = np.zeros(self.edge_len.shape[0] + 1, np.int64)
        np.cumsum(self.edge_len, out=qoff[1:])
        T = int(qoff[-1])
        parent = np.arange(-1, T - 1, dtype=np.int64)  # within an edge: the previous row
        rp = self.radix_parent
        first = qoff[:-1]
        parent[first] = np.where(rp < 0, -1, qoff[np.maximum(rp, 0) + 1] - 1)
        depth = np.repeat(self.first_char_depth.astype(np.int64) - first, self.edge_len) + np.arange(T)
        return parent.astype(np.int32), self.edge_tokens.copy(), depth.astype(np.int32)


def read_radix_subtree(path: str) -> RadixSubtree:
    lib = trie_lib()
    h = C.c_void_p()
    rc = lib.agpt_radix_read_subtree(str(path).encode(), C.byref(h))
    if rc:
        raise ValueError(f"{path}: not a readable radix subtree file (code {rc})")
    R, nc, ne = C.c_int64(), C.c_int64(), C.c_int64()
    rcid, mx = C.c_int32(), C.c_int32()
    lib.agpt_radix_info(h, C.byref(R), C.byref(nc), C.byref(ne), C.byref(rcid), C.byref(mx))
    a = [np.empty(R.value, np.int32) for _ in range(5)]
    et = np.empty(nc.value, np.int32)
    co = np.empty(R.value + 1, np.int32)
    ct = np.empty(ne.value, np.int32)
    cv = np.empty(ne.value, np.int32)
    lib.agpt_radix_export(h, *[_ptr(x) for x in a], _ptr(et), _ptr(co), _ptr(ct), _ptr(cv))
    lib.agpt_radix_free(h)
    return RadixSubtree(rcid.value, mx.value, *a, et, co, ct, cv)


def read_radix_manifest(path: str) -> list[tuple[int, int, int, int]]:
    """manifest.bin: (root_child_id, n_nodes, total_edge_chars, max_endpoint_depth) per subtree."""
    import struct
    data = open(path, "rb").read()
    magic, ver, n = struct.unpack_from("<Iii", data, 0)
    if magic != 0x52445841 or ver != 2:
        raise ValueError(f"{path}: not a v2 radix manifest")
    return [struct.unpack_from("<iiqi", data, 12 + 20 * i) for i in range(n)]


# BASELINE.json configs (synthetic tries). Seeds are fixed and recorded.
CONFIGS = {
    "C1": dict(n=200_000, order=3, vocab=65, zipf=1.1, depth=32, seed=1, H=4, hd=16, dtype="f32"),
    "C2": dict(n=1_100_000, order=5, vocab=65, zipf=1.1, depth=32, seed=2, H=8, hd=16, dtype="f32"),
    # C4 at full size is ~6e8 node-tokens (0.6 TB per bf16 [T, 512] tensor):
    # one GPU holds the 0.02 share (~1.3e7 node-tokens, ~0.15 TB of tensors).
    "C4": dict(n=5_000_000, order=8, vocab=256, zipf=1.2, depth=128, seed=4, H=8, hd=64,
               dtype="bf16", one_gpu_scale=0.02),
    "C5": dict(chains=512, chain_len=256, vocab=65, seed=5, H=4, hd=64, dtype="bf16"),
}


def config_trie(name: str, scale: float = 1.0, counts: bool = False) -> Trie:
    """The synthetic trie of a BASELINE config; scale < 1 shrinks the corpus."""
    c = CONFIGS[name]
    if "chains" in c:
        n_chains = max(1, int(c["chains"] * scale))
        tok = uniform_tokens(n_chains * c["chain_len"], c["vocab"], c["seed"])
        return build_chains(tok, n_chains, c["chain_len"])
    n = max(2, int(c["n"] * scale))
    tok = markov_corpus(n, c["order"], c["vocab"], c["zipf"], c["seed"])
    # "Build the leveled trie at max depth D, then radix-compress it":
    # the reference's on-disk pipeline.
    return build_radix_trie(tok, c["depth"], counts=counts)
