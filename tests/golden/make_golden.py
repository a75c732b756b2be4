"""Writes the committed fixtures under tests/golden/ (inputs + expected
outputs of the trie-attention path).

The reference holds no stored vectors for this path (its spec compares two
formulations at run time, spec/agpt_backward_attention_spec.cr:337-535), and
its implementation cannot run here (Crystal + the unvendored µGPT shard). The
expected outputs are therefore those of the C restatement (oracle/), which
tests/test_oracle.py pins against the spec's two-formulation agreement, torch
float64 autograd on masked dense attention, causal SDPA, finite differences
and closed forms.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(HERE))

import spec_model as SM  # noqa: E402
from agpt_amd import trie as trie_mod  # noqa: E402
from oracle import oracle as ORC  # noqa: E402


def scale_of(hd):
    return float(np.float32(1.0 / math.sqrt(hd)))


def spec_chain():
    """spec:299-429: the chain trie of tokens [0..7], max_depth 6, max_starts 1;
    one case per prefix_len 1..4 where only the query at that depth carries an
    upstream gradient and a seeded own accumulator."""
    tr = trie_mod.build_trie(np.arange(8, dtype=np.int32), 6, max_starts=1)
    cos_t, sin_t = ORC.rope_table(SM.SEQ_LEN, SM.HEAD_DIM)
    Q, K, V = SM.qkv(tr.token, tr.depth, cos_t, sin_t)
    T, H, hd = tr.n_nodes, SM.N_HEADS, SM.HEAD_DIM
    sc = scale_of(hd)
    O, W, lse = ORC.fwd(tr.parent, Q, K, V, H, hd, sc)
    out = dict(parent=tr.parent, token=tr.token, Q=Q, K=K, V=V, rope_cos=cos_t, rope_sin=sin_t,
               O=O, lse=lse, W=W)
    for p in range(1, 5):
        n = p - 1  # the chain's row at depth p
        assert tr.depth[n] == p
        dO = np.zeros((T, SM.D_MODEL), np.float32)
        dO[n] = SM.d_head_out(SM.chain_d_attn_proj(p))
        acc_k = np.zeros_like(dO)
        acc_v = np.zeros_like(dO)
        acc_k[n], acc_v[n] = SM.current_accum(p)
        dQ, dK, dV = ORC.bwd(tr.parent, Q, K, V, W, dO, H, hd, sc, acc_dk=acc_k, acc_dv=acc_v,
                             rope=(cos_t, sin_t))
        out.update({f"dO_{p}": dO, f"acc_dk_{p}": acc_k, f"acc_dv_{p}": acc_v, f"dQ_{p}": dQ,
                    f"dK_{p}": dK, f"dV_{p}": dV})
    return out


BRANCH_TOKENS = [0, 1, 2, 7, 0, 1, 3, 7, 0, 4, 2, 7, 0, 4, 3, 7]


def spec_branch():
    """spec:432-538: tokens BRANCH_TOKENS, max_depth 4; the first depth level
    with more than one node (depth 1) is the batch. Row i of the spec's
    d_attn_proj belongs to the i-th depth-1 node in first-insertion order."""
    tok = np.array(BRANCH_TOKENS, np.int32)
    tr = trie_mod.build_trie(tok, 4)
    cos_t, sin_t = ORC.rope_table(SM.SEQ_LEN, SM.HEAD_DIM)
    Q, K, V = SM.qkv(tr.token, tr.depth, cos_t, sin_t)
    T, H, hd = tr.n_nodes, SM.N_HEADS, SM.HEAD_DIM
    sc = scale_of(hd)
    O, W, lse = ORC.fwd(tr.parent, Q, K, V, H, hd, sc)
    first_seen = []
    for t in tok[:-1]:  # starts 0..n-2
        if t not in first_seen:
            first_seen.append(int(t))
    dO = np.zeros((T, SM.D_MODEL), np.float32)
    acc_k = np.zeros_like(dO)
    acc_v = np.zeros_like(dO)
    for i, t in enumerate(first_seen):
        row = int(np.flatnonzero((tr.depth == 1) & (tr.token == t))[0])
        dO[row] = SM.d_head_out(SM.branch_d_attn_proj(i))
        acc_k[row], acc_v[row] = SM.current_accum(1)
    dQ, dK, dV = ORC.bwd(tr.parent, Q, K, V, W, dO, H, hd, sc, acc_dk=acc_k, acc_dv=acc_v,
                         rope=(cos_t, sin_t))
    return dict(parent=tr.parent, token=tr.token, Q=Q, K=K, V=V, rope_cos=cos_t, rope_sin=sin_t,
                O=O, lse=lse, dO=dO, acc_dk=acc_k, acc_dv=acc_v, dQ=dQ, dK=dK, dV=dV)


def random_small():
    tok = trie_mod.markov_corpus(160, 2, 6, 1.1, seed=77)
    tr = trie_mod.build_trie(tok, 8)
    H, hd = 2, 8
    T, D = tr.n_nodes, H * hd
    rng = np.random.default_rng(2024)
    Q, K, V, dO = (rng.standard_normal((T, D)).astype(np.float32) for _ in range(4))
    acc_k, acc_v = (np.float32(0.1) * rng.standard_normal((T, D)).astype(np.float32)
                    for _ in range(2))
    cos_t, sin_t = ORC.rope_table(16, hd)
    sc = scale_of(hd)
    O, W, lse = ORC.fwd(tr.parent, Q, K, V, H, hd, sc)
    dQ, dK, dV = ORC.bwd(tr.parent, Q, K, V, W, dO, H, hd, sc, acc_dk=acc_k, acc_dv=acc_v,
                         rope=(cos_t, sin_t))
    return dict(parent=tr.parent, Q=Q, K=K, V=V, dO=dO, acc_dk=acc_k, acc_dv=acc_v,
                rope_cos=cos_t, rope_sin=sin_t, O=O, lse=lse, dQ=dQ, dK=dK, dV=dV, H=H, hd=hd)


def chains():
    tok = trie_mod.uniform_tokens(4 * 16, 65, seed=5)
    tr = trie_mod.build_chains(tok, 4, 16)
    H, hd = 2, 16
    T, D = tr.n_nodes, H * hd
    rng = np.random.default_rng(7)
    Q, K, V, dO = (rng.standard_normal((T, D)).astype(np.float32) for _ in range(4))
    sc = scale_of(hd)
    O, W, lse = ORC.fwd(tr.parent, Q, K, V, H, hd, sc)
    dQ, dK, dV = ORC.bwd(tr.parent, Q, K, V, W, dO, H, hd, sc)
    return dict(parent=tr.parent, Q=Q, K=K, V=V, dO=dO, O=O, lse=lse, dQ=dQ, dK=dK, dV=dV,
                H=H, hd=hd)


FIXTURES = {"spec_chain": spec_chain, "spec_branch": spec_branch,
            "random_small": random_small, "chains_4x16": chains}


def main():
    for name, fn in FIXTURES.items():
        data = fn()
        np.savez_compressed(HERE / f"{name}.npz", **data)
        print(f"wrote {name}.npz ({len(data)} arrays)")


if __name__ == "__main__":
    main()
