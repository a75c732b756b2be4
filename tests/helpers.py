"""Shared test helpers: seeded tries and tensors, tolerance checks."""
from __future__ import annotations

import math

import numpy as np

from agpt_amd import trie as trie_mod

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
