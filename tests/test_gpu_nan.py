"""NaN inputs surface in the outputs they reach.

The reference's divergence check is a NaN in the loss log
(tests/test_agpt_fundamentals.sh:121-134), so a NaN in Q, V or dO must not
vanish inside the attention (in a softmax max, a masked select or a
rescale). One NaN is planted per case; the CPU oracle (plain IEEE C)
computes which output elements it reaches. Bar: every element the oracle
makes NaN is NaN on the GPU, and every element finite on both sides
matches at the usual tolerance. The GPU may hold more NaN than the oracle,
but only near the affected rows: a 16x16 block pair multiplies its masked
(zero-weight) pairs by the operand rows as well, and 0 x NaN is NaN, so a
NaN row also reaches the other rows of the block pairs it takes part in.
Those rows lie in a 64-row tile that holds an affected row, or are
ancestors (prefix keys) of such a tile's rows.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import ATOL_BF16, ATOL_F32, RTOL_BF16, RTOL_F32, round_bf16, scale_of, small_trie, tensors
from oracle import oracle as ORC

pytestmark = pytest.mark.gpu


def _run(parent, Q, K, V, G, H, hd, dtype):
    import torch

    from agpt_amd.attention import TrieAttention
    tdt = torch.float32 if dtype == "f32" else torch.bfloat16
    att = TrieAttention(H, hd, max_depth=int(ORC.depths(parent).max()), dtype=tdt)
    att.plan(parent)
    q, k, v, g = (torch.from_numpy(x).cuda().to(tdt) for x in (Q, K, V, G))
    o, lse = att.forward(q, k, v)
    dq, dk, dv = att.backward(q, k, v, o, lse, g)
    torch.cuda.synchronize()
    out = [x.float().cpu().numpy() for x in (o, lse, dq, dk, dv)]
    att.close()
    return out


@pytest.mark.parametrize("dtype,H,hd", [("f32", 8, 16), ("f32", 2, 8), ("bf16", 2, 64)])
@pytest.mark.parametrize("where", ["Q", "V", "dO"])
def test_nan_surfaces(gpu, dtype, H, hd, where):
    tr = small_trie(n_tokens=500, depth=12, seed=17)
    T, D = tr.n_nodes, H * hd
    Q, K, V, G = tensors(T, D, seed=23)
    if dtype == "bf16":
        Q, K, V, G = (round_bf16(x) for x in (Q, K, V, G))
    # a row in the middle of the trie with ancestors and descendants
    depth = ORC.depths(tr.parent)
    row = int(np.flatnonzero((depth == 4) & (tr.subtree_end - np.arange(T) > 3))[0])
    {"Q": Q, "V": V, "dO": G}[where][row, hd + 1 if H > 1 else 1] = np.nan
    sc = scale_of(hd)
    Oo, W, lse_o = ORC.fwd(tr.parent, Q, K, V, H, hd, sc)
    dQ, dK, dV = ORC.bwd(tr.parent, Q, K, V, W, G, H, hd, sc)
    got = _run(tr.parent, Q, K, V, G, H, hd, dtype)
    rtol, atol = (RTOL_F32, ATOL_F32) if dtype == "f32" else (RTOL_BF16, ATOL_BF16)
    want = (Oo, lse_o, dQ, dK, dV)
    affected = np.zeros(T, bool)
    for w in want:
        affected |= np.isnan(w).reshape(T, -1).any(1)
    # rows of the 64-row tiles holding an affected row, and their ancestors
    near = np.isin(np.arange(T) // 64, np.unique(np.flatnonzero(affected) // 64))
    cur = np.flatnonzero(near)
    while cur.size:
        cur = tr.parent[cur]
        cur = cur[cur >= 0]
        cur = cur[~near[cur]]
        near[cur] = True
    n_reached = 0
    for name, g, w in zip(("O", "lse", "dQ", "dK", "dV"), got, want):
        wn, gn = np.isnan(w), np.isnan(g)
        n_reached += int(wn.sum())
        missed = wn & ~gn
        assert not missed.any(), f"{name}: {int(missed.sum())} NaN outputs of the oracle are not NaN"
        extra_rows = (gn & ~wn).reshape(T, -1).any(1)
        assert not (extra_rows & ~near).any(), f"{name}: NaN in rows away from the affected ones"
        both = ~wn & ~gn
        if dtype == "f32":
            err = np.abs(g - w)[both]
            assert (err <= atol + rtol * np.abs(w)[both]).all(), f"{name}: finite elements differ"
        # bf16 finite values are covered by the parity suite; here only NaN placement
    assert n_reached > 0
