"""Range batches of one trie on several streams (RangedTrieAttention.fwd_bwd,
agpt_attn_opts.ctx_wait): each range's forward then backward, the ranges
dealt over two streams, gives the same bytes as the ranges one after another
on one stream (the context rows' additions keep range order), and matches
the oracle on the whole trie."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import assert_close, assert_close_or_f64, f64_key_grads, scale_of, tensors
from oracle import oracle as ORC

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("cut", ["bigram", "rows"])
def test_ranges_on_two_streams(gpu, cut):
    import torch

    from agpt_amd import trie
    from agpt_amd.attention import RangedTrieAttention, partition_starts, range_batches

    tr = trie.config_trie("C2", scale=0.002)  # ~60K node-tokens, depth 32
    T, H, hd = tr.n_nodes, 8, 16
    D = H * hd
    if cut == "bigram":
        ranges = range_batches(T, 4000, partition_starts(tr.radix_head, tr.depth))
    else:
        ranges = range_batches(T, 1111)
    assert len(ranges) > 8
    Q, K, V, G = tensors(T, D, 9)
    q, k, v, g = (torch.from_numpy(x).cuda() for x in (Q, K, V, G))
    rt = ORC.rope_table(32, hd)
    rope = tuple(torch.from_numpy(x).cuda() for x in rt)
    ratt = RangedTrieAttention(H, hd, tr.parent, ranges, max_depth=32)
    outs = []
    for ns in (1, 2, 2):
        o, lse, (dq, dk, dv) = ratt.fwd_bwd(q, k, v, g, rope=rope, n_streams=ns)
        torch.cuda.synchronize()
        outs.append([x.clone() for x in (o, lse, dq, dk, dv)])
    for a, b in zip(outs[0], outs[1]):
        assert torch.equal(a, b)
    for a, b in zip(outs[1], outs[2]):
        assert torch.equal(a, b)
    ratt.close()
    o, lse, dq, dk, dv = (x.cpu().numpy() for x in outs[1])
    scale = scale_of(hd)
    Oo, W, lse_o = ORC.fwd(tr.parent, Q, K, V, H, hd, scale)
    dQ, dK, dV = ORC.bwd(tr.parent, Q, K, V, W, G, H, hd, scale, rope=rt)
    assert_close(o, Oo, what="O")
    assert_close(lse, lse_o, what="lse")
    assert_close(dq, dQ, what="dQ")
    f64 = lambda rows: f64_key_grads(tr.parent, Q, K, V, G, H, hd, scale, rows, rope=rt)
    assert_close_or_f64(dk, dK, lambda r: f64(r)[0], what="dK")
    assert_close_or_f64(dv, dV, lambda r: f64(r)[1], what="dV")
