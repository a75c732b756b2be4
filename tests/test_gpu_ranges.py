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


@pytest.mark.skip(reason="RangedTrieAttention.capture is switched off: capturing the two-stream range pass "
                         "ended in a segmentation fault at the end of capture (torch capture_end) on "
                         "MI355X, before any replay; no cause found in this code")
def test_ranges_graph_replay(gpu):
    """RangedTrieAttention.capture: the ranges' forward and backward on two
    streams captured once into a HIP graph. Every replay, with the outputs
    filled with NaN and eager work and synchronisations in between, writes
    the same bytes as the eager one-stream pass; an eager pass after the
    replays still does too."""
    import torch

    from agpt_amd import trie
    from agpt_amd.attention import RangedTrieAttention, partition_starts, range_batches

    tr = trie.config_trie("C2", scale=0.002)
    T, H, hd = tr.n_nodes, 8, 16
    D = H * hd
    ranges = range_batches(T, 4000, partition_starts(tr.radix_head, tr.depth))
    assert len(ranges) > 8
    Q, K, V, G = tensors(T, D, 11)
    q, k, v, g = (torch.from_numpy(x).cuda() for x in (Q, K, V, G))
    rope = tuple(torch.from_numpy(x).cuda() for x in ORC.rope_table(32, hd))
    ratt = RangedTrieAttention(H, hd, tr.parent, ranges, max_depth=32)
    o, lse, grads = ratt.fwd_bwd(q, k, v, g, rope=rope, n_streams=1)
    torch.cuda.synchronize()
    ref = [x.clone() for x in (o, lse, *grads)]
    out = torch.empty_like(q)
    lse_g = torch.empty(T, H, device=q.device, dtype=torch.float32)
    grads_g = tuple(torch.empty(T, D, device=q.device, dtype=torch.float32) for _ in range(3))
    graph = ratt.capture(q, k, v, g, out=out, lse=lse_g, grads=grads_g, rope=rope, n_streams=2)
    bufs = (out, lse_g, *grads_g)
    x = torch.randn(256, 256, device=q.device)
    for rep in range(3):
        for b in bufs:
            b.fill_(float("nan"))
        x = torch.tanh(x @ x)  # eager work between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("O", "lse", "dQ", "dK", "dV"), bufs, ref):
            assert torch.equal(a, b), f"replay {rep}: {name} differs from the eager pass"
    o2, lse2, grads2 = ratt.fwd_bwd(q, k, v, g, rope=rope, n_streams=2)
    torch.cuda.synchronize()
    for a, b in zip((o2, lse2, *grads2), ref):
        assert torch.equal(a, b)
    del graph
    ratt.close()
