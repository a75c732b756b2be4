"""agpt_attn_plan_static (the plan that allocates nothing: its device tables
and workspace live in the library's static scratch) against agpt_attn_plan,
through the C ABI: two static plans in a row on one handle, the second with
a smaller trie, each followed by fwd + bwd, give the same bytes as the
allocating plan; a later static plan on the device invalidates an earlier
handle's; a batch past the scratch is refused with its size; a handle with
an allocated plan is refused."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import scale_of, tensors

pytestmark = pytest.mark.gpu


def _fwd_bwd(att, T, D, seed, rope):
    import torch
    Q, K, V, G = (torch.from_numpy(x).cuda() for x in tensors(T, D, seed))
    acc = [torch.from_numpy(x).cuda() for x in tensors(T, D, seed + 1, n=2)]
    o, lse = att.forward(Q, K, V)
    dq, dk, dv = att.backward(Q, K, V, o, lse, G, acc_dk=acc[0], acc_dv=acc[1], rope=rope)
    torch.cuda.synchronize()
    return [x.clone() for x in (o, lse, dq, dk, dv)]


@pytest.mark.parametrize("H,hd", [(8, 16), (2, 64)])
def test_plan_static_matches_plan(gpu, H, hd):
    import torch

    from agpt_amd import trie
    from agpt_amd.attention import TrieAttention, rope_tables

    D = H * hd
    rope = rope_tables(32, hd)
    big = trie.config_trie("C2", scale=0.0015)     # ~40K node-tokens, depth 32
    small = trie.config_trie("C1", scale=0.002)    # a few thousand
    assert small.n_nodes < big.n_nodes
    st = TrieAttention(H, hd, max_depth=32)
    for tr, seed in ((big, 1), (small, 2)):
        st.plan_static(tr.parent)
        got = _fwd_bwd(st, tr.n_nodes, D, seed, rope)
        ref = TrieAttention(H, hd, max_depth=32)
        ref.plan(tr.parent)
        want = _fwd_bwd(ref, tr.n_nodes, D, seed, rope)
        ref.close()
        for name, g, w in zip(("O", "lse", "dQ", "dK", "dV"), got, want):
            assert torch.equal(g, w), f"{name} differs (T={tr.n_nodes})"
    st.close()


def test_plan_static_errors(gpu):
    import torch

    from agpt_amd import _native as N
    from agpt_amd import trie
    from agpt_amd.attention import TrieAttention

    tr = trie.config_trie("C1", scale=0.002)
    a = TrieAttention(4, 16, max_depth=32)
    b = TrieAttention(4, 16, max_depth=32)
    a.plan_static(tr.parent)
    b.plan_static(tr.parent)  # takes the device's scratch over
    q = torch.zeros(tr.n_nodes, 64, device="cuda")
    with pytest.raises(N.AgptError) as e:
        a.forward(q, q, q)
    assert e.value.code == N.AGPT_ERR_NO_PLAN
    o, lse = b.forward(q, q, q)
    torch.cuda.synchronize()
    # too large for the scratch: refused, with the bytes it needs
    big = trie.config_trie("C2", scale=0.01)
    with pytest.raises(N.AgptError) as e:
        b.plan_static(big.parent)
    assert e.value.code == N.AGPT_ERR_INVALID_ARG and "bytes" in str(e.value)
    # a handle holding an allocated plan is refused
    c = TrieAttention(4, 16, max_depth=32)
    c.plan(tr.parent)
    with pytest.raises(N.AgptError) as e:
        c.plan_static(tr.parent)
    assert e.value.code == N.AGPT_ERR_INVALID_ARG
    for x in (a, b, c):
        x.close()
