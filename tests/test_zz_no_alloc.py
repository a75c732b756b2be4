"""agpt_attn_plan_static (the plan that allocates nothing: its device tables
and workspace live in the library's static scratch) against agpt_attn_plan,
through the C ABI: two static plans in a row on one handle, the second with
a smaller trie, each followed by fwd + bwd, give the same bytes as the
allocating plan, and free device memory (hipMemGetInfo) is the same before
and after them (inputs and outputs allocated beforehand); a later static
plan on the device invalidates an earlier handle's; a batch past the scratch
is refused with its size; a handle with an allocated plan is refused."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import scale_of, tensors

pytestmark = pytest.mark.gpu


def _inputs(T, D, seed):
    import torch
    Q, K, V, G = (torch.from_numpy(x).cuda() for x in tensors(T, D, seed))
    acc = [torch.from_numpy(x).cuda() for x in tensors(T, D, seed + 1, n=2)]
    return Q, K, V, G, acc


def _outputs(T, D, H):
    import torch
    return [torch.empty(T, D, device="cuda"), torch.empty(T, H, device="cuda")] + \
        [torch.empty(T, D, device="cuda") for _ in range(3)]


def _fwd_bwd(att, inp, out, rope):
    Q, K, V, G, acc = inp
    o, lse, dq, dk, dv = out
    att.forward(Q, K, V, out=o, lse=lse)
    att.backward(Q, K, V, o, lse, G, acc_dk=acc[0], acc_dv=acc[1], rope=rope, out=(dq, dk, dv))


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
    cases = [(tr, _inputs(tr.n_nodes, D, seed), _outputs(tr.n_nodes, D, H)) for tr, seed in ((big, 1), (small, 2))]
    st = TrieAttention(H, hd, max_depth=32)
    # a first static plan and run loads the code objects and looks the
    # scratch up; what follows must not change free device memory
    st.plan_static(small.parent)
    _fwd_bwd(st, cases[1][1], cases[1][2], rope)
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    for tr, inp, out in cases:  # two calls in a row, the second smaller
        st.plan_static(tr.parent)
        _fwd_bwd(st, inp, out, rope)
        torch.cuda.synchronize()
        assert torch.cuda.mem_get_info()[0] == free0, f"device memory allocated (T={tr.n_nodes})"
    for tr, inp, g in cases:
        ref = TrieAttention(H, hd, max_depth=32)
        ref.plan(tr.parent)
        want = _outputs(tr.n_nodes, D, H)
        _fwd_bwd(ref, inp, want, rope)
        torch.cuda.synchronize()
        ref.close()
        for name, a, b in zip(("O", "lse", "dQ", "dK", "dV"), g, want):
            assert torch.equal(a, b), f"{name} differs (T={tr.n_nodes})"
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
    big = trie.config_trie("C2", scale=0.05)
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
