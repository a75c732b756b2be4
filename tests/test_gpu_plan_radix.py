"""agpt_attn_plan_radix through the C ABI, the call INTEGRATION's C++ host
makes: the radix tables of the reference's per-subtree files
(agpt_radix_read_subtree; format streaming_radix_builder.cr:388-426, read
side agpt_train.cu:495-669) planned as radix nodes, whose node-token rows
the library expands itself (agpt_train.cu:892-940 ancestor chains). Forward
and backward then equal the oracle on the expanded rows."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import (ATOL_BF16, RTOL_BF16, abs_terms, assert_close, assert_close_or_f64, assert_close_terms,
                     f64_key_grads, round_bf16, scale_of, tensors)
from oracle import oracle as ORC

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("H,hd,dtype", [(8, 16, "f32"), (2, 64, "bf16")])
def test_plan_radix_from_subtree_files(gpu, tmp_path, H, hd, dtype):
    import torch

    from agpt_amd import trie
    from agpt_amd.attention import TrieAttention

    tok = trie.markov_corpus(6000, 3, 9, 1.1, seed=31)
    trie.write_radix_files(tok, 24, str(tmp_path), 9)
    man = trie.read_radix_manifest(str(tmp_path / "manifest.bin"))
    rc = max(man, key=lambda m: m[2])[0]  # the subtree with the most node-tokens
    st = trie.read_radix_subtree(str(tmp_path / "subtrees" / f"radix_subtree_{rc:06d}.bin"))
    parent = st.rows()[0]
    T, D = parent.shape[0], H * hd
    assert T > 1000 and int(st.edge_len.max()) > 1
    tdt = torch.float32 if dtype == "f32" else torch.bfloat16
    att = TrieAttention(H, hd, max_depth=24, dtype=tdt)
    att.plan_radix(st.radix_parent, st.edge_len)
    assert att.plan_info()["n_nodes"] == T
    Q, K, V, G = tensors(T, D, seed=hd)
    if dtype == "bf16":
        Q, K, V, G = (round_bf16(x) for x in (Q, K, V, G))
    rope = ORC.rope_table(24, hd)
    cu = lambda x: torch.from_numpy(x).cuda().to(tdt).contiguous()
    q, k, v, g = (cu(x) for x in (Q, K, V, G))
    o, lse = att.forward(q, k, v)
    dq, dk, dv = att.backward(q, k, v, o, lse, g, rope=tuple(torch.from_numpy(x).cuda() for x in rope))
    torch.cuda.synchronize()
    att.close()
    scale = scale_of(hd)
    Oo, W, lse_o = ORC.fwd(parent, Q, K, V, H, hd, scale)
    dQ, dK, dV = ORC.bwd(parent, Q, K, V, W, G, H, hd, scale, rope=rope)
    assert_close(lse.cpu().numpy(), lse_o, *((RTOL_BF16, ATOL_BF16) if dtype == "bf16" else ()), what="lse")
    got = [x.float().cpu().numpy() for x in (o, dq, dk, dv)]
    if dtype == "bf16":
        terms = lambda kind: (lambda rows: abs_terms(kind, parent, Q, K, V, G, W, H, hd, scale, rows, rope=rope))
        for name, x, want in zip(("O", "dQ", "dK", "dV"), got, (Oo, dQ, dK, dV)):
            assert_close_terms(x, want, terms(name), RTOL_BF16, ATOL_BF16, name)
        return
    assert_close(got[0], Oo, what="O")
    assert_close(got[1], dQ, what="dQ")
    # a key's dK/dV sums its whole subtree (the subtree root: every row);
    # rows outside the bar against the oracle are held to it against float64
    f64 = lambda rows: f64_key_grads(parent, Q, K, V, G, H, hd, scale, rows, rope=rope)
    assert_close_or_f64(got[2], dK, lambda r: f64(r)[0], what="dK")
    assert_close_or_f64(got[3], dV, lambda r: f64(r)[1], what="dV")
