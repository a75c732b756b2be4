"""The reference's radix files (format v2, streaming_radix_builder.cr:10-32,
388-470; read side agpt_train.cu:495-669): a subtree file assembled here
byte by byte reads back into the documented tables in DFS order; files
written from a trie read back into exactly that trie's node-token rows,
with edges cut where the reference's rule cuts them; malformed files are
refused. CPU only."""
from __future__ import annotations

import os
import struct

import numpy as np
import pytest

from agpt_amd import trie

MAGIC = 0x52445841


def _rec(rid, par, fcd, edge, mass, entries):
    b = struct.pack("<4i", rid, par, fcd, len(edge)) + struct.pack(f"<{len(edge)}i", *edge)
    b += struct.pack("<2i", mass, len(entries))
    for t, c in entries:
        b += struct.pack("<2i", t, c)
    return b


def test_hand_built_subtree_file(tmp_path):
    # root child 7 = "ab" (depth 1-2) branching to 9 = "c" and 8 = "de"
    # (global ids, breadth first); 8 branches again to 12 = "f".
    recs = [_rec(7, 0, 1, [0, 1], 10, [(2, 6), (3, 4)]),
            _rec(9, 7, 3, [3], 4, [(5, 4)]),            # first token 3
            _rec(8, 7, 3, [2, 4], 6, [(5, 5), (6, 1)]),  # first token 2: DFS before 9
            _rec(12, 8, 5, [5], 5, [(0, 5)])]
    body = b"".join(recs)
    head = struct.pack("<Iiiiqi", MAGIC, 2, 7, len(recs), 6, 5)
    p = tmp_path / "radix_subtree_000007.bin"
    p.write_bytes(head + body)
    st = trie.read_radix_subtree(str(p))
    assert st.root_child_id == 7 and st.max_endpoint_depth == 5
    assert st.radix_id.tolist() == [7, 8, 12, 9]          # DFS, children by first token
    assert st.radix_parent.tolist() == [-1, 0, 1, 0]
    assert st.first_char_depth.tolist() == [1, 3, 5, 3]
    assert st.edge_len.tolist() == [2, 2, 1, 1]
    assert st.edge_mass.tolist() == [10, 6, 5, 4]
    assert st.edge_tokens.tolist() == [0, 1, 2, 4, 5, 3]
    assert st.counts_offset.tolist() == [0, 2, 4, 5, 6]
    assert st.counts_tok.tolist() == [2, 3, 5, 6, 0, 5] and st.counts_val.tolist() == [6, 4, 5, 1, 5, 4]
    parent, token, depth = st.rows()
    assert parent.tolist() == [-1, 0, 1, 2, 3, 1]
    assert token.tolist() == [0, 1, 2, 4, 5, 3] and depth.tolist() == [1, 2, 3, 4, 5, 3]
    for bad in (struct.pack("<I", 0x1234) + (head + body)[4:],        # magic
                head[:4] + struct.pack("<i", 1) + (head + body)[8:],  # version
                (head + body)[:-4],                                   # truncated
                head + body + b"\0"):                                  # trailing
        q = tmp_path / "bad.bin"
        q.write_bytes(bad)
        with pytest.raises(ValueError):
            trie.read_radix_subtree(str(q))


@pytest.mark.parametrize("pipeline", ["radix", "ingest"])
@pytest.mark.parametrize("n,order,vocab,depth", [(2000, 2, 6, 10), (5000, 3, 9, 16), (800, 1, 4, 32)])
def test_written_files_read_back_into_the_trie(tmp_path, n, order, vocab, depth, pipeline):
    tok = trie.markov_corpus(n, order, vocab, 1.1, seed=n)
    trie.write_radix_files(tok, depth, str(tmp_path), vocab, pipeline=pipeline)
    if pipeline == "radix":
        tr = trie.build_radix_trie(tok, depth, counts=True)
    else:
        tr = trie.build_trie(tok, depth, counts=True)
    man = trie.read_radix_manifest(str(tmp_path / "manifest.bin"))
    kids = {}
    for i, p in enumerate(tr.parent):
        kids.setdefault(int(p), []).append(i)
    nent = np.diff(tr.next_offsets)
    rows, base, seen = [], 0, 0
    for rc, nodes, chars, max_ep in man:
        st = trie.read_radix_subtree(str(tmp_path / "subtrees" / f"radix_subtree_{rc:06d}.bin"))
        assert (st.root_child_id, st.radix_id.shape[0], st.edge_tokens.shape[0]) == (rc, nodes, chars)
        p, t, d = st.rows()
        assert int(d.max()) == max_ep
        qoff = np.concatenate([[0], np.cumsum(st.edge_len)])
        for r in range(st.radix_id.shape[0]):  # per edge: mass = head's counts, counts = endpoint's
            head, end = base + qoff[r], base + qoff[r + 1] - 1
            h0, h1 = tr.next_offsets[head], tr.next_offsets[head + 1]
            assert st.edge_mass[r] == int(tr.next_val[h0:h1].sum())
            a, b = tr.next_offsets[end], tr.next_offsets[end + 1]
            c0, c1 = st.counts_offset[r], st.counts_offset[r + 1]
            assert st.counts_tok[c0:c1].tolist() == tr.next_tok[a:b].tolist()
            assert st.counts_val[c0:c1].tolist() == tr.next_val[a:b].tolist()
            # the reference's cut (streaming_radix_builder.cr:155-170): inside an
            # edge every node has one next-token entry and its child; the
            # endpoint has not, and it has at least one entry (:177-180)
            for x in range(head, end):
                assert nent[x] == 1 and len(kids.get(x, [])) == 1
            assert not (nent[end] == 1 and len(kids.get(end, [])) == 1)
            assert nent[end] >= 1
        rows.append(np.where(p < 0, -1, p + base))
        base += p.shape[0]
        seen += nodes
    assert (np.concatenate(rows) == tr.parent).all()
    meta = (tmp_path / "meta.bin").read_bytes()
    magic, ver, rcount, dfc, chars, ntok = struct.unpack_from("<Iiiiqi", meta, 0)
    assert (magic, ver, rcount, chars, ntok) == (MAGIC, 2, seen + 1, tr.n_nodes, n)
    assert dfc == tr.max_depth + 1


def test_model_batch_from_files_equals_batch_from_trie(tmp_path):
    """The C3 model's batch tables built from the radix files (the
    reference's loader path) equal those built from the in-memory trie."""
    import torch

    from agpt_amd import model

    tok = trie.markov_corpus(3000, 2, 7, 1.1, seed=3)
    trie.write_radix_files(tok, 10, str(tmp_path), 7)
    tr = trie.build_radix_trie(tok, 10, counts=True)
    cfg = model.ModelConfig(vocab=7, d_model=64, n_heads=4, n_layers=2, d_ff=128, max_depth=10)
    b1 = model.TrieBatch(tr, cfg, torch.device("cpu"))
    man = trie.read_radix_manifest(str(tmp_path / "manifest.bin"))
    sts = [trie.read_radix_subtree(str(tmp_path / "subtrees" / f"radix_subtree_{rc:06d}.bin"))
           for rc, _, _, _ in man]
    b2 = model.TrieBatch.from_radix(sts, cfg, torch.device("cpu"))
    assert (b1.parent == b2.parent).all()
    assert all(torch.equal(x, y) for x, y in zip(b1.loss_args, b2.loss_args))
    assert torch.equal(b1.mass, b2.mass) and torch.equal(b1.positions, b2.positions)


def test_subtree_groups_cover_the_rows_in_order():
    from agpt_amd import model

    tok = trie.markov_corpus(4000, 2, 6, 1.1, seed=11)
    tr = trie.build_trie(tok, 12, counts=True)
    roots = set(np.flatnonzero(tr.parent < 0).tolist()) | {tr.n_nodes}
    for max_rows in (1, 100, 1000, 1 << 30):
        g = model.subtree_groups(tr, max_rows)
        assert g[0][0] == 0 and g[-1][1] == tr.n_nodes
        assert all(a < b and b == c for (a, b), (c, _) in zip(g, g[1:] + [(tr.n_nodes, 0)]))
        assert all(a in roots and b in roots for a, b in g)  # whole root-child subtrees
        assert all(b - a <= max_rows or len([r for r in roots if a < r < b]) == 0 for a, b in g)
    empty = trie.build_trie(np.zeros(1, np.int32), 4, counts=True)
    assert model.subtree_groups(empty, 10) == []


def _radix_rows(rp, el, cap=None):
    import ctypes as C

    from agpt_amd import _native
    lib = _native.attn_lib()
    rp = np.ascontiguousarray(rp, np.int32)
    el = np.ascontiguousarray(el, np.int32)
    n = C.c_int64(-1)
    i32 = lambda a: a.ctypes.data_as(C.POINTER(C.c_int32))
    rc = lib.agpt_attn_radix_rows(i32(rp), i32(el), rp.shape[0], None, 0, C.byref(n))
    if rc:
        return rc, None, lib.agpt_last_error().decode()
    out = np.full(n.value if cap is None else cap, -7, np.int32)
    rc = lib.agpt_attn_radix_rows(i32(rp), i32(el), rp.shape[0], i32(out), out.shape[0], C.byref(n))
    return rc, out[:n.value], lib.agpt_last_error().decode()


def test_radix_rows_of_written_files_equal_the_trie(tmp_path):
    """agpt_attn_radix_rows, the row expansion agpt_attn_plan_radix plans
    from (agpt_train.cu:892-940 chains), turns each subtree file's radix
    tables into the node-token parent table of the trie the files were
    written from (an independent vectorised expansion, RadixSubtree.rows,
    and the builder's own trie)."""
    from agpt_amd import _native

    tok = trie.markov_corpus(5000, 3, 9, 1.1, seed=21)
    trie.write_radix_files(tok, 16, str(tmp_path), 9)
    tr = trie.build_radix_trie(tok, 16)
    rows, base = [], 0
    for rc, _, chars, _ in trie.read_radix_manifest(str(tmp_path / "manifest.bin")):
        st = trie.read_radix_subtree(str(tmp_path / "subtrees" / f"radix_subtree_{rc:06d}.bin"))
        code, par, _ = _radix_rows(st.radix_parent, st.edge_len)
        assert code == _native.AGPT_OK and par.shape[0] == chars
        assert (par == st.rows()[0]).all()
        rows.append(np.where(par < 0, -1, par + base))
        base += chars
    assert (np.concatenate(rows) == tr.parent).all()


def test_radix_rows_errors():
    from agpt_amd import _native
    ok, par, _ = _radix_rows([-1, 0, 0, -1], [2, 1, 3, 1])
    assert ok == _native.AGPT_OK and par.tolist() == [-1, 0, 1, 1, 3, 4, -1]
    code, _, msg = _radix_rows([-1, 1], [1, 1])           # a parent that is not an earlier node
    assert code == _native.AGPT_ERR_NOT_DFS and "radix_parent[1]" in msg
    code, _, msg = _radix_rows([-1, -2], [1, 1])
    assert code == _native.AGPT_ERR_NOT_DFS
    code, _, msg = _radix_rows([-1, 0], [1, 0])           # an empty edge
    assert code == _native.AGPT_ERR_INVALID_ARG and "edge_len[1] = 0" in msg
    code, _, msg = _radix_rows([-1, 0], [3, -2])
    assert code == _native.AGPT_ERR_INVALID_ARG
    code, _, msg = _radix_rows([-1, 0], [2, 2], cap=3)   # output too small
    assert code == _native.AGPT_ERR_INVALID_ARG and "cap" in msg
    code, _, _ = _radix_rows(np.zeros(0, np.int32), np.zeros(0, np.int32))
    assert code == _native.AGPT_ERR_INVALID_ARG
