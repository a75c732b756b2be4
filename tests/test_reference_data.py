"""The trie builder against what the reference recorded on its own corpus.

Fixtures in tests/golden/reference_data/ are data files the reference
holds, copied unchanged:
  input.txt         data/input.txt (the Shakespeare corpus, 1,115,394 chars)
  input.model       data/input.model (MGPT weights)
  sparsity_d*.txt   rnd/sparsity-profile/results/d{8,16,32}.txt: the output
                    of src/tools/trie_profile.cr on the radix tries the
                    reference built from input.txt at depths 8, 16, 32
  train_d*.log      bin/agpt_train logs on those tries (header lines printed
                    by load_radix_trie and run_radix_training,
                    agpt_train.cu:795-942, 3302, 3375, 3414, 3746):
                    d8  rnd/radix-saturation/logs/1step-d8-lr-3e-2-ep1_r1.log
                    d16 rnd/post-fix-baseline/logs/d16-det-wc-lr3e-4_r3.log
                    d32 rnd/post-fix-baseline/logs/d32-det-const-lr1e-3_r1.log

build_radix_trie restates the reference's on-disk pipeline
(StreamingLeveledBuilder, streaming_leveled_builder.cr:48-108, then
StreamingRadixBuilder, streaming_radix_builder.cr:149-180). Every figure
below is recomputed from its output with the formula of the tool that
printed it, formatted with the same printf pattern, and compared as text:
integer parity with the reference's own runs. CPU only.
"""
from __future__ import annotations

import re
from pathlib import Path

import numpy as np
import pytest

from agpt_amd import trie

DATA = Path(__file__).resolve().parent / "golden" / "reference_data"


def _corpus() -> np.ndarray:
    raw = (DATA / "input.txt").read_bytes()
    # Character ids: any one-to-one map gives the same counts; sorted bytes.
    lut = np.full(256, -1, np.int32)
    chars = sorted(set(raw))
    lut[chars] = np.arange(len(chars), dtype=np.int32)
    return lut[np.frombuffer(raw, np.uint8)]


class RadixView:
    """The radix records of a build_radix_trie result, as the reference's
    readers see them: per radix node (DFS order) its edge rows, endpoint
    counts and edge mass."""

    def __init__(self, tr: trie.Trie):
        T = tr.n_nodes
        self.T = T
        self.head = np.flatnonzero(tr.radix_head).astype(np.int64)
        self.last = np.append(self.head[1:], T) - 1              # endpoint row of each edge
        self.edge_len = (self.last - self.head + 1).astype(np.int64)
        self.first_depth = tr.depth[self.head].astype(np.int64)
        self.ep_depth = tr.depth[self.last].astype(np.int64)
        off = tr.next_offsets.astype(np.int64)
        self.n_entries = off[self.last + 1] - off[self.last]     # counts.size at the endpoint
        csum = np.concatenate([[0], np.cumsum(tr.next_val, dtype=np.int64)])
        self.ep_total = csum[off[self.last + 1]] - csum[off[self.last]]
        self.mass = csum[off[self.head + 1]] - csum[off[self.head]]  # v2 edge_mass
        radix_of = np.cumsum(tr.radix_head) - 1
        par = tr.parent[self.head]
        self.radix_parent = np.where(par < 0, -1, radix_of[np.maximum(par, 0)])
        self.depth_file_count = int(self.ep_depth.max()) + 1


_CACHE: dict[int, RadixView] = {}


def _view(depth: int) -> RadixView:
    if depth not in _CACHE:
        _CACHE[depth] = RadixView(trie.build_radix_trie(_corpus(), depth, counts=True))
    return _CACHE[depth]


def _profile_rows(v: RadixView) -> list[str]:
    """Per-depth table of src/tools/trie_profile.cr:94-119."""
    rows = []
    for d in range(1, v.depth_file_count):
        sel = v.ep_depth == d
        n = int(sel.sum())
        if n == 0:
            continue
        totals = np.sort(v.ep_total[sel])
        branches = v.n_entries[sel]
        lens = v.edge_len[sel]
        cap = d == v.depth_file_count - 1
        single = f"{100.0 * int((branches <= 1).sum()) / n:.2f}%" if cap else "   (n/a)"
        rows.append("  %5d  %9d  %13d  %10d  %9.2f  %9d  %9.2f  %12.2f  %14d  %s" % (
            d, n, int(totals.sum()), int(totals[n // 2]), float(totals.sum()) / n, int(totals[-1]),
            float(branches.sum()) / n, float(lens.sum()) / n, int(lens.sum()) - n, single))
    return rows


@pytest.mark.parametrize("depth", [8, 16, 32])
def test_sparsity_profile_matches_reference(depth):
    text = (DATA / f"sparsity_d{depth}.txt").read_text()
    v = _view(depth)
    want = [ln for ln in text.splitlines() if re.match(r"^\s+\d+\s+\d+\s+\d+\s+\d+\s+[\d.]+\s+\d+", ln)]
    got = _profile_rows(v)
    assert len(want) == depth
    assert got == want
    # TRIE SIZE block (trie_profile.cr:40-55)
    radix_count = v.head.shape[0] + 1  # + the virtual root
    assert f"radix_count        = {radix_count}" in text
    assert f"total_edge_chars   = {v.T}" in text
    assert f"compression        = {v.T / radix_count:.2f}x" in text
    assert f"depth_file_count   = {v.depth_file_count} " in text
    assert f"corpus_token_count = {_corpus().shape[0]}" in text
    # COMPRESSION SUMMARY (trie_profile.cr:128-135)
    absorbed = v.T - v.head.shape[0]
    assert f"radix endpoints          = {v.head.shape[0]}  " in text
    assert f"absorbed into edges      = {absorbed}  " in text
    assert f"{100.0 * absorbed / v.T:.2f}% of leveled nodes got compressed" in text


def _log_lines(v: RadixView) -> dict[str, str]:
    """The header lines bin/agpt_train prints about the radix trie."""
    R = v.head.shape[0]
    out = {
        "Radix trie:": "  Radix trie: %d nodes, %d total edge chars, %d endpoint depths" % (
            R + 1, v.T, v.depth_file_count),
        # total counts entries; ancestor chars = Σ over radix nodes of the
        # edge chars above them (agpt_train.cu:895-942)
        "Radix loaded:": "  Radix loaded: %d counts entries, %d ancestor char entries" % (
            int(v.n_entries.sum()), int((v.first_depth - 1).sum())),
        # agpt_train.cu:3290-3303
        "max edge_len:": "  max edge_len: %d, max ancestor chars: %d, max KV per node: %d, max endpoint depth: %d" % (
            int(v.edge_len.max()), int((v.first_depth - 1).max()),
            int((v.first_depth - 1).max() + v.edge_len.max()), int(v.ep_depth.max())),
    }
    # mass=1 compaction (agpt_train.cu:3355-3377): chars of edges with edge_mass == 1
    m1 = int(v.edge_len[v.mass == 1].sum())
    out["mass=1 compaction:"] = "  mass=1 compaction: %d / %d chars are mass=1 (%.1f%%); cache holds %d positions" % (
        m1, v.T, 100.0 * m1 / v.T, v.T - m1)
    # loop points (agpt_train.cu:3398-3416): radix leaves with edge_mass > 1
    nchild = np.bincount(v.radix_parent[v.radix_parent >= 0], minlength=R)
    heavy = v.mass > 1
    n_loop = int((heavy & (nchild == 0)).sum())
    out["loop points:"] = "  loop points: %d (mass>1 leaves; %.1f%% of %d mass>1 nodes)" % (
        n_loop, 100.0 * n_loop / max(int(heavy.sum()), 1), int(heavy.sum()))
    # root-child subtree sizes in radix nodes (agpt_train.cu:3603-3748)
    root = np.empty(R, np.int64)
    for r in range(R):  # parents precede children
        root[r] = r if v.radix_parent[r] < 0 else root[v.radix_parent[r]]
    sizes = np.bincount(root)[np.unique(root)]
    out["root-child subtrees:"] = "  %d root-child subtrees: sizes min=%d max=%d avg=%.1f (total=%d radix nodes)" % (
        sizes.shape[0], int(sizes.min()), int(sizes.max()), float(sizes.mean()), R)
    return out


@pytest.mark.parametrize("depth", [8, 16, 32])
def test_training_log_header_matches_reference(depth):
    log = (DATA / f"train_d{depth}.log").read_text().splitlines()
    v = _view(depth)
    checked = 0
    for key, line in _log_lines(v).items():
        hits = [ln for ln in log if key in ln]
        if not hits:  # the d8 log predates the compaction and loop-point lines
            assert depth == 8 and key in ("mass=1 compaction:", "loop points:")
            continue
        assert hits[0] == line, key
        checked += 1
    assert checked >= 4
    # Node-tokens per epoch (the metric's unit): "... N nodes)" on every epoch line.
    epochs = [ln for ln in log if ln.startswith("Epoch ")]
    assert epochs and all(ln.endswith(f" {v.T} nodes)") for ln in epochs)


def test_radix_files_of_reference_corpus(tmp_path):
    """The radix files written for input.txt at depth 8 hold the reference's
    counts: one subtree per root child, 845,539 radix nodes, 1,545,081 edge
    chars, the log's subtree sizes."""
    trie.write_radix_files(_corpus(), 8, str(tmp_path), 65)
    man = trie.read_radix_manifest(str(tmp_path / "manifest.bin"))
    sizes = np.array([m[1] for m in man])
    assert len(man) == 65 and int(sizes.sum()) == 845539 and sum(m[2] for m in man) == 1545081
    assert (int(sizes.min()), int(sizes.max()), round(float(sizes.mean()), 1)) == (1, 89208, 13008.3)
    assert max(m[3] for m in man) == 8
    import struct
    meta = (tmp_path / "meta.bin").read_bytes()
    magic, ver, rcount, dfc, chars, ntok, vocab = struct.unpack_from("<Iiiiqii", meta, 0)
    assert (rcount, dfc, chars, ntok, vocab) == (845540, 9, 1545081, 1115394, 65)
    v = _view(8)
    rc = man[int(np.argmax(sizes))][0]
    st = trie.read_radix_subtree(str(tmp_path / "subtrees" / f"radix_subtree_{rc:06d}.bin"))
    assert int(st.counts_offset[-1]) == int(st.counts_val.shape[0])
    # the file's records agree with the radix view of the same trie
    heads_in = int(st.radix_id.shape[0])
    assert heads_in == 89208 and int(st.edge_len.sum()) == int(st.edge_tokens.shape[0])
    assert int(st.edge_mass.max()) <= int(v.mass.max())


def test_reference_model_file_loads():
    """data/input.model: the header the training logs print (d=64 heads=4
    layers=2 ff=256 vocab=65 seq=128) and 108,481 weight floats
    ("Loaded 108481 weight floats (423.8 KB)")."""
    from agpt_amd import checkpoint

    cfg, flat = checkpoint.load_mgpt(str(DATA / "input.model"))
    assert (cfg.d_model, cfg.n_heads, cfg.n_layers, cfg.d_ff, cfg.vocab, cfg.max_depth) == (64, 4, 2, 256, 65, 128)
    assert flat.shape[0] == 108481
    assert f"Loaded {flat.shape[0]} weight floats ({flat.shape[0] * 4 / 1024:.1f} KB)" in \
        (DATA / "train_d32.log").read_text()
    assert np.isfinite(flat).all() and float(np.abs(flat).max()) > 0
    # Round trip through the writer is byte-identical.
    import tempfile, os
    with tempfile.TemporaryDirectory() as d:
        p = os.path.join(d, "m.model")
        checkpoint.save_mgpt(p, cfg, flat)
        assert open(p, "rb").read() == (DATA / "input.model").read_bytes()
