"""Head dim 64 with bf16 inputs on deep tries, at the configurations' own
head counts: C4 (8 heads x 64, radix trie to depth 128)
and C5 (4 heads x 64, independent chains of 256), through the C ABI, against
the oracle (batched_depth_forward.cr:836-971, batched_depth_backward.cr:605-695)
on reduced corpora.

A reduced trie has few tiles, so the plan-size defaults would pick the
small-plan unit shapes (two heads per unit, one-tile chunks without the path
carry). The deep kernels' shapes that a full-size plan takes are forced here
with the tuning overrides: 4 heads per forward unit (the C4 forward), 8 per
dQ unit (the C4 dQ kernel), key-side chunks of 96 tiles with the register
carry, tile-order claims (by XCD ranges, and from one counter); plus the
carry rows without registers, short chunks and the whole-key-set kernels.
C5's chains run on the dense-causal chain kernels (the backward in one
launch; AGPT_ATTN_CHAINFUSE=0 keeps two); with AGPT_ATTN_CHAIN=0
they take the general kernels, whose key side runs by subtree range unless
AGPT_ATTN_RANGE=0 sends it through the carry. A forest of 200 chains of
1..256 rows at 4 heads has more (chain, head) units than the chain kernels'
grid, so their snake deal gives workgroups a second round. The oracle
runs once per case.

Bar (bf16 inputs): 2e-2 relative + 2e-3 absolute, elementwise; an element
outside it must be within the same bar relative to the sum of its terms'
magnitudes (helpers.assert_close_terms), and such elements are counted.
"""
from __future__ import annotations

import types

import numpy as np
import pytest

from helpers import (ATOL_BF16, RTOL_BF16, abs_terms, assert_close, assert_close_terms, round_bf16,
                     run_gpu, run_gpu_ranges, scale_of, tensors)
from oracle import oracle as ORC

pytestmark = pytest.mark.gpu

DEEP_SHAPES = {
    "small_plan_defaults": {},
    "fwd_units_4_heads_chunk96": {"AGPT_ATTN_DHPU": "4", "AGPT_ATTN_CHUNK": "96", "AGPT_ATTN_LPT": "0"},
    "dq_units_8_heads_chunk96": {"AGPT_ATTN_DHPU": "8", "AGPT_ATTN_CHUNK": "96", "AGPT_ATTN_LPT": "0"},
    "chunk24_carry_rows_only": {"AGPT_ATTN_CHUNK": "24", "AGPT_ATTN_REGCARRY": "0"},
    "chunk2_one_head_units": {"AGPT_ATTN_CHUNK": "2", "AGPT_ATTN_DHPU": "1"},
    "whole_key_set": {"AGPT_ATTN_DEEP": "0"},
    "carry_two_register_blocks_chunk96": {"AGPT_ATTN_REGITERS": "2", "AGPT_ATTN_CHUNK": "96"},
    "dq_delta_pass_then_dq": {"AGPT_ATTN_DQ1": "0"},
    "one_claim_counter_tile_order": {"AGPT_ATTN_XCD": "0", "AGPT_ATTN_LPT": "0", "AGPT_ATTN_DHPU": "4"},
    "key_side_carry_not_subtree_range": {"AGPT_ATTN_RANGE": "0", "AGPT_ATTN_CHAIN": "0"},
    "general_kernels_not_chain_kernels": {"AGPT_ATTN_CHAIN": "0"},
    "chain_kernels_two_launch_backward": {"AGPT_ATTN_CHAINFUSE": "0"},
}
_KNOBS = ("AGPT_ATTN_VARIANT", "AGPT_ATTN_DHPU", "AGPT_ATTN_CHUNK", "AGPT_ATTN_LPT", "AGPT_ATTN_REGCARRY",
          "AGPT_ATTN_DEEP", "AGPT_ATTN_CARRY", "AGPT_ATTN_HG", "AGPT_ATTN_REGITERS", "AGPT_ATTN_DQ1",
          "AGPT_ATTN_XCD", "AGPT_ATTN_RANGE", "AGPT_ATTN_CHAIN", "AGPT_ATTN_CHAINFUSE")

_CASES: dict = {}


@pytest.fixture(params=list(DEEP_SHAPES))
def shape(request, monkeypatch):
    for k in _KNOBS:
        monkeypatch.delenv(k, raising=False)
    for k, v in DEEP_SHAPES[request.param].items():
        monkeypatch.setenv(k, v)
    return request.param


def _case(name):
    """Seeded trie, bf16-rounded tensors, RoPE table, accumulators and the
    oracle's outputs, computed once per case."""
    if name in _CASES:
        return _CASES[name]
    from agpt_amd import trie
    if name == "C4":
        tr = trie.config_trie("C4", scale=0.00008)  # 400 tokens: 34.6K node-tokens, depth 128
        H, hd, seed = 8, 64, 40
    elif name == "C5":
        tr = trie.config_trie("C5", scale=16 / 512)  # 16 chains of 256
        H, hd, seed = 4, 64, 50
    else:
        # 200 chains of 1..256 rows at C5's 4 heads: 800 (chain, head) units,
        # more than a grid of two chain workgroups per CU holds on 256 CUs,
        # so workgroups take units in a second round of the snake deal.
        rng = np.random.default_rng(60)
        parts, n = [], 0
        for L in rng.integers(1, 257, size=200):
            parts.append(np.concatenate([[-1], np.arange(n, n + int(L) - 1)]))
            n += int(L)
        parent = np.concatenate(parts).astype(np.int32)
        tr = types.SimpleNamespace(parent=parent, n_nodes=int(parent.shape[0]))
        H, hd, seed = 4, 64, 60
    T, D = tr.n_nodes, H * hd
    Q, K, V, G = (round_bf16(x) for x in tensors(T, D, seed))
    rng = np.random.default_rng(seed + 1)
    acc = [rng.standard_normal((T, D)).astype(np.float32) * np.float32(0.1) for _ in range(2)]
    rope = ORC.rope_table(256, hd)
    scale = scale_of(hd)
    print(f"oracle for {name}: T={T} H={H} hd={hd}", flush=True)
    O, W, lse = ORC.fwd(tr.parent, Q, K, V, H, hd, scale)
    dQ, dK, dV = ORC.bwd(tr.parent, Q, K, V, W, G, H, hd, scale, acc_dk=acc[0], acc_dv=acc[1], rope=rope)
    c = dict(tr=tr, H=H, hd=hd, T=T, inputs=(Q, K, V, G), acc=acc, rope=rope, scale=scale, W=W,
             want=(O, lse, dQ, dK, dV))
    _CASES[name] = c
    return c


def _compare(c, got):
    Q, K, V, G = c["inputs"]
    o, lse, dq, dk, dv = got
    O, lse_o, dQ, dK, dV = c["want"]
    assert_close(lse, lse_o, RTOL_BF16, ATOL_BF16, "lse")

    def terms(kind):
        # an element's terms depend on the inputs only: rows already summed
        # for this case (under another shape) are reused
        cache = c.setdefault("terms", {}).setdefault(kind, {})

        def rows_terms(rows):
            need = np.array([r for r in rows if int(r) not in cache], np.int64)
            if need.size:
                t = abs_terms(kind, c["tr"].parent, Q, K, V, G, c["W"], c["H"], c["hd"], c["scale"], need,
                              rope=c["rope"], acc=c["acc"])
                for r, row in zip(need, t):
                    cache[int(r)] = row
            return np.stack([cache[int(r)] for r in rows])
        return rows_terms
    for name, x, want in (("O", o, O), ("dQ", dq, dQ), ("dK", dk, dK), ("dV", dv, dV)):
        assert_close_terms(x, want, terms(name), RTOL_BF16, ATOL_BF16, name)


@pytest.mark.parametrize("name", ["C4", "C5", "chains_two_rounds"])
def test_deep_config_sample(gpu, shape, name):
    """The whole sample as one plan, at the config's head count."""
    c = _case(name)
    Q, K, V, G = c["inputs"]
    got = run_gpu(c["tr"].parent, Q, K, V, G, c["H"], c["hd"], "bf16", rope=c["rope"], acc=c["acc"])
    _compare(c, got)


@pytest.mark.parametrize("packed", [False, True])
def test_c4_sample_range_batches(gpu, shape, packed):
    """The C4 sample cut every 6,000 rows (cuts inside subtrees, contexts of
    any depth up to 127), one range plan each."""
    from agpt_amd.attention import range_batches
    c = _case("C4")
    Q, K, V, G = c["inputs"]
    ranges = range_batches(c["T"], 6000)
    assert len(ranges) >= 5
    got = run_gpu_ranges(c["tr"].parent, Q, K, V, G, c["H"], c["hd"], "bf16", ranges, packed, rope=c["rope"],
                         acc=c["acc"])
    _compare(c, got)
