"""The committed fixtures (tests/golden/*.npz, written by make_golden.py)
against the oracle and, on the GPU, against the HIP path.

spec_chain and spec_branch are the spec's own cases
(spec/agpt_backward_attention_spec.cr:299-429 and :432-538: closed-form
model weights, the chain [0..7] at prefix lengths 1..4 and the branching
batch, upstream gradients and seeded accumulators, RoPE at seq_len 8);
random_small is a seeded trie with RoPE and accumulators at head_dim 8;
chains_4x16 four dense causal chains at head_dim 16.

CPU: the oracle reproduces every stored output bit for bit (the fixtures
pin the oracle against regressions). GPU: the HIP path, through the C ABI,
matches every stored output at the fp32 bar (1e-4 relative / 1e-5 absolute).
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from helpers import ATOL_F32, RTOL_F32, assert_close, scale_of
from oracle import oracle as ORC

HERE = Path(__file__).resolve().parent / "golden"
NAMES = ["spec_chain", "spec_branch", "random_small", "chains_4x16"]
SPEC_H, SPEC_HD = 2, 4  # spec model: d_model 8 = 2 heads x 4 (spec:12-51)


def _load(name):
    z = np.load(HERE / f"{name}.npz")
    d = {k: z[k] for k in z.files}
    H, hd = (int(d["H"]), int(d["hd"])) if "H" in d else (SPEC_H, SPEC_HD)
    return d, H, hd


def _cases(d):
    """(dO, acc_dk, acc_dv, expected dQ, dK, dV) per backward case."""
    if "dO_1" in d:
        return [(d[f"dO_{p}"], d[f"acc_dk_{p}"], d[f"acc_dv_{p}"], d[f"dQ_{p}"], d[f"dK_{p}"], d[f"dV_{p}"])
                for p in range(1, 5)]
    return [(d["dO"], d.get("acc_dk"), d.get("acc_dv"), d["dQ"], d["dK"], d["dV"])]


@pytest.mark.parametrize("name", NAMES)
def test_oracle_reproduces_fixture(name):
    d, H, hd = _load(name)
    sc = scale_of(hd)
    O, W, lse = ORC.fwd(d["parent"], d["Q"], d["K"], d["V"], H, hd, sc)
    assert np.array_equal(O, d["O"]) and np.array_equal(lse, d["lse"])
    rope = (d["rope_cos"], d["rope_sin"]) if "rope_cos" in d else None
    for dO, ak, av, dQ, dK, dV in _cases(d):
        gq, gk, gv = ORC.bwd(d["parent"], d["Q"], d["K"], d["V"], W, dO, H, hd, sc, acc_dk=ak, acc_dv=av,
                             rope=rope)
        assert np.array_equal(gq, dQ) and np.array_equal(gk, dK) and np.array_equal(gv, dV)


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
def test_hip_matches_fixture(gpu, name):
    import torch

    from agpt_amd.attention import TrieAttention

    d, H, hd = _load(name)
    dev = gpu
    cu = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    att = TrieAttention(H, hd, max_depth=int(ORC.depths(d["parent"]).max()))
    att.plan(d["parent"])
    q, k, v = cu(d["Q"]), cu(d["K"]), cu(d["V"])
    o, lse = att.forward(q, k, v)
    torch.cuda.synchronize()
    assert_close(o.cpu().numpy(), d["O"], RTOL_F32, ATOL_F32, f"{name} O")
    assert_close(lse.cpu().numpy(), d["lse"], RTOL_F32, ATOL_F32, f"{name} lse")
    rope = (cu(d["rope_cos"]), cu(d["rope_sin"])) if "rope_cos" in d else None
    for i, (dO, ak, av, dQ, dK, dV) in enumerate(_cases(d)):
        gq, gk, gv = att.backward(q, k, v, o, lse, cu(dO), acc_dk=cu(ak), acc_dv=cu(av), rope=rope)
        torch.cuda.synchronize()
        assert_close(gq.cpu().numpy(), dQ, RTOL_F32, ATOL_F32, f"{name}[{i}] dQ")
        assert_close(gk.cpu().numpy(), dK, RTOL_F32, ATOL_F32, f"{name}[{i}] dK")
        assert_close(gv.cpu().numpy(), dV, RTOL_F32, ATOL_F32, f"{name}[{i}] dV")
    att.close()
