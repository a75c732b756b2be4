"""HIP per-query AGPT loss (agpt_loss_per_query through the C ABI) vs the
pinned C oracle (oracle/loss_oracle.c) on seeded radix batches.

Bar: fp32, 1e-4 relative / 1e-5 absolute on d_logits and the loss (the
softmax sums run in another order than the oracle's; nothing else differs).
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import ATOL_F32, RTOL_F32, assert_close, loss_batch
from oracle import oracle as ORC

pytestmark = pytest.mark.gpu

ARGS = ("logits", "query_to_node", "query_offsets", "radix_ids", "token_ids", "counts_offset",
        "counts_tok", "counts_val")


def _gpu(b, mass=None, **kw):
    import torch

    from agpt_amd import loss

    dev = torch.device("cuda:0")
    t = [torch.from_numpy(np.ascontiguousarray(b[k])).to(dev) for k in ARGS]
    m = None if mass is None else torch.from_numpy(mass).to(dev)
    g, lo = loss.loss_per_query(*t, mass_weights=m, **kw)
    torch.cuda.synchronize()
    return g.cpu().numpy(), lo.cpu().numpy()


def _both(b, mass=None, **kw):
    g, lo = _gpu(b, mass, **kw)
    g0, lo0 = ORC.loss_per_query(*(b[k] for k in ARGS), mass_weights=mass, **kw)
    assert_close(g, g0, RTOL_F32, ATOL_F32, "d_logits")
    assert_close(lo, lo0, RTOL_F32, ATOL_F32, "loss")
    return g, lo


@pytest.mark.parametrize("V", [1, 3, 16, 17, 48, 65, 80, 96, 128, 129, 256, 300, 1000, 1024])
def test_loss_parity_vocab_sizes(gpu, V):
    _both(loss_batch(300, V, seed=V, max_entries=min(V, 70)))


@pytest.mark.parametrize("opts", [dict(entropy_lambda=0.5), dict(intermediate_weight=0.25),
                                  dict(ce_only=True), dict(mass=True),
                                  dict(mass=True, entropy_lambda=1.5, intermediate_weight=0.5)])
@pytest.mark.parametrize("V", [65, 256])
def test_loss_parity_options(gpu, V, opts):
    b = loss_batch(400, V, seed=7 + V)
    mass = None
    if opts.pop("mass", False):
        rng = np.random.default_rng(3)
        mass = rng.uniform(0.1, 4.0, b["logits"].shape[0]).astype(np.float32)
    _both(b, mass, **opts)


def test_loss_repeated_tokens_and_long_count_lists(gpu):
    # more count entries than lanes per row (16 / 64), tokens repeated
    _both(loss_batch(200, 65, seed=11, dup=True, max_entries=150, empty_frac=0.0))
    _both(loss_batch(100, 300, seed=12, dup=True, max_entries=200, empty_frac=0.0))


def test_loss_edge_shapes(gpu):
    # a single query (an endpoint with counts), one without counts, and the
    # sharp-logit case where p underflows to 0 (loss = -log 1e-10)
    b = loss_batch(1, 65, seed=1, max_edge=1, empty_frac=0.0)
    _both(b)
    b = loss_batch(1, 65, seed=1, max_edge=1, empty_frac=1.0)
    g, lo = _both(b)
    assert lo[0] == 0.0
    b = loss_batch(50, 65, seed=2, logit_scale=60.0)
    _both(b)


def test_loss_empty_batch_and_errors(gpu):
    import torch

    from agpt_amd import _native, loss

    dev = torch.device("cuda:0")
    z = torch.zeros(0, dtype=torch.int32, device=dev)
    o = torch.zeros(1, dtype=torch.int32, device=dev)
    g, lo = loss.loss_per_query(torch.zeros(0, 5, device=dev), z, o, z, z, o, z, z)
    assert g.shape == (0, 5) and lo.shape == (0,)
    b = loss_batch(4, 1025, seed=1)
    with pytest.raises(_native.AgptError, match="V > 1024"):
        _gpu(b)


def test_loss_large_batch_rows_match(gpu):
    """2M queries at V = 65 (C2's character vocabulary): every row against the
    oracle."""
    b = loss_batch(800_000, 65, seed=21, max_edge=4, max_entries=8)
    _both(b, intermediate_weight=0.7)


def test_loss_deterministic(gpu):
    b = loss_batch(5000, 65, seed=4)
    g1, l1 = _gpu(b, entropy_lambda=0.3)
    g2, l2 = _gpu(b, entropy_lambda=0.3)
    assert (g1 == g2).all() and (l1 == l2).all()
