"""GPU: the projection epilogue and RMSProp against the oracle, and one C3
training step (agpt_amd.model: trie attention, epilogue, loss and RMSProp
native; GEMMs and norms torch) against the float64 CPU reference model.

Bars: epilogue and RMSProp within a few ulp of the oracle (fp32, fused
multiply-adds on the GPU); the C3 step's loss within 1e-4 relative and every
parameter's gradient within 2e-4 of its largest |value| (fp32 through two
layers against float64)."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import small_trie
from oracle import oracle as ORC

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("H,hd,rope,bias", [(4, 16, True, True), (2, 64, True, False), (8, 16, False, True),
                                            (3, 32, True, True)])
def test_bias_rope_matches_oracle(gpu, H, hd, rope, bias):
    import torch

    from agpt_amd import block

    rng = np.random.default_rng(H * hd)
    T, seq = 1037, 24
    x = rng.standard_normal((T, H * hd)).astype(np.float32)
    b = rng.standard_normal(H * hd).astype(np.float32) if bias else None
    pos = rng.integers(-2, seq + 5, T).astype(np.int32)  # clamped to [0, seq-1]
    cos_t, sin_t = ORC.rope_table(seq, hd)
    want = ORC.bias_rope(x, b, np.clip(pos, 0, seq - 1), cos_t if rope else None, sin_t if rope else None, H, hd)
    xt = torch.from_numpy(x).to(gpu)
    c, s = (torch.from_numpy(t).to(gpu) for t in (cos_t, sin_t))  # the same tables on both sides
    block.bias_rope_(xt, None if b is None else torch.from_numpy(b).to(gpu),
                     torch.from_numpy(pos).to(gpu), c if rope else None, s if rope else None, H)
    np.testing.assert_allclose(xt.cpu().numpy(), want, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("H,hd,bias", [(8, 16, True), (2, 64, False)])
def test_bias_rope_split_matches_oracle(gpu, H, hd, bias):
    import torch

    from agpt_amd import block

    rng = np.random.default_rng(7 * H + hd)
    T, seq, D = 2049, 32, H * hd
    x = rng.standard_normal((T, 3 * D)).astype(np.float32)
    b = rng.standard_normal(3 * D).astype(np.float32) if bias else None
    pos = rng.integers(0, seq + 3, T).astype(np.int32)
    cos_t, sin_t = ORC.rope_table(seq, hd)
    p = np.clip(pos, 0, seq - 1)
    want = [ORC.bias_rope(np.ascontiguousarray(x[:, i * D:(i + 1) * D]), None if b is None else b[i * D:(i + 1) * D],
                          p, cos_t if i < 2 else None, sin_t if i < 2 else None, H, hd) for i in range(3)]
    c, s = (torch.from_numpy(t).to(gpu) for t in (cos_t, sin_t))
    got = block.bias_rope_split(torch.from_numpy(x).to(gpu), None if b is None else torch.from_numpy(b).to(gpu),
                                torch.from_numpy(pos).to(gpu), c, s, H)
    for g_, w_ in zip(got, want):
        np.testing.assert_allclose(g_.cpu().numpy(), w_, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("n", [1, 4, 1001, 1 << 20])
def test_rmsprop_matches_oracle(gpu, n):
    import torch

    from agpt_amd import block

    rng = np.random.default_rng(n)
    p = rng.standard_normal(n).astype(np.float32)
    s = np.zeros(n, np.float32)
    pt, st = torch.from_numpy(p).to(gpu), torch.from_numpy(s).to(gpu)
    for _ in range(3):
        g = rng.standard_normal(n).astype(np.float32)
        p, s = ORC.rmsprop(p, g, s, 1e-3, 0.999, 1e-8)
        block.rmsprop_(pt, torch.from_numpy(g).to(gpu), st, 1e-3, 0.999, 1e-8)
    np.testing.assert_allclose(pt.cpu().numpy(), p, rtol=2e-6, atol=1e-6)
    np.testing.assert_allclose(st.cpu().numpy(), s, rtol=2e-6)


@pytest.mark.parametrize("norm,max_rows", [("rms", 1 << 20), ("layer", 1 << 20), ("rms", 400)])
def test_c3_step_matches_float64(gpu, norm, max_rows):
    import torch

    from agpt_amd import model, trie
    from c3_reference import step_f64

    tok = trie.markov_corpus(260, 2, 7, 1.1, seed=5)
    tr = trie.build_trie(tok, 10, counts=True)
    cfg = model.ModelConfig(vocab=7, d_model=64, n_heads=4, n_layers=2, d_ff=128, max_depth=10, norm=norm)
    m = model.TrieGPT(cfg, device=gpu, seed=3)
    m.plan(tr, max_rows=max_rows)  # 400: several batches, gradients accumulated over them
    assert len(m.groups) == (1 if max_rows > tr.n_nodes else len(model.subtree_groups(tr, max_rows)))
    flat0 = m.flat.detach().cpu().numpy().copy()
    loss = float(m.step())
    torch.cuda.synchronize()
    grad = m.flat.grad.detach().cpu().numpy()
    mass = np.concatenate([b.mass.cpu().numpy() for _, b in m.groups])
    want_loss, want_grad = step_f64(cfg, flat0, tr, mass)
    assert abs(loss - want_loss) <= 1e-4 * abs(want_loss), (loss, want_loss)
    off = 0
    for name, shape in model.param_shapes(cfg):
        k = int(np.prod(shape))
        g, w = grad[off:off + k], want_grad[off:off + k]
        bound = 2e-4 * max(np.abs(w).max(), 1e-6)
        assert np.abs(g - w).max() <= bound, (name, np.abs(g - w).max(), np.abs(w).max())
        off += k
    # the update is RMSProp on the step's own gradient
    p1, _ = ORC.rmsprop(flat0, grad, np.zeros_like(flat0), m.lr, m.beta, m.eps)
    np.testing.assert_allclose(m.flat.detach().cpu().numpy(), p1, rtol=2e-6, atol=1e-6)
    m.close()


@pytest.mark.parametrize("max_rows", [1 << 20, 700])
def test_c3_config_step(gpu, max_rows):
    """C3's own model (4 layers, d_model 128, 8 heads x
    16, FFN 512, RMSNorm, vocab 65) on a C1-corpus radix trie of ~2K rows
    (depth 32), linear mass weights, one step against the float64 CPU
    model: loss within 1e-4 relative, every parameter's gradient within
    2e-4 of its largest |value|, the update RMSProp on that gradient."""
    import torch

    from agpt_amd import model, trie
    from c3_reference import step_f64

    tr = trie.config_trie("C1", scale=0.0005, counts=True)
    assert 1500 < tr.n_nodes < 4000 and tr.max_depth == 32
    cfg = model.ModelConfig()
    assert (cfg.n_layers, cfg.d_model, cfg.n_heads, cfg.d_ff, cfg.vocab, cfg.norm) == (4, 128, 8, 512, 65, "rms")
    m = model.TrieGPT(cfg, device=gpu, seed=7)
    m.plan(tr, max_rows=max_rows)
    # The GPU's ReLU decisions, per layer over the batches in row order: with
    # 4.4M ReLU inputs some lie within float32 rounding of zero (the
    # smallest here is ~1e-7 of the mean), where float32 and float64 may take
    # different sides of the kink; the reference takes the GPU's side.
    masks = {l: [] for l in range(cfg.n_layers)}
    m.relu_hook = lambda l, h: masks[l].append((h > 0).cpu())
    flat0 = m.flat.detach().cpu().numpy().copy()
    loss = float(m.step())
    torch.cuda.synchronize()
    grad = m.flat.grad.detach().cpu().numpy()
    mass = np.concatenate([b.mass.cpu().numpy() for _, b in m.groups])
    want_loss, want_grad = step_f64(cfg, flat0, tr, mass,
                                    relu_masks=[torch.cat(masks[l]) for l in range(cfg.n_layers)])
    # a differing decision is only ever a kink within rounding
    for l, fl in enumerate(step_f64.relu_flips):
        assert fl.size == 0 or float(fl.max()) < 1e-5, (l, fl)
    assert abs(loss - want_loss) <= 1e-4 * abs(want_loss), (loss, want_loss)
    off = 0
    for name, shape in model.param_shapes(cfg):
        k = int(np.prod(shape))
        g, w = grad[off:off + k], want_grad[off:off + k]
        bound = 2e-4 * max(np.abs(w).max(), 1e-6)
        assert np.abs(g - w).max() <= bound, (name, np.abs(g - w).max(), np.abs(w).max())
        off += k
    p1, _ = ORC.rmsprop(flat0, grad, np.zeros_like(flat0), m.lr, m.beta, m.eps)
    np.testing.assert_allclose(m.flat.detach().cpu().numpy(), p1, rtol=2e-6, atol=1e-6)
    m.close()


def test_c3_checkpoint_round_trip_through_the_model(gpu, tmp_path):
    from agpt_amd import model

    cfg = model.ModelConfig(vocab=7, d_model=64, n_heads=4, n_layers=2, d_ff=128, max_depth=10, norm="layer")
    a = model.TrieGPT(cfg, device=gpu, seed=1)
    b = model.TrieGPT(cfg, device=gpu, seed=2)
    a.save(str(tmp_path / "a.mgpt"))
    b.load(str(tmp_path / "a.mgpt"))
    assert (a.flat.detach() == b.flat.detach()).all()


def test_c3_step_from_radix_files(gpu, tmp_path):
    """Planning from the reference's radix files gives the same step as
    planning from the trie (loss and gradient bit for bit: same tables)."""
    from agpt_amd import model, trie

    tok = trie.markov_corpus(3000, 2, 7, 1.1, seed=3)
    trie.write_radix_files(tok, 10, str(tmp_path), 7)
    tr = trie.build_radix_trie(tok, 10, counts=True)
    cfg = model.ModelConfig(vocab=7, d_model=64, n_heads=4, n_layers=2, d_ff=128, max_depth=10)
    a, b = model.TrieGPT(cfg, device=gpu, seed=3), model.TrieGPT(cfg, device=gpu, seed=3)
    a.plan(tr, max_rows=2000)
    b.plan_radix_dir(str(tmp_path), max_rows=2000)
    assert [g[1].T for g in a.groups] == [g[1].T for g in b.groups]
    la, lb = float(a.step()), float(b.step())
    assert la == lb
    assert (a.flat.grad == b.flat.grad).all()
    a.close()
    b.close()


@pytest.mark.parametrize("D", [64, 128, 256, 512])
@pytest.mark.parametrize("layer", [True, False])
def test_norm_matches_oracle(gpu, D, layer):
    import torch

    from agpt_amd import block

    rng = np.random.default_rng(D + layer)
    T = 5003
    x = (rng.standard_normal((T, D)) * 1.5 + 0.3).astype(np.float32)
    w = rng.standard_normal(D).astype(np.float32)
    b = rng.standard_normal(D).astype(np.float32) if layer else None
    dy = rng.standard_normal((T, D)).astype(np.float32)
    y0, mu0, rs0 = ORC.norm_fwd(x, w, b, 1e-5)
    to = lambda a: None if a is None else torch.from_numpy(a).to(gpu)
    y, mu, rs = block.norm_fwd(to(x), to(w), to(b), 1e-5)
    np.testing.assert_allclose(y.cpu().numpy(), y0, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(rs.cpu().numpy(), rs0, rtol=1e-6)
    dx0, dw0, db0 = ORC.norm_bwd(dy, x, w, mu0, rs0, layer)
    dx, dw, db = block.norm_bwd(to(dy), to(x), to(w), mu, rs, layer)
    np.testing.assert_allclose(dx.cpu().numpy(), dx0, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(dw.cpu().numpy(), dw0, rtol=1e-4, atol=1e-3)  # sums of 5003 rows
    if layer:
        np.testing.assert_allclose(db.cpu().numpy(), db0, rtol=1e-4, atol=1e-3)
    dx2, dw2, _ = block.norm_bwd(to(dy), to(x), to(w), mu, rs, layer)
    assert torch.equal(dx, dx2) and torch.equal(dw, dw2)  # fixed-order sums
    # dres (a residual stream's gradient at x) is added into dx only
    r = rng.standard_normal((T, D)).astype(np.float32)
    dxr, dwr, dbr = block.norm_bwd(to(dy), to(x), to(w), mu, rs, layer, dres=to(r))
    np.testing.assert_allclose(dxr.cpu().numpy(), dx0 + r, rtol=1e-4, atol=1e-5)
    assert torch.equal(dwr, dw) and (not layer or torch.equal(dbr, db))


@pytest.mark.parametrize("W", [128, 512])
def test_relu_bwd(gpu, W):
    """agpt_relu_bwd against torch fp32: dh exact, db = the column sum of dh
    (fixed order: two calls give identical bytes); in place allowed."""
    import ctypes

    import torch

    from agpt_amd import _native, block

    g = torch.Generator().manual_seed(W)
    T = 7001
    dy = torch.randn(T, W, generator=g).to(gpu)
    h = torch.relu(torch.randn(T, W, generator=g)).to(gpu)
    h[3, :] = 0.0  # a row with no live units
    dh, db = block.relu_bwd(dy, h)
    ref = torch.where(h > 0, dy, torch.zeros((), device=gpu))
    assert torch.equal(dh, ref)
    torch.testing.assert_close(db.double().cpu(), ref.double().sum(0).cpu(), rtol=1e-5, atol=1e-3)
    dh2, db2 = block.relu_bwd(dy, h)
    assert torch.equal(dh, dh2) and torch.equal(db, db2)
    lib = _native.attn_lib()
    ws = torch.empty(lib.agpt_norm_workspace_floats(W), device=gpu)
    d3 = torch.empty(W, device=gpu)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    y = dy.clone()
    assert lib.agpt_relu_bwd(p(y), p(h), p(y), p(d3), p(ws), ws.numel(), T, W, None) == 0
    torch.cuda.synchronize()
    assert torch.equal(y, ref) and torch.equal(d3, db)
