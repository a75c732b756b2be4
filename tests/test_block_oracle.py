"""Pins the C restatement of the projection epilogue (bias + RoPE,
agpt_train.cu:4676-4687 and :1305-1326) and of the RMSProp update
(oracle/block_oracle.c) before it checks the GPU kernels. CPU only."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import oracle as ORC


def test_bias_rope_known_angle_and_norm():
    H, hd, seq = 2, 8, 10
    cos_t, sin_t = ORC.rope_table(seq, hd)
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, H * hd)).astype(np.float32)
    pos = np.array([0, 1, 3, 9, 40], np.int32)  # 40 clamps to 9
    y = ORC.bias_rope(x, None, pos, cos_t, sin_t, H, hd)
    np.testing.assert_array_equal(y[0], x[0])  # position 0: identity
    for t, p in enumerate(np.minimum(pos, seq - 1)):
        for h in range(H):
            for i in range(hd // 2):
                th = p / 10000.0 ** (2 * i / hd)
                a, b = x[t, h * hd + 2 * i], x[t, h * hd + 2 * i + 1]
                np.testing.assert_allclose(y[t, h * hd + 2 * i], a * math.cos(th) - b * math.sin(th), atol=2e-6)
                np.testing.assert_allclose(y[t, h * hd + 2 * i + 1], a * math.sin(th) + b * math.cos(th), atol=2e-6)
    np.testing.assert_allclose(np.linalg.norm(y.reshape(5, H, hd // 2, 2), axis=-1),
                               np.linalg.norm(x.reshape(5, H, hd // 2, 2), axis=-1), rtol=1e-6)


def test_bias_rope_bias_then_rotation_and_inverse():
    H, hd, seq = 3, 16, 32
    cos_t, sin_t = ORC.rope_table(seq, hd)
    rng = np.random.default_rng(1)
    x = rng.standard_normal((7, H * hd)).astype(np.float32)
    bias = rng.standard_normal(H * hd).astype(np.float32)
    pos = rng.integers(0, seq, 7).astype(np.int32)
    y = ORC.bias_rope(x, bias, pos, cos_t, sin_t, H, hd)
    np.testing.assert_allclose(ORC.bias_rope(x + bias, None, pos, cos_t, sin_t, H, hd), y, atol=1e-6)
    back = y.copy()
    for t in range(7):  # the trie oracle's inverse rotation (batched_depth_backward.cr:738-748)
        for h in range(H):
            seg = np.ascontiguousarray(back[t, h * hd:(h + 1) * hd])
            ORC.lib().oracle_rope_inverse(ORC._fp(seg), hd, ORC._fp(cos_t), ORC._fp(sin_t), int(pos[t]))
            back[t, h * hd:(h + 1) * hd] = seg
    np.testing.assert_allclose(back, x + bias, atol=2e-6)
    np.testing.assert_array_equal(ORC.bias_rope(x, bias, None, None, None, H, hd), x + bias)


@pytest.mark.parametrize("beta,lr,eps", [(0.999, 1e-3, 1e-8), (0.9, 0.05, 1e-6)])
def test_rmsprop_matches_torch(beta, lr, eps):
    rng = np.random.default_rng(2)
    p = rng.standard_normal(1001).astype(np.float32)
    s = np.zeros(1001, np.float32)
    pt = torch.tensor(p.copy(), requires_grad=True)
    # The update takes beta as a float32 (the kernel argument) and forms
    # 1 - beta from it; torch is given the same float32 value.
    opt = torch.optim.RMSprop([pt], lr=lr, alpha=float(np.float32(beta)), eps=eps, momentum=0.0,
                              centered=False)
    for step in range(3):
        g = rng.standard_normal(1001).astype(np.float32)
        p, s = ORC.rmsprop(p, g, s, lr, beta, eps)
        pt.grad = torch.tensor(g)
        opt.step()
        np.testing.assert_allclose(p, pt.detach().numpy(), rtol=2e-6, atol=1e-6)  # a few ulp (fused forms)
        np.testing.assert_allclose(s, opt.state[pt]["square_avg"].numpy(), rtol=2e-6)


@pytest.mark.parametrize("layer", [True, False])
def test_norm_oracle_matches_torch_float64(layer):
    """The row norms' restatement against torch's layer_norm / rms_norm and
    autograd in float64 (library routines)."""
    rng = np.random.default_rng(3)
    T, D, eps = 37, 64, 1e-5
    x = (rng.standard_normal((T, D)) * 2 + 0.5).astype(np.float32)
    w = rng.standard_normal(D).astype(np.float32)
    b = rng.standard_normal(D).astype(np.float32) if layer else None
    dy = rng.standard_normal((T, D)).astype(np.float32)
    y, mu, rs = ORC.norm_fwd(x, w, b, eps)
    dx, dw, db = ORC.norm_bwd(dy, x, w, mu, rs, layer)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    wt = torch.tensor(w, dtype=torch.float64, requires_grad=True)
    if layer:
        bt = torch.tensor(b, dtype=torch.float64, requires_grad=True)
        yt = torch.nn.functional.layer_norm(xt, (D,), wt, bt, eps)
    else:
        yt = torch.nn.functional.rms_norm(xt, (D,), wt, eps)
    yt.backward(torch.tensor(dy, dtype=torch.float64))
    np.testing.assert_allclose(y, yt.detach().numpy(), rtol=2e-6, atol=2e-6)
    np.testing.assert_allclose(dx, xt.grad.numpy(), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(dw, wt.grad.numpy(), rtol=1e-5, atol=1e-5)
    if layer:
        np.testing.assert_allclose(db, bt.grad.numpy(), rtol=1e-6, atol=1e-6)
