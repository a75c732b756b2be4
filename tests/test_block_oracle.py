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
