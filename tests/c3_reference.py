"""Float64 CPU reference of the C3 training step (agpt_amd.model), written
independently of the kernels: attention as a dense softmax over each row's
ancestor-or-self mask, RoPE by rotation matrices from the oracle's table,
the per-query loss from its definition (log-sum-exp), torch autograd for the
gradients. Test infrastructure."""
from __future__ import annotations

import math

import numpy as np
import torch

from agpt_amd.model import param_shapes
from oracle import oracle as ORC


def ancestor_mask(parent: np.ndarray) -> torch.Tensor:
    T = parent.shape[0]
    m = np.zeros((T, T), bool)
    for i in range(T):
        j = i
        while j >= 0:
            m[i, j] = True
            j = parent[j]
    return torch.from_numpy(m)


def _rope(x, pos, cos_t, sin_t, H, hd):
    c = cos_t[pos].reshape(-1, 1, hd)  # [T, 1, hd]
    s = sin_t[pos].reshape(-1, 1, hd)
    x = x.reshape(x.shape[0], H, hd)
    x0, x1 = x[..., 0::2], x[..., 1::2]
    y0 = x0 * c[..., 0::2] - x1 * s[..., 0::2]
    y1 = x0 * s[..., 0::2] + x1 * c[..., 0::2]
    return torch.stack([y0, y1], dim=-1).reshape(x.shape[0], H * hd)


def step_f64(cfg, flat: np.ndarray, tr, mass: np.ndarray | None, dt=torch.float64, relu_masks=None):
    """Returns (loss, grad of the flat buffer) in float64 (dt=torch.float32
    gives the same model in float32 on the CPU: how far plain float32
    arithmetic lands from float64 on a given model and trie).

    relu_masks (per layer, bool [T, d_ff]) replaces the ReLU's own decision
    (input > 0) by the given one: the gradient of the model that took the
    same side of every kink. step_f64.relu_flips then holds, per layer, the
    relative size |input| / mean |input| of the inputs where the given mask
    differs from the float64 decision."""
    fl = torch.tensor(flat, dtype=dt, requires_grad=True)
    P, off = {}, 0
    for name, shape in param_shapes(cfg):
        n = int(np.prod(shape))
        P[name] = fl[off:off + n].view(shape)
        off += n
    H, D = cfg.n_heads, cfg.d_model
    hd = D // H
    cos_t, sin_t = (torch.tensor(t, dtype=dt) for t in ORC.rope_table(cfg.max_depth, hd))
    pos = torch.from_numpy(np.minimum(tr.depth - 1, cfg.max_depth - 1).astype(np.int64))
    mask = ancestor_mask(tr.parent)
    scale = 1.0 / math.sqrt(hd)

    def norm(x, w, b):
        if cfg.norm == "rms":
            return x / torch.sqrt((x * x).mean(-1, keepdim=True) + cfg.eps) * w
        mu = x.mean(-1, keepdim=True)
        var = ((x - mu) ** 2).mean(-1, keepdim=True)
        return (x - mu) / torch.sqrt(var + cfg.eps) * w + b

    x = P["tok_emb"][torch.from_numpy(tr.token.astype(np.int64))]
    T = x.shape[0]
    margins, flips = [], []
    for l in range(cfg.n_layers):
        n1 = norm(x, P[f"n1_w{l}"], P[f"n1_b{l}"])
        q = _rope(n1 @ P[f"wq{l}"].T + P[f"bq{l}"], pos, cos_t, sin_t, H, hd).reshape(T, H, hd)
        k = _rope(n1 @ P[f"wk{l}"].T + P[f"bk{l}"], pos, cos_t, sin_t, H, hd).reshape(T, H, hd)
        v = (n1 @ P[f"wv{l}"].T + P[f"bv{l}"]).reshape(T, H, hd)
        s = torch.einsum("ihd,jhd->hij", q, k) * scale
        s = s.masked_fill(~mask[None], float("-inf"))
        o = torch.einsum("hij,jhd->ihd", torch.softmax(s, -1), v).reshape(T, D)
        x = x + o @ P[f"wo{l}"].T + P[f"bo{l}"]
        n2 = norm(x, P[f"n2_w{l}"], P[f"n2_b{l}"])
        pre = n2 @ P[f"w1{l}"].T + P[f"b1{l}"]
        a = pre.detach().abs()
        margins.append(float(a.min() / a.mean()))
        if relu_masks is not None:
            mk = torch.as_tensor(relu_masks[l])
            flip = mk != (pre.detach() > 0)
            flips.append((a[flip] / a.mean()).numpy())
            act = torch.where(mk, pre, torch.zeros((), dtype=dt))
        else:
            act = torch.relu(pre)
        x = x + act @ P[f"w2{l}"].T + P[f"b2{l}"]
    logits = norm(x, P["nf_w"], P["nf_b"]) @ P["w_out"].T + P["b_out"]
    logp = torch.log_softmax(logits, -1)
    p = logp.exp()
    # target distributions (agpt_train.cu:2121-2193 without entropy weighting)
    heads = np.flatnonzero(tr.radix_head)
    ends = np.append(heads[1:], T) - 1
    tgt = torch.zeros(T, cfg.vocab, dtype=dt)
    is_end = np.zeros(T, bool)
    is_end[ends] = True
    for q_ in range(T):
        if is_end[q_]:
            a, b = tr.next_offsets[q_], tr.next_offsets[q_ + 1]
            c = tr.next_val[a:b].astype(np.float64)
            if c.size:
                tgt[q_, torch.from_numpy(tr.next_tok[a:b].astype(np.int64))] += torch.from_numpy(c / c.sum())
        else:
            tgt[q_, int(tr.token[q_ + 1])] = 1.0
    w = torch.ones(T, dtype=dt) if mass is None else torch.tensor(mass, dtype=dt)
    loss = -(w[:, None] * tgt * torch.log(p + 1e-10)).sum()
    loss.backward()
    # ReLU inputs nearest zero, relative to their mean size: an input within
    # rounding of the kink may fall on the other side in float32, which
    # changes the gradient by a whole unit's term (not by rounding).
    step_f64.relu_margin = min(margins) if margins else float("inf")
    step_f64.relu_flips = flips
    return float(loss.detach()), fl.grad.numpy()
