"""The closed-form inputs of spec/agpt_backward_attention_spec.cr, restated.

make_deterministic_model (spec:12-51): d_model 8, 2 heads x 4, seq_len 8,
vocab 8, every matrix filled with (((offset + r*cols + c) % 37) + 1) * scale
(fill_mat!, spec:3-10). The attention inputs of a node are
LN1(token_emb[token]) @ W + b (incremental_forward.cr:30-41; LN as
ln_row_with_state, incremental_forward.cr:143-163), split into heads and
rotated by RoPE at position depth-1 (incremental_forward.cr:44-48).
Upstream gradients and accumulator seeds follow spec:278-296, 311-314,
439-444.
"""
from __future__ import annotations

import numpy as np

D_MODEL, N_HEADS, HEAD_DIM, SEQ_LEN, VOCAB = 8, 2, 4, 8, 8


def fill_mat(rows: int, cols: int, scale: float, offset: int) -> np.ndarray:
    r = np.arange(rows)[:, None]
    c = np.arange(cols)[None, :]
    return ((((offset + r * cols + c) % 37) + 1).astype(np.float32) * np.float32(scale))


def model():
    m = {
        "token_emb": fill_mat(VOCAB, D_MODEL, 0.01, 1),
        "ln1_gamma": fill_mat(1, D_MODEL, 0.02, 2),
        "ln1_beta": fill_mat(1, D_MODEL, 0.01, 3),
        "wq": fill_mat(D_MODEL, D_MODEL, 0.01, 6), "bq": fill_mat(1, D_MODEL, 0.01, 7),
        "wk": fill_mat(D_MODEL, D_MODEL, 0.01, 8), "bk": fill_mat(1, D_MODEL, 0.01, 9),
        "wv": fill_mat(D_MODEL, D_MODEL, 0.01, 10), "bv": fill_mat(1, D_MODEL, 0.01, 11),
        "wo": fill_mat(D_MODEL, D_MODEL, 0.01, 12),
    }
    return m


def layer_norm_row(x: np.ndarray, gamma: np.ndarray, beta: np.ndarray) -> np.ndarray:
    """ln_row_with_state (incremental_forward.cr:143-163): float32 mean and
    variance, std_inv = 1/sqrt(var + 1e-5) rounded to float32."""
    d = x.shape[0]
    mean = np.float32(0.0)
    for j in range(d):
        mean = np.float32(mean + x[j])
    mean = np.float32(mean / np.float32(d))
    var = np.float32(0.0)
    for j in range(d):
        diff = np.float32(x[j] - mean)
        var = np.float32(var + diff * diff)
    var = np.float32(var / np.float32(d))
    std_inv = np.float32(1.0 / np.sqrt(np.float64(var + np.float32(1e-5))))
    out = np.empty(d, np.float32)
    for j in range(d):
        normed = np.float32((x[j] - mean) * std_inv)
        out[j] = np.float32(normed * gamma[0, j] + beta[0, j])
    return out


def matmul_row(x: np.ndarray, w: np.ndarray, b: np.ndarray) -> np.ndarray:
    out = np.empty(w.shape[1], np.float32)
    for j in range(w.shape[1]):
        acc = np.float32(0.0)
        for i in range(w.shape[0]):
            acc = np.float32(acc + x[i] * w[i, j])
        out[j] = np.float32(acc + b[0, j])
    return out


def qkv(tokens: np.ndarray, depth: np.ndarray, cos_t: np.ndarray, sin_t: np.ndarray):
    """Post-RoPE Q, K and V rows [T, 8] of nodes with the given tokens/depths."""
    m = model()
    T = tokens.shape[0]
    Q = np.zeros((T, D_MODEL), np.float32)
    K = np.zeros_like(Q)
    V = np.zeros_like(Q)
    for n in range(T):
        x = layer_norm_row(m["token_emb"][tokens[n]], m["ln1_gamma"], m["ln1_beta"])
        q = matmul_row(x, m["wq"], m["bq"])
        k = matmul_row(x, m["wk"], m["bk"])
        v = matmul_row(x, m["wv"], m["bv"])
        pos = int(depth[n]) - 1
        for h in range(N_HEADS):
            sl = slice(h * HEAD_DIM, (h + 1) * HEAD_DIM)
            q[sl] = rope_row(q[sl], cos_t, sin_t, pos)
            k[sl] = rope_row(k[sl], cos_t, sin_t, pos)
        Q[n], K[n], V[n] = q, k, v
    return Q, K, V


def rope_row(x, cos_t, sin_t, pos):
    """apply_rope_at! (incremental_forward.cr:195-206)."""
    y = x.copy()
    for i in range(x.shape[0] // 2):
        c, s = cos_t[pos, 2 * i], sin_t[pos, 2 * i]
        x0, x1 = x[2 * i], x[2 * i + 1]
        y[2 * i] = np.float32(x0 * c - x1 * s)
        y[2 * i + 1] = np.float32(x0 * s + x1 * c)
    return y


def d_head_out(values: np.ndarray) -> np.ndarray:
    """d_concat = d_attn_proj * wo.w^T (spec:311-315, 439-447), one row."""
    wo = model()["wo"]
    out = np.empty(D_MODEL, np.float32)
    for i in range(D_MODEL):
        acc = np.float32(0.0)
        for j in range(D_MODEL):
            acc = np.float32(acc + values[j] * wo[i, j])
        out[i] = acc
    return out


def chain_d_attn_proj(prefix_len: int) -> np.ndarray:
    """spec:311-314: 0.01 * (prefix_len + j + 1)."""
    return (np.float32(0.01) * (prefix_len + np.arange(D_MODEL) + 1).astype(np.float32)).astype(np.float32)


def branch_d_attn_proj(i: int) -> np.ndarray:
    """spec:439-444: 0.005 * (i * d_model + j + 1)."""
    return (np.float32(0.005) * (i * D_MODEL + np.arange(D_MODEL) + 1).astype(np.float32)).astype(np.float32)


def current_accum(prefix_len: int):
    """seed_current_accum (spec:278-287): dk 0.001*(p+hi+j+1), dv 0.002*(...)."""
    dk = np.zeros(D_MODEL, np.float32)
    dv = np.zeros(D_MODEL, np.float32)
    for hi in range(N_HEADS):
        for j in range(HEAD_DIM):
            dk[hi * HEAD_DIM + j] = np.float32(0.001) * np.float32(prefix_len + hi + j + 1)
            dv[hi * HEAD_DIM + j] = np.float32(0.002) * np.float32(prefix_len + hi + j + 1)
    return dk, dv
