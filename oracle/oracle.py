"""numpy front end of the C restatement (liboracle.so). TEST INFRASTRUCTURE:
imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
_lib = None

_f = C.POINTER(C.c_float)
_i = C.POINTER(C.c_int32)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        path = HERE / "liboracle.so"
        if not path.exists():
            from .build import build
            build()
        _lib = C.CDLL(str(path))
    return _lib


def _fp(a):
    return None if a is None else a.ctypes.data_as(_f)


def _ip(a):
    return None if a is None else a.ctypes.data_as(_i)


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def _i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


def rope_table(max_seq: int, dim: int, base: float = 10000.0):
    c = np.empty((max_seq, dim), np.float32)
    s = np.empty((max_seq, dim), np.float32)
    lib().oracle_rope_table(max_seq, dim, C.c_float(base), _fp(c), _fp(s))
    return c, s


def depths(parent: np.ndarray) -> np.ndarray:
    d = np.zeros(parent.shape[0], np.int32)
    for i, p in enumerate(parent):
        d[i] = 1 if p < 0 else d[p] + 1
    return d


def fwd(parent, Q, K, V, H, hd, scale, depth=None, per_node=False):
    """Returns (O [T,D], W [T,H,maxd], lse [T,H])."""
    parent = _i32(parent)
    depth = _i32(depths(parent) if depth is None else depth)
    T = parent.shape[0]
    maxd = int(depth.max()) if T else 1
    Q, K, V = _f32(Q), _f32(K), _f32(V)
    O = np.zeros((T, H * hd), np.float32)
    W = np.zeros((T, H, maxd), np.float32)
    lse = np.zeros((T, H), np.float32)
    if per_node:
        lib().oracle_fwd_per_node(C.c_int64(T), H, hd, _ip(parent), _ip(depth), _fp(Q), _fp(K),
                                  _fp(V), C.c_float(scale), _fp(O), _fp(W), maxd)
        lse[:] = np.nan
    else:
        lib().oracle_fwd_grouped(C.c_int64(T), H, hd, _ip(parent), _ip(depth), _fp(Q), _fp(K),
                                 _fp(V), C.c_float(scale), _fp(O), _fp(W), maxd, _fp(lse))
    return O, W, lse


def bwd(parent, Q, K, V, W, dO, H, hd, scale, acc_dk=None, acc_dv=None, rope=None,
        depth=None, matrix_form=False):
    """Whole-trie backward (deepest level first). Returns (dQ, dK, dV)."""
    parent = _i32(parent)
    depth = _i32(depths(parent) if depth is None else depth)
    T = parent.shape[0]
    Q, K, V, dO = _f32(Q), _f32(K), _f32(V), _f32(dO)
    W = _f32(W)
    acc_dk, acc_dv = _f32(acc_dk), _f32(acc_dv)
    dQ = np.zeros((T, H * hd), np.float32)
    dK = np.zeros_like(dQ)
    dV = np.zeros_like(dQ)
    cos_t = sin_t = None
    seq = 1
    if rope is not None:
        cos_t, sin_t = _f32(rope[0]), _f32(rope[1])
        seq = cos_t.shape[0]
    lib().oracle_bwd_trie(C.c_int64(T), H, hd, _ip(parent), _ip(depth), _fp(Q), _fp(K), _fp(V),
                          _fp(W), W.shape[2], _fp(dO), _fp(acc_dk), _fp(acc_dv), _fp(cos_t),
                          _fp(sin_t), seq, C.c_float(scale), 1 if matrix_form else 0, _fp(dQ),
                          _fp(dK), _fp(dV))
    return dQ, dK, dV


def varlen_fwd(q, k, v, kv_offsets, kv_lengths, n_nodes, H, hd, max_len, scale):
    out = np.zeros((n_nodes * H * hd,), np.float32)
    w = np.zeros((n_nodes * H * max_len,), np.float32)
    q, k, v = _f32(q), _f32(k), _f32(v)
    lib().oracle_varlen_fwd(n_nodes, H, hd, _fp(q), _fp(k), _fp(v), _ip(_i32(kv_offsets)),
                            _ip(_i32(kv_lengths)), _fp(out), _fp(w), max_len, C.c_float(scale))
    return out, w


def varlen_bwd(q, k, v, w, d_out, kv_offsets, kv_lengths, n_nodes, H, hd, max_len, scale,
               total_kv):
    dq = np.zeros((n_nodes * H * hd,), np.float32)
    dk = np.zeros((total_kv * H * hd,), np.float32)
    dv = np.zeros_like(dk)
    args = [_f32(x) for x in (q, k, v, w, d_out)]
    lib().oracle_varlen_bwd(n_nodes, H, hd, *[_fp(a) for a in args], _ip(_i32(kv_offsets)),
                            _ip(_i32(kv_lengths)), _fp(dq), _fp(dk), _fp(dv), max_len,
                            C.c_float(scale))
    return dq, dk, dv


def varlen_L_fwd(q, k, v, q2n, qoff, kv_offsets, kv_lengths, T_q, H, hd, max_len, scale):
    out = np.zeros((T_q * H * hd,), np.float32)
    w = np.zeros((T_q * H * max_len,), np.float32)
    q, k, v = _f32(q), _f32(k), _f32(v)
    lib().oracle_varlen_L_fwd(T_q, H, hd, _fp(q), _fp(k), _fp(v), _ip(_i32(q2n)), _ip(_i32(qoff)),
                              _ip(_i32(kv_offsets)), _ip(_i32(kv_lengths)), _fp(out), _fp(w),
                              max_len, C.c_float(scale))
    return out, w


def varlen_L_bwd(q, k, v, w, d_out, q2n, qoff, kv_offsets, kv_lengths, T_q, H, hd, max_len,
                 scale, total_kv, dk=None, dv=None):
    dq = np.zeros((T_q * H * hd,), np.float32)
    dk = np.zeros((total_kv * H * hd,), np.float32) if dk is None else _f32(dk).copy()
    dv = np.zeros((total_kv * H * hd,), np.float32) if dv is None else _f32(dv).copy()
    args = [_f32(x) for x in (q, k, v, w, d_out)]
    lib().oracle_varlen_L_bwd(T_q, H, hd, *[_fp(a) for a in args], _ip(_i32(q2n)), _ip(_i32(qoff)),
                              _ip(_i32(kv_offsets)), _ip(_i32(kv_lengths)), _fp(dq), _fp(dk),
                              _fp(dv), max_len, C.c_float(scale))
    return dq, dk, dv


def loss_per_query(logits, query_to_node, query_offsets, radix_ids, token_ids, counts_offset,
                   counts_tok, counts_val, mass_weights=None, entropy_lambda=0.0,
                   intermediate_weight=1.0, ce_only=False):
    """agpt_train.cu:2069-2194 restated (loss_oracle.c); returns (d_logits, loss)."""
    lg = _f32(logits)
    T_q, V = lg.shape
    g = np.empty_like(lg)
    lo = np.empty(T_q, np.float32)
    ints = [_i32(x) for x in (query_to_node, query_offsets, radix_ids, token_ids, counts_offset,
                              counts_tok, counts_val)]
    lib().oracle_loss_per_query(_fp(lg), *(_ip(x) for x in ints), _fp(_f32(mass_weights)), _fp(g),
                                _fp(lo), T_q, V, C.c_float(entropy_lambda),
                                C.c_float(intermediate_weight), int(bool(ce_only)))
    return g, lo


def loss_mass_weights(radix_ids, edge_mass, edge_lens, query_offsets, T_q, mode):
    """agpt_train.cu:4608-4637 restated (loss_oracle.c)."""
    a = [_i32(x) for x in (radix_ids, edge_mass, edge_lens, query_offsets)]
    out = np.empty(T_q, np.float32)
    lib().oracle_loss_mass_weights(*(_ip(x) for x in a), len(a[0]), T_q, mode, _fp(out))
    return out


def bias_rope(x, bias, positions, cos_t, sin_t, n_heads, head_dim):
    """cuda_bias_add + rope_batched_kernel restated (block_oracle.c); returns a copy."""
    y = np.array(x, dtype=np.float32, copy=True, order="C")
    T = y.shape[0]
    seq = 0 if cos_t is None else cos_t.shape[0]
    lib().oracle_bias_rope(_fp(y), _fp(_f32(bias)), None if positions is None else _ip(_i32(positions)),
                           _fp(_f32(cos_t)), _fp(_f32(sin_t)), seq, C.c_int64(T), n_heads, head_dim)
    return y


def rmsprop(params, grads, sq_avg, lr, beta, eps):
    """Textbook RMSProp restated (block_oracle.c); returns (params, sq_avg) copies."""
    p = np.array(params, dtype=np.float32, copy=True)
    s = np.array(sq_avg, dtype=np.float32, copy=True)
    g = _f32(grads)
    lib().oracle_rmsprop(_fp(p), _fp(g), _fp(s), C.c_float(lr), C.c_float(beta), C.c_float(eps),
                         C.c_int64(p.size))
    return p, s


def norm_fwd(x, w, b, eps):
    """LayerNorm (b given) / RMSNorm restated (block_oracle.c); returns (y, mean, rstd)."""
    x = _f32(x)
    T, D = x.shape
    y = np.empty_like(x)
    rs = np.empty(T, np.float32)
    mu = np.empty(T, np.float32) if b is not None else None
    lib().oracle_norm_fwd(_fp(x), _fp(_f32(w)), _fp(_f32(b)), _fp(y), _fp(mu), _fp(rs), C.c_int64(T), D,
                          C.c_float(eps))
    return y, mu, rs


def norm_bwd(dy, x, w, mean, rstd, layer):
    x = _f32(x)
    T, D = x.shape
    dx = np.empty_like(x)
    dw = np.empty(D, np.float32)
    db = np.empty(D, np.float32) if layer else None
    lib().oracle_norm_bwd(_fp(_f32(dy)), _fp(x), _fp(_f32(w)), _fp(_f32(mean)), _fp(_f32(rstd)), _fp(dx),
                          _fp(dw), _fp(db), C.c_int64(T), D)
    return dx, dw, db
