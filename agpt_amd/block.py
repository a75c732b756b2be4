"""Kernels around the trie-attention path in a training step
(include/agpt_block.h): the projection epilogue (bias + RoPE, in place), the
row norms and the RMSProp update. Torch CUDA tensors, current stream; no CPU
fallback."""
from __future__ import annotations

import ctypes as C

from . import _native


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream(t) -> C.c_void_p:
    import torch
    return C.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def bias_rope_(x, bias=None, positions=None, cos_t=None, sin_t=None, n_heads: int = 1):
    """In place on x [T, D] fp32: x += bias, then (cos_t given) RoPE of each
    head at row position positions[t] (int32 [T]). Returns x."""
    if not x.is_cuda or not x.is_contiguous() or x.dim() != 2:
        raise ValueError("x must be a contiguous CUDA [T, D] tensor")
    T, D = x.shape
    if D % n_heads:
        raise ValueError("D must be a multiple of n_heads")
    seq = 0 if cos_t is None else cos_t.shape[0]
    _native.check(_native.attn_lib().agpt_bias_rope(
        _ptr(x), _ptr(bias), _ptr(positions), _ptr(cos_t), _ptr(sin_t), seq, T, n_heads, D // n_heads,
        _stream(x)))
    return x


def bias_rope_split(qkv, bias=None, positions=None, cos_t=None, sin_t=None, n_heads: int = 1):
    """qkv [T, 3D] -> contiguous (q, k, v) [T, D]: bias on all, RoPE on q, k."""
    import torch
    if not qkv.is_cuda or not qkv.is_contiguous() or qkv.dim() != 2 or qkv.shape[1] % 3:
        raise ValueError("qkv must be a contiguous CUDA [T, 3D] tensor")
    T, D3 = qkv.shape
    D = D3 // 3
    if D % n_heads:
        raise ValueError("D must be a multiple of n_heads")
    q, k, v = (torch.empty(T, D, device=qkv.device, dtype=qkv.dtype) for _ in range(3))
    seq = 0 if cos_t is None else cos_t.shape[0]
    _native.check(_native.attn_lib().agpt_bias_rope_split(
        _ptr(qkv), _ptr(bias), _ptr(positions), _ptr(cos_t), _ptr(sin_t), seq, T, n_heads, D // n_heads,
        _ptr(q), _ptr(k), _ptr(v), _stream(qkv)))
    return q, k, v


def rmsprop_(params, grads, sq_avg, lr: float, beta: float, eps: float = 1e-8):
    """In place: sq_avg = beta sq_avg + (1-beta) g^2; params -= lr g / (sqrt(sq_avg) + eps)."""
    for t in (params, grads, sq_avg):
        if not t.is_cuda or not t.is_contiguous():
            raise ValueError("params, grads and sq_avg must be contiguous CUDA tensors")
    n = params.numel()
    if grads.numel() != n or sq_avg.numel() != n:
        raise ValueError("params, grads and sq_avg must have the same size")
    _native.check(_native.attn_lib().agpt_rmsprop(
        _ptr(params), _ptr(grads), _ptr(sq_avg), C.c_float(lr), C.c_float(beta), C.c_float(eps), n,
        _stream(params)))


def relu_bwd(dy, h):
    """Returns (dh, db): dh = dy where h > 0 else 0 ([T, width]), db = its
    column sum [width] (fixed order), in one pass."""
    import torch
    for t in (dy, h):
        if not t.is_cuda or not t.is_contiguous() or t.dim() != 2 or t.dtype != torch.float32:
            raise ValueError("dy and h must be contiguous float32 CUDA [T, width] tensors")
    if dy.shape != h.shape:
        raise ValueError("dy and h must have the same shape")
    T, W = dy.shape
    lib = _native.attn_lib()
    ws = torch.empty(lib.agpt_norm_workspace_floats(W), device=dy.device, dtype=torch.float32)
    dh = torch.empty_like(dy)
    db = torch.empty(W, device=dy.device, dtype=torch.float32)
    _native.check(lib.agpt_relu_bwd(_ptr(dy), _ptr(h), _ptr(dh), _ptr(db), _ptr(ws), ws.numel(), T, W,
                                    _stream(dy)))
    return dh, db


def norm_fwd(x, w, b=None, eps: float = 1e-5):
    """LayerNorm (b given) or RMSNorm of the rows of x [T, D]; returns
    (y, mean or None, rstd)."""
    import torch
    T, D = x.shape
    y = torch.empty_like(x)
    rstd = torch.empty(T, device=x.device, dtype=torch.float32)
    mean = torch.empty(T, device=x.device, dtype=torch.float32) if b is not None else None
    _native.check(_native.attn_lib().agpt_norm_fwd(
        _ptr(x), _ptr(w), _ptr(b), _ptr(y), _ptr(mean), _ptr(rstd), T, D, C.c_float(eps), _stream(x)))
    return y, mean, rstd


def norm_bwd(dy, x, w, mean, rstd, layer: bool, dres=None):
    """Returns (dx, dw, db or None) of norm_fwd; dres [T, D] (a residual
    stream's gradient at x) is added into dx in the same pass."""
    import torch
    T, D = x.shape
    if dres is not None and (not dres.is_cuda or not dres.is_contiguous() or dres.shape != x.shape):
        raise ValueError("dres must be a contiguous CUDA tensor shaped as x")
    lib = _native.attn_lib()
    ws = torch.empty(lib.agpt_norm_workspace_floats(D), device=x.device, dtype=torch.float32)
    dx = torch.empty_like(x)
    dw = torch.empty(D, device=x.device, dtype=torch.float32)
    db = torch.empty(D, device=x.device, dtype=torch.float32) if layer else None
    _native.check(lib.agpt_norm_bwd(_ptr(dy), _ptr(dres), _ptr(x), _ptr(w), _ptr(mean), _ptr(rstd), _ptr(dx), _ptr(dw),
                                    _ptr(db), _ptr(ws), ws.numel(), T, D, _stream(x)))
    return dx, dw, db
