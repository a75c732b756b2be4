"""Per-query AGPT loss over radix queries (include/agpt_loss.h), the host
mirror of launch_agpt_loss_per_query (agpt_train.cu:2199-2216) and the
corpus-mass weights (agpt_train.cu:4608-4637).

Tensors are torch CUDA tensors; the kernels run on the current stream. There
is no CPU fallback: a missing library or GPU raises.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _native

MASS_OFF, MASS_LOG, MASS_SQRT, MASS_LINEAR = 0, 1, 2, 3


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def loss_per_query(logits, query_to_node, query_offsets, radix_ids, token_ids, counts_offset,
                   counts_tok, counts_val, mass_weights=None, entropy_lambda: float = 0.0,
                   intermediate_weight: float = 1.0, ce_only: bool = False, d_logits=None,
                   loss_out=None):
    """Returns (d_logits [T_q, V] fp32, loss [T_q] fp32); see agpt_loss.h for
    the meaning of every argument. Integer tensors are int32, floats fp32,
    all contiguous on the logits' device."""
    import torch

    if not logits.is_cuda:
        raise ValueError("logits must be a CUDA tensor (the loss runs on the GPU only)")
    if logits.dtype != torch.float32 or logits.dim() != 2 or not logits.is_contiguous():
        raise ValueError("logits must be a contiguous fp32 [T_q, V] tensor")
    T_q, V = logits.shape
    ints = (query_to_node, query_offsets, radix_ids, token_ids, counts_offset, counts_tok, counts_val)
    for t in ints:
        if t.dtype != torch.int32 or not t.is_contiguous() or t.device != logits.device:
            raise ValueError("index tensors must be contiguous int32 on the logits' device")
    # An empty CSR (no count entries) has no storage; the C ABI takes any
    # valid device address for it, since nothing is read.
    ints = tuple(t if t.numel() else torch.zeros(1, dtype=torch.int32, device=logits.device)
                 for t in ints)
    if query_to_node.numel() != T_q or token_ids.numel() != T_q:
        raise ValueError("query_to_node and token_ids need T_q entries")
    if mass_weights is not None and (mass_weights.dtype != torch.float32 or mass_weights.numel() != T_q):
        raise ValueError("mass_weights must be fp32 [T_q]")
    if d_logits is None:
        d_logits = torch.empty_like(logits)
    if loss_out is None:
        loss_out = torch.empty(T_q, device=logits.device, dtype=torch.float32)
    stream = torch.cuda.current_stream(logits.device).cuda_stream
    lib = _native.attn_lib()
    _native.check(lib.agpt_loss_per_query(
        _ptr(logits), *(_ptr(t) for t in ints), _ptr(mass_weights), _ptr(d_logits), _ptr(loss_out),
        T_q, V, C.c_float(entropy_lambda), C.c_float(intermediate_weight), int(bool(ce_only)),
        C.c_void_p(stream)))
    return d_logits, loss_out


def mass_weights(radix_ids, edge_mass, edge_lens, query_offsets, T_q: int, mode: int) -> np.ndarray:
    """Host: per-query weights f(edge_mass) / mean (agpt_train.cu:4608-4637)."""
    a = [np.ascontiguousarray(x, dtype=np.int32) for x in (radix_ids, edge_mass, edge_lens, query_offsets)]
    out = np.empty(T_q, np.float32)
    p = [x.ctypes.data_as(C.POINTER(C.c_int32)) for x in a]
    _native.check(_native.attn_lib().agpt_loss_mass_weights(
        *p, len(a[0]), T_q, mode, out.ctypes.data_as(C.POINTER(C.c_float))))
    return out


def radix_queries(radix_parent: np.ndarray, edge_len: np.ndarray):
    """Query layout of a radix batch (agpt_train.cu:4444-4479): radix node i
    owns queries query_offsets[i] .. query_offsets[i+1]-1, one per edge token.
    Returns (query_to_node [T_q], query_offsets [R+1]) int32."""
    edge_len = np.asarray(edge_len, np.int64)
    off = np.zeros(edge_len.shape[0] + 1, np.int64)
    np.cumsum(edge_len, out=off[1:])
    q2n = np.repeat(np.arange(edge_len.shape[0], dtype=np.int32), edge_len)
    return q2n, off.astype(np.int32)
