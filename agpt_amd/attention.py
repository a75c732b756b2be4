"""Host-side mirror of the reference's trie-attention operator interface.

`TrieAttention` is the batched form of the reference's per-depth calls
(BatchedDepthForward#cpu_grouped_attention, batched_depth_forward.cr:836-971;
BatchedDepthBackward#optimized_attention_backward_head,
batched_depth_backward.cr:605-695): one plan per subtree batch, then forward
and backward over all of its node-tokens at once. The `batched_varlen_*`
functions keep the argument meaning of the µGPT externs the reference binds
(agpt_train.cu:73-86, 3120-3132).

Tensors are torch tensors on the GPU (PyTorch is the device-memory and
stream plumbing only); every computation runs in libagpt_attn.so. Errors are
raised as AgptError with the library's message, mirroring the reference's
CUDA_CHECK failures (agpt_train.cu:26-33) without exiting.
"""
from __future__ import annotations

import ctypes as C
import math

import numpy as np
import torch

from . import _native as N

_DTYPES = {torch.float32: N.AGPT_DTYPE_F32, torch.bfloat16: N.AGPT_DTYPE_BF16}


def rope_tables(max_seq: int, head_dim: int, base: float = 10000.0,
                device="cuda") -> tuple[torch.Tensor, torch.Tensor]:
    """RoPE cos/sin tables [max_seq, head_dim] laid out as build_rope_cache
    (agpt_train.cu:2298-2321): theta = pos / base^(2i/dim), each value stored
    in lanes 2i and 2i+1. Computed in float32 like the reference."""
    pos = np.arange(max_seq, dtype=np.float32)[:, None]
    i = np.arange(head_dim // 2, dtype=np.float32)[None, :]
    theta = pos / np.power(np.float32(base), np.float32(2.0) * i / np.float32(head_dim))
    theta = theta.astype(np.float32)
    c = np.repeat(np.cos(theta), 2, axis=1).astype(np.float32)
    s = np.repeat(np.sin(theta), 2, axis=1).astype(np.float32)
    return torch.from_numpy(c).to(device), torch.from_numpy(s).to(device)


def _addr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream_handle(stream) -> int | None:
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream or None


class TrieAttention:
    """Trie-scoped attention on one GPU.

    plan(parent): rows in DFS preorder, parent[i] < i or -1 (depth-1 node).
    forward(q, k, v) -> (o, lse); backward(q, k, v, o, lse, d_o) -> (dq, dk, dv).
    q and k are post-RoPE (batched_depth_forward.cr:417-425); with `rope`
    given, dq and dk come back in pre-RoPE space (batched_depth_backward.cr:693-694).
    """

    def __init__(self, n_heads: int, head_dim: int, max_depth: int = 32,
                 dtype: torch.dtype = torch.float32):
        self.n_heads = n_heads
        self.head_dim = head_dim
        self.d_model = n_heads * head_dim
        self.dtype = dtype
        self._lib = N.attn_lib()
        cfg = N.AttnConfig(n_heads, head_dim, max_depth, _DTYPES[dtype])
        h = C.c_void_p()
        N.check(self._lib.agpt_attn_create(C.byref(cfg), C.byref(h)))
        self._h = h
        self.n_nodes = 0
        self.n_ctx = 0

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.agpt_attn_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- plan ---------------------------------------------------------------
    def plan(self, parent: np.ndarray) -> None:
        par = np.ascontiguousarray(parent, dtype=np.int32)
        N.check(self._lib.agpt_attn_plan(self._h, par.ctypes.data_as(C.POINTER(C.c_int32)),
                                         par.shape[0]))
        self.n_nodes = int(par.shape[0])
        self.n_ctx = 0

    def plan_range(self, parent: np.ndarray, row_begin: int, row_end: int, packed: bool = False) -> None:
        """Plans rows [row_begin, row_end) of the trie `parent` (its whole DFS
        table) as one batch (agpt_attn_plan_range). packed=False: forward /
        backward take the whole trie's tensors, and the backward adds the
        batch's share of dK/dV of its context rows (the ancestors of
        row_begin before the range) into their rows: run the ranges of a
        trie in ascending order. packed=True: the tensors hold the n_ctx
        context rows (root first) and then the range's rows; the backward
        writes the context rows' share into rows 0..n_ctx-1."""
        par = np.ascontiguousarray(parent, dtype=np.int32)
        mode = N.AGPT_CTX_PACKED if packed else N.AGPT_CTX_GLOBAL
        N.check(self._lib.agpt_attn_plan_range(self._h, par.ctypes.data_as(C.POINTER(C.c_int32)),
                                               par.shape[0], int(row_begin), int(row_end), mode))
        self.n_ctx = 0
        a = int(par[row_begin])
        while a >= 0:
            self.n_ctx += 1
            a = int(par[a])
        self.n_nodes = (row_end - row_begin + self.n_ctx) if packed else int(par.shape[0])

    def plan_static(self, parent: np.ndarray) -> None:
        """plan() with every device table and workspace in the library's
        static scratch (agpt_attn_plan_static: no device allocation; one
        such plan is live per device at a time)."""
        par = np.ascontiguousarray(parent, dtype=np.int32)
        N.check(self._lib.agpt_attn_plan_static(self._h, par.ctypes.data_as(C.POINTER(C.c_int32)),
                                                par.shape[0]))
        self.n_nodes = int(par.shape[0])

    def plan_radix(self, radix_parent: np.ndarray, edge_len: np.ndarray) -> None:
        rp = np.ascontiguousarray(radix_parent, dtype=np.int32)
        el = np.ascontiguousarray(edge_len, dtype=np.int32)
        N.check(self._lib.agpt_attn_plan_radix(self._h, rp.ctypes.data_as(C.POINTER(C.c_int32)),
                                               el.ctypes.data_as(C.POINTER(C.c_int32)), rp.shape[0]))
        self.n_nodes = int(el.astype(np.int64).sum())

    def plan_info(self) -> dict:
        n, nt, sd = C.c_int64(), C.c_int64(), C.c_int64()
        md = C.c_int32()
        N.check(self._lib.agpt_attn_plan_info(self._h, C.byref(n), C.byref(nt), C.byref(sd),
                                              C.byref(md)))
        return dict(n_nodes=n.value, n_tiles=nt.value, sum_depth=sd.value, max_depth=md.value)

    def describe(self) -> str:
        return self._lib.agpt_attn_describe(self._h).decode()

    # -- compute ------------------------------------------------------------
    def _opts(self, scale, rope, stream, events=None) -> N.AttnOpts:
        o = N.AttnOpts()
        if events:
            arr = (C.c_void_p * len(events))(*events)
            o.prof_events = C.cast(arr, C.POINTER(C.c_void_p))
            o.n_prof_events = len(events)
            o._keep = arr  # keeps the array alive as long as the struct
        o.scale = 0.0 if scale is None else float(scale)
        if rope is not None:
            cos_t, sin_t = rope
            assert cos_t.dtype == torch.float32 and cos_t.is_contiguous()
            assert cos_t.shape[1] == self.head_dim
            o.rope_cos, o.rope_sin = cos_t.data_ptr(), sin_t.data_ptr()
            o.rope_seq_len = int(cos_t.shape[0])
        o.stream = _stream_handle(stream)
        return o

    def _check_rows(self, *ts: torch.Tensor) -> None:
        for t in ts:
            if t is None:
                continue
            if not t.is_cuda or not t.is_contiguous():
                raise ValueError("tensors must be contiguous device tensors")
            if t.shape[0] != self.n_nodes:
                raise ValueError(f"tensor has {t.shape[0]} rows, plan has {self.n_nodes}")

    def forward(self, q, k, v, *, scale=None, stream=None, out=None, lse=None, events=None):
        self._check_rows(q, k, v)
        for t in (q, k, v):
            if t.dtype != self.dtype or t.shape[1] != self.d_model:
                raise ValueError("q/k/v must be [T, D] of the configured dtype")
        o = out if out is not None else torch.empty_like(q)
        l = lse if lse is not None else torch.empty(self.n_nodes, self.n_heads,
                                                    device=q.device, dtype=torch.float32)
        opts = self._opts(scale, None, stream, events)
        N.check(self._lib.agpt_attn_fwd(self._h, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                        o.data_ptr(), l.data_ptr(), C.byref(opts)))
        return o, l

    def backward(self, q, k, v, o, lse, d_o, *, acc_dk=None, acc_dv=None, rope=None,
                 scale=None, stream=None, out=None, events=None, ctx_wait=None):
        """ctx_wait: a torch.cuda.Event (recorded) that a range plan's
        context-row reduction waits for (agpt_attn_opts.ctx_wait)."""
        self._check_rows(q, k, v, o, lse, d_o, acc_dk, acc_dv)
        if out is None:
            out = tuple(torch.empty(self.n_nodes, self.d_model, device=q.device,
                                    dtype=torch.float32) for _ in range(3))
        for t in out:
            if (not t.is_cuda or t.dtype != torch.float32 or not t.is_contiguous()
                    or tuple(t.shape) != (self.n_nodes, self.d_model)):
                raise ValueError("out must be three contiguous float32 CUDA [n_nodes, d_model] tensors")
        dq, dk, dv = out
        opts = self._opts(scale, rope, stream, events)
        if ctx_wait is not None:
            opts.ctx_wait = ctx_wait.cuda_event
        N.check(self._lib.agpt_attn_bwd(self._h, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                        o.data_ptr(), lse.data_ptr(), d_o.data_ptr(),
                                        dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                                        _addr(acc_dk), _addr(acc_dv), C.byref(opts)))
        return dq, dk, dv


def partition_starts(radix_head: np.ndarray, depth: np.ndarray) -> np.ndarray:
    """First rows of the bigram partitions (streaming_radix_builder.cr:212-240)
    of a DFS-ordered trie: each root child whose radix edge is longer than
    one token is one partition (key: its first two tokens); a root child
    whose edge is one token is a partition of its own (second token 255),
    and each subtree below it is one more (key: first token, that
    subtree's first token)."""
    rh = np.asarray(radix_head)
    d = np.asarray(depth)
    return np.flatnonzero((d == 1) | ((d == 2) & (rh != 0)))


def range_batches(n_rows: int, max_rows: int, starts: np.ndarray | None = None) -> list[tuple[int, int]]:
    """Contiguous row ranges covering [0, n_rows), each at most max_rows long
    unless a single unit is longer; ranges are cut only at `starts` (the
    units' first rows, e.g. partition_starts), or anywhere when None."""
    if starts is None:
        return [(a, min(a + max_rows, n_rows)) for a in range(0, n_rows, max_rows)]
    bounds = np.append(np.asarray(starts, dtype=np.int64), n_rows)
    if bounds[0] != 0:
        raise ValueError("the first unit must start at row 0")
    out, a = [], 0
    for r in range(1, bounds.shape[0]):
        if bounds[r] - a > max_rows and bounds[r - 1] > a:
            out.append((a, int(bounds[r - 1])))
            a = int(bounds[r - 1])
    if n_rows > a:
        out.append((a, n_rows))
    return out


class RangedTrieAttention:
    """A trie processed as contiguous row ranges, one plan each (exact:
    every range reads its context rows as keys and returns their share of
    dK/dV). Forward and backward take the whole trie's [T, D] tensors; the
    ranges run in ascending order on one stream."""

    def __init__(self, n_heads: int, head_dim: int, parent: np.ndarray, ranges, max_depth: int = 32,
                 dtype: torch.dtype = torch.float32):
        self.ranges = [(int(a), int(b)) for a, b in ranges]
        self.parts = []
        par = np.ascontiguousarray(parent, dtype=np.int32)
        # Each range adds its share of dK/dV into the rows of earlier ranges,
        # and the outputs start uninitialised: the ranges must tile the trie
        # in ascending order from row 0.
        if not self.ranges or self.ranges[0][0] != 0 or self.ranges[-1][1] != par.shape[0] or any(
                b <= a for a, b in self.ranges) or any(
                self.ranges[i][1] != self.ranges[i + 1][0] for i in range(len(self.ranges) - 1)):
            raise ValueError("ranges must be non-empty, contiguous, ascending, start at row 0 and end at n_nodes")
        for a, b in self.ranges:
            att = TrieAttention(n_heads, head_dim, max_depth=max_depth, dtype=dtype)
            att.plan_range(par, a, b)
            self.parts.append(att)
        self.n_nodes = int(par.shape[0])
        self.n_heads, self.d_model, self.dtype = n_heads, n_heads * head_dim, dtype

    def forward(self, q, k, v, *, scale=None, stream=None):
        o = torch.empty_like(q)
        lse = torch.empty(self.n_nodes, self.n_heads, device=q.device, dtype=torch.float32)
        for att in self.parts:
            att.forward(q, k, v, scale=scale, stream=stream, out=o, lse=lse)
        return o, lse

    def backward(self, q, k, v, o, lse, d_o, *, acc_dk=None, acc_dv=None, rope=None, scale=None, stream=None):
        out = tuple(torch.empty(self.n_nodes, self.d_model, device=q.device, dtype=torch.float32)
                    for _ in range(3))
        for att in self.parts:
            att.backward(q, k, v, o, lse, d_o, acc_dk=acc_dk, acc_dv=acc_dv, rope=rope, scale=scale,
                         stream=stream, out=out)
        return out

    def fwd_bwd(self, q, k, v, d_o, *, out=None, lse=None, grads=None, acc_dk=None, acc_dv=None, rope=None,
                scale=None, n_streams=2, events=None):
        """Per range: forward, then backward (a per-subtree trainer's order),
        the ranges dealt round robin over n_streams streams of default
        priority so that one range's launch tails overlap the next range's
        kernels. Each backward's context-row reduction (additions into rows
        an earlier range wrote) waits for the previous range's backward, so
        the results are the bytes of the one-stream order. events: per range
        a pair of prof_events lists (forward, backward) or None. Returns
        (o, lse, (dq, dk, dv)); the caller's current stream waits for all."""
        dev = q.device
        cur = torch.cuda.current_stream(dev)
        o = out if out is not None else torch.empty_like(q)
        lse = lse if lse is not None else torch.empty(self.n_nodes, self.n_heads, device=dev, dtype=torch.float32)
        if grads is None:
            grads = tuple(torch.empty(self.n_nodes, self.d_model, device=dev, dtype=torch.float32)
                          for _ in range(3))
        streams = self._streams(dev, n_streams)
        ready = torch.cuda.Event()
        ready.record(cur)
        for s in streams:
            s.wait_event(ready)
        prev = None
        for j, att in enumerate(self.parts):
            s = streams[j % len(streams)]
            ev = events[j] if events is not None else (None, None)
            att.forward(q, k, v, scale=scale, stream=s, out=o, lse=lse, events=ev[0])
            att.backward(q, k, v, o, lse, d_o, acc_dk=acc_dk, acc_dv=acc_dv, rope=rope, scale=scale, stream=s,
                         out=grads, events=ev[1], ctx_wait=prev)
            prev = torch.cuda.Event()
            prev.record(s)
        for s in streams:
            cur.wait_stream(s)
        return o, lse, grads

    def capture(self, q, k, v, d_o, *, out, lse, grads, acc_dk=None, acc_dv=None, rope=None, scale=None,
                n_streams=2):
        """fwd_bwd over every range captured once into a HIP graph, so that a
        replay reruns the pass from one host call instead of two library
        calls per range. Switched off: capturing the pass (two forked
        streams, the ranges' context reductions waiting on events recorded
        on the other stream) ended in a segmentation fault inside the
        runtime's end of capture on MI355X, before any replay, and no cause
        in this code has been found."""
        raise RuntimeError("RangedTrieAttention.capture is switched off: its stream capture ended in a "
                           "segmentation fault at the end of capture, cause not found; use fwd_bwd")

    def _streams(self, dev, n):
        if getattr(self, "_stream_pool", None) is None or len(self._stream_pool) != n:
            self._stream_pool = [torch.cuda.Stream(dev) for _ in range(max(1, n))]
        return self._stream_pool

    def close(self) -> None:
        for att in self.parts:
            att.close()
        self.parts = []


# -- packed varlen drop-ins (µGPT extern argument meaning) --------------------

def batched_varlen_attention(q_packed, k_packed, v_packed, kv_offsets, kv_lengths, output,
                             weights_out, n_nodes, n_heads, head_dim, max_len, scale,
                             stream=None):
    lib = N.attn_lib()
    N.check(lib.agpt_varlen_attention(q_packed.data_ptr(), k_packed.data_ptr(),
                                      v_packed.data_ptr(), kv_offsets.data_ptr(),
                                      kv_lengths.data_ptr(), output.data_ptr(),
                                      weights_out.data_ptr(), n_nodes, n_heads, head_dim,
                                      max_len, scale, _stream_handle(stream)))


def batched_varlen_attention_backward(q_packed, k_packed, v_packed, attn_weights, d_out,
                                      kv_offsets, kv_lengths, dq, dk_full, dv_full, n_nodes,
                                      n_heads, head_dim, max_len, scale, stream=None):
    lib = N.attn_lib()
    N.check(lib.agpt_varlen_attention_backward(
        q_packed.data_ptr(), k_packed.data_ptr(), v_packed.data_ptr(), attn_weights.data_ptr(),
        d_out.data_ptr(), kv_offsets.data_ptr(), kv_lengths.data_ptr(), dq.data_ptr(),
        dk_full.data_ptr(), dv_full.data_ptr(), n_nodes, n_heads, head_dim, max_len, scale,
        _stream_handle(stream)))


def unpack_batched_attn_output(packed, unpacked, n_nodes, n_heads, head_dim, stream=None):
    lib = N.attn_lib()
    N.check(lib.agpt_unpack_batched_attn_output(packed.data_ptr(), unpacked.data_ptr(), n_nodes,
                                                n_heads, head_dim, _stream_handle(stream)))


def batched_varlen_attention_L_queries(q_packed, k_packed, v_packed, query_to_node,
                                       query_offsets, kv_offsets, kv_lengths, output,
                                       weights_out, T_q, n_heads, head_dim, max_kv_len, scale,
                                       stream=None):
    lib = N.attn_lib()
    N.check(lib.agpt_varlen_attention_L_queries(
        q_packed.data_ptr(), k_packed.data_ptr(), v_packed.data_ptr(), query_to_node.data_ptr(),
        query_offsets.data_ptr(), kv_offsets.data_ptr(), kv_lengths.data_ptr(), output.data_ptr(),
        weights_out.data_ptr(), T_q, n_heads, head_dim, max_kv_len, scale,
        _stream_handle(stream)))


def batched_varlen_attention_L_queries_backward(q_packed, k_packed, v_packed, attn_weights,
                                                d_out, query_to_node, query_offsets,
                                                kv_offsets, kv_lengths, dq, dk_full, dv_full,
                                                T_q, n_heads, head_dim, max_kv_len, scale,
                                                stream=None):
    lib = N.attn_lib()
    N.check(lib.agpt_varlen_attention_L_queries_backward(
        q_packed.data_ptr(), k_packed.data_ptr(), v_packed.data_ptr(), attn_weights.data_ptr(),
        d_out.data_ptr(), query_to_node.data_ptr(), query_offsets.data_ptr(),
        kv_offsets.data_ptr(), kv_lengths.data_ptr(), dq.data_ptr(), dk_full.data_ptr(),
        dv_full.data_ptr(), T_q, n_heads, head_dim, max_kv_len, scale, _stream_handle(stream)))


def default_scale(head_dim: int) -> float:
    """(1.0 / Math.sqrt(hd.to_f64)).to_f32 — batched_depth_forward.cr:878."""
    return float(np.float32(1.0 / math.sqrt(head_dim)))
