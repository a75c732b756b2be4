"""µGPT-style transformer over one trie batch: the training step of config C3
around the trie-attention path (the forward of agpt_train.cu:4640-4830 and
its backward, one subtree batch).

Per layer: x1 = x + Wo·attn(rope(Wq·n1(x) + bq), rope(Wk·n1(x) + bk),
Wv·n1(x) + bv) + bo; x = x1 + W2·relu(W1·n2(x1) + b1) + b2. Then n_f, the
output projection, the per-query AGPT loss (sum over queries), and an RMSProp
update of every parameter (one flat fp32 buffer, as the reference's
d_weights). X = tok_emb[token]; positions enter through RoPE at depth - 1.

Native (libagpt_attn.so): trie attention fwd/bwd, the bias + RoPE epilogue,
the row norms, the loss and RMSProp. The plain GEMMs are torch's
(hipBLASLt), ReLU and the residual adds torch's elementwise kernels; torch
autograd strings them together.
`norm="rms"` (BASELINE.json's C3 text) or `"layer"` (the reference code's
LayerNorm, agpt_train.cu:4671). Norm eps is 1e-5: µGPT's is not in the
reference (parity unpinned).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F

from . import block, loss as L
from .attention import TrieAttention, rope_tables


@dataclass
class ModelConfig:
    vocab: int = 65
    d_model: int = 128
    n_heads: int = 8
    n_layers: int = 4
    d_ff: int = 512
    max_depth: int = 32
    norm: str = "rms"
    eps: float = 1e-5


def param_shapes(cfg: ModelConfig) -> list[tuple[str, tuple[int, ...]]]:
    """Names and shapes of the flat parameter buffer, in order."""
    D, Fd, V = cfg.d_model, cfg.d_ff, cfg.vocab
    out = [("tok_emb", (V, D))]
    for l in range(cfg.n_layers):
        # wq, wk, wv (and bq, bk, bv) adjacent: one [3D, D] projection
        out += [(f"n1_w{l}", (D,)), (f"n1_b{l}", (D,)),
                (f"wq{l}", (D, D)), (f"wk{l}", (D, D)), (f"wv{l}", (D, D)),
                (f"bq{l}", (D,)), (f"bk{l}", (D,)), (f"bv{l}", (D,)), (f"wo{l}", (D, D)), (f"bo{l}", (D,)),
                (f"n2_w{l}", (D,)), (f"n2_b{l}", (D,)),
                (f"w1{l}", (Fd, D)), (f"b1{l}", (Fd,)), (f"w2{l}", (D, Fd)), (f"b2{l}", (D,))]
    out += [("nf_w", (D,)), ("nf_b", (D,)), ("w_out", (V, D)), ("b_out", (V,))]
    return out


def init_params(cfg: ModelConfig, seed: int = 0) -> np.ndarray:
    """Flat fp32 buffer: projections N(0, 0.02^2), embeddings N(0, 1) * 0.02,
    norm weights 1, biases 0 (seeded)."""
    rng = np.random.default_rng(seed)
    parts = []
    for name, shape in param_shapes(cfg):
        n = int(np.prod(shape))
        if name.startswith(("n1_w", "n2_w", "nf_w")):
            parts.append(np.ones(n, np.float32))
        elif name.startswith(("b", "n1_b", "n2_b", "nf_b")) or name in ("b_out",):
            parts.append(np.zeros(n, np.float32))
        else:
            parts.append((rng.standard_normal(n) * 0.02).astype(np.float32))
    return np.concatenate(parts)


def subtree_groups(tr, max_rows: int) -> list[tuple[int, int]]:
    """Contiguous DFS row ranges of whole root-child subtrees, each at most
    max_rows long unless one subtree alone is longer (the batching of the
    reference's per-subtree trainer, agpt_train.cu:423-428)."""
    roots = np.flatnonzero(tr.parent < 0)
    bounds = np.append(roots, tr.n_nodes)
    out, a = [], 0
    for r in range(1, bounds.shape[0]):
        if bounds[r] - a > max_rows and bounds[r - 1] > a:
            out.append((a, int(bounds[r - 1])))
            a = int(bounds[r - 1])
    if tr.n_nodes > a:
        out.append((a, tr.n_nodes))
    return out


class TrieBatch:
    """The device tables of one batch of whole root-child subtrees: DFS
    parents, RoPE positions, and the loss's radix query layout (one query
    per node-token, radix nodes in DFS order, each endpoint's next-token
    counts, edge_mass = the sum of the edge head's counts). Mass weights
    are normalised over the batch."""

    def __init__(self, tr, cfg: ModelConfig, device, mass_mode: int = L.MASS_LINEAR, rows=None):
        """From a trie with corpus counts (build_radix_trie or build_trie
        with counts=True), rows a..b (whole root-child subtrees)."""
        if tr.visits is None:
            raise ValueError("the trie needs corpus counts (build_trie(..., counts=True))")
        a0, b0 = rows if rows is not None else (0, tr.n_nodes)
        par = tr.parent[a0:b0]
        heads = np.flatnonzero(tr.radix_head[a0:b0])
        qoff = np.append(heads, b0 - a0).astype(np.int64)
        ends = qoff[1:] - 1 + a0
        a, b = tr.next_offsets[ends], tr.next_offsets[ends + 1]
        cnt = (b - a).astype(np.int64)
        coff = np.zeros(heads.shape[0] + 1, np.int64)
        np.cumsum(cnt, out=coff[1:])
        sel = np.repeat(a.astype(np.int64) - coff[:-1], cnt) + np.arange(int(coff[-1]))
        # edge_mass: the sum of the edge head's counts (streaming_radix_builder.cr:150-153)
        csum = np.concatenate([[0], np.cumsum(tr.next_val, dtype=np.int64)])
        h = heads + a0
        mass = (csum[tr.next_offsets[h + 1]] - csum[tr.next_offsets[h]]).astype(np.int32)
        self._build(cfg, device, mass_mode, np.where(par < 0, -1, par - a0), tr.token[a0:b0],
                    tr.depth[a0:b0], qoff, mass, coff, tr.next_tok[sel], tr.next_val[sel])

    @classmethod
    def from_radix(cls, subtrees, cfg: ModelConfig, device, mass_mode: int = L.MASS_LINEAR):
        """From radix subtree files read by trie.read_radix_subtree (the
        reference's per-subtree loader, agpt_train.cu:495-669), concatenated."""
        self = cls.__new__(cls)
        parts = [st.rows() for st in subtrees]
        base = np.cumsum([0] + [p[0].shape[0] for p in parts])
        parent = np.concatenate([np.where(p < 0, -1, p + o) for (p, _, _), o in zip(parts, base)])
        qoff = [np.zeros(1, np.int64)]
        coff = [np.zeros(1, np.int64)]
        for st, o in zip(subtrees, base):
            qoff.append(np.cumsum(st.edge_len).astype(np.int64) + o)
            coff.append(st.counts_offset[1:].astype(np.int64) + coff[-1][-1])
        self._build(cfg, device, mass_mode, parent, np.concatenate([p[1] for p in parts]),
                    np.concatenate([p[2] for p in parts]), np.concatenate(qoff),
                    np.concatenate([st.edge_mass for st in subtrees]), np.concatenate(coff),
                    np.concatenate([st.counts_tok for st in subtrees]),
                    np.concatenate([st.counts_val for st in subtrees]))
        return self

    def _build(self, cfg, dev, mass_mode, parent, token, depth, qoff, edge_mass, coff, ctok, cval):
        self.T = int(parent.shape[0])
        self.parent = np.ascontiguousarray(parent, dtype=np.int32)
        if int(token.max(initial=0)) >= cfg.vocab:
            raise ValueError("trie tokens exceed the model vocabulary")
        self.tokens = torch.from_numpy(token.astype(np.int64)).to(dev)
        self.positions = torch.from_numpy((depth - 1).astype(np.int32)).to(dev)
        R = qoff.shape[0] - 1
        edge_len = np.diff(qoff).astype(np.int32)
        q2n = np.repeat(np.arange(R, dtype=np.int32), edge_len)
        rid = np.arange(R, dtype=np.int32)
        self.mass = None
        if mass_mode != L.MASS_OFF:
            self.mass = torch.from_numpy(L.mass_weights(rid, edge_mass, edge_len, qoff, self.T, mass_mode)).to(dev)

        def to(x):
            return torch.from_numpy(np.ascontiguousarray(x, dtype=np.int32)).to(dev)
        self.loss_args = [to(q2n), to(qoff), to(rid), to(token), to(coff), to(ctok), to(cval)]


class _QKVAttn(torch.autograd.Function):
    """x -> fused Q|K|V projection x·Wᵀ ([T, 3D]) -> bias + RoPE epilogue ->
    trie attention. The backward writes dq, dk, dv (pre-RoPE, i.e. gradients
    of the projection's output before its bias) into one [3, T, D] buffer and
    forms dx as three accumulating products dq·Wq + dk·Wk + dv·Wv, so the
    three gradients are never concatenated into [T, 3D]."""

    @staticmethod
    def forward(ctx, x, w, b, m, grp):
        att, batch = grp
        qkv = F.linear(x, w)
        q, k, v = block.bias_rope_split(qkv, b.detach(), batch.positions, m.cos, m.sin, m.cfg.n_heads)
        del qkv
        m._hook()
        o, lse = att.forward(q, k, v)
        m._hook()
        ctx.save_for_backward(x, w, q, k, v, o, lse)
        ctx.m, ctx.att = m, att
        return o

    @staticmethod
    def backward(ctx, d_o):
        x, w, q, k, v, o, lse = ctx.saved_tensors
        m = ctx.m
        T, D = q.shape
        d3 = torch.empty(3, T, D, device=q.device, dtype=q.dtype)
        m._hook()
        ctx.att.backward(q, k, v, o, lse, d_o.contiguous(), rope=(m.cos, m.sin), out=(d3[0], d3[1], d3[2]))
        m._hook()
        w = w.detach()
        dx = d3[0] @ w[:D]
        dx.addmm_(d3[1], w[D:2 * D])
        dx.addmm_(d3[2], w[2 * D:])
        dw = torch.cat([_wgrad(d3[j], x) for j in range(3)])
        # The bias gradient as matrix-vector products (a column sum over ~1M
        # rows as a plain reduction keeps only D outputs in flight).
        ones = torch.ones(1, T, device=q.device, dtype=q.dtype)
        db = torch.matmul(ones, d3).view(3 * D)
        return dx, dw, db, None, None


def _col_sum(dy: torch.Tensor, rows: int = 64) -> torch.Tensor:
    """Sum over the rows of dy [T, V] in two wide stages: [T/rows, rows*V]
    summed over its first dimension, then the rows blocks (a plain column
    sum of a narrow matrix, V = 65, leaves the reduction nearly serial)."""
    T, V = dy.shape
    m = T // rows * rows
    out = dy[:m].view(-1, rows * V).sum(0).view(rows, V).sum(0)
    return out + dy[m:].sum(0) if m < T else out


def _wgrad(dy: torch.Tensor, x: torch.Tensor, splits: int = 64) -> torch.Tensor:
    """dyᵀ·x [out, in] over T ≈ 1M rows, split along the rows into `splits`
    batched products summed in order: a single product has only out·in/1024
    output tiles (16 for 128 x 128) to spread over 256 CUs."""
    T = dy.shape[0]
    m = T // splits * splits
    if m == 0:
        return dy.t() @ x
    a = dy[:m].view(splits, m // splits, dy.shape[1]).transpose(1, 2)  # [S, out, T/S]
    b = x[:m].contiguous().view(splits, m // splits, x.shape[1])       # [S, T/S, in]
    w = torch.bmm(a, b).sum(0)
    return w + dy[m:].t() @ x[m:] if m < T else w


class _Lin(torch.autograd.Function):
    """x·Wᵀ (+ b, hipBLASLt's fused bias epilogue). Backward: dx = dy·W, the
    weight gradient by _wgrad, the bias gradient by _col_sum when the output
    is narrow (the vocabulary) and a plain column sum otherwise."""

    @staticmethod
    def forward(ctx, x, w, b):
        ctx.save_for_backward(x, w)
        ctx.has_b = b is not None
        return F.linear(x, w, b)

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        db = None
        if ctx.has_b:
            db = _col_sum(dy) if dy.shape[1] < 128 else dy.sum(0)
        return dy @ w, _wgrad(dy, x), db


class _LinRelu(torch.autograd.Function):
    """relu(x·Wᵀ + b) with bias and ReLU in the GEMM's epilogue; backward
    masks dy by the saved output (> 0) and sums the bias gradient in one
    native pass (agpt_relu_bwd), then dx and dW as _Lin."""

    @staticmethod
    def forward(ctx, x, w, b):
        h = torch._addmm_activation(b, x, w.t(), use_gelu=False)
        ctx.save_for_backward(x, w, h)
        return h

    @staticmethod
    def backward(ctx, dy):
        x, w, h = ctx.saved_tensors
        dh, db = block.relu_bwd(dy.contiguous(), h)
        return dh @ w, _wgrad(dh, x), db


class _Embed(torch.autograd.Function):
    """X = onehot(token)·E; dE = onehotᵀ·dX by _wgrad (V x D outputs)."""

    @staticmethod
    def forward(ctx, tokens, emb):
        oh = F.one_hot(tokens, emb.shape[0]).to(emb.dtype)
        ctx.save_for_backward(oh)
        return oh @ emb

    @staticmethod
    def backward(ctx, dx):
        (oh,) = ctx.saved_tensors
        return None, _wgrad(oh, dx)


class _Norm(torch.autograd.Function):
    """Row norm on the native kernels (agpt_norm_fwd / agpt_norm_bwd)."""

    @staticmethod
    def forward(ctx, x, w, b, eps, layer):
        x = x.contiguous()
        y, mu, rs = block.norm_fwd(x, w.detach(), b.detach() if layer else None, eps)
        ctx.save_for_backward(x, w, mu, rs)
        ctx.layer = layer
        return y

    @staticmethod
    def backward(ctx, dy):
        x, w, mu, rs = ctx.saved_tensors
        dx, dw, db = block.norm_bwd(dy.contiguous(), x, w.detach(), mu, rs, ctx.layer)
        return dx, dw, db, None, None


class _NormRes(torch.autograd.Function):
    """(norm(x), x) for an x that also continues as the residual stream: the
    backward adds the stream's gradient into dx inside the norm kernel
    (agpt_norm_bwd's dres), so autograd has no add of its own at x."""

    @staticmethod
    def forward(ctx, x, w, b, eps, layer):
        ctx.set_materialize_grads(False)
        x = x.contiguous()
        y, mu, rs = block.norm_fwd(x, w.detach(), b.detach() if layer else None, eps)
        ctx.save_for_backward(x, w, mu, rs)
        ctx.layer = layer
        return y, x.view_as(x)

    @staticmethod
    def backward(ctx, dy, dres):
        x, w, mu, rs = ctx.saved_tensors
        if dy is None:
            dy = torch.zeros_like(x)
        dx, dw, db = block.norm_bwd(dy.contiguous(), x, w.detach(), mu, rs, ctx.layer,
                                    None if dres is None else dres.contiguous())
        return dx, dw, db, None, None


class _Loss(torch.autograd.Function):
    """Sum over queries of the per-query AGPT loss; the kernel's d_logits is
    the gradient of that sum (agpt_train.cu:4810-4830)."""

    @staticmethod
    def forward(ctx, logits, batch):
        d_logits, loss_q = L.loss_per_query(logits.detach().contiguous(), *batch.loss_args,
                                            mass_weights=batch.mass)
        ctx.save_for_backward(d_logits)
        return loss_q.sum()

    @staticmethod
    def backward(ctx, g):
        (d_logits,) = ctx.saved_tensors
        return d_logits * g, None


class TrieGPT:
    def __init__(self, cfg: ModelConfig, device="cuda", seed: int = 0, lr: float = 3e-4,
                 beta: float = 0.999, eps: float = 1e-8):
        if cfg.d_model not in (64, 128, 256, 512) or cfg.d_ff not in (64, 128, 256, 512):
            raise ValueError("the native row kernels take d_model and d_ff of 64, 128, 256 or 512")
        self.cfg = cfg
        self.dev = torch.device(device)
        self.flat = torch.from_numpy(init_params(cfg, seed)).to(self.dev).requires_grad_(True)
        self.sq_avg = torch.zeros_like(self.flat, requires_grad=False)
        self.lr, self.beta, self.eps = lr, beta, eps
        hd = cfg.d_model // cfg.n_heads
        self.cos, self.sin = rope_tables(cfg.max_depth, hd, device=self.dev)
        self.groups = []  # (TrieAttention, TrieBatch) per batch of subtrees
        self.attn_hook = None  # called before and after every attention fwd / bwd (timing)
        self.relu_hook = None  # called with (layer, FFN activation) after each ReLU (inspection)

    def plan(self, tr, mass_mode: int = L.MASS_LINEAR, max_rows: int = 1 << 20) -> None:
        """Splits the trie into batches of whole root-child subtrees (at most
        max_rows rows each) and plans each batch's attention and loss tables."""
        self.close()
        hd = self.cfg.d_model // self.cfg.n_heads
        for a, b in subtree_groups(tr, max_rows):
            batch = TrieBatch(tr, self.cfg, self.dev, mass_mode, rows=(a, b))
            att = TrieAttention(self.cfg.n_heads, hd, max_depth=self.cfg.max_depth)
            att.plan(batch.parent)
            self.groups.append((att, batch))

    def plan_radix_dir(self, radix_dir: str, mass_mode: int = L.MASS_LINEAR, max_rows: int = 1 << 20) -> None:
        """Plans from the reference's radix files (manifest.bin +
        subtrees/radix_subtree_%06d.bin): subtrees in manifest order, packed
        into batches of at most max_rows node-tokens (a larger subtree alone)."""
        import os

        from . import trie as trie_mod
        self.close()
        hd = self.cfg.d_model // self.cfg.n_heads
        man = trie_mod.read_radix_manifest(os.path.join(radix_dir, "manifest.bin"))
        pending, rows = [], 0

        def flush():
            if pending:
                batch = TrieBatch.from_radix(pending, self.cfg, self.dev, mass_mode)
                att = TrieAttention(self.cfg.n_heads, hd, max_depth=self.cfg.max_depth)
                att.plan(batch.parent)
                self.groups.append((att, batch))
        for rc, _, chars, _ in man:
            if pending and rows + chars > max_rows:
                flush()
                pending, rows = [], 0
            pending.append(trie_mod.read_radix_subtree(
                os.path.join(radix_dir, "subtrees", f"radix_subtree_{rc:06d}.bin")))
            rows += chars
        flush()

    def _hook(self) -> None:
        if self.attn_hook is not None:
            self.attn_hook()

    def params(self) -> dict[str, torch.Tensor]:
        """Views into the flat buffer by name, plus wqkv{l} [3D, D] and
        bqkv{l} [3D] over the adjacent q, k, v blocks."""
        out, off, at = {}, 0, {}
        for name, shape in param_shapes(self.cfg):
            n = int(np.prod(shape))
            out[name] = self.flat[off:off + n].view(shape)
            at[name] = off
            off += n
        D = self.cfg.d_model
        for l in range(self.cfg.n_layers):
            out[f"wqkv{l}"] = self.flat[at[f"wq{l}"]:at[f"wq{l}"] + 3 * D * D].view(3 * D, D)
            out[f"bqkv{l}"] = self.flat[at[f"bq{l}"]:at[f"bq{l}"] + 3 * D]
        return out

    def _norm(self, x, w, b):
        return _Norm.apply(x, w, b, self.cfg.eps, self.cfg.norm == "layer")

    def _norm_res(self, x, w, b):
        return _NormRes.apply(x, w, b, self.cfg.eps, self.cfg.norm == "layer")

    def loss(self, grp) -> torch.Tensor:
        """Forward over one planned batch: the summed per-query loss."""
        P, cfg = self.params(), self.cfg
        batch = grp[1]
        # X = onehot(token) · tok_emb: the backward is a product onehotᵀ · dX
        # (the gather's backward would scatter-add 1M rows into 65).
        x = _Embed.apply(batch.tokens, P["tok_emb"])
        for l in range(cfg.n_layers):
            # x feeds the norm and the residual add: _NormRes passes it on so
            # both gradients meet inside the norm backward.
            n1, x = self._norm_res(x, P[f"n1_w{l}"], P[f"n1_b{l}"])
            o = _QKVAttn.apply(n1, P[f"wqkv{l}"], P[f"bqkv{l}"], self, grp)
            x = x + _Lin.apply(o, P[f"wo{l}"], P[f"bo{l}"])
            n2, x = self._norm_res(x, P[f"n2_w{l}"], P[f"n2_b{l}"])
            h = _LinRelu.apply(n2, P[f"w1{l}"], P[f"b1{l}"])
            if self.relu_hook is not None:
                self.relu_hook(l, h)
            x = x + _Lin.apply(h, P[f"w2{l}"], P[f"b2{l}"])
        logits = _Lin.apply(self._norm(x, P["nf_w"], P["nf_b"]), P["w_out"], P["b_out"])
        return _Loss.apply(logits, batch)

    def step(self) -> torch.Tensor:
        """One training step over every planned batch: forward and backward
        per batch (gradients accumulate in the flat buffer), then one
        RMSProp update. Returns the summed loss as a device scalar."""
        self.flat.grad = None
        total = torch.zeros((), device=self.dev)
        for grp in self.groups:
            lv = self.loss(grp)
            lv.backward()
            total += lv.detach()
        if self.flat.grad is not None:  # no planned rows: nothing to update
            with torch.no_grad():
                block.rmsprop_(self.flat.data, self.flat.grad, self.sq_avg, self.lr, self.beta, self.eps)
        return total

    def save(self, path: str) -> None:
        """Writes the parameters as an MGPT checkpoint (agpt_train.cu:1262-1296)."""
        from .checkpoint import save_mgpt
        save_mgpt(path, self.cfg, self.flat.detach().cpu().numpy())

    def load(self, path: str) -> None:
        """Reads an MGPT checkpoint of this model's shape into the parameters."""
        from .checkpoint import load_mgpt
        cfg, flat = load_mgpt(path, norm=self.cfg.norm)
        if (cfg.vocab, cfg.d_model, cfg.n_heads, cfg.n_layers, cfg.d_ff) != (
                self.cfg.vocab, self.cfg.d_model, self.cfg.n_heads, self.cfg.n_layers, self.cfg.d_ff):
            raise ValueError("checkpoint shape differs from the model's")
        with torch.no_grad():
            self.flat.copy_(torch.from_numpy(flat))

    def close(self) -> None:
        for att, _ in self.groups:
            att.close()
        self.groups = []
