"""MGPT model checkpoints (the reference's weight file), read into and
written from TrieGPT's flat parameter buffer.

Format (load_model_weights / save_model_weights, agpt_train.cu:1211-1296;
offsets compute_offsets :258-310), little-endian:
    u32 magic 0x4D475054, i32 d_model, n_heads, n_layers, d_ff, vocab, seq_len,
    then matrices as (i32 rows, i32 cols, f32 data[rows*cols]) in the order
    token_emb [V, D]; per layer: wq [D, D], bq [1, D], wk, bk, wv, bv, wo, bo,
    ln1 gamma [1, D], ln1 beta, l1 [D, F], l1 bias [1, F], l2 [F, D],
    l2 bias [1, D], ln2 gamma, ln2 beta; final gamma [1, D], final beta,
    out [D, V], out bias [1, V].
Matrices are stored [in, out] (the reference multiplies x·W with
column-major GEMMs); TrieGPT keeps [out, in] (torch's linear), so every
projection is transposed on the way in and out. seq_len is the RoPE table
length (ModelConfig.max_depth).
"""
from __future__ import annotations

import struct

import numpy as np

from .model import ModelConfig, param_shapes

MGPT_MAGIC = 0x4D475054


def _file_order(cfg: ModelConfig) -> list[tuple[str, bool]]:
    """(our parameter name, stored transposed) in the file's matrix order."""
    out = [("tok_emb", False)]
    for l in range(cfg.n_layers):
        out += [(f"wq{l}", True), (f"bq{l}", False), (f"wk{l}", True), (f"bk{l}", False),
                (f"wv{l}", True), (f"bv{l}", False), (f"wo{l}", True), (f"bo{l}", False),
                (f"n1_w{l}", False), (f"n1_b{l}", False), (f"w1{l}", True), (f"b1{l}", False),
                (f"w2{l}", True), (f"b2{l}", False), (f"n2_w{l}", False), (f"n2_b{l}", False)]
    out += [("nf_w", False), ("nf_b", False), ("w_out", True), ("b_out", False)]
    return out


def _offsets(cfg: ModelConfig) -> dict[str, tuple[int, tuple[int, ...]]]:
    out, off = {}, 0
    for name, shape in param_shapes(cfg):
        out[name] = (off, shape)
        off += int(np.prod(shape))
    return out


def save_mgpt(path: str, cfg: ModelConfig, flat: np.ndarray) -> None:
    flat = np.ascontiguousarray(flat, dtype=np.float32)
    offs = _offsets(cfg)
    with open(path, "wb") as f:
        f.write(struct.pack("<I6i", MGPT_MAGIC, cfg.d_model, cfg.n_heads, cfg.n_layers, cfg.d_ff,
                            cfg.vocab, cfg.max_depth))
        for name, transposed in _file_order(cfg):
            off, shape = offs[name]
            w = flat[off:off + int(np.prod(shape))].reshape(shape)
            m = w.T if transposed else (w if w.ndim == 2 else w.reshape(1, -1))
            f.write(struct.pack("<2i", m.shape[0], m.shape[1]))
            f.write(np.ascontiguousarray(m, dtype="<f4").tobytes())


def load_mgpt(path: str, norm: str = "layer") -> tuple[ModelConfig, np.ndarray]:
    """Returns (config, flat parameter buffer in TrieGPT's layout). The
    reference's blocks use LayerNorm (gamma and beta), hence norm="layer"."""
    with open(path, "rb") as f:
        data = f.read()
    if len(data) < 28:
        raise ValueError(f"{path}: too short for an MGPT header")
    magic, D, H, L, Fd, V, seq = struct.unpack_from("<I6i", data, 0)
    if magic != MGPT_MAGIC:
        raise ValueError(f"{path}: bad model magic {magic:#x}")
    cfg = ModelConfig(vocab=V, d_model=D, n_heads=H, n_layers=L, d_ff=Fd, max_depth=seq, norm=norm)
    offs = _offsets(cfg)
    flat = np.empty(sum(int(np.prod(s)) for _, s in param_shapes(cfg)), np.float32)
    pos = 28
    for name, transposed in _file_order(cfg):
        off, shape = offs[name]
        rows, cols = struct.unpack_from("<2i", data, pos)
        pos += 8
        want = (shape[1], shape[0]) if transposed else (shape if len(shape) == 2 else (1, shape[0]))
        if (rows, cols) != tuple(want):
            raise ValueError(f"{path}: matrix {name} is {rows}x{cols}, expected {want[0]}x{want[1]}")
        n = rows * cols
        if pos + 4 * n > len(data):
            raise ValueError(f"{path}: truncated at {name}")
        m = np.frombuffer(data, dtype="<f4", count=n, offset=pos).reshape(rows, cols)
        pos += 4 * n
        flat[off:off + n] = (m.T if transposed else m).reshape(-1)
    if pos != len(data):
        raise ValueError(f"{path}: {len(data) - pos} trailing bytes")
    return cfg, flat
