"""MGPT checkpoints (agpt_train.cu:1211-1296): a file assembled here byte by
byte from the format loads into the right parameters (transposed where the
reference stores [in, out]); save then load is the identity; malformed
files are refused. CPU only."""
from __future__ import annotations

import struct

import numpy as np
import pytest

from agpt_amd import checkpoint, model


def _mats(cfg, rng):
    """The file's matrices in order, as the reference's save writes them."""
    D, F, V = cfg.d_model, cfg.d_ff, cfg.vocab
    m = [("emb", rng.standard_normal((V, D)))]
    for l in range(cfg.n_layers):
        for nm, shape in (("wq", (D, D)), ("bq", (1, D)), ("wk", (D, D)), ("bk", (1, D)), ("wv", (D, D)),
                          ("bv", (1, D)), ("wo", (D, D)), ("bo", (1, D)), ("g1", (1, D)), ("be1", (1, D)),
                          ("l1", (D, F)), ("l1b", (1, F)), ("l2", (F, D)), ("l2b", (1, D)), ("g2", (1, D)),
                          ("be2", (1, D))):
            m.append((f"{nm}{l}", rng.standard_normal(shape)))
    m += [("gf", rng.standard_normal((1, D))), ("bf", rng.standard_normal((1, D))),
          ("out", rng.standard_normal((D, V))), ("outb", rng.standard_normal((1, V)))]
    return [(n, a.astype(np.float32)) for n, a in m]


def _write(path, cfg, mats, magic=0x4D475054):
    with open(path, "wb") as f:
        f.write(struct.pack("<I", magic))
        for v in (cfg.d_model, cfg.n_heads, cfg.n_layers, cfg.d_ff, cfg.vocab, cfg.max_depth):
            f.write(struct.pack("<i", v))
        for _, a in mats:
            f.write(struct.pack("<ii", *a.shape))
            f.write(a.astype("<f4").tobytes())


def test_hand_built_file_loads_into_the_model_layout(tmp_path):
    cfg = model.ModelConfig(vocab=7, d_model=8, n_heads=2, n_layers=2, d_ff=12, max_depth=5, norm="layer")
    mats = dict(_mats(cfg, np.random.default_rng(0)))
    p = tmp_path / "m.bin"
    _write(p, cfg, list(mats.items()))
    cfg2, flat = checkpoint.load_mgpt(str(p))
    assert (cfg2.d_model, cfg2.n_heads, cfg2.n_layers, cfg2.d_ff, cfg2.vocab, cfg2.max_depth) == (8, 2, 2, 12, 7, 5)
    P, off = {}, 0
    for name, shape in model.param_shapes(cfg2):
        n = int(np.prod(shape))
        P[name] = flat[off:off + n].reshape(shape)
        off += n
    np.testing.assert_array_equal(P["tok_emb"], mats["emb"])
    for l in range(2):
        # y = x·W_file (agpt_train.cu:4675-4680) = torch linear with W_file transposed
        np.testing.assert_array_equal(P[f"wq{l}"], mats[f"wq{l}"].T)
        np.testing.assert_array_equal(P[f"wo{l}"], mats[f"wo{l}"].T)
        np.testing.assert_array_equal(P[f"w1{l}"], mats[f"l1{l}"].T)
        np.testing.assert_array_equal(P[f"w2{l}"], mats[f"l2{l}"].T)
        np.testing.assert_array_equal(P[f"bv{l}"], mats[f"bv{l}"][0])
        np.testing.assert_array_equal(P[f"n1_b{l}"], mats[f"be1{l}"][0])
        np.testing.assert_array_equal(P[f"n2_w{l}"], mats[f"g2{l}"][0])
    np.testing.assert_array_equal(P["w_out"], mats["out"].T)
    np.testing.assert_array_equal(P["nf_b"], mats["bf"][0])
    x = np.random.default_rng(1).standard_normal((3, 8)).astype(np.float32)
    np.testing.assert_allclose(x @ P["w1" + "1"].T, x @ mats["l11"], rtol=1e-6)


def test_save_load_round_trip_and_errors(tmp_path):
    cfg = model.ModelConfig(vocab=65, d_model=32, n_heads=2, n_layers=3, d_ff=64, max_depth=32, norm="layer")
    flat = model.init_params(cfg, seed=4)
    flat += np.random.default_rng(2).standard_normal(flat.shape).astype(np.float32)
    p = tmp_path / "ck.bin"
    checkpoint.save_mgpt(str(p), cfg, flat)
    cfg2, flat2 = checkpoint.load_mgpt(str(p))
    assert cfg2 == cfg
    np.testing.assert_array_equal(flat2, flat)
    raw = p.read_bytes()
    (tmp_path / "bad.bin").write_bytes(b"XXXX" + raw[4:])
    with pytest.raises(ValueError, match="magic"):
        checkpoint.load_mgpt(str(tmp_path / "bad.bin"))
    (tmp_path / "short.bin").write_bytes(raw[:-8])
    with pytest.raises(ValueError, match="truncated"):
        checkpoint.load_mgpt(str(tmp_path / "short.bin"))
    (tmp_path / "long.bin").write_bytes(raw + b"\0" * 4)
    with pytest.raises(ValueError, match="trailing"):
        checkpoint.load_mgpt(str(tmp_path / "long.bin"))
