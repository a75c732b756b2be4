"""ctypes bindings of the two native libraries (include/agpt_attn.h,
include/agpt_loss.h and include/agpt_block.h in libagpt_attn.so;
include/agpt_trie.h in libagpt_trie.so).

The attention library is the product path: if it is missing or fails to load,
every call raises — there is no Python or CPU fallback.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_DIR = Path(__file__).resolve().parent / "lib"

# status codes (include/agpt_attn.h)
AGPT_OK = 0
AGPT_ERR_INVALID_ARG = 1
AGPT_ERR_NOT_DFS = 2
AGPT_ERR_NO_PLAN = 3
AGPT_ERR_UNSUPPORTED = 4
AGPT_ERR_DEVICE = 5
AGPT_ERR_TOO_DEEP = 6

AGPT_CTX_GLOBAL = 0
AGPT_CTX_PACKED = 1
AGPT_DTYPE_F32 = 0
AGPT_DTYPE_BF16 = 1

_i32p = C.POINTER(C.c_int32)
_i64p = C.POINTER(C.c_int64)
_vp = C.c_void_p
_fp = C.c_void_p  # device float* passed as raw addresses


class AttnConfig(C.Structure):
    _fields_ = [("n_heads", C.c_int), ("head_dim", C.c_int), ("max_depth", C.c_int),
                ("dtype", C.c_int)]


class AttnOpts(C.Structure):
    _fields_ = [("scale", C.c_float), ("rope_cos", _vp), ("rope_sin", _vp),
                ("rope_seq_len", C.c_int), ("stream", _vp),
                ("prof_events", C.POINTER(_vp)), ("n_prof_events", C.c_int), ("ctx_wait", _vp)]


class AgptError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"agpt status {code}: {msg}")
        self.code = code


# Every symbol include/agpt_attn.h declares, with (restype, argtypes).
ATTN_SYMBOLS = {
    "agpt_last_error": (C.c_char_p, []),
    "agpt_version": (C.c_char_p, []),
    "agpt_attn_create": (C.c_int, [C.POINTER(AttnConfig), C.POINTER(_vp)]),
    "agpt_attn_destroy": (C.c_int, [_vp]),
    "agpt_attn_plan": (C.c_int, [_vp, _i32p, C.c_int64]),
    "agpt_attn_plan_static": (C.c_int, [_vp, _i32p, C.c_int64]),
    "agpt_attn_plan_range": (C.c_int, [_vp, _i32p, C.c_int64, C.c_int64, C.c_int64, C.c_int]),
    "agpt_attn_plan_radix": (C.c_int, [_vp, _i32p, _i32p, C.c_int64]),
    "agpt_attn_radix_rows": (C.c_int, [_i32p, _i32p, C.c_int64, _i32p, C.c_int64, C.POINTER(C.c_int64)]),
    "agpt_attn_plan_info": (C.c_int, [_vp, _i64p, _i64p, _i64p, _i32p]),
    "agpt_attn_describe": (C.c_char_p, [_vp]),
    "agpt_attn_fwd": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, C.POINTER(AttnOpts)]),
    "agpt_attn_bwd": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                C.POINTER(AttnOpts)]),
    "agpt_attn_check_tree": (C.c_int, [_i32p, C.c_int64, _i32p, _i32p]),
    "agpt_attn_dfs_order": (C.c_int, [_i32p, C.c_int64, _i32p]),
    "agpt_varlen_attention": (C.c_int, [_vp] * 7 + [C.c_int] * 4 + [C.c_float, _vp]),
    "agpt_varlen_attention_backward": (C.c_int, [_vp] * 10 + [C.c_int] * 4 + [C.c_float, _vp]),
    "agpt_unpack_batched_attn_output": (C.c_int, [_vp, _vp, C.c_int, C.c_int, C.c_int, _vp]),
    "agpt_varlen_attention_L_queries": (C.c_int, [_vp] * 9 + [C.c_int] * 4 + [C.c_float, _vp]),
    "agpt_varlen_attention_L_queries_backward": (C.c_int, [_vp] * 12 + [C.c_int] * 4 +
                                                 [C.c_float, _vp]),
    "agpt_sync": (C.c_int, []),
}

# include/agpt_loss.h (same library as the attention entry points).
LOSS_SYMBOLS = {
    "agpt_loss_per_query": (C.c_int, [_vp] * 11 + [C.c_int, C.c_int, C.c_float, C.c_float, C.c_int,
                                                   _vp]),
    "agpt_loss_mass_weights": (C.c_int, [_i32p] * 4 + [C.c_int, C.c_int, C.c_int,
                                                       C.POINTER(C.c_float)]),
}

# include/agpt_block.h (same library as the attention entry points).
BLOCK_SYMBOLS = {
    "agpt_bias_rope": (C.c_int, [_vp, _vp, _vp, _vp, _vp, C.c_int, C.c_int64, C.c_int, C.c_int, _vp]),
    "agpt_bias_rope_split": (C.c_int, [_vp] * 5 + [C.c_int, C.c_int64, C.c_int, C.c_int, _vp, _vp, _vp, _vp]),
    "agpt_rmsprop": (C.c_int, [_vp, _vp, _vp, C.c_float, C.c_float, C.c_float, C.c_int64, _vp]),
    "agpt_norm_fwd": (C.c_int, [_vp] * 6 + [C.c_int64, C.c_int, C.c_float, _vp]),
    "agpt_norm_bwd": (C.c_int, [_vp] * 10 + [C.c_int64, C.c_int64, C.c_int, _vp]),
    "agpt_norm_workspace_floats": (C.c_int64, [C.c_int]),
    "agpt_relu_bwd": (C.c_int, [_vp] * 5 + [C.c_int64, C.c_int64, C.c_int, _vp]),
}

TRIE_SYMBOLS = {
    "agpt_markov_corpus": (C.c_int, [C.c_uint64, C.c_int, C.c_int, C.c_double, C.c_double,
                                     C.c_int64, _i32p]),
    "agpt_uniform_tokens": (C.c_int, [C.c_uint64, C.c_int, C.c_int64, _i32p]),
    "agpt_trie_build": (C.c_int, [_i32p, C.c_int64, C.c_int, C.c_int64, C.POINTER(_vp)]),
    "agpt_trie_build_radix": (C.c_int, [_i32p, C.c_int64, C.c_int, C.POINTER(_vp)]),
    "agpt_trie_build_radix_part": (C.c_int, [_i32p, C.c_int64, C.c_int, C.c_int32, C.POINTER(_vp)]),
    "agpt_trie_build_chains": (C.c_int, [_i32p, C.c_int64, C.c_int, C.POINTER(_vp)]),
    "agpt_trie_stats": (C.c_int, [_vp, _i64p, _i64p, _i64p, _i32p, _i64p, _i64p]),
    "agpt_trie_export": (C.c_int, [_vp, _i32p, _i32p, _i32p, _i32p, _i32p, _i32p]),
    "agpt_trie_export_radix": (C.c_int, [_vp, _i32p, _i32p]),
    "agpt_trie_next_counts": (C.c_int, [_vp, _i32p, _i64p, _i32p, _i32p, _i32p]),
    "agpt_radix_write_subtrees": (C.c_int, [_vp, C.c_char_p, C.c_int32]),
    "agpt_radix_read_subtree": (C.c_int, [C.c_char_p, C.POINTER(_vp)]),
    "agpt_radix_info": (C.c_int, [_vp, _i64p, _i64p, _i64p, _i32p, _i32p]),
    "agpt_radix_export": (C.c_int, [_vp] + [_i32p] * 9),
    "agpt_radix_free": (None, [_vp]),
    "agpt_trie_free": (None, [_vp]),
}

_attn = None
_trie = None


def _load(name: str, symbols: dict) -> C.CDLL:
    path = LIB_DIR / name
    if not path.exists():
        raise OSError(f"{path} is not built: run `python -m agpt_amd.build` "
                      "(or __graft_entry__.build())")
    lib = C.CDLL(str(path))
    for sym, (res, args) in symbols.items():
        fn = getattr(lib, sym)
        fn.restype = res
        fn.argtypes = args
    return lib


def attn_lib() -> C.CDLL:
    global _attn
    if _attn is None:
        _attn = _load("libagpt_attn.so", {**ATTN_SYMBOLS, **LOSS_SYMBOLS, **BLOCK_SYMBOLS})
    return _attn


def trie_lib() -> C.CDLL:
    global _trie
    if _trie is None:
        _trie = _load("libagpt_trie.so", TRIE_SYMBOLS)
    return _trie


def check(rc: int) -> None:
    if rc != AGPT_OK:
        msg = attn_lib().agpt_last_error().decode(errors="replace")
        raise AgptError(rc, msg)
