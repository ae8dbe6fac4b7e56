"""ctypes binding of libukv.so (the gfx950 kernels behind the C ABI in include/ukv.h).

The library is loaded from this package directory only. There is no fallback:
if it is missing or fails to load, ``load()`` raises and the drop-in modules
report themselves unavailable, the way the reference reports a missing Triton
(core/page16_native.py:6-13).
"""
from __future__ import annotations

import ctypes
import functools
import os
from pathlib import Path
from typing import Optional

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libukv.so"

UKV_DTYPE_F16 = 0
UKV_DTYPE_BF16 = 1

UKV_OK = 0
UKV_ERR_INVALID_ARGUMENT = -1
UKV_ERR_EMPTY = -2
UKV_ERR_GQA = -3
UKV_ERR_HEAD_DIM = -4
UKV_ERR_DTYPE = -5
UKV_ERR_WORKSPACE = -6
UKV_ERR_LAUNCH = -7
UKV_ERR_NO_DEVICE = -8

_c_void_p = ctypes.c_void_p
_c_int = ctypes.c_int
_c_i64p = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes); every symbol declared in include/ukv.h.
SIGNATURES = {
    "ukv_version": (_c_int, []),
    "ukv_status_string": (ctypes.c_char_p, [_c_int]),
    "ukv_page16_workspace_bytes": (ctypes.c_size_t, [_c_int, _c_int, _c_int, _c_int]),
    "ukv_copy_2d": (
        _c_int, [_c_void_p, ctypes.c_size_t, _c_void_p, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t, _c_void_p]),
    "ukv_page16_decode": (
        _c_int,
        [
            _c_void_p, _c_void_p, _c_void_p,  # q, k_cache, v_cache
            _c_void_p, _c_void_p, _c_void_p,  # block_table, seqlens, out
            _c_int, _c_int, _c_int, _c_int, _c_int,  # batch, Hq, Hkv, D, n_rep
            _c_int, _c_int,  # max_blocks, num_pages
            _c_i64p, _c_i64p, _c_i64p,  # q/k/v strides
            ctypes.c_float, _c_int,  # softmax_scale, dtype
            _c_void_p, ctypes.c_size_t, _c_void_p,  # workspace, bytes, stream
        ],
    ),
    "ukv_page16_decode_noalloc": (
        _c_int,
        [
            _c_void_p, _c_void_p, _c_void_p,  # q, k_cache, v_cache
            _c_void_p, _c_void_p, _c_void_p,  # block_table, seqlens, out
            _c_int, _c_int, _c_int, _c_int, _c_int,  # batch, Hq, Hkv, D, n_rep
            _c_int, _c_int,  # max_blocks, num_pages
            _c_i64p, _c_i64p, _c_i64p,  # q/k/v strides
            ctypes.c_float, _c_int, _c_void_p,  # softmax_scale, dtype, stream
        ],
    ),
    "ukv_kv_scatter_tokens": (
        _c_int,
        [_c_void_p, _c_i64p, _c_void_p, _c_i64p, _c_void_p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
         _c_void_p],
    ),
    "ukv_kv_gather_tokens": (
        _c_int,
        [_c_void_p, _c_i64p, _c_void_p, _c_i64p, _c_void_p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
         _c_void_p],
    ),
    "ukv_page_copy": (
        _c_int,
        [
            ctypes.POINTER(_c_void_p), ctypes.POINTER(_c_void_p), _c_int,  # src pools, dst pools, npools
            _c_i64p, _c_i64p,  # src / dst strides {layer, page}
            _c_void_p, ctypes.c_int64, _c_void_p, ctypes.c_int64,  # src ids, stride, dst ids, stride
            _c_int, _c_int, _c_int, _c_int, _c_int, _c_void_p,  # n, layers, page_elems, src/dst pages, stream
        ],
    ),
    "ukv_retain_writeback_dense": (
        _c_int,
        [
            ctypes.POINTER(_c_void_p), ctypes.POINTER(_c_void_p), _c_i64p,  # k/v layer bases (host), strides
            _c_int, _c_int, _c_int,  # src_len, sink_len, obs_len
            _c_void_p, ctypes.c_int64, _c_int, _c_int,  # sel, sel layer stride, k, pad_blocks
            _c_void_p, _c_void_p, _c_i64p,  # k/v pools, pool strides
            _c_void_p, _c_int, _c_int,  # dst ids, n_dst_ids, num_pages
            _c_int, _c_int, _c_int, _c_void_p,  # layers, heads, head_dim, stream
        ],
    ),
    "ukv_retain_compact_pages": (
        _c_int,
        [
            _c_void_p, _c_void_p, _c_i64p,  # k/v source pools, strides
            _c_void_p, _c_int, _c_int, _c_int,  # src ids, n_src_ids, src_num_pages, src_len
            _c_int, _c_int,  # sink_len, obs_len
            _c_void_p, ctypes.c_int64, _c_int, _c_int,  # sel, sel layer stride, k, pad_blocks
            _c_void_p, _c_void_p, _c_i64p,  # k/v pools, pool strides
            _c_void_p, _c_int, _c_int,  # dst ids, n_dst_ids, num_pages
            _c_int, _c_int, _c_int, _c_void_p,  # layers, heads, head_dim, stream
        ],
    ),
    "ukv_kv_append": (
        _c_int,
        [
            _c_void_p, _c_void_p, _c_i64p, _c_i64p,  # k/v pool layers, strides
            _c_void_p, _c_void_p, _c_i64p,  # k_new, v_new, strides
            _c_void_p, _c_int, _c_void_p, _c_void_p,  # block_table, max_blocks, old_lens, new_lens
            _c_int, _c_int, _c_int, _c_int, _c_int, _c_void_p,  # batch, block_size, heads, head_dim, pages, stream
        ],
    ),
    "ukv_page16_decode_append": (
        _c_int,
        [
            _c_void_p, _c_void_p, _c_void_p,  # q, k_cache, v_cache
            _c_void_p, _c_void_p,  # block_table, seqlens
            _c_void_p, _c_void_p, _c_i64p, _c_void_p,  # k_new, v_new, new strides, out
            _c_int, _c_int, _c_int, _c_int, _c_int,  # batch, Hq, Hkv, D, n_rep
            _c_int, _c_int,  # max_blocks, num_pages
            _c_i64p, _c_i64p, _c_i64p,  # q/k/v strides
            ctypes.c_float, _c_int,  # softmax_scale, dtype
            _c_void_p, ctypes.c_size_t, _c_void_p,  # workspace, bytes, stream
        ],
    ),
    "ukv_decode_prologue": (
        _c_int,
        [
            _c_void_p, _c_int, _c_int,  # block_table, max_blocks, batch
            _c_void_p, _c_void_p,  # lens_in, lens_out
            ctypes.POINTER(ctypes.c_int32), _c_int, _c_void_p,  # host (row, col, id) triples, n_new, stream
        ],
    ),
    "ukv_kv_write_varlen": (
        _c_int,
        [
            _c_void_p, _c_void_p, _c_i64p, _c_i64p, _c_void_p, _c_void_p, _c_i64p,  # pools, strides, k/v new
            _c_void_p, _c_int, _c_void_p, _c_void_p,  # block_table, max_blocks, cu_seqlens_q, kv_lens
            _c_int, _c_int, _c_int, _c_int, _c_int, _c_void_p,  # batch, max_chunk, heads, head_dim, pages, stream
        ],
    ),
    "ukv_paged_prefill": (
        _c_int,
        [
            _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,  # q k v bt cu kv_lens out
            _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,  # batch total_q max_chunk Hq Hkv D n_rep
            _c_int, _c_int, _c_i64p, _c_i64p, _c_i64p,  # max_blocks num_pages strides
            ctypes.c_float, _c_int, _c_void_p,  # scale dtype stream
        ],
    ),
    "ukv_paged_prefill_obs_stats": (
        _c_int,
        [
            _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,  # q k v bt cu kv_lens out
            _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,  # batch total_q max_chunk Hq Hkv D n_rep
            _c_int, _c_int, _c_i64p, _c_i64p, _c_i64p,  # max_blocks num_pages strides
            ctypes.c_float, _c_int,  # scale dtype
            _c_int, _c_int, _c_void_p, ctypes.c_int64, _c_void_p,  # sink obs stats stats_seq_stride stream
        ],
    ),
    "ukv_snapkv_block_count": (_c_int, [_c_int, _c_int, _c_int, _c_int]),
    "ukv_snapkv_workspace_bytes": (
        ctypes.c_size_t, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int]),
    "ukv_snapkv_scores": (
        _c_int,
        [
            _c_void_p, _c_i64p, _c_void_p, _c_i64p,  # q_obs, strides, k, strides
            _c_void_p, _c_int, _c_int,  # block_table, max_blocks, num_pages
            _c_int, _c_int, _c_int, _c_int, _c_int,  # layers, seqs, seq_len, sink, obs
            _c_int, _c_int, _c_int, _c_int, _c_int,  # Hq, Hkv, D, n_rep, block_size
            ctypes.c_float, _c_int, _c_void_p, ctypes.c_int64,  # scale, dtype, scores, stride
            _c_void_p, ctypes.c_size_t, _c_void_p,  # workspace, bytes, stream
        ],
    ),
    "ukv_snapkv_scores_from_stats": (
        _c_int,
        [
            _c_void_p, _c_i64p, _c_void_p, _c_i64p,  # q_obs, strides, k, strides
            _c_void_p, _c_int, _c_int,  # block_table, max_blocks, num_pages
            _c_int, _c_int, _c_int, _c_int, _c_int,  # layers, seqs, seq_len, sink, obs
            _c_int, _c_int, _c_int, _c_int, _c_int,  # Hq, Hkv, D, n_rep, block_size
            ctypes.c_float, _c_int, _c_void_p,  # scale, dtype, obs_stats
            _c_void_p, ctypes.c_int64,  # scores, stride
            _c_void_p, ctypes.c_size_t, _c_void_p,  # workspace, bytes, stream
        ],
    ),
    "ukv_select_topk": (
        _c_int,
        [_c_void_p, ctypes.c_int64, _c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_void_p, ctypes.c_int64,
         _c_void_p],
    ),
}

_lib: Optional[ctypes.CDLL] = None
_load_error: Optional[str] = None


def load() -> ctypes.CDLL:
    """Load libukv.so once and attach the C signatures. Raises on failure."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        _load_error = f"{LIB_PATH} is not built (run __graft_entry__.build())"
        raise OSError(_load_error)
    try:
        lib = ctypes.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | os.RTLD_LOCAL)
    except OSError as exc:
        _load_error = str(exc)
        raise
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def available() -> bool:
    try:
        load()
        return True
    except OSError:
        return False


def load_error() -> Optional[str]:
    return _load_error


def status_string(code: int) -> str:
    return load().ukv_status_string(int(code)).decode()


def i64_array(values) -> ctypes.Array:
    vals = [int(v) for v in values]
    return (ctypes.c_int64 * len(vals))(*vals)


@functools.lru_cache(maxsize=512)
def i64_tuple(values: tuple) -> ctypes.Array:
    """i64_array of a tuple of ints, built once per distinct tuple (the C side only reads it)."""
    return i64_array(values)


def ptr_array(values) -> ctypes.Array:
    vals = [ctypes.c_void_p(int(v)) for v in values]
    return (ctypes.c_void_p * len(vals))(*vals)


def check(code: int, what: str) -> None:
    if code != UKV_OK:
        raise RuntimeError(f"{what}: ukv status {code} ({status_string(code)})")
