"""TEST INFRASTRUCTURE ONLY - CPU oracle of the Page16 hot path.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this module, and only as the checker or as the reported CPU
baseline. The product (``unifiedkv_amd`` / ``libukv.so``) never imports it.

Restatements (all cite BP-KV, the reference repository):

* ``page16_decode_pageloop`` - the reference's Page16 program
  (core/page16_native.py:34-80), fp32 page loop with natural exp, in C
  (oracle/page16_oracle.c), parallel over (sequence, head) with OpenMP.
* ``page16_decode_dense`` - closed form in fp64: gather the sequence's pages
  into a dense [L, H_kv, D] KV (the dense-rebuild formulation of
  core/engine.py:4021-4115, ``index_select`` of the block table then slice to
  ``seq_len``) and apply softmax attention with the GQA map h // n_rep
  (core/page16_native.py:36, core/compress.py:7-20).
* ``page16_decode_bruteforce`` - pure-Python scalar loops, tiny inputs only.

Pinning (tests/test_oracle.py): the three formulations agree with each other;
closed-form special cases (L = 1 gives V_0, constant K gives the mean of V,
scale 0 gives the mean of V, n_rep = 1 equals MHA over repeat_kv); invariants
(page permutation, garbage past L or in spare table columns); and planted
mistakes in the C restatement (``mutation`` 1-5) each fail at least one check.
"""
from __future__ import annotations

import ctypes
import math
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

DT_F16 = 0
DT_BF16 = 1


# --------------------------------------------------------------------------
# 16-bit storage helpers (values are kept as uint16 bit patterns)
# --------------------------------------------------------------------------
def bf16_bits_to_f32(u16: np.ndarray) -> np.ndarray:
    return (np.asarray(u16, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (NaN -> quiet NaN)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r.astype(np.uint16)


def f16_bits_to_f32(u16: np.ndarray) -> np.ndarray:
    return np.asarray(u16, dtype=np.uint16).view(np.float16).astype(np.float32)


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def bits_to_f32(u16: np.ndarray, dtype: int) -> np.ndarray:
    return bf16_bits_to_f32(u16) if dtype == DT_BF16 else f16_bits_to_f32(u16)


def f32_to_bits(x: np.ndarray, dtype: int) -> np.ndarray:
    return f32_to_bf16_bits(x) if dtype == DT_BF16 else f32_to_f16_bits(x)


# --------------------------------------------------------------------------
# C page-loop restatement
# --------------------------------------------------------------------------
_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def _load():
    """Load liboracle.so. Never builds it: the callers (tests, bench.py) may already hold a GPU
    context, and a fork + exec of make from such a process is not allowed; build() does it ahead."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it first (__graft_entry__.build() or make -C oracle)")
        lib = ctypes.CDLL(str(LIB_PATH))
        P = ctypes.c_void_p
        I = ctypes.c_int
        lib.ukvo_page16_decode.restype = I
        lib.ukvo_page16_decode.argtypes = [P, P, P, P, P, P, I, I, I, I, I, I, I, ctypes.c_float, I, I]
        lib.ukvo_set_threads.restype = None
        lib.ukvo_set_threads.argtypes = [I]
        _lib = lib
    return _lib


def page16_decode_pageloop(q, k_cache, v_cache, block_table, seqlens, *, softmax_scale, n_rep, dtype,
                           mutation: int = 0) -> np.ndarray:
    """fp32 restatement of core/page16_native.py:34-80; returns fp32 [B, Hq, D] (unrounded).

    q: uint16 [B, Hq, D]; k_cache/v_cache: uint16 [N, 16, Hkv, D]; block_table int32
    [B, max_blocks]; seqlens int32 [B]; dtype DT_F16 / DT_BF16.
    """
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k_cache, dtype=np.uint16)
    v = np.ascontiguousarray(v_cache, dtype=np.uint16)
    bt = np.ascontiguousarray(block_table, dtype=np.int32)
    lens = np.ascontiguousarray(seqlens, dtype=np.int32)
    B, Hq, D = q.shape
    N, page, Hkv, Dk = k.shape
    assert page == 16 and Dk == D and v.shape == k.shape and bt.shape[0] == B and lens.shape == (B,)
    out = np.empty((B, Hq, D), dtype=np.float32)
    rc = _load().ukvo_page16_decode(
        q.ctypes.data, k.ctypes.data, v.ctypes.data, bt.ctypes.data, lens.ctypes.data, out.ctypes.data,
        B, Hq, Hkv, D, int(n_rep), int(bt.shape[1]), N, float(softmax_scale), int(dtype), int(mutation))
    if rc != 0:
        raise ValueError("oracle rejected the arguments")
    return out


def set_threads(n: int) -> None:
    """OpenMP threads of page16_decode_pageloop."""
    _load().ukvo_set_threads(int(n))


def page16_decode_torch_dense(q, k_cache, v_cache, block_table, seqlens, *, softmax_scale, n_rep, dtype):
    """The dense-fallback formulation on the CPU in torch fp32: for each sequence, gather its pages
    (``index_select`` as _rebuild_pkv does, core/engine.py:4021-4115), convert to fp32, repeat the
    KV heads and run eager attention softmax(q K^T * scale) V. Inputs as page16_decode_pageloop;
    returns fp32 [B, Hq, D]."""
    import torch

    tdt = torch.bfloat16 if int(dtype) == DT_BF16 else torch.float16
    kt = torch.from_numpy(np.ascontiguousarray(k_cache, dtype=np.uint16).view(np.int16)).view(tdt)
    vt = torch.from_numpy(np.ascontiguousarray(v_cache, dtype=np.uint16).view(np.int16)).view(tdt)
    qt = torch.from_numpy(np.ascontiguousarray(q, dtype=np.uint16).view(np.int16)).view(tdt).float()
    B, Hq, D = qt.shape
    Hkv = kt.shape[2]
    out = torch.empty((B, Hq, D), dtype=torch.float32)
    for b in range(B):
        L = int(seqlens[b])
        n = (L + 15) // 16
        ids = torch.from_numpy(np.ascontiguousarray(block_table[b, :n], dtype=np.int64))
        K = kt.index_select(0, ids).reshape(n * 16, Hkv, D)[:L].float().transpose(0, 1)  # [Hkv, L, D]
        V = vt.index_select(0, ids).reshape(n * 16, Hkv, D)[:L].float().transpose(0, 1)
        K = K.repeat_interleave(n_rep, dim=0)  # q head h reads KV head h // n_rep
        V = V.repeat_interleave(n_rep, dim=0)
        s = torch.bmm(qt[b].unsqueeze(1), K.transpose(1, 2).contiguous()) * softmax_scale  # [Hq, 1, L]
        out[b] = torch.bmm(torch.softmax(s, dim=-1), V).squeeze(1)
    return out.numpy()


# --------------------------------------------------------------------------
# Closed forms (numpy fp64)
# --------------------------------------------------------------------------
def _gather_tokens(cache_f, block_table_row, L, num_pages):
    """Dense [L, Hkv, D] rows of one sequence; rows of out-of-range pages are dropped."""
    n_pages = (L + 15) // 16
    ids = np.asarray(block_table_row[:n_pages], dtype=np.int64)
    ok = (ids >= 0) & (ids < num_pages)
    pages = cache_f[np.where(ok, ids, 0)]  # [n_pages, 16, Hkv, D]
    tok_ok = np.repeat(ok, 16)[:L]
    rows = pages.reshape(n_pages * 16, *cache_f.shape[2:])[:L]
    return rows[tok_ok]


def page16_decode_dense(q_f, k_f, v_f, block_table, seqlens, *, softmax_scale, n_rep) -> np.ndarray:
    """fp64 dense softmax attention; inputs already in float. Returns fp64 [B, Hq, D].

    A sequence with no valid token yields NaN (0/0), as the reference's acc/l does.
    """
    q_f = np.asarray(q_f, dtype=np.float64)
    k_f = np.asarray(k_f, dtype=np.float64)
    v_f = np.asarray(v_f, dtype=np.float64)
    B, Hq, D = q_f.shape
    max_blocks = block_table.shape[1]
    N = k_f.shape[0]
    out = np.full((B, Hq, D), np.nan)
    for b in range(B):
        L = int(min(max(int(seqlens[b]), 0), 16 * max_blocks))
        if L == 0:
            continue
        K = _gather_tokens(k_f, block_table[b], L, N)
        V = _gather_tokens(v_f, block_table[b], L, N)
        if K.shape[0] == 0:
            continue
        for h in range(Hq):
            g = h // n_rep
            s = (K[:, g, :] @ q_f[b, h]) * softmax_scale
            s = s - s.max()
            p = np.exp(s)
            out[b, h] = (p @ V[:, g, :]) / p.sum()
    return out


def page16_decode_bruteforce(q_f, k_f, v_f, block_table, seqlens, *, softmax_scale, n_rep):
    """Scalar Python loops straight from the definition (tiny inputs only)."""
    B, Hq, D = len(q_f), len(q_f[0]), len(q_f[0][0])
    out = [[[float("nan")] * D for _ in range(Hq)] for _ in range(B)]
    for b in range(B):
        L = min(max(int(seqlens[b]), 0), 16 * len(block_table[b]))
        for h in range(Hq):
            g = h // n_rep
            scores, rows = [], []
            for t in range(L):
                pid = int(block_table[b][t // 16])
                if pid < 0 or pid >= len(k_f):
                    continue
                kr = k_f[pid][t % 16][g]
                scores.append(softmax_scale * sum(float(kr[d]) * float(q_f[b][h][d]) for d in range(D)))
                rows.append(v_f[pid][t % 16][g])
            if not scores:
                continue
            mx = max(scores)
            w = [math.exp(s - mx) for s in scores]
            z = sum(w)
            out[b][h] = [sum(w[i] * float(rows[i][d]) for i in range(len(w))) / z for d in range(D)]
    return np.array(out, dtype=np.float64)


def allclose_report(actual, expected, atol, rtol):
    """(ok, max_abs_err, worst_excess) with NaN positions required to match."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    nan_a, nan_e = np.isnan(a), np.isnan(e)
    if not np.array_equal(nan_a, nan_e):
        return False, float("inf"), float("inf")
    fin = ~nan_e
    if not fin.any():
        return True, 0.0, 0.0
    err = np.abs(a[fin] - e[fin])
    excess = err - (atol + rtol * np.abs(e[fin]))
    return bool((excess <= 0).all()), float(err.max()), float(excess.max())
