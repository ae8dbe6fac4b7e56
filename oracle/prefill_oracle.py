"""TEST INFRASTRUCTURE ONLY - CPU closed form of chunked prefill over pages (row a9).

Only tests/ and bench.py's cpu_baseline leg may import this module.

The reference prefills densely (core/engine.py:1826-1854, HF attention over the
past KV; core/varlen.py:19-42, flash_attn_varlen_func(causal=True)): query i of
a chunk of C queries appended after P keys attends to keys 0 .. P + i. flash-attn
is not installed here and no reference test pins its values (benchmarks/tests.py:
57-75 checks shapes only), so this restatement is pinned by its closed form and
by tests/test_prefill.py's checks: the last chunk query equals Page16 decode of
the same keys, P = 0 with C = 1 returns V_0, and causal rows never see later keys.
"""
from __future__ import annotations

import numpy as np


def write_chunk(cache_f: np.ndarray, table_row, start: int, rows: np.ndarray) -> None:
    """cache_f [N, 16, H, D]; rows [C, H, D] go to positions start .. start + C - 1."""
    for i in range(rows.shape[0]):
        pos = start + i
        cache_f[table_row[pos // 16], pos % 16] = rows[i]


def prefill_dense(q_f, k_f, v_f, block_table, cu_q, kv_lens, *, softmax_scale, n_rep, rows=None):
    """fp64 outputs [total_q, Hq, D] (or only the requested (row, head) pairs as a dict)."""
    q_f = np.asarray(q_f, dtype=np.float64)
    total_q, Hq, D = q_f.shape
    out = np.full((total_q, Hq, D), np.nan) if rows is None else {}
    B = len(kv_lens)
    for b in range(B):
        C = int(cu_q[b + 1] - cu_q[b])
        if C == 0:
            continue  # no queries in this sequence's chunk
        Lk = int(kv_lens[b])
        P = Lk - C
        n_pages = (Lk + 15) // 16
        ids = np.asarray(block_table[b][:n_pages], dtype=np.int64)
        K = np.asarray(k_f[ids], dtype=np.float64).reshape(n_pages * 16, -1, D)[:Lk]
        V = np.asarray(v_f[ids], dtype=np.float64).reshape(n_pages * 16, -1, D)[:Lk]
        wanted = range(C) if rows is None else [r - int(cu_q[b]) for r, _ in rows if cu_q[b] <= r < cu_q[b + 1]]
        for i in wanted:
            row = int(cu_q[b]) + i
            n_keys = P + i + 1
            heads = range(Hq) if rows is None else [h for r, h in rows if r == row]
            for h in heads:
                g = h // n_rep
                s = (K[:n_keys, g, :] @ q_f[row, h]) * softmax_scale
                s -= s.max()
                p = np.exp(s)
                val = (p @ V[:n_keys, g, :]) / p.sum()
                if rows is None:
                    out[row, h] = val
                else:
                    out[(row, h)] = val
    return out


def prefill_rows_f32(q_rows, K, V, positions, *, softmax_scale, n_rep):
    """Dense fp32 causal attention of some chunk rows of one sequence (the CPU baseline formulation).

    q_rows [n, Hq, D]; K, V [Lk, Hkv, D] in logical order; row j sees keys 0 .. positions[j].
    The reference's CPU path is this eager matmul-softmax-matmul (HF attention over the
    past KV, core/engine.py:1826-1854), here with numpy's BLAS.
    """
    q_rows = np.asarray(q_rows, dtype=np.float32)
    n, Hq, D = q_rows.shape
    pos = np.asarray(positions)
    n_keys = int(pos.max()) + 1
    mask = np.arange(n_keys)[None, :] > pos[:, None]
    out = np.empty((n, Hq, D), dtype=np.float32)
    for h in range(Hq):
        g = h // n_rep
        s = (q_rows[:, h, :] @ K[:n_keys, g, :].T) * np.float32(softmax_scale)
        s[mask] = -np.inf
        s -= s.max(axis=1, keepdims=True)
        p = np.exp(s)
        out[:, h, :] = (p @ V[:n_keys, g, :]) / p.sum(axis=1, keepdims=True)
    return out
