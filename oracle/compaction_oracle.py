"""TEST INFRASTRUCTURE ONLY - CPU restatement of block compression's budget, selection and gather.

Only tests/ may import this module. Each function follows the cited BP-KV lines:

* ``selection_budget``   core/scheduler.py:547-563
* ``snapkv_arithmetic``  core/compress.py:75-94, 99-114, 133-145 (segment split, alignment, k, L_final)
* ``select_topk``        core/scheduler.py:613-616 (topk then sorted); ties broken toward the lower
                         index (the reference's torch.topk leaves them unspecified)
* ``retained_pages``     core/scheduler.py:762-779 (sink blocks, Ls/B + selected, obs blocks)
* ``compact``            core/scheduler.py:805-878 + 702-733: per sequence FIFO destination pages,
                         per layer ``pool[l, dst[j]] = pool[l, table[keep_l[j]]]``
"""
from __future__ import annotations

import math

import numpy as np


def selection_budget(L, block_size=16, sink_len=16, obs_len=16, retain_ratio=0.20, retain_budget_tokens=0):
    B = block_size
    budget = int(retain_budget_tokens or 0)
    if budget > 0 and L <= budget:
        return 0, L, "input_le_budget"
    if L < sink_len + obs_len + B:
        return 0, L, "too_short"
    mid_tokens = max(0, L - sink_len - obs_len)
    mid_blocks = int(math.ceil(mid_tokens / B))
    if budget > 0:
        mid_budget = max(0, budget - sink_len - obs_len)
        k = max(0, min(mid_blocks, int(math.floor(mid_budget / B))))
        return k, sink_len + k * B + obs_len, "fixed_budget"
    k = max(1, min(mid_blocks, int(math.floor(float(retain_ratio) * mid_blocks))))
    return k, sink_len + k * B + obs_len, "ratio"


def snapkv_arithmetic(L, block_size=16, sink_len=64, obs_len=64, retain_ratio=0.20, retain_budget_tokens=0):
    """The debug record of BlockAlignedSnapKV.compress without the tensors."""
    B = block_size
    budget = int(retain_budget_tokens)
    if budget > 0 and L <= budget:
        return dict(compression_skipped="input_le_budget", effective_retained_tokens=L)
    premid = L - sink_len - obs_len
    aligned = math.ceil(premid / B) * B
    N = aligned // B
    if budget > 0:
        k = max(0, min(N, int(math.floor(max(0, budget - sink_len - obs_len) / B))))
        mode = "fixed_budget"
    else:
        k = max(1, int(math.floor(retain_ratio * N)))
        mode = "ratio"
    return dict(mid_tokens_before_align=premid, mid_tokens_aligned=aligned, mid_block_count=N,
                retained_block_count=k, effective_retained_tokens=sink_len + k * B + obs_len, compression_mode=mode)


def select_topk(scores: np.ndarray, k: int) -> np.ndarray:
    """Rows of ascending indices of the k largest scores, ties to the lower index, NaN first."""
    scores = np.asarray(scores, dtype=np.float32)
    out = np.empty((scores.shape[0], k), dtype=np.int32)
    for r, row in enumerate(scores):
        idx = np.arange(row.shape[0])
        with np.errstate(invalid="ignore"):  # signalling-NaN payloads warn on the widening cast
            key = np.where(np.isnan(row), np.inf, row.astype(np.float64))
        nan_first = np.isnan(row)
        order = np.lexsort((idx, -key, ~nan_first))  # NaN first, then score desc, then index asc
        out[r] = np.sort(order[:k])
    return out


def retained_pages(L, selected_mid, block_size=16, sink_len=16, obs_len=16):
    sel = np.asarray(selected_mid)
    layers = sel.shape[0]
    sink = np.broadcast_to(np.arange(sink_len // block_size), (layers, sink_len // block_size))
    obs_blocks = np.arange((L - obs_len) // block_size, L // block_size)
    obs = np.broadcast_to(obs_blocks, (layers, len(obs_blocks)))
    return np.concatenate([sink, sel + sink_len // block_size, obs], axis=1).astype(np.int32)


def compact(k_pool: np.ndarray, v_pool: np.ndarray, allocator, seq_page_lists, retained):
    """k_pool / v_pool [L, N, ...]; allocator = pool_oracle.FifoAllocator. Returns new page lists."""
    new_lists = []
    for pages, keep in zip(seq_page_lists, retained):
        keep = np.asarray(keep)
        ids = allocator.allocate_blocks(keep.shape[1])
        assert len(ids) == keep.shape[1]
        pages = np.asarray(pages)
        for layer in range(k_pool.shape[0]):
            src = pages[keep[layer]]
            k_pool[layer, ids] = k_pool[layer, src]
            v_pool[layer, ids] = v_pool[layer, src]
        new_lists.append(list(ids))
    return new_lists
