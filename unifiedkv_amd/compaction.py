"""Fixed-budget block compression on the paged pool: retain-set selection and compaction.

Rows a6 / a7 of the hot path (BP-KV's selected writeback):

* ``selection_budget_blocks`` - how many middle blocks survive, and the
  resulting token count (core/scheduler.py:547-563; the same arithmetic as
  core/compress.py:76-94, 133-145);
* ``select_blocks`` - per (layer, sequence) row the k best middle blocks by
  score, ascending (core/scheduler.py:613-616), on the GPU with a defined tie
  rule (score descending, then index ascending) - torch.topk leaves ties open;
* ``retained_pages`` - sink blocks, selected middle blocks, observation-window
  blocks (the block-aligned fast path of core/scheduler.py:762-779);
* ``compact`` - FIFO-allocate each sequence's destination pages in sequence
  order (core/scheduler.py:817, core/pool.py:101-109), then one gfx950 page-copy
  launch for every layer, sequence and K/V page:
  ``pool[l, dst[j]] = pool[l, src_l[j]]`` with per-layer sources and shared
  destinations (core/scheduler.py:702-733, 805-878). The new block-table rows
  are the destination lists. No host synchronisation: selections stay on the
  device and only the page counts, known from the budget arithmetic, drive the
  host-side allocation.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import torch

from . import _ext, page_ops


def selection_budget_blocks(L: int, *, block_size: int = 16, sink_len: int = 16, obs_len: int = 16,
                            retain_ratio: float = 0.20, retain_budget_tokens: int = 0) -> Tuple[int, int, str]:
    """(k_blocks, effective_len, mode) of core/scheduler.py:547-563."""
    B = int(block_size)
    budget = int(retain_budget_tokens or 0)
    Ls, Lo, L = int(sink_len), int(obs_len), int(L)
    if budget > 0 and L <= budget:
        return 0, L, "input_le_budget"
    if L < Ls + Lo + B:
        return 0, L, "too_short"
    mid_tokens = max(0, L - Ls - Lo)
    mid_blocks = int(math.ceil(mid_tokens / B))
    if budget > 0:
        mid_budget = max(0, budget - Ls - Lo)
        k_blocks = max(0, min(mid_blocks, int(math.floor(mid_budget / B))))
        return int(k_blocks), int(Ls + k_blocks * B + Lo), "fixed_budget"
    k_blocks = max(1, min(mid_blocks, int(math.floor(float(retain_ratio) * mid_blocks))))
    return int(k_blocks), int(Ls + k_blocks * B + Lo), "ratio"


def select_blocks(scores: torch.Tensor, k: int, n_valid: Optional[torch.Tensor] = None,
                  k_per_row: Optional[torch.Tensor] = None) -> torch.Tensor:
    """int32 [rows, k]: per row the k best indices (score desc, index asc), ascending; -1 pads.

    scores float32 [rows, n] on the GPU; optional int32 [rows] valid lengths / per-row k.
    """
    if scores.dtype != torch.float32 or scores.dim() != 2:
        raise ValueError("select_blocks: float32 [rows, n] scores required")
    if scores.stride(1) != 1:
        scores = scores.contiguous()
    rows, n = int(scores.shape[0]), int(scores.shape[1])
    dev = scores.device
    out = torch.empty((rows, max(int(k), 0)), dtype=torch.int32, device=dev)
    if rows == 0 or k <= 0:
        return out
    rn = n_valid.to(device=dev, dtype=torch.int32).contiguous() if n_valid is not None else None
    rk = k_per_row.to(device=dev, dtype=torch.int32).contiguous() if k_per_row is not None else None
    code = _ext.load().ukv_select_topk(
        scores.data_ptr(), int(scores.stride(0)), rn.data_ptr() if rn is not None else None,
        rk.data_ptr() if rk is not None else None, rows, n, int(k), out.data_ptr(), int(out.stride(0)),
        torch.cuda.current_stream(dev).cuda_stream)
    _ext.check(code, "ukv_select_topk")
    return out


def retained_pages(L: int, selected_mid: torch.Tensor, *, block_size: int = 16, sink_len: int = 16,
                   obs_len: int = 16) -> torch.Tensor:
    """Logical source pages per layer: [layers, sink + k + obs] (block-aligned fast path).

    selected_mid int32 [layers, k] (ascending middle-block indices, from select_blocks).
    Requires L, sink_len and obs_len to be multiples of block_size (core/scheduler.py:762-779).
    """
    B = int(block_size)
    if L % B or sink_len % B or obs_len % B:
        raise ValueError("retained_pages: the page-granular path needs block-aligned L, sink and window")
    layers = int(selected_mid.shape[0])
    dev = selected_mid.device
    sink = torch.arange(sink_len // B, dtype=torch.int32, device=dev).expand(layers, -1)
    obs = torch.arange((L - obs_len) // B, L // B, dtype=torch.int32, device=dev).expand(layers, -1)
    return torch.cat([sink, selected_mid + sink_len // B, obs], dim=1)


@dataclass
class CompactionResult:
    page_lists: List[List[int]]  # new physical pages per sequence (shared by all layers)
    block_table: torch.Tensor    # int32 [batch, max_pages] device table of page_lists
    seq_lens: List[int]          # resident tokens per sequence (effective length)


def compact(pool, seq_page_lists: Sequence[Sequence[int]], retained: Sequence[torch.Tensor],
            seq_lens: Sequence[int]) -> CompactionResult:
    """Gather each sequence's retained pages into freshly allocated pages of the same pool.

    seq_page_lists  physical pages of each sequence (shared by all layers, as in core/offload.py:486-509)
    retained        per sequence, int32 [num_layers, n_keep] logical page indices into its list
    seq_lens        resident tokens after compaction (the effective lengths)
    Destination pages come from ``pool.allocate_blocks`` in sequence order; if the pool runs
    out, the pages taken by this call are returned and MemoryError is raised (the rollback of
    core/scheduler.py:872-878).
    """
    dev = pool.device
    L = pool.num_layers
    dst_lists: List[List[int]] = []
    try:
        for s, keep in enumerate(retained):
            n_keep = int(keep.shape[1])
            ids = pool.allocate_blocks(n_keep) if n_keep > 0 else []
            if len(ids) != n_keep:
                raise MemoryError(f"Cannot allocate {n_keep} blocks for sequence {s}")
            dst_lists.append(ids)
    except MemoryError:
        for ids in dst_lists:
            pool.free_blocks_by_ids(ids)
        raise
    src_parts = []
    for pages, keep in zip(seq_page_lists, retained):
        if int(keep.shape[1]) == 0:
            continue
        table = torch.tensor(list(pages), dtype=torch.int32).pin_memory().to(dev, non_blocking=True)
        src_parts.append(table[keep.to(device=dev, dtype=torch.long)])  # [L, n_keep] physical ids
    if src_parts:
        src = torch.cat(src_parts, dim=1).contiguous()
        flat_dst = [p for ids in dst_lists for p in ids]
        dst = torch.tensor(flat_dst, dtype=torch.int32).pin_memory().to(dev, non_blocking=True)
        if int(src.shape[0]) != L:
            raise ValueError("compact: retained index rows must match the pool's layers")
        pool.copy_pages(src, dst)
    table = pool.block_table_for([list(x) for x in dst_lists]) if dst_lists else None
    return CompactionResult(page_lists=dst_lists, block_table=table, seq_lens=[int(x) for x in seq_lens])
