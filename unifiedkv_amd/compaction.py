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
  destinations (core/scheduler.py:702-733, 805-878); optionally freeing each
  sequence's old pages after its copy (core/offload.py:1262);
* ``compact_selected`` - the token-granular form for any L, sink and window
  alignment: sink tokens, each selected middle block zero-padded to 16, the
  window (core/scheduler.py:781-799), from pool-resident pages;
* ``selected_writeback`` / ``write_block_indexed_layer`` - the same map from the
  scheduler's dense raw KV [H_kv, L, D] of every layer (core/scheduler.py:702-733,
  735-799, 805-878), one launch for all layers;
* ``prune_window`` - the pool->pool page movement of prune_sequence_window
  (core/offload.py:1236-1262).
The new block-table rows are the destination lists. Selections stay on the
device and only the page counts, known from the budget arithmetic, drive the
host-side allocation; the one host synchronisation is the range check of the
retained indices (out-of-range entries would otherwise copy the wrong page).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import numpy as np
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
    if dev.type != "cuda":
        raise RuntimeError(f"select_blocks: scores must be on a GPU, got {dev}")
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
    n_mid = (L - sink_len - obs_len) // B
    if selected_mid.numel() and bool(((selected_mid < 0) | (selected_mid >= n_mid)).any()):
        # select_blocks pads short rows with -1, which the sink offset would turn into a real page
        raise ValueError(f"retained_pages: selected middle blocks outside [0, {n_mid})")
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


def _stream(dev) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _host_ids(ids, dev) -> torch.Tensor:
    return torch.tensor([int(x) for x in ids], dtype=torch.int32).pin_memory().to(dev, non_blocking=True)


def _check_pool_ids(pool, ids, what):
    bad = [int(x) for x in ids if not 0 <= int(x) < pool.N_total]
    if bad:
        raise ValueError(f"{what}: page ids outside the pool: {bad[:4]}")


def _check_keep(keep: torch.Tensor, n_pages: int, what: str) -> None:
    """Logical page indices must address the sequence's list; one device check, one sync."""
    if keep.numel() and bool(((keep < 0) | (keep >= n_pages)).any()):
        raise ValueError(f"{what}: retained page indices outside [0, {n_pages})")


def compact(pool, seq_page_lists: Sequence[Sequence[int]], retained: Sequence[torch.Tensor],
            seq_lens: Sequence[int], *, free_sources: bool = False) -> CompactionResult:
    """Gather each sequence's retained pages into freshly allocated pages of the same pool.

    seq_page_lists  physical pages of each sequence (shared by all layers, as in core/offload.py:486-509)
    retained        per sequence, int32 [num_layers, n_keep] logical page indices into its list
    seq_lens        resident tokens after compaction (the effective lengths)
    free_sources    return each sequence's old pages to the free list, in list order, right after
                    its copy (core/offload.py:1262); sequences are then handled one after another
                    (allocate, copy, free), as the reference's per-sequence calls do, so a later
                    sequence may receive an earlier one's old pages
    Destination pages come from ``pool.allocate_blocks`` in sequence order. Without
    free_sources, every copy is one launch, and if the pool runs out the pages taken by this
    call are returned and MemoryError is raised (the rollback of core/scheduler.py:872-878);
    with it, sequences finished before the failure stay compacted (``err.partial``).
    """
    dev = pool.device
    L = pool.num_layers
    keeps = []
    for s, (pages, keep) in enumerate(zip(seq_page_lists, retained)):
        if keep.dim() != 2 or int(keep.shape[0]) != L:
            raise ValueError("compact: retained index rows must match the pool's layers")
        _check_pool_ids(pool, pages, f"compact: sequence {s}")
        keep = keep.to(device=dev, dtype=torch.long)
        _check_keep(keep, len(pages), f"compact: sequence {s}")
        keeps.append(keep)
    if free_sources:
        dst_lists: List[List[int]] = []
        for s, (pages, keep) in enumerate(zip(seq_page_lists, keeps)):
            n_keep = int(keep.shape[1])
            ids = pool.allocate_blocks(n_keep) if n_keep > 0 else []
            if len(ids) != n_keep:
                err = MemoryError(f"Cannot allocate {n_keep} blocks for sequence {s}")
                err.partial = dst_lists
                raise err
            if n_keep:
                src = _host_ids(pages, dev)[keep].to(torch.int32).contiguous()
                pool.copy_pages(src, _host_ids(ids, dev))
            pool.free_blocks_by_ids(list(pages))
            dst_lists.append(ids)
    else:
        dst_lists = []
        try:
            for s, keep in enumerate(keeps):
                n_keep = int(keep.shape[1])
                ids = pool.allocate_blocks(n_keep) if n_keep > 0 else []
                if len(ids) != n_keep:
                    raise MemoryError(f"Cannot allocate {n_keep} blocks for sequence {s}")
                dst_lists.append(ids)
        except MemoryError:
            for ids in dst_lists:
                pool.free_blocks_by_ids(ids)
            raise
        src_parts = [_host_ids(pages, dev)[keep] for pages, keep in zip(seq_page_lists, keeps)
                     if int(keep.shape[1]) > 0]
        if src_parts:
            src = torch.cat(src_parts, dim=1).to(torch.int32).contiguous()  # [L, n] physical ids
            pool.copy_pages(src, _host_ids([p for ids in dst_lists for p in ids], dev))
    table = pool.block_table_for([list(x) for x in dst_lists]) if dst_lists else None
    return CompactionResult(page_lists=dst_lists, block_table=table, seq_lens=[int(x) for x in seq_lens])


# ------------------------------------------------------------------------- token granular
def _selection_tensor(selected, layers: int, dev) -> torch.Tensor:
    """int32 [layers, k] on dev from a device tensor [layers, k] / [k], a per-layer dict or list of
    lists, or one list shared by every layer (the forms core/scheduler.py:841-844 accepts)."""
    if torch.is_tensor(selected):
        t = selected.to(device=dev, dtype=torch.int32)
        if t.dim() == 1:
            t = t.unsqueeze(0).expand(layers, -1)
        if t.dim() != 2 or int(t.shape[0]) != layers:
            raise ValueError("selection must be [layers, k]")
        return t.contiguous()
    if isinstance(selected, dict):
        rows = [list(selected.get(int(l), [])) for l in range(layers)]
    elif len(selected) and isinstance(selected[0], (list, tuple, np.ndarray)):
        rows = [list(r) for r in selected]
    else:
        rows = [list(selected)] * layers
    if len(rows) != layers or len({len(r) for r in rows}) > 1:
        raise RuntimeError("selected_writeback_len_mismatch: every layer must keep the same number of blocks")
    if any(int(x) < 0 for r in rows for x in r):
        raise ValueError("selection: negative middle-block index")
    k = len(rows[0]) if rows else 0
    host = torch.tensor([[int(x) for x in r] for r in rows], dtype=torch.int32).reshape(layers, k)
    return host.pin_memory().to(dev, non_blocking=True)


def _retain_map(L: int, mode: str, sink_len: int, obs_len: int, k: int) -> Tuple[int, int, int, int]:
    """(sink, obs, k, dst_len) of the writeback map: the pass-through modes keep the first
    effective_len = L tokens, the others the sink, k padded blocks and the window."""
    if mode in ("input_le_budget", "too_short"):
        return L, 0, 0, L
    obs_start = max(0, L - obs_len)
    return sink_len, obs_len, k, sink_len + 16 * k + (L - obs_start)


def _pool_strides(pool):
    k = pool.k_cache
    if pool.v_cache.stride() != k.stride():
        raise ValueError("pool K and V must share strides")
    return _ext.i64_array(k.stride()[:4])


def write_block_indexed_layer(pool, layer_id: int, block_ids: Sequence[int], K: torch.Tensor, V: torch.Tensor,
                              source_block_indices: Sequence[int]) -> bool:
    """core/scheduler.py:702-733 for one layer: whole source blocks of the dense raw K/V [H, L, D]
    into ``block_ids``, one launch. Returns False in the reference's bail-out cases (mismatched
    lengths, L not a multiple of the block, a source block outside [0, L/B))."""
    B = int(pool.B)
    if not source_block_indices or len(source_block_indices) != len(block_ids):
        return False
    if int(K.shape[1]) % B != 0 or int(V.shape[1]) % B != 0:
        return False
    idx = [int(x) for x in source_block_indices]
    if max(idx) < 0 or max(idx) >= int(K.shape[1]) // B:
        return False
    if min(idx) < 0:
        raise IndexError("index out of range in self")  # torch.index_select's refusal
    _writeback(pool, [(K, V)], layer_id, list(block_ids), idx, src_len=int(K.shape[1]), sink=0, obs=0, pad=True)
    return True


def selected_writeback(pool, raw_by_layer: Sequence[Tuple[torch.Tensor, torch.Tensor]], selected_mid_blocks_by_layer,
                       effective_len: int, mode: str, *, sink_len: int, obs_len: int) -> List[int]:
    """One sequence's selected writeback from the dense raw KV of every layer (core/scheduler.py:805-878
    with the writes of :735-799), in one launch for all layers.

    raw_by_layer[l] = (K, V), each [H_kv, L, D] (the scheduler's raw_kv_cache entries);
    selected_mid_blocks_by_layer: a dict layer -> list, a list of lists, one shared list, or an int32
    device tensor [layers, k] (e.g. from select_blocks; entries must lie in [0, middle blocks));
    effective_len and mode as _compute_per_layer_selected_blocks returns them. Allocates
    ceil(max(1, effective_len) / B) pages FIFO and returns them (every layer's new block map);
    when the allocation fails MemoryError is raised, and when the write is refused the pages are
    freed again before the error propagates, as the reference's transaction does. A selection
    entry outside the middle blocks (a -1 pad of select_blocks, an index past the middle) raises
    ValueError before any page is taken (one host synchronisation for a device selection)."""
    if len(raw_by_layer) != pool.num_layers:
        raise RuntimeError(f"selected_writeback_missing_raw layers={len(raw_by_layer)}")
    L = int(raw_by_layer[0][0].shape[1])
    sel = _selection_tensor(selected_mid_blocks_by_layer, pool.num_layers, pool.device) \
        if mode not in ("input_le_budget", "too_short") else None
    if sel is not None and sel.numel():
        n_mid = max(1, -(-(L - int(sink_len) - int(obs_len)) // 16))
        if bool(((sel < 0) | (sel >= n_mid)).any()):
            raise ValueError("selected_writeback: a selection entry lies outside the middle blocks")
    n_req = int(math.ceil(max(1, int(effective_len)) / int(pool.B)))
    block_ids = pool.allocate_blocks(n_req)
    if not block_ids:
        raise MemoryError(f"Cannot allocate {n_req} blocks")
    try:
        k = int(sel.shape[1]) if sel is not None else 0
        sink, obs, k, dst_len = _retain_map(L, mode, int(sink_len), int(obs_len), k)
        if dst_len != int(effective_len):
            raise RuntimeError(f"selected_writeback_len_mismatch got={dst_len} expected={int(effective_len)}")
        _writeback(pool, raw_by_layer, None, block_ids, sel, src_len=L, sink=sink, obs=obs, pad=True)
    except Exception:
        pool.free_blocks_by_ids(block_ids)
        raise
    return block_ids


def _writeback(pool, raw_by_layer, layer_id, block_ids, sel, *, src_len, sink, obs, pad):
    """Launch ukv_retain_writeback_dense for all layers (layer_id None) or one layer."""
    dev = pool.device
    layers = list(range(pool.num_layers)) if layer_id is None else [int(layer_id)]
    if layer_id is not None and not 0 <= int(layer_id) < pool.num_layers:
        raise IndexError(f"layer {layer_id} is outside the pool's {pool.num_layers} layers")
    ks, vs = [], []
    for K, V in raw_by_layer:
        if K.dim() != 3 or tuple(K.shape) != tuple(V.shape) or int(K.shape[1]) != src_len:
            raise RuntimeError("selected_writeback_bad_raw_shape")
        if tuple(K.shape[::2]) != (pool.num_kv_heads, pool.head_dim):
            raise RuntimeError("selected_writeback_bad_raw_shape")
        K = K.to(device=dev, dtype=pool.dtype)
        V = V.to(device=dev, dtype=pool.dtype)
        if K.stride(2) != 1 or V.stride() != K.stride():
            K, V = K.contiguous(), V.contiguous()
        ks.append(K)
        vs.append(V)
    strides = ks[0].stride()[:2]
    if any(t.stride()[:2] != strides for t in ks + vs):
        ks = [t.contiguous() for t in ks]
        vs = [t.contiguous() for t in vs]
        strides = ks[0].stride()[:2]
    if isinstance(sel, list):
        sel = _host_ids(sel, dev).unsqueeze(0)
    k = int(sel.shape[1]) if sel is not None else 0
    dst = _host_ids(block_ids, dev)
    kc, vc = pool.k_cache, pool.v_cache
    if layer_id is not None:  # one layer: address its slice of the pool as a one-layer pool
        kc, vc = kc[layer_id:layer_id + 1], vc[layer_id:layer_id + 1]
    code = _ext.load().ukv_retain_writeback_dense(
        _ext.ptr_array([t.data_ptr() for t in ks]), _ext.ptr_array([t.data_ptr() for t in vs]),
        _ext.i64_array(strides), int(src_len), int(sink), int(obs),
        sel.data_ptr() if sel is not None else None, int(sel.stride(0)) if sel is not None and sel.shape[0] > 1 else 0,
        k, 1 if pad else 0, kc.data_ptr(), vc.data_ptr(), _ext.i64_array(kc.stride()[:4]), dst.data_ptr(),
        len(block_ids), int(pool.N_total), len(layers), pool.num_kv_heads, pool.head_dim, _stream(dev))
    _ext.check(code, "ukv_retain_writeback_dense")


def compact_selected(pool, seq_page_lists: Sequence[Sequence[int]], seq_lens: Sequence[int],
                     selections: Sequence[Optional[torch.Tensor]], *, sink_len: int, obs_len: int,
                     free_sources: bool = False) -> CompactionResult:
    """Token-granular compaction of pool-resident sequences (any L, sink and window alignment).

    For sequence s of seq_lens[s] tokens in pages seq_page_lists[s] (shared by all layers),
    selections[s] holds the kept middle blocks, int32 [layers, k] ascending (select_blocks'
    rows of that sequence), or None to keep the sequence whole (the pass-through modes). The
    new pages hold the sink, each selected 16-token block of the middle zero-padded where the
    middle ends, then the window - the layout of core/scheduler.py:781-799 - one launch per
    sequence for all layers (``ukv_retain_compact_pages``). Destination pages are allocated
    FIFO in sequence order; with free_sources each sequence's old pages are freed, in list
    order, right after its copy (core/offload.py:1262). On MemoryError the sequences finished
    before stay compacted (``err.partial``) unless free_sources is False, in which case every
    page taken by this call is returned. Invalid input (a page outside the pool, a length beyond
    its pages or below its sink, a selection outside the middle) raises ValueError before any
    page is taken."""
    dev = pool.device
    layers = pool.num_layers
    results: List[List[int]] = []
    eff_lens: List[int] = []
    # Every input is checked before any page is taken, so that a refusal leaves the pool as it
    # was; the selections are range-checked on the device with one host synchronisation for the
    # whole call (one per sequence would leave the GPU idle between the launches).
    plan, checks = [], []
    for s, (pages, L, sel) in enumerate(zip(seq_page_lists, seq_lens, selections)):
        L = int(L)
        pages = [int(x) for x in pages]
        _check_pool_ids(pool, pages, f"compact_selected: sequence {s}")
        if L > 16 * len(pages) or L < 0:
            raise ValueError(f"compact_selected: sequence {s} holds {len(pages)} pages for {L} tokens")
        selt = None if sel is None else _selection_tensor(sel, layers, dev)
        mode, k = ("too_short", 0) if selt is None else ("ratio", int(selt.shape[1]))
        sink, obs, k, dst_len = _retain_map(L, mode, int(sink_len), int(obs_len), k)
        if sink > L:
            raise ValueError(f"compact_selected: sequence {s} is shorter than its sink")
        if selt is not None and k:
            n_mid = max(1, -(-(L - sink_len - obs_len) // 16))
            checks.append(((selt < 0) | (selt >= n_mid)).any())
        else:
            checks.append(torch.zeros((), dtype=torch.bool, device=dev))
        plan.append((pages, L, selt, sink, obs, k, dst_len))
    if checks:
        bad = torch.stack(checks)
        if bool(bad.any()):
            s = int(torch.nonzero(bad)[0, 0])
            raise ValueError(f"compact_selected: sequence {s} selects blocks outside the middle")
    try:
        for s, (pages, L, selt, sink, obs, k, dst_len) in enumerate(plan):
            n_req = int(math.ceil(max(1, dst_len) / int(pool.B)))
            ids = pool.allocate_blocks(n_req)
            if len(ids) != n_req:
                raise MemoryError(f"Cannot allocate {n_req} blocks for sequence {s}")
            results.append(ids)
            eff_lens.append(dst_len)
            _compact_pages(pool, pages, L, ids, selt, sink=sink, obs=obs, k=k, pad=True)
            if free_sources:
                pool.free_blocks_by_ids(pages)
    except MemoryError as err:
        if not free_sources:
            for ids in results:
                pool.free_blocks_by_ids(ids)
        else:
            err.partial = results
        raise
    table = pool.block_table_for([list(x) for x in results]) if results else None
    return CompactionResult(page_lists=results, block_table=table, seq_lens=eff_lens)


def _compact_pages(pool, src_pages, src_len, dst_ids, sel, *, sink, obs, k, pad):
    dev = pool.device
    src = _host_ids(src_pages, dev)
    dst = _host_ids(dst_ids, dev)
    strides = _pool_strides(pool)
    code = _ext.load().ukv_retain_compact_pages(
        pool.k_cache.data_ptr(), pool.v_cache.data_ptr(), strides, src.data_ptr(), len(src_pages),
        int(pool.N_total), int(src_len), int(sink), int(obs),
        sel.data_ptr() if sel is not None else None, int(sel.stride(0)) if sel is not None and sel.shape[0] > 1 else 0,
        int(k), 1 if pad else 0, pool.k_cache.data_ptr(), pool.v_cache.data_ptr(), strides, dst.data_ptr(),
        len(dst_ids), int(pool.N_total), pool.num_layers, pool.num_kv_heads, pool.head_dim, _stream(dev))
    _ext.check(code, "ukv_retain_compact_pages")


def prune_window(pool, old_block_ids: Sequence[int], old_len: int, kept_blocks: Sequence[int]) -> Optional[List[int]]:
    """The page movement of prune_sequence_window (core/offload.py:1236-1262): FIFO-allocate
    ceil(max(1, kept tokens) / B) pages, copy the kept blocks' tokens of every layer (a partial
    last block included) into them, then free the old ids in list order. kept_blocks are block
    indices into old_block_ids; the reference passes them sorted and unique, and so must the
    caller. Returns the new ids, or None when the pool cannot supply them (nothing changes)."""
    B = int(pool.B)
    old = [int(x) for x in old_block_ids]
    kept = [int(b) for b in kept_blocks]
    if kept != sorted(set(kept)) or (kept and kept[0] < 0):
        raise ValueError("prune_window: kept blocks must be sorted, unique and non-negative")
    if old_len > B * len(old) or old_len < 0:
        raise ValueError("prune_window: old_len exceeds the old pages")
    _check_pool_ids(pool, old, "prune_window")
    kept = [b for b in kept if b * B < old_len]  # empty spans add nothing (core/offload.py:1243-1245)
    keep_len = sum(min(old_len, (b + 1) * B) - b * B for b in kept)
    if not kept:
        raise RuntimeError("No kept blocks while pruning sequence")
    n_new = int(math.ceil(max(1, keep_len) / B))
    new_ids = pool.allocate_blocks(n_new)
    if not new_ids:
        return None
    sel = _host_ids(kept, pool.device).unsqueeze(0)
    _compact_pages(pool, old, old_len, new_ids, sel, sink=0, obs=0, k=len(kept), pad=False)
    pool.free_blocks_by_ids(old)
    return new_ids
