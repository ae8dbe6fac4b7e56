"""Per-sequence offload / prefetch over a pinned page arena (BP-KV's offload policy entry points).

BP-KV's ``offload_sequence_blocks`` / ``prefetch_sequence_blocks`` (core/offload.py:547-599,
620-691) move one (layer, page) at a time: a fresh pinned host tensor per K and per V block
(``torch.empty_like(..., pin_memory=True)``), a small copy each, on a transfer stream that does
not wait for the compute stream before reading the pages (core/offload.py:578). Completion is
polled later (``_try_finalize_offload`` / ``_try_finalize_prefetch``, core/offload.py:362-449),
which frees the GPU pages or publishes the new map.

``SequenceOffloader`` keeps those two entry points, their return values, the per-sequence states
(ON_GPU / MIXED / ON_CPU / OFFLOAD_INFLIGHT / PREFETCH_INFLIGHT), the CPU byte accounting and
the FIFO page allocation, with a different data path:

* host memory is one pinned arena allocated up front (``PinnedArena``: K and V
  ``[layers, capacity, page]``), handed out in extents of page slots, never allocated per call;
* pages move in chunks of every layer: the gfx950 page-copy kernel gathers a chunk into a device
  staging buffer and one strided DMA (``ukv_copy_2d``, one row per layer) moves it to or from its
  arena slots; prefetch does the reverse into freshly allocated pages;
* ordering: the side stream waits for the compute stream before reading or overwriting pages
  (so this step's appends land first); every arena read and write is on that one stream, so
  slots freed by a prefetch are reused safely without a host wait; GPU pages of an offload go
  back to the pool only once its event has completed, and a prefetched map is published only
  once its event has completed (host-side ``query``, or ``synchronize`` with ``force_sync``).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import torch

from . import _ext, page_ops

ON_GPU, MIXED, ON_CPU = "ON_GPU", "MIXED", "ON_CPU"
OFFLOAD_INFLIGHT, PREFETCH_INFLIGHT = "OFFLOAD_INFLIGHT", "PREFETCH_INFLIGHT"


class ExtentAllocator:
    """First-fit allocator of slot extents over [0, capacity); frees coalesce with neighbours."""

    def __init__(self, capacity: int):
        self.capacity = int(capacity)
        self._free: List[Tuple[int, int]] = [(0, self.capacity)] if capacity > 0 else []

    @property
    def n_free(self) -> int:
        return sum(n for _, n in self._free)

    @property
    def free_extents(self) -> List[Tuple[int, int]]:
        return list(self._free)

    def alloc(self, n: int) -> Optional[List[Tuple[int, int]]]:
        """n slots as extents (start, count) in ascending order, lowest addresses first; None if
        fewer than n slots are free."""
        n = int(n)
        if n < 0 or n > self.n_free:
            return None
        out, rest, need = [], [], n
        for start, cnt in self._free:
            if need == 0:
                rest.append((start, cnt))
                continue
            take = min(cnt, need)
            out.append((start, take))
            need -= take
            if take < cnt:
                rest.append((start + take, cnt - take))
        self._free = rest
        return out

    def free(self, extents: Sequence[Tuple[int, int]]) -> None:
        spans = sorted(self._free + [(int(s), int(c)) for s, c in extents if int(c) > 0])
        merged: List[Tuple[int, int]] = []
        for s, c in spans:
            if merged and merged[-1][0] + merged[-1][1] > s:
                raise ValueError("extent freed twice")
            if merged and merged[-1][0] + merged[-1][1] == s:
                merged[-1] = (merged[-1][0], merged[-1][1] + c)
            else:
                merged.append((s, c))
        self._free = merged


def runs_of(slots: Sequence[int]) -> List[Tuple[int, int, int]]:
    """Maximal runs of consecutive slots in the given order: (position, first slot, count)."""
    out = []
    i = 0
    while i < len(slots):
        j = i + 1
        while j < len(slots) and slots[j] == slots[j - 1] + 1:
            j += 1
        out.append((i, int(slots[i]), j - i))
        i = j
    return out


class PinnedArena:
    """Pinned host page slots for every layer of a pool: K and V ``[layers, capacity, page]``."""

    def __init__(self, pool, capacity_pages: int):
        self.capacity = int(capacity_pages)
        self.page_elems = pool.B * pool.num_kv_heads * pool.head_dim
        shape = (pool.num_layers, self.capacity, self.page_elems)
        self.k = torch.empty(shape, dtype=pool.dtype, pin_memory=True)
        self.v = torch.empty(shape, dtype=pool.dtype, pin_memory=True)
        self.slots = ExtentAllocator(self.capacity)

    @property
    def page_bytes(self) -> int:
        return self.page_elems * self.k.element_size()


@dataclass
class _Seq:
    maps: List[List[int]]                 # per layer: logical block -> page id, -1 when on the host
    seq_len: int
    state: str = ON_GPU
    slot_of: Dict[int, int] = field(default_factory=dict)   # logical block -> arena slot
    pending_maps: Optional[List[List[int]]] = None
    pending_idx: Optional[List[int]] = None
    event: Optional[torch.cuda.Event] = None


class SequenceOffloader:
    """``offload_sequence_blocks`` / ``prefetch_sequence_blocks`` over a ``PinnedArena``."""

    def __init__(self, pool, arena_pages: int, chunk_pages: int = 256,
                 offload_budget_blocks: Optional[int] = None, prefetch_budget_blocks: Optional[int] = None):
        pool.ensure_allocated()
        self.pool = pool
        self.dev = pool.device
        self.arena = PinnedArena(pool, arena_pages)
        self.chunk = int(chunk_pages)
        self.stream = torch.cuda.Stream(device=self.dev)  # default priority
        shape = (pool.num_layers, self.chunk, pool.B, pool.num_kv_heads, pool.head_dim)
        self.stage_k = torch.empty(shape, dtype=pool.dtype, device=self.dev)
        self.stage_v = torch.empty_like(self.stage_k)
        self._iota = torch.arange(self.chunk, dtype=torch.int32, device=self.dev)
        self.seqs: Dict[int, _Seq] = {}
        self.stats: Dict[str, int] = {}
        # Per-step block budgets (core/offload.py:221-236); None = unlimited.
        self.offload_budget_blocks = offload_budget_blocks
        self.prefetch_budget_blocks = prefetch_budget_blocks
        self._offload_used = 0
        self._prefetch_used = 0

    # ------------------------------------------------------------------ bookkeeping
    def _inc(self, key: str, n: int = 1) -> None:
        self.stats[key] = self.stats.get(key, 0) + n

    def new_step(self) -> None:
        """Reset the per-step budgets."""
        self._offload_used = 0
        self._prefetch_used = 0

    def _consume(self, kind: str, n: int) -> bool:
        budget = self.offload_budget_blocks if kind == "offload" else self.prefetch_budget_blocks
        used = self._offload_used if kind == "offload" else self._prefetch_used
        if budget is not None and used + n > budget:
            return False
        if kind == "offload":
            self._offload_used += n
        else:
            self._prefetch_used += n
        return True

    def add_sequence(self, seq_id: int, gpu_block_map, seq_len: int) -> None:
        """Register a resident sequence: one page list shared by every layer, or one per layer."""
        L = self.pool.num_layers
        if gpu_block_map and isinstance(gpu_block_map[0], (list, tuple)):
            maps = [[int(x) for x in m] for m in gpu_block_map]
            if len(maps) != L or len({len(m) for m in maps}) != 1:
                raise ValueError("one page list per layer, all of one length")
        else:
            maps = [[int(x) for x in gpu_block_map] for _ in range(L)]
        st = _Seq(maps=maps, seq_len=int(seq_len))
        self._update_state(st)
        self.seqs[int(seq_id)] = st

    def gpu_block_map(self, seq_id: int, layer_id: int = 0) -> List[int]:
        return list(self.seqs[int(seq_id)].maps[layer_id])

    def state(self, seq_id: int) -> str:
        return self.seqs[int(seq_id)].state

    def _update_state(self, st: _Seq) -> None:
        """core/offload.py:146-156: by the resident blocks of the (first) layer's map."""
        resident = sum(1 for b in st.maps[0] if b >= 0)
        logical = len(st.maps[0])
        st.state = ON_CPU if resident <= 0 else (ON_GPU if resident >= logical else MIXED)

    def _bytes(self, st: _Seq, idx: Sequence[int]) -> int:
        """core/offload.py:181-187 for every layer: 2 (K, V) x heads x tokens x dim x 2 bytes."""
        B, H, D = self.pool.B, self.pool.num_kv_heads, self.pool.head_dim
        per_layer = sum(2 * H * max(0, min(st.seq_len, i * B + B) - i * B) * D * 2 for i in idx)
        return per_layer * self.pool.num_layers

    # ------------------------------------------------------------------ data path
    def _ids_dev(self, rows: List[List[int]]) -> torch.Tensor:
        ids = torch.tensor(rows, dtype=torch.int32).pin_memory().to(self.dev, non_blocking=True)
        ids.record_stream(self.stream)
        return ids

    def _copy(self, dst: torch.Tensor, dst_pitch: int, src: torch.Tensor, src_pitch: int, width: int) -> None:
        code = _ext.load().ukv_copy_2d(dst, dst_pitch, src, src_pitch, width, self.pool.num_layers,
                                       self.stream.cuda_stream)
        _ext.check(code, "ukv_copy_2d")

    def _move(self, ids: torch.Tensor, slots: List[int], to_host: bool) -> None:
        """Pages ids[:, j] <-> arena slots[j] for every layer, K and V, on the side stream."""
        a, pool = self.arena, self.pool
        pb = a.page_bytes
        host_pitch = a.capacity * pb
        stage_pitch = self.chunk * pb
        for pos, first, count in runs_of(slots):
            for off in range(0, count, self.chunk):
                c = min(self.chunk, count - off)
                cols = ids[:, pos + off:pos + off + c]
                width = c * pb
                if to_host:
                    page_ops.page_copy([pool.k_cache, pool.v_cache], [self.stage_k, self.stage_v], cols,
                                       self._iota[:c])
                for host, stage in ((a.k, self.stage_k), (a.v, self.stage_v)):
                    hp = host.data_ptr() + (first + off) * pb
                    if to_host:
                        self._copy(hp, host_pitch, stage.data_ptr(), stage_pitch, width)
                    else:
                        self._copy(stage.data_ptr(), stage_pitch, hp, host_pitch, width)
                if not to_host:
                    page_ops.page_copy([self.stage_k, self.stage_v], [pool.k_cache, pool.v_cache], self._iota[:c],
                                       cols)

    # ------------------------------------------------------------------ finalize
    def finalize_offload(self, seq_id: int, force_sync: bool = False) -> bool:
        """core/offload.py:362-397: once the copy is done, publish the map and free the GPU pages."""
        st = self.seqs[int(seq_id)]
        if st.state != OFFLOAD_INFLIGHT:
            return True
        if st.event is not None:
            if force_sync:
                st.event.synchronize()
            elif not st.event.query():
                return False
        freed = set()
        for old, new in zip(st.maps, st.pending_maps):
            for o, n in zip(old, new):
                if o >= 0 and n < 0:
                    freed.add(o)
        st.maps, st.pending_maps, st.pending_idx, st.event = st.pending_maps, None, None, None
        self._update_state(st)
        if freed:
            self.pool.free_blocks_by_ids(sorted(freed))
        self._inc("offload_success")
        return True

    def finalize_prefetch(self, seq_id: int, force_sync: bool = False) -> bool:
        """core/offload.py:399-449: once the copy is done, publish the map and drop the host copies."""
        st = self.seqs[int(seq_id)]
        if st.state != PREFETCH_INFLIGHT:
            return st.state == ON_GPU
        if st.event is not None:
            if force_sync:
                st.event.synchronize()
            elif not st.event.query():
                return False
        self.pool.cpu_used_bytes = max(0, self.pool.cpu_used_bytes - self._bytes(st, st.pending_idx))
        st.maps, st.pending_maps, st.pending_idx, st.event = st.pending_maps, None, None, None
        self._update_state(st)
        self._inc("prefetch_success")
        return True

    # ------------------------------------------------------------------ entry points
    def offload_sequence_blocks(self, seq_id: int, logical_block_indices: Sequence[int]) -> bool:
        """core/offload.py:547-599. True when the copy was issued (pages freed at finalize)."""
        self._inc("offload_calls")
        st = self.seqs.get(int(seq_id))
        if st is None:
            self._inc("offload_fail")
            return False
        self.finalize_offload(seq_id)
        self.finalize_prefetch(seq_id)
        if st.state not in (ON_GPU, MIXED):
            self._inc("offload_fail")
            return False
        first = st.maps[0]
        selected = sorted({int(i) for i in logical_block_indices if 0 <= int(i) < len(first) and first[int(i)] >= 0})
        if not selected:
            self._inc("offload_fail")
            return False
        if not self._consume("offload", len(selected)):
            self._inc("offload_fail")
            return False
        need = self._bytes(st, selected)
        if self.pool.cpu_used_bytes + need > self.pool.cpu_budget:
            self._inc("offload_fail")
            return False
        extents = self.arena.slots.alloc(len(selected))
        if extents is None:
            self._inc("offload_fail")
            return False
        slots = [s for start, cnt in extents for s in range(start, start + cnt)]
        rows = [[m[i] for i in selected] for m in st.maps]
        self.stream.wait_stream(torch.cuda.current_stream(self.dev))  # this step's writes land first
        ev = torch.cuda.Event()
        with torch.cuda.stream(self.stream):
            self._move(self._ids_dev(rows), slots, to_host=True)
            ev.record(self.stream)
        pending = [list(m) for m in st.maps]
        for m in pending:
            for i in selected:
                m[i] = -1
        for i, sl in zip(selected, slots):
            st.slot_of[i] = sl
        st.pending_maps, st.pending_idx, st.event, st.state = pending, selected, ev, OFFLOAD_INFLIGHT
        self.pool.cpu_used_bytes += need
        return True

    def prefetch_sequence_blocks(self, seq_id: int, logical_block_indices: Sequence[int]) -> bool:
        """core/offload.py:620-691. True when the blocks are resident (finalized or nothing to do);
        False after issuing a prefetch (call again, or finalize_prefetch, to publish it) or on failure."""
        self._inc("prefetch_calls")
        st = self.seqs.get(int(seq_id))
        if st is None:
            self._inc("prefetch_noop")
            self._inc("prefetch_success")
            return True
        if self.finalize_prefetch(seq_id):
            return True
        if st.state == PREFETCH_INFLIGHT:
            self._inc("prefetch_inflight")
            return False
        if st.state not in (ON_CPU, MIXED):
            self._inc("prefetch_noop")
            self._inc("prefetch_success")
            return True
        first = st.maps[0]
        selected = sorted({int(i) for i in logical_block_indices
                           if 0 <= int(i) < len(first) and first[int(i)] < 0 and int(i) in st.slot_of})
        if not selected:
            self._inc("prefetch_noop")
            self._inc("prefetch_success")
            return True
        if not self._consume("prefetch", len(selected)):
            self._inc("prefetch_fail")
            return False
        block_ids = self.pool.allocate_blocks(len(selected))
        if len(block_ids) != len(selected):
            if block_ids:
                self.pool.free_blocks_by_ids(block_ids)
            self._inc("prefetch_fail")
            return False
        slots = [st.slot_of.pop(i) for i in selected]
        rows = [list(block_ids) for _ in range(self.pool.num_layers)]  # one new id per block, every layer
        self.stream.wait_stream(torch.cuda.current_stream(self.dev))  # earlier users of these pages are done
        ev = torch.cuda.Event()
        with torch.cuda.stream(self.stream):
            self._move(self._ids_dev(rows), slots, to_host=False)
            ev.record(self.stream)
        # Later arena writes run on the same stream, after these reads: the slots are free now.
        self.arena.slots.free([(s, n) for _, s, n in runs_of(sorted(slots))])
        pending = [list(m) for m in st.maps]
        for m in pending:
            for i, bid in zip(selected, block_ids):
                m[i] = int(bid)
        st.pending_maps, st.pending_idx, st.event, st.state = pending, selected, ev, PREFETCH_INFLIGHT
        return False

    def offload_sequence(self, seq_id: int) -> bool:
        """Every block of the sequence (core/offload.py:601-618)."""
        st = self.seqs.get(int(seq_id))
        if st is None or not st.maps[0]:
            self._inc("offload_fail")
            return False
        if self.offload_sequence_blocks(seq_id, range(len(st.maps[0]))):
            return True
        if st.state == OFFLOAD_INFLIGHT:
            return True
        return self.finalize_offload(seq_id)

    def prefetch_sequence(self, seq_id: int) -> bool:
        st = self.seqs.get(int(seq_id))
        if st is None:
            self._inc("prefetch_noop")
            self._inc("prefetch_success")
            return True
        return self.prefetch_sequence_blocks(seq_id, range(len(st.maps[0])))

    def wait(self, seq_id: int) -> None:
        """Make the current stream wait for the sequence's in-flight copy (no host wait)."""
        st = self.seqs[int(seq_id)]
        if st.event is not None:
            torch.cuda.current_stream(self.dev).wait_event(st.event)


__all__ = ["ExtentAllocator", "PinnedArena", "SequenceOffloader", "runs_of", "ON_GPU", "MIXED", "ON_CPU",
           "OFFLOAD_INFLIGHT", "PREFETCH_INFLIGHT"]
