"""Device-resident decode step over the paged pool (the fused decode prologue).

What BP-KV does for one page16_native decode step, all on the host:

* ``reserve_decode_slot`` per sequence, in batch order (core/offload.py:780-866,
  called from core/scheduler.py:1101-1104): when ``seq_len % B == 0`` it allocates
  one page (FIFO) and appends it to the block list of every layer of the sequence;
* per layer, ``build_block_table`` with one host-to-device copy per row
  (core/pool.py:174-189) and a ``cache_seqlens`` tensor
  (core/scheduler.py:1106-1160): 32 layers x B rows of small copies per step;
* per layer, ``block_pos = old_lens // B``, ``tok_pos = old_lens % B``, two
  ``index_put_`` of the new K/V row, ``attn_lens = old_lens + 1`` and the decode
  call (core/scheduler.py:401-418);
* ``commit_paged_direct_decode``: ``seq_len += 1`` for every (sequence, layer)
  (core/scheduler.py:1247-1265).

``DecodeBatch`` keeps the block table and the lengths on the device for the
life of the batch. ``begin_step`` allocates the step's new pages on the host in
the reference's order (so every page id is the reference's) and hands them to
one prologue kernel (``ukv_decode_prologue``) that writes them into the table
and produces the attention lengths; that kernel is the only per-step
host-to-device traffic (the page ids ride in its arguments). The table and
lengths serve every layer. ``attention`` appends the layer's token rows
(``ukv_kv_append``) and attends (``ukv_page16_decode``); with
``fused_append=True`` it is one fused call per layer
(``ukv_page16_decode_append``), which measured under 1 % faster over a
32-layer step and relies on no sequence attending another's page - guaranteed
here by the checks at construction (distinct pages, lists covering their
lengths). ``end_step`` commits the host copy of the lengths. No call
synchronises with the device.
"""
from __future__ import annotations

import ctypes
from typing import Callable, Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

from . import _ext, page16_native, page_ops
from .pool import PagedKVPool, pack_block_table

_TABLE_ALIGN = 64  # table width granularity in pages (1024 tokens)


def plan_decode_pages(allocate: Callable[[int], List[int]], page_lists: List[List[int]], seq_lens: Sequence[int],
                      block_size: int, seq_ids: Optional[Sequence[int]] = None,
                      on_pool_full: Optional[Callable[[int], bool]] = None) -> List[Tuple[int, int, int]]:
    """The allocation side of ``reserve_decode_slot`` for a batch (core/offload.py:838-866).

    For each sequence i in order: when ``seq_lens[i] % block_size == 0`` one page is
    allocated with ``allocate(1)`` and appended to ``page_lists[i]`` (in place), giving the
    triple ``(i, column, page id)`` with column = the list length before the append. When
    the pool has no free page, ``on_pool_full(seq_id)`` may free some (the reference's
    ``_evict_until_free``); without it, or when it returns False, the step fails with
    ``page16_native_blocked:direct_decode_expand_evict_failed``, and with
    ``...:direct_decode_expand_alloc_failed`` when the retry finds no page either. As in the
    reference, pages given to earlier sequences of the batch stay with them when a later one
    fails; the triples of those pages are attached to the raised error as ``.triples``.
    """
    triples: List[Tuple[int, int, int]] = []
    for i, L in enumerate(seq_lens):
        if int(L) % block_size != 0:
            continue
        ids = allocate(1)
        if not ids:
            sid = int(seq_ids[i]) if seq_ids is not None else i
            reason = "direct_decode_expand_evict_failed"
            if on_pool_full is not None and on_pool_full(sid):
                ids = allocate(1)
                reason = "direct_decode_expand_alloc_failed"
            if not ids:
                err = RuntimeError(f"page16_native_blocked:{reason}")
                err.triples = triples
                raise err
        col = len(page_lists[i])
        page_lists[i].append(int(ids[0]))
        triples.append((i, col, int(ids[0])))
    return triples


class DecodeBatch:
    """A batch of sequences decoding over ``pool``: device block table + lengths, fused steps.

    ``seq_page_lists[i]`` is sequence i's page list (its ``gpu_block_map``, shared by all
    layers) and ``seq_lens[i]`` its current length. The lists are owned by the batch from
    here on (``page_lists`` returns them).

    Streams: the device table and lengths are written on the stream current at construction
    and at each ``begin_step`` and read on the stream current at each layer call; a caller that
    runs the calls of one batch on several streams orders them itself (``wait_stream``).
    """

    def __init__(self, pool: PagedKVPool, seq_page_lists: Sequence[Sequence[int]], seq_lens: Sequence[int], *,
                 seq_ids: Optional[Sequence[int]] = None, capacity_blocks: Optional[int] = None,
                 on_pool_full: Optional[Callable[[int], bool]] = None, fused_append: bool = False):
        if len(seq_page_lists) == 0:
            raise RuntimeError("page16_native_empty_batch")
        if len(seq_lens) != len(seq_page_lists):
            raise ValueError("seq_lens and seq_page_lists differ in length")
        self.pool = pool
        self.seq_ids = [int(s) for s in seq_ids] if seq_ids is not None else list(range(len(seq_page_lists)))
        self._lists = [[int(x) for x in ids] for ids in seq_page_lists]
        self._lens = [int(x) for x in seq_lens]
        for sid, ids, L in zip(self.seq_ids, self._lists, self._lens):
            # The resident checks of core/offload.py:797-830, same reasons.
            if any(x < 0 for x in ids):
                raise RuntimeError(f"page16_native_blocked:direct_decode_resident_missing seq={sid}")
            if not ids:
                raise RuntimeError(f"page16_native_blocked:direct_decode_no_gpu_blocks seq={sid}")
            if any(x >= pool.N_total for x in ids):
                raise ValueError(f"page id outside the pool for seq={sid}")
            if L < 0:
                raise ValueError(f"negative length for seq={sid}")
            if -(-L // pool.B) > len(ids):
                # The device table is zero padded: a length past its list would attend page 0
                # (another sequence's page) and the fused append would write into it.
                raise ValueError(f"seq={sid}: length {L} needs {-(-L // pool.B)} pages, its list holds {len(ids)}")
        owned = [x for ids in self._lists for x in ids]
        if len(set(owned)) != len(owned):
            # A page in two sequences' lists would be attended by one while the other appends to it.
            raise ValueError("a page appears in more than one sequence's list")
        self.on_pool_full = on_pool_full
        self.fused_append = bool(fused_append)
        pool.ensure_allocated()
        self.device = pool.device
        self.batch = len(self._lists)
        want = max(max(len(ids) for ids in self._lists) + 1, int(capacity_blocks or 0))
        width = -(-want // _TABLE_ALIGN) * _TABLE_ALIGN
        packed = pack_block_table(self._lists)
        host = np.zeros((self.batch, width), dtype=np.int32)
        host[:, : packed.shape[1]] = packed
        self._table = torch.from_numpy(host).pin_memory().to(self.device, non_blocking=True)
        lens = torch.tensor(self._lens, dtype=torch.int32).pin_memory().to(self.device, non_blocking=True)
        self._lens_dev = [lens, torch.empty_like(lens)]  # [old lengths, attention lengths] of a step
        self._cur = 0
        self._open = False
        self._table_version = 0

    # ------------------------------------------------------------------ state
    @property
    def block_table(self) -> torch.Tensor:
        """int32 [batch, width] device table (zero padded), shared by every layer."""
        return self._table

    @property
    def cache_seqlens(self) -> torch.Tensor:
        """int32 [batch] device lengths before the current step's token (the reference's cache_seqlens)."""
        return self._lens_dev[self._cur]

    @property
    def attn_lens(self) -> torch.Tensor:
        """int32 [batch] device lengths including the step's token (valid between begin_step and end_step)."""
        if not self._open:
            raise RuntimeError("decode_step_not_open")
        return self._lens_dev[self._cur ^ 1]

    @property
    def step_parity(self) -> int:
        """0 or 1: which of the two device length buffers holds the lengths before this step. The
        per-layer calls of an open step read the table, those lengths and the other buffer's; a
        HIP graph captured from them replays correctly at steps of the same parity while
        ``table_version`` is unchanged."""
        return self._cur

    @property
    def table_version(self) -> int:
        """Counts the reallocations of the device table (a step whose new page lies past its
        width; ``capacity_blocks`` sizes it ahead). Graphs captured from the per-layer calls read
        the table they were captured with and must be captured again when this changes."""
        return self._table_version

    @property
    def seq_lens(self) -> List[int]:
        return list(self._lens)

    @property
    def page_lists(self) -> List[List[int]]:
        return self._lists

    # ------------------------------------------------------------------- step
    def begin_step(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """Reserve the step's pages and launch the prologue; returns (block_table, attn_lens)."""
        if self._open:
            raise RuntimeError("decode_step_already_open")
        B = self.pool.B
        for sid, ids, L in zip(self.seq_ids, self._lists, self._lens):
            # page_lists hands out the lists themselves: re-check that each still covers its
            # length (the planner then adds the page a length L % B == 0 needs for its token).
            if -(-L // B) > len(ids):
                raise RuntimeError(f"page16_native_blocked:direct_decode_slot_missing seq={sid}")
        try:
            triples = plan_decode_pages(self.pool.allocate_blocks, self._lists, self._lens, self.pool.B,
                                        self.seq_ids, self.on_pool_full)
        except RuntimeError as err:
            # Pages already given to earlier sequences stay theirs (as in the reference):
            # put them in the device table, leave the lengths as they are.
            done = getattr(err, "triples", [])
            if done:
                self._launch(done, lens=False)
            raise
        self._launch(triples, lens=True)
        self._open = True
        return self._table, self._lens_dev[self._cur ^ 1]

    def attention(self, layer_id: int, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, *,
                  softmax_scale: float, n_rep: int) -> torch.Tensor:
        """Append the step's K/V rows of ``layer_id`` and attend (core/scheduler.py:401-418)."""
        if not self._open:
            raise RuntimeError("decode_step_not_open")
        k_layer, v_layer = self.pool.k_cache[layer_id], self.pool.v_cache[layer_id]
        attn_lens = self._lens_dev[self._cur ^ 1]
        if self.fused_append:
            return page16_native.page16_decode_append_attention(
                q, k_layer, v_layer, self._table, attn_lens, k_new, v_new, softmax_scale=softmax_scale, n_rep=n_rep)
        self.append(layer_id, k_new, v_new)
        return page16_native.page16_decode_attention(q, k_layer, v_layer, self._table, attn_lens,
                                                     softmax_scale=softmax_scale, n_rep=n_rep)

    def append(self, layer_id: int, k_new: torch.Tensor, v_new: torch.Tensor) -> None:
        """Only the append of ``layer_id`` (for callers that run their own attention)."""
        if not self._open:
            raise RuntimeError("decode_step_not_open")
        pool = self.pool
        page_ops.kv_append(pool.k_cache[layer_id], pool.v_cache[layer_id], self._table, self._lens_dev[self._cur],
                           pool._as_pool_rows(k_new), pool._as_pool_rows(v_new), return_new_lens=False)

    def end_step(self) -> None:
        """Commit: every length grows by one (core/scheduler.py:1247-1265)."""
        if not self._open:
            raise RuntimeError("decode_step_not_open")
        self._lens = [L + 1 for L in self._lens]
        self._cur ^= 1
        self._open = False

    def context(self) -> Dict[str, object]:
        """The dict ``prepare_page16_native_context`` returns (core/scheduler.py:1150-1160), for
        callers that index it; every layer view shares the one device table."""
        views = {lid: {"k_cache": self.pool.k_cache[lid], "v_cache": self.pool.v_cache[lid],
                       "block_table": self._table} for lid in range(self.pool.num_layers)}
        return {
            "backend": "page16_native",
            "seq_ids": list(self.seq_ids),
            "seq_lens": list(self._lens),
            "logical_seq_lens": list(self._lens),
            "cache_seqlens": self.cache_seqlens,
            "layer_views": views,
            "resident_missing_blocks": 0,
            "materialized_blocks": int(self._table.numel()) * self.pool.num_layers,
        }

    # --------------------------------------------------------------- internal
    def _grow(self, need_cols: int) -> None:
        width = int(self._table.shape[1])
        new_w = max(2 * width, -(-need_cols // _TABLE_ALIGN) * _TABLE_ALIGN)
        table = torch.zeros((self.batch, new_w), dtype=torch.int32, device=self.device)
        table[:, :width].copy_(self._table)
        self._table = table
        self._table_version += 1

    def _launch(self, triples: List[Tuple[int, int, int]], lens: bool) -> None:
        if triples:
            need = max(c for _, c, _ in triples) + 1
            if need > int(self._table.shape[1]):
                self._grow(need)
        flat = (ctypes.c_int32 * (3 * len(triples) or 1))(*[v for t in triples for v in t])
        lens_in = self._lens_dev[self._cur]
        lens_out = self._lens_dev[self._cur ^ 1] if lens else None
        stream = torch.cuda.current_stream(self.device).cuda_stream
        code = _ext.load().ukv_decode_prologue(
            self._table.data_ptr(), int(self._table.shape[1]), self.batch, lens_in.data_ptr(),
            lens_out.data_ptr() if lens_out is not None else None, flat, len(triples), stream)
        _ext.check(code, "ukv_decode_prologue")


__all__ = ["DecodeBatch", "plan_decode_pages"]
