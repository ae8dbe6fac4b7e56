"""Drop-in ``PagedKVPool`` for MI355X (core/pool.py of BP-KV).

Same constructor, attributes and methods as core/pool.py:7-189, same layout
``[num_layers, N_total, block_size, num_kv_heads, head_dim]`` per K and V,
same FIFO allocation order (it decides the page ids of every later block
table, so it is kept bit-exact), same sizing formula. What changes:

* token I/O (``write_kv_to_blocks`` / ``read_kv_from_blocks``) is one gfx950
  scatter / gather kernel per call instead of a Python loop of per-page
  transposed slices (core/pool.py:134-141, 160-172);
* ``build_block_table`` packs all rows on the host and uploads them with one
  pinned H2D copy instead of one copy per row (core/pool.py:181-188), and
  reuses the device table while the page lists are unchanged - the scheduler
  asks for the same lists once per layer (core/scheduler.py:1109-1146);
* the free list is a deque (O(n) in the pages moved, not in the pool size).

Extra entry points used by the fused decode prologue and by compaction:
``block_table_for``, ``append_decode_tokens``, ``copy_pages``.
"""
from __future__ import annotations

import threading
from collections import deque
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

from . import page_ops
from .page16_native import _current_stream


def pack_block_table(seq_block_ids_list: Sequence[Sequence[int]]) -> np.ndarray:
    """Host int32 [batch, max_len], row i = the page ids of sequence i, zero padded (core/pool.py:179-188)."""
    batch = len(seq_block_ids_list)
    max_blocks = max(len(ids) for ids in seq_block_ids_list)
    host = np.zeros((batch, max_blocks), dtype=np.int32)
    for i, ids in enumerate(seq_block_ids_list):
        if len(ids):
            host[i, : len(ids)] = ids
    return host


class PagedKVPool:
    """Paged KV storage: k_cache / v_cache [num_layers, N_total, B, h_kv, d]; tables pad with 0."""

    def __init__(
        self,
        block_size: int,
        num_layers: int,
        num_kv_heads: int,
        head_dim: int,
        dtype: torch.dtype = torch.float16,
        gpu_mem_frac: float = 0.75,
        cpu_mem_gb: float = 48.0,
        *,
        num_blocks: Optional[int] = None,
        device=None,
    ):
        self.B = block_size
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self.device = torch.device(device) if device is not None else torch.device("cuda", 0)

        if num_blocks is None:
            # core/pool.py:36-45: a fraction of (total - allocated - 10 % reserve), 2 bytes per element.
            total_gpu = torch.cuda.get_device_properties(self.device).total_memory
            model_used = torch.cuda.memory_allocated(self.device)
            reserve = int(0.10 * total_gpu)
            available = total_gpu - model_used - reserve
            max_kv_mem = int(available * gpu_mem_frac)
            bytes_per_block = 2 * num_layers * block_size * num_kv_heads * head_dim * 2
            self.N_total = max(1, int(max_kv_mem / bytes_per_block))
        else:
            self.N_total = max(1, int(num_blocks))

        self._k_cache: Optional[torch.Tensor] = None
        self._v_cache: Optional[torch.Tensor] = None

        self.lock = threading.Lock()
        self._free = deque(range(self.N_total))
        self.used_blocks: Dict[int, int] = {}

        self.cpu_budget = int(cpu_mem_gb * 1024**3)
        self.cpu_used_bytes = 0

        self.N_wm_low = max(1, int(0.15 * self.N_total))
        self.N_wm_high = max(2, int(0.40 * self.N_total))

        # The last block table uploaded (page lists, stream, device table).
        self._table_cache: Optional[Tuple[List[List[int]], int, torch.Tensor]] = None
        # The last id list token I/O uploaded (list, stream, device ids): callers pass the same
        # list once per layer.
        self._ids_cache: Optional[Tuple[List[int], int, torch.Tensor]] = None

    # ------------------------------------------------------------------ storage
    @property
    def is_allocated(self) -> bool:
        return self._k_cache is not None and self._v_cache is not None

    def ensure_allocated(self) -> None:
        if self.is_allocated:
            return
        shape = (self.num_layers, self.N_total, self.B, self.num_kv_heads, self.head_dim)
        self._k_cache = torch.zeros(shape, dtype=self.dtype, device=self.device)
        self._v_cache = torch.zeros_like(self._k_cache)

    @property
    def k_cache(self) -> torch.Tensor:
        self.ensure_allocated()
        assert self._k_cache is not None
        return self._k_cache

    @property
    def v_cache(self) -> torch.Tensor:
        self.ensure_allocated()
        assert self._v_cache is not None
        return self._v_cache

    def release_if_empty(self) -> bool:
        with self.lock:
            empty = len(self.used_blocks) == 0
        if not empty or not self.is_allocated:
            return False
        self._k_cache = None
        self._v_cache = None
        self._table_cache = None
        self._ids_cache = None
        if torch.cuda.is_available():
            torch.cuda.empty_cache()
        return True

    # --------------------------------------------------------------- allocation
    @property
    def free_blocks(self) -> List[int]:
        """The free list in allocation order (a copy)."""
        with self.lock:
            return list(self._free)

    @property
    def n_free(self) -> int:
        with self.lock:
            return len(self._free)

    def allocate_blocks(self, n: int) -> List[int]:
        """First n free ids in FIFO order, or [] when fewer than n are free (core/pool.py:101-109)."""
        with self.lock:
            if len(self._free) < n:
                return []
            if n < 0:  # list-slice semantics of the reference: free[:n]
                keep = -n
                ids = [self._free.popleft() for _ in range(len(self._free) - keep)]
            else:
                ids = [self._free.popleft() for _ in range(n)]
            for bid in ids:
                self.used_blocks[bid] = 1
            return ids

    def free_blocks_by_ids(self, block_ids: List[int]):
        """Appends every id to the free list, in order (core/pool.py:111-116)."""
        with self.lock:
            for bid in block_ids:
                if bid in self.used_blocks:
                    del self.used_blocks[bid]
                self._free.append(bid)

    def check_watermark(self, n_required: int) -> str:
        with self.lock:
            n = len(self._free)
        if n < n_required:
            return "VRAM_FULL"
        if n < self.N_wm_high:
            return "WARNING"
        return "OK"

    # ---------------------------------------------------------------- token I/O
    def _as_pool_rows(self, X: torch.Tensor) -> torch.Tensor:
        if X.device != self.device or X.dtype != self.dtype:
            X = X.to(device=self.device, dtype=self.dtype)
        if X.stride(-1) != 1:
            X = X.contiguous()
        return X

    def _device_ids(self, block_ids) -> torch.Tensor:
        """int32 device copy of block_ids, reused while the caller passes an equal list on the same
        stream (the exact list compare costs ~1 % of a pinned upload). The copy is ordered on the
        stream it was uploaded on, so a call on another stream uploads its own; list, stream and
        tensor are kept as one tuple, so a concurrent caller never pairs one list with another's ids."""
        ids = [int(x) for x in block_ids] if not isinstance(block_ids, list) else block_ids
        stream = _current_stream(self.device)
        cached = self._ids_cache
        if cached is not None and cached[1] == stream and cached[0] == ids:
            return cached[2]
        dev = torch.tensor(ids, dtype=torch.int32).pin_memory().to(self.device, non_blocking=True)
        self._ids_cache = (list(ids), stream, dev)
        return dev

    def write_kv_to_blocks(self, layer_id: int, block_ids: List[int], K: torch.Tensor, V: torch.Tensor):
        """K/V [h_kv, T, d]: token t -> page block_ids[t // B], slot t % B (core/pool.py:127-141)."""
        n = min(int(K.shape[1]), self.B * len(block_ids))
        if n <= 0:
            return
        ids = self._device_ids(block_ids)
        page_ops.scatter_tokens(self.k_cache[layer_id], ids, self._as_pool_rows(K), n)
        page_ops.scatter_tokens(self.v_cache[layer_id], ids, self._as_pool_rows(V), n)

    def write_one_token(self, layer_id: int, block_id: int, pos_in_block: int, k_tok: torch.Tensor,
                        v_tok: torch.Tensor):
        self.k_cache[layer_id, block_id, pos_in_block] = k_tok.squeeze(1)
        self.v_cache[layer_id, block_id, pos_in_block] = v_tok.squeeze(1)

    def read_kv_from_blocks(self, layer_id: int, block_ids: List[int], seq_len: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """[h_kv, min(seq_len, B * len(block_ids)), d] K and V (core/pool.py:154-172)."""
        n = max(0, min(int(seq_len), self.B * len(block_ids)))
        if n == 0:
            K = torch.empty(self.num_kv_heads, 0, self.head_dim, dtype=self.dtype, device=self.device)
            return K, torch.empty_like(K)
        ids = self._device_ids(block_ids)
        return (page_ops.gather_tokens(self.k_cache[layer_id], ids, n),
                page_ops.gather_tokens(self.v_cache[layer_id], ids, n))

    # ------------------------------------------------------------- block tables
    def block_table_for(self, seq_block_ids_list: Sequence[Sequence[int]]) -> torch.Tensor:
        """Zero-padded int32 [batch, max_len] device table; one pinned H2D copy, reused while unchanged
        and asked for on the stream it was uploaded on (the copy is ordered on that stream only)."""
        cacheable = isinstance(seq_block_ids_list, list) and all(isinstance(x, list) for x in seq_block_ids_list)
        stream = _current_stream(self.device)
        cached = self._table_cache
        if cacheable and cached is not None and cached[1] == stream and cached[0] == seq_block_ids_list:
            return cached[2]
        host = pack_block_table(seq_block_ids_list)
        table = torch.from_numpy(host).pin_memory().to(self.device, non_blocking=True)
        # list, stream and table as one tuple: a concurrent caller never pairs one with another's
        self._table_cache = ([list(ids) for ids in seq_block_ids_list], stream, table) if cacheable else None
        return table

    def build_block_table(self, layer_id: int, seq_block_ids_list: List[List[int]]
                          ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """(k_cache[layer], v_cache[layer], int32 [batch, max_blocks]) as core/pool.py:174-189.

        The returned table may be shared by several layers (the page lists are shared by all
        layers of a sequence); callers treat it as read-only, as the reference's callers do.
        """
        table = self.block_table_for(seq_block_ids_list)
        return self.k_cache[layer_id], self.v_cache[layer_id], table

    # ------------------------------------------------------------ fused helpers
    def append_decode_tokens(self, layer_id: int, block_table: torch.Tensor, old_lens: torch.Tensor,
                             k_new: torch.Tensor, v_new: torch.Tensor) -> torch.Tensor:
        """One kernel for core/scheduler.py:401-408: token b goes to page block_table[b, len//B],
        slot len % B; returns the attention lengths old_lens + 1."""
        return page_ops.kv_append(self.k_cache[layer_id], self.v_cache[layer_id], block_table, old_lens,
                                  self._as_pool_rows(k_new), self._as_pool_rows(v_new))

    def copy_pages(self, src_ids, dst_ids) -> None:
        """pool[l, dst_ids(l)[j]] = pool[l, src_ids(l)[j]] for K and V of every layer l.

        Id lists are int32 [n] (shared by all layers) or [num_layers, n] (per layer); destination
        pages must not be source pages of the same call."""
        k, v = self.k_cache, self.v_cache
        page_ops.page_copy([k, v], [k, v], src_ids, dst_ids)
