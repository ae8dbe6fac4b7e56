"""TEST INFRASTRUCTURE ONLY - CPU restatement of the paged pool's integer and copy semantics.

Only tests/ may import this module. Each function follows the cited lines of BP-KV:

* ``FifoAllocator``        core/pool.py:51-58, 96-125 (free list, allocate first n, free appends)
* ``write_kv_to_blocks``   core/pool.py:127-141 (page i gets tokens 16i .. min(16i+16, T))
* ``read_kv_from_blocks``  core/pool.py:154-172
* ``build_block_table``    core/pool.py:174-189 (zero padded int32 [B, max_len])
* ``kv_append``            core/scheduler.py:401-408 (token at len -> page bt[b, len//16], slot len%16)
* ``reserve_decode_slots`` core/offload.py:838-866 per sequence in batch order (core/scheduler.py:1101-1104):
                           len % 16 == 0 -> one FIFO page appended to the sequence's block list
* ``prefill_chunk_pages``  pages for a prefill chunk written straight into the pool: each sequence
                           takes the FIFO pages its new length needs, in batch order (the pool-side
                           replacement of register / writeback, core/offload.py:451-470, core/pool.py:127-141)
* ``decode_steps``         the page16_native decode loop: reserve, per layer table + append + attention
                           over old_len + 1 (core/scheduler.py:1092-1160, 401-418), commit (1247-1265)
* ``pool_size``            core/pool.py:36-45 (N_total from free memory)

Caches here are numpy arrays [N, 16, H, D] of one layer (any dtype; the copies are bit-exact).
"""
from __future__ import annotations

from typing import List

import numpy as np


class FifoAllocator:
    def __init__(self, n_total: int):
        self.N_total = n_total
        self.free_blocks: List[int] = list(range(n_total))
        self.used_blocks = {}
        self.N_wm_low = max(1, int(0.15 * n_total))
        self.N_wm_high = max(2, int(0.40 * n_total))

    @property
    def n_free(self) -> int:
        return len(self.free_blocks)

    def allocate_blocks(self, n: int) -> List[int]:
        if len(self.free_blocks) < n:
            return []
        ids = self.free_blocks[:n]
        self.free_blocks = self.free_blocks[n:]
        for bid in ids:
            self.used_blocks[bid] = 1
        return ids

    def free_blocks_by_ids(self, block_ids):
        for bid in block_ids:
            if bid in self.used_blocks:
                del self.used_blocks[bid]
            self.free_blocks.append(bid)

    def check_watermark(self, n_required: int) -> str:
        n = len(self.free_blocks)
        if n < n_required:
            return "VRAM_FULL"
        if n < self.N_wm_high:
            return "WARNING"
        return "OK"


def pool_size(total_bytes: int, used_bytes: int, gpu_mem_frac: float, num_layers: int, block_size: int,
              num_kv_heads: int, head_dim: int) -> int:
    reserve = int(0.10 * total_bytes)
    available = total_bytes - used_bytes - reserve
    max_kv_mem = int(available * gpu_mem_frac)
    bytes_per_block = 2 * num_layers * block_size * num_kv_heads * head_dim * 2
    return max(1, int(max_kv_mem / bytes_per_block))


def write_kv_to_blocks(cache: np.ndarray, block_ids, K: np.ndarray) -> None:
    """cache [N, 16, H, D] (one layer); K [H, T, D]."""
    seq_len = K.shape[1]
    for i, bid in enumerate(block_ids):
        start = i * 16
        end = min(start + 16, seq_len)
        chunk = end - start
        if chunk > 0:
            cache[bid, :chunk] = K[:, start:end].transpose(1, 0, 2)


def read_kv_from_blocks(cache: np.ndarray, block_ids, seq_len: int) -> np.ndarray:
    chunks = []
    for i, bid in enumerate(block_ids):
        start = i * 16
        end = min(start + 16, seq_len)
        chunk = end - start
        if chunk > 0:
            chunks.append(cache[bid, :chunk].transpose(1, 0, 2))
    if not chunks:
        return np.empty((cache.shape[2], 0, cache.shape[3]), dtype=cache.dtype)
    return np.concatenate(chunks, axis=1)


def build_block_table(seq_block_ids_list) -> np.ndarray:
    batch = len(seq_block_ids_list)
    max_blocks = max(len(ids) for ids in seq_block_ids_list)
    bt = np.zeros((batch, max_blocks), dtype=np.int32)
    for i, ids in enumerate(seq_block_ids_list):
        if ids:
            bt[i, : len(ids)] = np.asarray(ids, dtype=np.int32)
    return bt


def kv_append(k_cache: np.ndarray, v_cache: np.ndarray, block_table: np.ndarray, old_lens: np.ndarray,
              k_new: np.ndarray, v_new: np.ndarray, block_size: int = 16) -> np.ndarray:
    """k_new / v_new [B, H, D]; returns attn_lens = old_lens + 1."""
    B = block_table.shape[0]
    block_pos = old_lens.astype(np.int64) // block_size
    tok_pos = old_lens.astype(np.int64) % block_size
    block_ids = block_table[np.arange(B), block_pos]
    k_cache[block_ids.astype(np.int64), tok_pos] = k_new
    v_cache[block_ids.astype(np.int64), tok_pos] = v_new
    return (old_lens + 1).astype(np.int32)


def reserve_decode_slots(allocator, page_lists, seq_lens, block_size: int = 16):
    """Returns the page given to each sequence this step (None where none was needed); page_lists
    are extended in place. Raises like the reference with no page to evict."""
    got = []
    for i, L in enumerate(seq_lens):
        if int(L) % block_size == 0:
            new_ids = allocator.allocate_blocks(1)
            if not new_ids:
                raise RuntimeError("page16_native_blocked:direct_decode_expand_evict_failed")
            page_lists[i].extend(new_ids)
            got.append(int(new_ids[0]))
        else:
            got.append(None)
    return got


def decode_steps(allocator, k_pool, v_pool, page_lists, seq_lens, tokens, attend, block_size: int = 16):
    """k_pool / v_pool: per-layer lists of [N, 16, H, D] arrays (modified in place);
    tokens[step][layer] = (q, k_new, v_new) with k_new / v_new [B, H, D];
    attend(layer, q, block_table, attn_lens) -> output. Returns (outputs[step][layer], seq_lens)."""
    lens = np.asarray(seq_lens, dtype=np.int32).copy()
    outs = []
    for step_tokens in tokens:
        reserve_decode_slots(allocator, page_lists, lens, block_size)
        bt = build_block_table(page_lists)
        row = []
        for layer, (q, k_new, v_new) in enumerate(step_tokens):
            attn_lens = kv_append(k_pool[layer], v_pool[layer], bt, lens, k_new, v_new, block_size)
            row.append(attend(layer, q, bt, attn_lens))
        outs.append(row)
        lens = lens + 1
    return outs, lens


def prefill_chunk_pages(allocator, page_lists, seq_lens, chunk_lens, block_size: int = 16):
    """Extends page_lists in place; returns the ids each sequence took (empty lists where none)."""
    need = [max(0, -(-(int(L) + int(c)) // block_size) - len(ids)) for L, c, ids in zip(seq_lens, chunk_lens,
                                                                                          page_lists)]
    if sum(need) > allocator.n_free:
        raise RuntimeError("prefill_pages_alloc_failed")
    took = []
    for ids, n in zip(page_lists, need):
        got = allocator.allocate_blocks(n) if n else []
        ids.extend(got)
        took.append(got)
    return took
