"""TEST INFRASTRUCTURE ONLY - CPU restatement of block compression's budget, selection and gather.

Only tests/ may import this module. Each function follows the cited BP-KV lines:

* ``selection_budget``   core/scheduler.py:547-563
* ``snapkv_arithmetic``  core/compress.py:75-94, 99-114, 133-145 (segment split, alignment, k, L_final)
* ``select_topk``        core/scheduler.py:613-616 (topk then sorted); ties broken toward the lower
                         index (the reference's torch.topk leaves them unspecified)
* ``retained_pages``     core/scheduler.py:762-779 (sink blocks, Ls/B + selected, obs blocks)
* ``compact``            core/scheduler.py:805-878 + 702-733: per sequence FIFO destination pages,
                         per layer ``pool[l, dst[j]] = pool[l, table[keep_l[j]]]``
* ``write_piece_to_blocks``      core/scheduler.py:666-690 (token-granular write at a page offset)
* ``pad_piece_to_block``         core/scheduler.py:692-700 (zero rows up to one block)
* ``write_block_indexed_layer``  core/scheduler.py:702-733 (aligned fast path, with its bail-outs)
* ``write_selected_layer``       core/scheduler.py:735-799 (pass-through modes, the aligned fast
                                 path, else sink / padded middle blocks / window as pieces)
* ``selected_writeback``         core/scheduler.py:805-878 (FIFO pages for ceil(max(1, eff)/B) blocks,
                                 every layer written, the pages freed again when a write fails)
* ``prune_copy``                 core/offload.py:1236-1262 (new FIFO pages for the kept blocks'
                                 tokens, every layer read, concatenated and written, old ids freed)
* ``compress_tensors``           core/compress.py:99-175 (the tensor result of BlockAlignedSnapKV:
                                 F.pad of the middle, gather of whole blocks, cat with sink and window)
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


# --------------------------------------------------------------- selected writeback (dense raw KV)
def write_piece_to_blocks(k_cache, v_cache, block_ids, dst_offset, K_piece, V_piece, B=16):
    """k_cache / v_cache one layer [N, B, H, D]; pieces [H, T, D]; returns the next position."""
    if K_piece.shape[1] != V_piece.shape[1]:
        raise RuntimeError("selected_writeback_piece_len_mismatch")
    total = int(K_piece.shape[1])
    src, pos = 0, int(dst_offset)
    while src < total:
        block_idx, off = pos // B, pos % B
        if block_idx >= len(block_ids):
            raise RuntimeError("selected_writeback_block_overflow")
        take = min(total - src, B - off)
        bid = int(block_ids[block_idx])
        k_cache[bid, off:off + take] = K_piece[:, src:src + take, :].transpose(1, 0, 2)
        v_cache[bid, off:off + take] = V_piece[:, src:src + take, :].transpose(1, 0, 2)
        src += take
        pos += take
    return pos


def pad_piece_to_block(K_piece, V_piece, B=16):
    missing = B - int(K_piece.shape[1])
    if missing <= 0:
        return K_piece, V_piece
    pad = np.zeros((K_piece.shape[0], missing, K_piece.shape[2]), dtype=K_piece.dtype)
    return np.concatenate([K_piece, pad], axis=1), np.concatenate([V_piece, pad.astype(V_piece.dtype)], axis=1)


def write_block_indexed_layer(k_cache, v_cache, block_ids, K, V, source_block_indices, B=16):
    """One K and one V scatter of whole source blocks; False where the reference bails out."""
    if not source_block_indices or len(source_block_indices) != len(block_ids):
        return False
    if K.shape[1] % B != 0 or V.shape[1] % B != 0:
        return False
    raw_blocks = K.shape[1] // B
    max_src = max(int(x) for x in source_block_indices)
    if max_src < 0 or max_src >= raw_blocks:
        return False
    idx = np.asarray([int(x) for x in source_block_indices], dtype=np.int64)
    if (idx < 0).any():  # torch's index_select rejects negative indices
        raise IndexError("index out of range in self")
    Kb = K.reshape(K.shape[0], raw_blocks, B, K.shape[2])[:, idx].transpose(1, 2, 0, 3)  # [n, B, H, D]
    Vb = V.reshape(V.shape[0], raw_blocks, B, V.shape[2])[:, idx].transpose(1, 2, 0, 3)
    dst = np.asarray([int(x) for x in block_ids], dtype=np.int64)
    k_cache[dst] = Kb
    v_cache[dst] = Vb
    return True


def write_selected_layer(k_cache, v_cache, block_ids, K, V, selected_mid_blocks, effective_len, mode, Ls, Lo,
                         B=16, allow_fast=True):
    """K / V one layer [H, L, D] of raw KV; allow_fast=False forces the piecewise path (for tests)."""
    L = int(K.shape[1])
    if mode in ("input_le_budget", "too_short"):
        if allow_fast and effective_len % B == 0 and L >= effective_len:
            if write_block_indexed_layer(k_cache, v_cache, block_ids, K[:, :effective_len], V[:, :effective_len],
                                         list(range(effective_len // B)), B):
                return
        write_piece_to_blocks(k_cache, v_cache, block_ids, 0, K[:, :effective_len], V[:, :effective_len], B)
        return
    if (allow_fast and Ls % B == 0 and Lo % B == 0 and L % B == 0 and effective_len % B == 0
            and len(block_ids) == effective_len // B):
        source = (list(range(Ls // B)) + [Ls // B + int(x) for x in selected_mid_blocks]
                  + list(range((L - Lo) // B, L // B)))
        if len(source) == len(block_ids):
            if write_block_indexed_layer(k_cache, v_cache, block_ids, K, V, source, B):
                return
    pos = write_piece_to_blocks(k_cache, v_cache, block_ids, 0, K[:, :Ls], V[:, :Ls], B)
    mid_start, mid_end = Ls, max(Ls, L - Lo)
    for mid_idx in selected_mid_blocks:
        start = mid_start + int(mid_idx) * B
        end = min(start + B, mid_end)
        if end > start:
            Kp, Vp = K[:, start:end], V[:, start:end]
        else:
            Kp, Vp = K[:, :0], V[:, :0]
        Kp, Vp = pad_piece_to_block(Kp, Vp, B)
        pos = write_piece_to_blocks(k_cache, v_cache, block_ids, pos, Kp, Vp, B)
    obs_start = max(0, L - Lo)
    pos = write_piece_to_blocks(k_cache, v_cache, block_ids, pos, K[:, obs_start:L], V[:, obs_start:L], B)
    if pos != effective_len:
        raise RuntimeError(f"selected_writeback_len_mismatch got={pos} expected={effective_len}")


def selected_writeback(k_pool, v_pool, allocator, raw_by_layer, selected_by_layer, effective_len, mode, Ls, Lo,
                       B=16):
    """k_pool / v_pool [layers, N, B, H, D]; raw_by_layer[l] = (K, V) [H, L, D]; selected_by_layer a
    list of per-layer lists or one shared list. Returns the new page ids (shared by every layer)."""
    n_req = int(math.ceil(max(1, int(effective_len)) / B))
    block_ids = allocator.allocate_blocks(n_req)
    if not block_ids:
        raise MemoryError(f"Cannot allocate {n_req} blocks")
    try:
        for layer, (K, V) in enumerate(raw_by_layer):
            sel = selected_by_layer[layer] if isinstance(selected_by_layer[0], (list, tuple, np.ndarray)) \
                else selected_by_layer
            write_selected_layer(k_pool[layer], v_pool[layer], block_ids, K, V, list(sel), effective_len, mode, Ls,
                                 Lo, B)
    except Exception:
        allocator.free_blocks_by_ids(block_ids)
        raise
    return list(block_ids)


# ------------------------------------------------------------------ pool -> pool prune copy
def prune_copy(k_pool, v_pool, allocator, old_block_ids, old_len, kept_blocks, B=16):
    """The page movement of prune_sequence_window; returns the new ids or None on failure."""
    keep_len = sum(max(0, min(old_len, (bi + 1) * B) - bi * B) for bi in kept_blocks)
    n_new = int(math.ceil(max(1, keep_len) / B))
    new_ids = allocator.allocate_blocks(n_new)
    if not new_ids:
        return None
    for layer in range(k_pool.shape[0]):
        parts_k, parts_v = [], []
        Kf = pool_read(k_pool[layer], old_block_ids, old_len, B)
        Vf = pool_read(v_pool[layer], old_block_ids, old_len, B)
        for bi in kept_blocks:
            bs, be = bi * B, min(old_len, (bi + 1) * B)
            if be <= bs:
                continue
            parts_k.append(Kf[:, bs:be])
            parts_v.append(Vf[:, bs:be])
        Kk, Vk = np.concatenate(parts_k, axis=1), np.concatenate(parts_v, axis=1)
        pool_write(k_pool[layer], new_ids, Kk, B)
        pool_write(v_pool[layer], new_ids, Vk, B)
    allocator.free_blocks_by_ids(old_block_ids)
    return list(new_ids)


def pool_read(cache, block_ids, seq_len, B=16):
    """read_kv_from_blocks of core/pool.py:154-172 for any block size: [H, T, D]."""
    chunks = []
    for i, bid in enumerate(block_ids):
        end = min(i * B + B, seq_len)
        if end - i * B > 0:
            chunks.append(cache[bid, :end - i * B].transpose(1, 0, 2))
    if not chunks:
        return np.empty((cache.shape[2], 0, cache.shape[3]), dtype=cache.dtype)
    return np.concatenate(chunks, axis=1)


def pool_write(cache, block_ids, K, B=16):
    """write_kv_to_blocks of core/pool.py:127-141 for any block size."""
    T = K.shape[1]
    for i, bid in enumerate(block_ids):
        end = min(i * B + B, T)
        if end - i * B > 0:
            cache[bid, :end - i * B] = K[:, i * B:end].transpose(1, 0, 2)


# ----------------------------------------------------------- the compressor's tensor result
def compress_tensors(K, V, selected_mid, Ls, Lo, B=16):
    """BlockAlignedSnapKV.compress's K_final / V_final for a given selection, from its own steps:
    split into sink / middle / window, zero-pad the middle to whole blocks, gather the selected
    blocks, concatenate. K / V [H, L, D]."""
    L = K.shape[1]
    K_sink, V_sink = K[:, :Ls], V[:, :Ls]
    K_obs, V_obs = K[:, L - Lo:] if Lo else K[:, L:], V[:, L - Lo:] if Lo else V[:, L:]
    K_mid, V_mid = K[:, Ls:L - Lo], V[:, Ls:L - Lo]
    premid = K_mid.shape[1]
    aligned = int(math.ceil(premid / B)) * B
    if aligned > premid:
        pad = ((0, 0), (0, aligned - premid), (0, 0))
        K_mid, V_mid = np.pad(K_mid, pad), np.pad(V_mid, pad)
    N = aligned // B
    idx = np.asarray(selected_mid, dtype=np.int64)
    Kmb = K_mid.reshape(K.shape[0], N, B, K.shape[2])[:, idx].reshape(K.shape[0], len(idx) * B, K.shape[2])
    Vmb = V_mid.reshape(V.shape[0], N, B, V.shape[2])[:, idx].reshape(V.shape[0], len(idx) * B, V.shape[2])
    return np.concatenate([K_sink, Kmb, K_obs], axis=1), np.concatenate([V_sink, Vmb, V_obs], axis=1)
