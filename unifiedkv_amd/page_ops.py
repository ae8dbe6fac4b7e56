"""Python entry points of libukv.so's page-movement kernels (bit-exact copies).

Every function enqueues on the current stream and returns without a host
synchronisation; tensors must live on the same GPU, 16-bit K/V dtypes.
"""
from __future__ import annotations

from typing import Optional, Sequence

import torch

from . import _ext


def _stream(dev) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _i32(ids, dev) -> torch.Tensor:
    if torch.is_tensor(ids):
        return ids.to(device=dev, dtype=torch.int32).contiguous()
    return torch.tensor(list(ids), dtype=torch.int32, device=dev)


def _check_rows(t: torch.Tensor, what: str):
    if t.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError(f"{what}: 16-bit float tensor required, got {t.dtype}")
    if t.stride(-1) != 1:
        raise ValueError(f"{what}: last dimension must be contiguous")


def _check_gpu(dev: torch.device, others, fn: str):
    """Every tensor the kernel dereferences on the one GPU ``dev``, checked before any launch."""
    if dev.type != "cuda":
        raise RuntimeError(f"{fn}: tensors must be on a GPU, got {dev}")
    for t, w in others:
        if t.device != dev:
            raise RuntimeError(f"{fn}: {w} is on {t.device}, the pool on {dev}")


def scatter_tokens(pool_layer: torch.Tensor, page_ids, dense: torch.Tensor, n_tokens: Optional[int] = None) -> None:
    """pool_layer[page_ids[t // bs], t % bs, h, :] = dense[h, t, :] for t < n_tokens (bs = pool_layer.shape[1]).

    pool_layer [N, bs, H, D]; dense [H, T, D]; n_tokens defaults to min(T, bs * len(page_ids)).
    """
    _check_rows(pool_layer, "pool_layer")
    _check_rows(dense, "dense")
    dev = pool_layer.device
    if pool_layer.dim() != 4 or dense.dim() != 3 or dense.dtype != pool_layer.dtype:
        raise ValueError("scatter_tokens: pool_layer [N, bs, H, D] and dense [H, T, D] of one dtype required")
    if int(dense.shape[0]) != int(pool_layer.shape[2]) or int(dense.shape[2]) != int(pool_layer.shape[3]):
        raise ValueError(f"scatter_tokens: dense {list(dense.shape)} does not hold the pool's "
                         f"{int(pool_layer.shape[2])} heads x {int(pool_layer.shape[3])} dims")
    _check_gpu(dev, [(dense, "dense")], "scatter_tokens")
    ids = _i32(page_ids, dev)
    bs = int(pool_layer.shape[1])
    T = int(dense.shape[1]) if n_tokens is None else min(int(n_tokens), int(dense.shape[1]))
    T = min(T, bs * int(ids.numel()))
    if T <= 0:
        return
    code = _ext.load().ukv_kv_scatter_tokens(
        pool_layer.data_ptr(), _ext.i64_array(pool_layer.stride()[:3]), dense.data_ptr(),
        _ext.i64_array(dense.stride()[:2]), ids.data_ptr(), int(ids.numel()), int(pool_layer.shape[0]), T, bs,
        int(pool_layer.shape[2]), int(pool_layer.shape[3]), _stream(dev))
    _ext.check(code, "ukv_kv_scatter_tokens")


def gather_tokens(pool_layer: torch.Tensor, page_ids, n_tokens: int) -> torch.Tensor:
    """[H, n, D] with row t = pool_layer[page_ids[t // bs], t % bs], n = min(n_tokens, bs * len(ids))."""
    _check_rows(pool_layer, "pool_layer")
    dev = pool_layer.device
    if pool_layer.dim() != 4:
        raise ValueError("gather_tokens: pool_layer [N, bs, H, D] required")
    _check_gpu(dev, [], "gather_tokens")
    ids = _i32(page_ids, dev)
    bs = int(pool_layer.shape[1])
    H, D = int(pool_layer.shape[2]), int(pool_layer.shape[3])
    T = max(0, min(int(n_tokens), bs * int(ids.numel())))
    out = torch.empty((H, T, D), dtype=pool_layer.dtype, device=dev)
    if T == 0:
        return out
    code = _ext.load().ukv_kv_gather_tokens(
        pool_layer.data_ptr(), _ext.i64_array(pool_layer.stride()[:3]), out.data_ptr(),
        _ext.i64_array(out.stride()[:2]), ids.data_ptr(), int(ids.numel()), int(pool_layer.shape[0]), T, bs, H, D,
        _stream(dev))
    _ext.check(code, "ukv_kv_gather_tokens")
    return out


def page_copy(src_pools: Sequence[torch.Tensor], dst_pools: Sequence[torch.Tensor], src_ids, dst_ids) -> None:
    """dst[l, dst_ids(l)[j]] = src[l, src_ids(l)[j]] for every layer l and pool pair.

    Pools are [L, N, 16, H, D] (or any [L, N, ...] with contiguous pages); src_ids / dst_ids are
    int32 [n] (shared by all layers) or [L, n] (per layer).
    """
    if len(src_pools) != len(dst_pools) or not 1 <= len(src_pools) <= 2:
        raise ValueError("page_copy: one or two (src, dst) pool pairs")
    s0, d0 = src_pools[0], dst_pools[0]
    dev = s0.device
    _check_gpu(dev, [(t, "a pool") for t in list(src_pools[1:]) + list(dst_pools)], "page_copy")
    L = int(s0.shape[0])
    page_elems = int(s0[0, 0].numel())
    for s, d in zip(src_pools, dst_pools):
        _check_rows(s, "src pool")
        _check_rows(d, "dst pool")
        if int(d.shape[0]) != L or int(d[0, 0].numel()) != page_elems or s.dtype != d.dtype:
            raise ValueError("page_copy: pools disagree in layers, page size or dtype")
        if not (s[0, 0].is_contiguous() and d[0, 0].is_contiguous()):
            raise ValueError("page_copy: pages must be contiguous")
        if s.stride()[:2] != s0.stride()[:2] or d.stride()[:2] != d0.stride()[:2]:
            raise ValueError("page_copy: K and V pools must share strides")
    si = _i32(src_ids, dev)
    di = _i32(dst_ids, dev)
    n = int(si.shape[-1])
    if int(di.shape[-1]) != n:
        raise ValueError("page_copy: src and dst id lists differ in length")
    for ids in (si, di):
        if ids.dim() == 2 and int(ids.shape[0]) != L:
            raise ValueError("page_copy: per-layer id lists need one row per layer")
    code = _ext.load().ukv_page_copy(
        _ext.ptr_array([t.data_ptr() for t in src_pools]), _ext.ptr_array([t.data_ptr() for t in dst_pools]),
        len(src_pools), _ext.i64_array(s0.stride()[:2]), _ext.i64_array(d0.stride()[:2]),
        si.data_ptr(), n if si.dim() == 2 else 0, di.data_ptr(), n if di.dim() == 2 else 0,
        n, L, page_elems, int(s0.shape[1]), int(d0.shape[1]), _stream(dev))
    _ext.check(code, "ukv_page_copy")


def kv_append(k_layer: torch.Tensor, v_layer: torch.Tensor, block_table: torch.Tensor, old_lens: torch.Tensor,
              k_new: torch.Tensor, v_new: torch.Tensor, return_new_lens: bool = True) -> Optional[torch.Tensor]:
    """Write the decode token of each sequence at position old_lens[b] (core/scheduler.py:401-408).

    k_layer/v_layer [N, bs, H, D]; block_table int32 [B, max_blocks]; old_lens int32 [B];
    k_new/v_new [B, H, D] (or [B, 1, H, D]). Returns old_lens + 1 (int32) when asked.
    """
    for t, w in ((k_layer, "k_layer"), (v_layer, "v_layer"), (k_new, "k_new"), (v_new, "v_new")):
        _check_rows(t, w)
    dev = k_layer.device
    # Everything the kernel dereferences is checked here, before any launch: a short
    # length vector or a mis-shaped row tensor would otherwise be read out of bounds.
    for t, w in ((v_layer, "v_layer"), (k_new, "k_new"), (v_new, "v_new"), (block_table, "block_table"),
                 (old_lens, "old_lens")):
        if t.device != dev:
            raise RuntimeError(f"kv_append: {w} is on {t.device}, the pool layer on {dev}")
    if k_layer.dim() != 4 or tuple(v_layer.shape) != tuple(k_layer.shape) or v_layer.dtype != k_layer.dtype:
        raise RuntimeError("kv_append: k_layer / v_layer must be equal [N, bs, H, D] tensors")
    if block_table.dim() != 2:
        raise RuntimeError("kv_append: block_table must be [batch, max_blocks]")
    if k_new.dim() == 4:
        if int(k_new.shape[1]) != 1 or int(v_new.shape[1]) != 1:
            raise RuntimeError("kv_append: k_new / v_new must be [batch, H, D] or [batch, 1, H, D]")
        k_new, v_new = k_new[:, 0], v_new[:, 0]
    B = int(block_table.shape[0])
    want = (B, int(k_layer.shape[2]), int(k_layer.shape[3]))
    if tuple(k_new.shape) != want or tuple(v_new.shape) != want:
        raise RuntimeError(f"kv_append: k_new / v_new must be {list(want)}, got {list(k_new.shape)} / "
                           f"{list(v_new.shape)}")
    if k_new.dtype != k_layer.dtype or v_new.dtype != k_layer.dtype:
        raise RuntimeError("kv_append: new rows must have the pool's dtype")
    if int(old_lens.numel()) != B:
        raise RuntimeError(f"kv_append: old_lens has {int(old_lens.numel())} entries for a batch of {B}")
    if dev.type != "cuda":
        raise RuntimeError(f"kv_append: tensors must be on a GPU, got {dev}")
    if k_new.stride() != v_new.stride():
        v_new = v_new.contiguous()
        k_new = k_new.contiguous()
    bt = block_table if block_table.dtype == torch.int32 else block_table.to(torch.int32)
    bt = bt.contiguous()
    lens = old_lens.to(torch.int32).contiguous()
    new_lens = torch.empty_like(lens) if return_new_lens else None
    code = _ext.load().ukv_kv_append(
        k_layer.data_ptr(), v_layer.data_ptr(), _ext.i64_array(k_layer.stride()[:3]),
        _ext.i64_array(v_layer.stride()[:3]), k_new.data_ptr(), v_new.data_ptr(), _ext.i64_array(k_new.stride()[:2]),
        bt.data_ptr(), int(bt.shape[1]), lens.data_ptr(), new_lens.data_ptr() if new_lens is not None else None,
        B, int(k_layer.shape[1]), int(k_layer.shape[2]), int(k_layer.shape[3]), int(k_layer.shape[0]), _stream(dev))
    _ext.check(code, "ukv_kv_append")
    return new_lens
