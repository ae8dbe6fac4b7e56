"""Chunked prefill over the paged pool (row a9): chunk K/V into pages, then causal attention.

The reference prefills densely: the HF model runs over a chunk with the past
KV in a DynamicCache (core/engine.py:1826-1854; core/chunked_prefill.py:9-33),
flash-attn's varlen kernel for a single causal chunk (core/varlen.py:19-42);
the pool is only written after compression. Here the chunk's K/V go straight
into 16-token pages and the attention reads prefix and chunk through the block
table, with the argument conventions of flash_attn_varlen_func (packed
queries, cu_seqlens_q) and flash_attn_with_kvcache (block_table, cache lengths).
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _ext

_DTYPE_CODES = {torch.float16: _ext.UKV_DTYPE_F16, torch.bfloat16: _ext.UKV_DTYPE_BF16}


def _i32(t, dev):
    if not torch.is_tensor(t):
        t = torch.tensor(list(t), dtype=torch.int32)
    return t.to(device=dev, dtype=torch.int32).contiguous()


def _max_chunk(cu_seqlens_q, max_chunk):
    if max_chunk is not None:
        return int(max_chunk)
    cu = cu_seqlens_q.tolist() if torch.is_tensor(cu_seqlens_q) else list(cu_seqlens_q)  # host sync if on device
    return max((cu[i + 1] - cu[i] for i in range(len(cu) - 1)), default=0)


def write_chunk_kv(k_layer: torch.Tensor, v_layer: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                   block_table: torch.Tensor, cu_seqlens_q, kv_lens, max_chunk: Optional[int] = None) -> None:
    """Row cu[b] + i of k_new / v_new ([total, H_kv, D]) -> position kv_lens[b] - C_b + i of sequence b."""
    dev = k_layer.device
    for t in (k_layer, v_layer, k_new, v_new):
        if t.dtype != k_layer.dtype or t.stride(-1) != 1:
            raise ValueError("write_chunk_kv: one 16-bit dtype, contiguous last dimension")
    if k_new.stride() != v_new.stride():
        k_new, v_new = k_new.contiguous(), v_new.contiguous()
    cu = _i32(cu_seqlens_q, dev)
    lens = _i32(kv_lens, dev)
    bt = _i32(block_table, dev)
    B = int(lens.numel())
    mc = _max_chunk(cu_seqlens_q, max_chunk)
    code = _ext.load().ukv_kv_write_varlen(
        k_layer.data_ptr(), v_layer.data_ptr(), _ext.i64_array(k_layer.stride()[:3]),
        _ext.i64_array(v_layer.stride()[:3]), k_new.data_ptr(), v_new.data_ptr(), _ext.i64_array(k_new.stride()[:2]),
        bt.data_ptr(), int(bt.shape[1]), cu.data_ptr(), lens.data_ptr(), B, mc, int(k_layer.shape[2]),
        int(k_layer.shape[3]), int(k_layer.shape[0]), torch.cuda.current_stream(dev).cuda_stream)
    _ext.check(code, "ukv_kv_write_varlen")


def paged_prefill_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                            block_table: torch.Tensor, cu_seqlens_q, kv_lens, *, softmax_scale: float, n_rep: int,
                            max_chunk: Optional[int] = None) -> torch.Tensor:
    """Causal attention of packed chunk queries q [total_q, H_q, D] over their sequences' pages.

    Query i of sequence b is at position kv_lens[b] - C_b + i and sees keys 0 .. that position.
    Returns [total_q, H_q, D] in q's dtype.
    """
    if q.dim() != 3 or k_cache.dim() != 4 or v_cache.dim() != 4 or int(k_cache.shape[1]) != 16:
        raise RuntimeError("paged_prefill_shape_unsupported")
    if q.dtype not in _DTYPE_CODES or k_cache.dtype != q.dtype or v_cache.dtype != q.dtype:
        raise RuntimeError("paged_prefill_shape_unsupported:dtype")
    if q.stride(-1) != 1 or k_cache.stride(-1) != 1 or v_cache.stride(-1) != 1:
        raise RuntimeError("paged_prefill_shape_unsupported:stride")
    dev = q.device
    total_q, Hq, D = (int(x) for x in q.shape)
    Hkv = int(k_cache.shape[2])
    if int(k_cache.shape[3]) != D or tuple(v_cache.shape[1:]) != tuple(k_cache.shape[1:]):
        raise RuntimeError("paged_prefill_shape_unsupported:kv_cache")
    cu = _i32(cu_seqlens_q, dev)
    lens = _i32(kv_lens, dev)
    bt = _i32(block_table, dev)
    B = int(lens.numel())
    if int(cu.numel()) != B + 1 or int(bt.shape[0]) != B:
        raise RuntimeError("paged_prefill_shape_unsupported:batch")
    mc = _max_chunk(cu_seqlens_q, max_chunk)
    out = torch.empty((total_q, Hq, D), dtype=q.dtype, device=dev)
    code = _ext.load().ukv_paged_prefill(
        q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), bt.data_ptr(), cu.data_ptr(), lens.data_ptr(),
        out.data_ptr(), B, total_q, mc, Hq, Hkv, D, int(n_rep), int(bt.shape[1]),
        min(int(k_cache.shape[0]), int(v_cache.shape[0])), _ext.i64_array(q.stride()[:2]),
        _ext.i64_array(k_cache.stride()[:3]), _ext.i64_array(v_cache.stride()[:3]), float(softmax_scale),
        _DTYPE_CODES[q.dtype], torch.cuda.current_stream(dev).cuda_stream)
    if code != _ext.UKV_OK:
        raise RuntimeError(f"paged_prefill_error:{_ext.status_string(code)}")
    return out


def chunked_prefill(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, k_cache: torch.Tensor,
                    v_cache: torch.Tensor, block_table: torch.Tensor, cu_seqlens_q, kv_lens, *,
                    softmax_scale: float, n_rep: int, max_chunk: Optional[int] = None) -> torch.Tensor:
    """Write the chunk's K/V into its pages, then run paged causal attention for its queries."""
    mc = _max_chunk(cu_seqlens_q, max_chunk)
    write_chunk_kv(k_cache, v_cache, k_new, v_new, block_table, cu_seqlens_q, kv_lens, mc)
    return paged_prefill_attention(q, k_cache, v_cache, block_table, cu_seqlens_q, kv_lens,
                                   softmax_scale=softmax_scale, n_rep=n_rep, max_chunk=mc)
