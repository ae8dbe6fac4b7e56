"""Drop-in replacement for BP-KV's ``page16_native`` module on MI355X.

Keeps the call surface of core/page16_native.py: the ``HAS_TRITON`` flag the
scheduler probes (core/scheduler.py:14, 203-212) and
``page16_decode_attention(q, k_cache, v_cache, block_table, cache_seqlens, *,
softmax_scale, n_rep)`` with the reference's argument checks, their order and
their exact RuntimeError strings (core/page16_native.py:101-124), the output
allocation ``empty_like(q)`` and the launch on the current stream without a
host synchronisation (core/page16_native.py:126-150).

The computation runs in libukv.so (gfx950 HIP kernels, C ABI in
include/ukv.h). There is no CPU or PyTorch fallback: without the library the
module reports ``HAS_TRITON = False`` and the call raises the reference's
``page16_native_unavailable:triton_not_available``.
"""
from __future__ import annotations

import functools

import torch

from . import _ext

# Name kept for the reference's importers (core/scheduler.py:14). True iff the
# native library loaded.
HAS_TRITON = _ext.available()
HAS_UKV = HAS_TRITON

_DTYPE_CODES = {torch.float16: _ext.UKV_DTYPE_F16, torch.bfloat16: _ext.UKV_DTYPE_BF16}


def _status_message(code: int, head_dim: int) -> str:
    if code == _ext.UKV_ERR_EMPTY:
        return "page16_native_shape_unsupported:empty"
    if code == _ext.UKV_ERR_GQA:
        return "page16_native_shape_unsupported:gqa"
    if code == _ext.UKV_ERR_HEAD_DIM:
        return f"page16_native_shape_unsupported:head_dim_{head_dim}"
    if code == _ext.UKV_ERR_DTYPE:
        return "page16_native_shape_unsupported:dtype"
    return f"page16_native_runtime_error:{_ext.status_string(code)}"


def _prepare(q, k_cache, v_cache, block_table, cache_seqlens):
    """The reference's argument checks, in its order (core/page16_native.py:101-124),
    then the native kernels' own; returns the normalised call arguments."""
    if not HAS_TRITON:
        raise RuntimeError("page16_native_unavailable:triton_not_available")
    if q.dim() != 3:
        raise RuntimeError(f"page16_native_shape_unsupported:q_dim_{q.dim()}")
    if k_cache.dim() != 4 or v_cache.dim() != 4:
        raise RuntimeError("page16_native_shape_unsupported:cache_rank")
    if int(k_cache.shape[1]) != 16:
        raise RuntimeError(f"page16_native_shape_unsupported:block_size_{int(k_cache.shape[1])}")
    if block_table.dim() != 2:
        raise RuntimeError("page16_native_shape_unsupported:block_table_rank")
    batch, num_q_heads, head_dim = [int(x) for x in q.shape]
    num_kv_heads = int(k_cache.shape[2])
    if batch <= 0 or num_q_heads <= 0 or head_dim <= 0:
        raise RuntimeError("page16_native_shape_unsupported:empty")
    if int(v_cache.shape[1]) != 16 or int(v_cache.shape[2]) != num_kv_heads or int(v_cache.shape[3]) != head_dim:
        raise RuntimeError("page16_native_shape_unsupported:v_cache")
    if num_q_heads % num_kv_heads != 0:
        raise RuntimeError("page16_native_shape_unsupported:gqa")
    if int(block_table.shape[0]) != batch:
        raise RuntimeError("page16_native_shape_unsupported:block_table_batch")
    if int(cache_seqlens.numel()) != batch:
        raise RuntimeError("page16_native_shape_unsupported:seqlens")
    if head_dim > 256:
        raise RuntimeError(f"page16_native_shape_unsupported:head_dim_{head_dim}")
    # Checks beyond the reference: the native kernels read 16-bit rows directly,
    # so dtypes must agree, the K rows must match head_dim, the last dimension
    # must be contiguous and everything must sit on one GPU.
    if q.dtype not in _DTYPE_CODES or k_cache.dtype != q.dtype or v_cache.dtype != q.dtype:
        raise RuntimeError("page16_native_shape_unsupported:dtype")
    if int(k_cache.shape[3]) != head_dim:
        raise RuntimeError("page16_native_shape_unsupported:k_cache")
    if int(k_cache.stride(3)) != 1 or int(v_cache.stride(3)) != 1:
        raise RuntimeError("page16_native_shape_unsupported:cache_stride")
    dev = q.device
    if dev.type != "cuda" or any(t.device != dev for t in (k_cache, v_cache, block_table, cache_seqlens)):
        raise RuntimeError("page16_native_unavailable:device")

    q = q.contiguous()
    if block_table.dtype != torch.int32:
        block_table = block_table.to(torch.int32)
    block_table = block_table.contiguous()
    cache_seqlens = cache_seqlens.to(dtype=torch.int32).contiguous()
    return q, block_table, cache_seqlens, batch, num_q_heads, num_kv_heads, head_dim, dev


@functools.lru_cache(maxsize=256)
def _workspace_bytes(dev_index, batch, num_q_heads, head_dim, max_blocks) -> int:
    # The size depends on the shape and the device's CU count only.
    with torch.cuda.device(dev_index):
        return max(int(_ext.load().ukv_page16_workspace_bytes(batch, num_q_heads, head_dim, max_blocks)), 256)


# One workspace per (device, stream), reused by every eager call on that stream (calls on one
# stream are ordered; the workspace needs no initialisation, include/ukv.h). A workspace outgrown
# by a larger shape is replaced and the old one kept alive for the calls still queued on it.
# Under graph capture every call gets a workspace of its own from the graph's memory pool, never
# the cached one: a graph may be replayed on another stream, beside eager calls or other graphs
# captured on the same stream, and a shared buffer would race there.
_WORKSPACES = {}
_RETIRED = []


def _workspace(batch, num_q_heads, head_dim, max_blocks, dev, stream) -> torch.Tensor:
    need = _workspace_bytes(dev.index, batch, num_q_heads, head_dim, max_blocks)
    if torch.cuda.is_current_stream_capturing():
        return torch.empty(need, dtype=torch.uint8, device=dev)
    key = (dev.index, stream)
    ws = _WORKSPACES.get(key)
    if ws is not None and ws.numel() >= need:
        return ws
    fresh = torch.empty(need if ws is None else max(need, 2 * ws.numel()), dtype=torch.uint8, device=dev)
    if ws is not None:
        _RETIRED.append(ws)
    _WORKSPACES[key] = fresh
    return fresh


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _current_stream(dev) -> int:
    """Handle of dev's current stream. torch's raw query costs ~0.2 us per call against ~4 us for
    torch.cuda.current_stream(dev).cuda_stream, which matters for small, launch-bound batches."""
    if _raw_stream is not None:
        return _raw_stream(dev.index)
    return torch.cuda.current_stream(dev).cuda_stream


def page16_decode_attention(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    cache_seqlens: torch.Tensor,
    *,
    softmax_scale: float,
    n_rep: int,
) -> torch.Tensor:
    """Decode-only paged attention over 16-token blocks.

    Args:
        q: [batch, num_q_heads, head_dim] fp16/bf16 device tensor.
        k_cache/v_cache: [num_blocks, 16, num_kv_heads, head_dim], last dim contiguous.
        block_table: [batch, max_blocks] int32 device tensor (zero padded).
        cache_seqlens: [batch] device tensor, including the current token.

    Same contract as core/page16_native.py:83-150; q head h reads KV head h // n_rep.
    """
    q, block_table, cache_seqlens, batch, num_q_heads, num_kv_heads, head_dim, dev = _prepare(
        q, k_cache, v_cache, block_table, cache_seqlens)
    out = torch.empty_like(q)
    max_blocks = int(block_table.shape[1])
    num_pages = min(int(k_cache.shape[0]), int(v_cache.shape[0]))

    lib = _ext.load()
    stream = _current_stream(dev)
    workspace = _workspace(batch, num_q_heads, head_dim, max_blocks, dev, stream)
    code = lib.ukv_page16_decode(
        q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
        block_table.data_ptr(), cache_seqlens.data_ptr(), out.data_ptr(),
        batch, num_q_heads, num_kv_heads, head_dim, int(n_rep),
        max_blocks, num_pages,
        _ext.i64_tuple(q.stride()[:2]),
        _ext.i64_tuple(k_cache.stride()[:3]),
        _ext.i64_tuple(v_cache.stride()[:3]),
        float(softmax_scale), _DTYPE_CODES[q.dtype],
        workspace.data_ptr(), workspace.numel(), stream,
    )
    if code != _ext.UKV_OK:
        raise RuntimeError(_status_message(code, head_dim))
    return out


def page16_decode_append_attention(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    cache_seqlens: torch.Tensor,
    k_new: torch.Tensor,
    v_new: torch.Tensor,
    *,
    softmax_scale: float,
    n_rep: int,
) -> torch.Tensor:
    """The decode step's token append and ``page16_decode_attention`` in one call.

    ``cache_seqlens`` are the attention lengths (old lengths + 1, as passed to the
    decode call); ``k_new``/``v_new`` are the step's [batch, num_kv_heads, head_dim]
    (or [batch, 1, num_kv_heads, head_dim]) rows, written to position
    cache_seqlens[b] - 1 of sequence b before it is attended. Same result and pool
    contents as core/scheduler.py:401-418 (block_pos / tok_pos, the two
    ``index_put_``, ``attn_lens = old_lens + 1``, ``page16_decode_attention``),
    provided no page one sequence attends is another sequence's append target
    (true for the pool's per-sequence pages; a length beyond its table row
    attends the zero padding, page 0, and the reference rejects such a length).
    """
    q, block_table, cache_seqlens, batch, num_q_heads, num_kv_heads, head_dim, dev = _prepare(
        q, k_cache, v_cache, block_table, cache_seqlens)
    if k_new.dim() == 4:
        k_new, v_new = k_new[:, 0], v_new[:, 0]
    if tuple(k_new.shape) != (batch, num_kv_heads, head_dim) or tuple(v_new.shape) != tuple(k_new.shape):
        raise RuntimeError("page16_native_shape_unsupported:new_token")
    if k_new.dtype != q.dtype or v_new.dtype != q.dtype:
        raise RuntimeError("page16_native_shape_unsupported:dtype")
    if k_new.device != dev or v_new.device != dev:
        raise RuntimeError("page16_native_unavailable:device")
    if k_new.stride(2) != 1 or v_new.stride(2) != 1 or k_new.stride()[:2] != v_new.stride()[:2]:
        k_new, v_new = k_new.contiguous(), v_new.contiguous()
    out = torch.empty_like(q)
    max_blocks = int(block_table.shape[1])
    num_pages = min(int(k_cache.shape[0]), int(v_cache.shape[0]))

    lib = _ext.load()
    stream = _current_stream(dev)
    workspace = _workspace(batch, num_q_heads, head_dim, max_blocks, dev, stream)
    code = lib.ukv_page16_decode_append(
        q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
        block_table.data_ptr(), cache_seqlens.data_ptr(),
        k_new.data_ptr(), v_new.data_ptr(), _ext.i64_tuple(k_new.stride()[:2]), out.data_ptr(),
        batch, num_q_heads, num_kv_heads, head_dim, int(n_rep),
        max_blocks, num_pages,
        _ext.i64_tuple(q.stride()[:2]),
        _ext.i64_tuple(k_cache.stride()[:3]),
        _ext.i64_tuple(v_cache.stride()[:3]),
        float(softmax_scale), _DTYPE_CODES[q.dtype],
        workspace.data_ptr(), workspace.numel(), stream,
    )
    if code != _ext.UKV_OK:
        raise RuntimeError(_status_message(code, head_dim))
    return out


__all__ = ["HAS_TRITON", "HAS_UKV", "page16_decode_attention", "page16_decode_append_attention"]
