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
from .page16_native import _current_stream
from .snapkv import ObsStats

_DTYPE_CODES = {torch.float16: _ext.UKV_DTYPE_F16, torch.bfloat16: _ext.UKV_DTYPE_BF16}


def _i32(t, dev):
    if not torch.is_tensor(t):
        t = torch.tensor(list(t), dtype=torch.int32)
    return t.to(device=dev, dtype=torch.int32).contiguous()


def _chunk_lens_on_host(cu_seqlens_q):
    """The chunk lengths when ``cu_seqlens_q`` lives on the host (a sequence or a CPU tensor), else None."""
    if torch.is_tensor(cu_seqlens_q):
        if cu_seqlens_q.device.type != "cpu":
            return None
        cu = cu_seqlens_q.tolist()
    else:
        cu = [int(x) for x in cu_seqlens_q]
    return [cu[i + 1] - cu[i] for i in range(len(cu) - 1)]


def _max_chunk(cu_seqlens_q, max_chunk, chunk_lens=None):
    """The longest chunk: derived from the lengths when no ``max_chunk`` is given (as
    core/varlen.py:28-29 derives max_seqlen; a device synchronisation when ``cu_seqlens_q`` is on
    the device), checked against them when they are on the host. A ``max_chunk`` given with
    device-only lengths is trusted; a chunk longer than it comes out as NaN rows."""
    if chunk_lens is None:
        chunk_lens = _chunk_lens_on_host(cu_seqlens_q)
    if max_chunk is None:
        if chunk_lens is None:
            cu = cu_seqlens_q.tolist()  # host sync
            chunk_lens = [cu[i + 1] - cu[i] for i in range(len(cu) - 1)]
        return max(chunk_lens, default=0)
    mc = int(max_chunk)
    if mc < 0 or (chunk_lens is not None and mc < max(chunk_lens, default=0)):
        raise RuntimeError("paged_prefill_shape_unsupported:max_chunk")
    return mc


def write_chunk_kv(k_layer: torch.Tensor, v_layer: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                   block_table: torch.Tensor, cu_seqlens_q, kv_lens, max_chunk: Optional[int] = None) -> None:
    """Row cu[b] + i of k_new / v_new ([total, H_kv, D]) -> position kv_lens[b] - C_b + i of sequence b."""
    dev = k_layer.device
    for t in (k_layer, v_layer, k_new, v_new):
        if t.dtype != k_layer.dtype or t.stride(-1) != 1:
            raise ValueError("write_chunk_kv: one 16-bit dtype, contiguous last dimension")
    # Everything the kernel dereferences, checked before the launch: the rows it reads are
    # k_new[cu[b] + i] for i < C_b, so the chunk rows must hold every head and dim of the pool.
    if k_layer.dim() != 4 or tuple(v_layer.shape) != tuple(k_layer.shape):
        raise ValueError("write_chunk_kv: k_layer / v_layer must be equal [N, 16, H_kv, D] tensors")
    if k_new.dim() != 3 or tuple(k_new.shape[1:]) != tuple(k_layer.shape[2:]) or v_new.shape != k_new.shape:
        raise ValueError(f"write_chunk_kv: k_new / v_new must be [total, {int(k_layer.shape[2])}, "
                         f"{int(k_layer.shape[3])}] tensors of one shape")
    if dev.type != "cuda" or any(t.device != dev for t in (v_layer, k_new, v_new)):
        raise RuntimeError("paged_prefill_unavailable:device")
    chunk_lens = _chunk_lens_on_host(cu_seqlens_q)
    if chunk_lens is not None and sum(chunk_lens) > int(k_new.shape[0]):
        raise ValueError(f"write_chunk_kv: the chunks hold {sum(chunk_lens)} rows, k_new {int(k_new.shape[0])}")
    if k_new.stride() != v_new.stride():
        k_new, v_new = k_new.contiguous(), v_new.contiguous()
    cu = _i32(cu_seqlens_q, dev)
    lens = _i32(kv_lens, dev)
    bt = _i32(block_table, dev)
    B = int(lens.numel())
    if int(cu.numel()) != B + 1 or bt.dim() != 2 or int(bt.shape[0]) != B:
        raise RuntimeError("paged_prefill_shape_unsupported:batch")
    mc = _max_chunk(cu_seqlens_q, max_chunk, chunk_lens)
    code = _ext.load().ukv_kv_write_varlen(
        k_layer.data_ptr(), v_layer.data_ptr(), _ext.i64_array(k_layer.stride()[:3]),
        _ext.i64_array(v_layer.stride()[:3]), k_new.data_ptr(), v_new.data_ptr(), _ext.i64_array(k_new.stride()[:2]),
        bt.data_ptr(), int(bt.shape[1]), cu.data_ptr(), lens.data_ptr(), B, mc, int(k_layer.shape[2]),
        int(k_layer.shape[3]), int(k_layer.shape[0]), torch.cuda.current_stream(dev).cuda_stream)
    _ext.check(code, "ukv_kv_write_varlen")


def _host_ints(x):
    return [int(v) for v in (x.tolist() if torch.is_tensor(x) else x)]


def paged_prefill_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                            block_table: torch.Tensor, cu_seqlens_q, kv_lens, *, softmax_scale: float, n_rep: int,
                            max_chunk: Optional[int] = None, obs_stats: Optional[ObsStats] = None,
                            layer_id: Optional[int] = None, host_lens=None) -> torch.Tensor:
    """Causal attention of packed chunk queries q [total_q, H_q, D] over their sequences' pages.

    Query i of sequence b is at position kv_lens[b] - C_b + i and sees keys 0 .. that position.
    Returns [total_q, H_q, D] in q's dtype.

    With ``obs_stats`` (and ``layer_id``), the chunk must be each sequence's last, holding at
    least ``obs_stats.obs_len`` queries: layer ``layer_id``'s SnapKV normalisers of the last
    ``obs_len`` queries are written alongside (ukv_paged_prefill_obs_stats). ``host_lens``:
    (chunk lengths, sequence lengths) as host lists, saving the synchronisation that reading
    device ``cu_seqlens_q`` / ``kv_lens`` back would cost.
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
    stats_view = None
    if obs_stats is not None:
        if layer_id is None:
            raise ValueError("paged_prefill_attention: obs_stats needs layer_id")
        if not isinstance(obs_stats, ObsStats):
            raise TypeError("obs_stats must be an ObsStats")
        if obs_stats.seqs != B or obs_stats.num_q_heads != Hq or obs_stats.data.device != dev:
            raise RuntimeError("paged_prefill_shape_unsupported:obs_stats")
        if not obs_stats.same_scale(softmax_scale):
            raise RuntimeError("paged_prefill_shape_unsupported:obs_stats_scale")
        # host copies of the chunk and sequence lengths (a sync when they are device tensors)
        chunk_lens, seq_lens = host_lens if host_lens is not None else (None, None)
        if chunk_lens is None:
            cu_h = _host_ints(cu_seqlens_q)
            chunk_lens = [cu_h[i + 1] - cu_h[i] for i in range(B)]
            seq_lens = _host_ints(kv_lens)
        if any(c < obs_stats.obs_len for c in chunk_lens):
            raise RuntimeError("paged_prefill_shape_unsupported:obs_window_spans_chunks")
        stats_view = obs_stats.layer_view(layer_id)
        host_lens = (chunk_lens, seq_lens)
    if dev.type != "cuda" or any(t.device != dev for t in (k_cache, v_cache, bt, cu, lens)):
        raise RuntimeError("paged_prefill_unavailable:device")
    mc = _max_chunk(cu_seqlens_q, max_chunk, None if host_lens is None else host_lens[0])
    out = torch.empty((total_q, Hq, D), dtype=q.dtype, device=dev)
    args = [q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), bt.data_ptr(), cu.data_ptr(), lens.data_ptr(),
            out.data_ptr(), B, total_q, mc, Hq, Hkv, D, int(n_rep), int(bt.shape[1]),
            min(int(k_cache.shape[0]), int(v_cache.shape[0])), _ext.i64_array(q.stride()[:2]),
            _ext.i64_array(k_cache.stride()[:3]), _ext.i64_array(v_cache.stride()[:3]), float(softmax_scale),
            _DTYPE_CODES[q.dtype]]
    stream = torch.cuda.current_stream(dev).cuda_stream
    if stats_view is None:
        code = _ext.load().ukv_paged_prefill(*args, stream)
    else:
        code = _ext.load().ukv_paged_prefill_obs_stats(*args, obs_stats.sink_len, obs_stats.obs_len, *stats_view,
                                                        stream)
        if code == _ext.UKV_OK:
            obs_stats.mark(layer_id, seq_lens)
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


class PrefillPages:
    """Chunked prefill of a batch of sequences straight into the paged pool.

    BP-KV keeps a chunked prefill's past in a DynamicCache (core/engine.py:1826-1854: each
    chunk's forward concatenates its K/V onto the past of every layer), stages the finished KV
    on the host and writes it into the pool only after compression (core/engine.py:1856-1882:
    capture_prefill_kv, post_prefill_compress, then write_kv_to_blocks, core/pool.py:127-141).
    Here each chunk's K/V land in their 16-token pages as each layer computes them:

    * ``begin_chunk(chunk_lens)`` reserves the pages the chunk needs: for each sequence in batch
      order, FIFO from the pool, one id per block shared by every layer; if the pool cannot
      hold the whole chunk nothing is allocated and ``prefill_pages_alloc_failed`` is raised;
      the block table, ``cu_seqlens_q`` and the new lengths go to the device in one copy each;
    * ``attention(layer, q, k, v, ...)`` writes the layer's chunk K/V into the pages and runs
      the paged causal attention (``write`` alone for callers with their own attention);
    * ``end_chunk()`` commits the lengths.

    ``page_lists`` / ``seq_lens`` are what ``DecodeBatch``, ``snapkv.score_blocks`` and
    ``compaction.compact`` take next; no dense copy of the prefill KV is ever made.

    Streams: the chunk's table and lengths are uploaded on the stream current at ``begin_chunk``
    and read on the stream current at each later call; a caller that moves to another stream
    orders it after the upload itself (``wait_stream``), as for any tensor handed across
    streams. Each other stream a chunk's tensors are read on is recorded with the caching
    allocator, so ``end_chunk`` never frees them under that stream's pending kernels.
    """

    def __init__(self, pool, num_seqs: Optional[int] = None, *, page_lists=None, seq_lens=None):
        if page_lists is None:
            page_lists = [[] for _ in range(int(num_seqs or 0))]
        if seq_lens is None:
            seq_lens = [0] * len(page_lists)
        if len(page_lists) != len(seq_lens) or not page_lists:
            raise ValueError("PrefillPages: one page list and one length per sequence")
        for ids, L in zip(page_lists, seq_lens):
            if len(ids) * pool.B < int(L):
                raise ValueError("PrefillPages: a sequence has fewer pages than its length needs")
        pool.ensure_allocated()
        self.pool = pool
        self.dev = pool.device
        self._lists = [[int(x) for x in ids] for ids in page_lists]
        self._lens = [int(x) for x in seq_lens]
        self._chunk = None
        self._strides = None

    @property
    def page_lists(self):
        return self._lists

    @property
    def seq_lens(self):
        return list(self._lens)

    @property
    def block_table(self) -> torch.Tensor:
        if self._chunk is None:
            raise RuntimeError("prefill_chunk_not_open")
        return self._chunk["bt"]

    def begin_chunk(self, chunk_lens):
        """Reserve pages for ``chunk_lens[b]`` new tokens of each sequence; returns
        (block_table, cu_seqlens_q, kv_lens, max_chunk) for the chunk (device tensors, host int)."""
        if self._chunk is not None:
            raise RuntimeError("prefill_chunk_already_open")
        chunk_lens = [int(c) for c in chunk_lens]
        if len(chunk_lens) != len(self._lists) or any(c < 0 for c in chunk_lens):
            raise ValueError("PrefillPages: one non-negative chunk length per sequence")
        B = self.pool.B
        need = [max(0, -(-(L + c) // B) - len(ids)) for L, c, ids in zip(self._lens, chunk_lens, self._lists)]
        if sum(need) > self.pool.n_free:
            raise RuntimeError("prefill_pages_alloc_failed")
        for ids, n in zip(self._lists, need):
            if n:
                ids.extend(self.pool.allocate_blocks(n))
        width = max(1, max(len(ids) for ids in self._lists))
        host = torch.zeros((len(self._lists), width), dtype=torch.int32)
        for i, ids in enumerate(self._lists):
            if ids:
                host[i, :len(ids)] = torch.tensor(ids, dtype=torch.int32)
        cu = [0]
        for c in chunk_lens:
            cu.append(cu[-1] + c)
        kv = [L + c for L, c in zip(self._lens, chunk_lens)]
        small = torch.tensor(cu + kv, dtype=torch.int32).pin_memory().to(self.dev, non_blocking=True)
        self._chunk = dict(bt=host.pin_memory().to(self.dev, non_blocking=True), small=small, cu=small[:len(cu)],
                           kv=small[len(cu):], max_chunk=max(chunk_lens), lens=chunk_lens, total=cu[-1],
                           streams={_current_stream(self.dev)})
        return self._chunk["bt"], self._chunk["cu"], self._chunk["kv"], self._chunk["max_chunk"]

    def _open(self):
        if self._chunk is None:
            raise RuntimeError("prefill_chunk_not_open")
        return self._chunk

    def _read_here(self, c) -> None:
        """Before a launch that reads the chunk's tensors: on a stream other than the upload's,
        record them there, so that the caching allocator keeps them for its pending kernels."""
        cur = _current_stream(self.dev)
        if cur not in c["streams"]:
            s = torch.cuda.current_stream(self.dev)
            c["bt"].record_stream(s)
            c["small"].record_stream(s)
            c["streams"].add(cur)

    def write(self, layer_id: int, k_new: torch.Tensor, v_new: torch.Tensor) -> None:
        """The layer's chunk K/V, packed [total_q, H_kv, D] in batch order, into their pages."""
        c = self._open()
        pool = self.pool
        layer_id = int(layer_id)
        if not 0 <= layer_id < pool.num_layers:  # the fast path below computes the layer's address itself
            raise IndexError(f"layer {layer_id} is outside the pool's {pool.num_layers} layers")
        if c["total"] == 0:
            return
        self._read_here(c)
        if (k_new.dtype != pool.dtype or v_new.dtype != pool.dtype or k_new.device != self.dev
                or tuple(k_new.shape) != (c["total"], pool.num_kv_heads, pool.head_dim)
                or k_new.stride() != v_new.stride() or k_new.stride(-1) != 1):
            # unusual inputs: the general wrapper converts and checks them
            write_chunk_kv(pool.k_cache[layer_id], pool.v_cache[layer_id], k_new, v_new, c["bt"], c["cu"], c["kv"],
                           c["max_chunk"])
            return
        if self._strides is None:  # the pool's layer strides, fixed for its life
            kl = pool.k_cache[0]
            self._strides = (_ext.i64_array(kl.stride()[:3]), _ext.i64_array(pool.v_cache[0].stride()[:3]),
                             int(pool.k_cache.stride(0)) * pool.k_cache.element_size(),
                             int(pool.v_cache.stride(0)) * pool.v_cache.element_size())
        ks, vs, kl_bytes, vl_bytes = self._strides
        code = _ext.load().ukv_kv_write_varlen(
            pool.k_cache.data_ptr() + layer_id * kl_bytes, pool.v_cache.data_ptr() + layer_id * vl_bytes, ks, vs,
            k_new.data_ptr(), v_new.data_ptr(), _ext.i64_array(k_new.stride()[:2]), c["bt"].data_ptr(),
            int(c["bt"].shape[1]), c["cu"].data_ptr(), c["kv"].data_ptr(), len(self._lists), c["max_chunk"],
            pool.num_kv_heads, pool.head_dim, pool.N_total, torch.cuda.current_stream(self.dev).cuda_stream)
        _ext.check(code, "ukv_kv_write_varlen")

    def attention(self, layer_id: int, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, *,
                  softmax_scale: float, n_rep: int, obs_stats: Optional[ObsStats] = None) -> torch.Tensor:
        """Write the layer's chunk K/V, then causal attention of q [total_q, H_q, D] over prefix + chunk.

        ``obs_stats``: this is the sequences' final chunk; also record layer ``layer_id``'s
        SnapKV normalisers of the last ``obs_len`` queries (see ``snapkv.ObsStats``)."""
        c = self._open()
        if c["total"] == 0 and obs_stats is None:
            return torch.empty_like(q)
        self.write(layer_id, k_new, v_new)
        self._read_here(c)
        host_lens = None
        if obs_stats is not None:
            host_lens = (c["lens"], [L + n for L, n in zip(self._lens, c["lens"])])
        return paged_prefill_attention(q, self.pool.k_cache[layer_id], self.pool.v_cache[layer_id], c["bt"], c["cu"],
                                       c["kv"], softmax_scale=softmax_scale, n_rep=n_rep, max_chunk=c["max_chunk"],
                                       obs_stats=obs_stats, layer_id=layer_id, host_lens=host_lens)

    def end_chunk(self) -> None:
        c = self._open()
        self._lens = [L + n for L, n in zip(self._lens, c["lens"])]
        self._chunk = None
