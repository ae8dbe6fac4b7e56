"""SnapKV observation-window block scores on the GPU (the input of retain-set selection).

``score_layer_blocks(K, Q_obs, ...)`` keeps the contract of BP-KV's
``_score_layer_blocks_for_selection`` (core/scheduler.py:565-592): K is one layer's
dense ``[H_kv, L, D]`` keys, ``Q_obs`` the last ``obs_len`` queries ``[H_q, obs, D]``,
the result the ``N`` smoothed block scores (fp32, on the device), empty when the
sequence is too short. ``score_blocks`` scores many (sequence, layer) items in one
call, reading K straight from the paged pool through the block table, and returns
``[seqs * layers, N]`` rows in the order ``compaction.select_blocks`` takes them.

Both run ``ukv_snapkv_scores`` (csrc/snapkv_score.hip). There is no CPU fallback.

``ObsStats`` carries the scores' softmax normalisers from the prefill: passed to the
prefill attention of a sequence batch's final chunk (``PrefillPages.attention(...,
obs_stats=...)``), it is filled while the kernel streams the keys, and ``score_blocks(...,
obs_stats=...)`` then skips its own pass over the keys for them.
"""
from __future__ import annotations

import struct
from typing import Optional

import torch

from . import _ext

_DTYPES = {torch.float16: _ext.UKV_DTYPE_F16, torch.bfloat16: _ext.UKV_DTYPE_BF16}


class ObsStats:
    """Row statistics of the observation window for ``seqs`` sequences x ``layers`` layers.

    ``data`` [seqs, layers, H_q, obs_len, 2] fp32 on ``device``: (log2 of the softmax
    normaliser of the query's scores over the middle keys, flag), as
    ``ukv_paged_prefill_obs_stats`` writes them. A layer's rows are valid once the prefill
    attention of the sequences' final chunk ran for it with this object; ``seq_lens`` are the
    sequence lengths that chunk ended at, which ``score_blocks`` checks.
    """

    def __init__(self, seqs: int, layers: int, num_q_heads: int, *, sink_len: int, obs_len: int,
                 softmax_scale: float, device):
        if seqs <= 0 or layers <= 0 or num_q_heads <= 0 or obs_len <= 0 or sink_len < 0:
            raise ValueError("ObsStats: positive sizes, non-negative sink_len")
        self.seqs, self.layers, self.num_q_heads = int(seqs), int(layers), int(num_q_heads)
        self.sink_len, self.obs_len = int(sink_len), int(obs_len)
        self.softmax_scale = float(softmax_scale)
        self.data = torch.empty((self.seqs, self.layers, self.num_q_heads, self.obs_len, 2), dtype=torch.float32,
                                device=device)
        self.seq_lens = [None] * self.layers
        self.written = [False] * self.layers

    def layer_view(self, layer_id: int):
        """(address, sequence stride in pairs) of layer ``layer_id``'s rows, for the prefill kernel."""
        if not 0 <= int(layer_id) < self.layers:
            raise IndexError(f"layer {layer_id} is outside the statistics' {self.layers} layers")
        return (self.data.data_ptr() + int(layer_id) * self.num_q_heads * self.obs_len * 8,
                self.layers * self.num_q_heads * self.obs_len)

    def same_scale(self, softmax_scale: float) -> bool:
        """Whether the kernels would use the same scale: they take it as fp32."""
        f32 = lambda x: struct.unpack("f", struct.pack("f", float(x)))[0]  # noqa: E731
        return f32(self.softmax_scale) == f32(softmax_scale)

    def mark(self, layer_id: int, seq_lens) -> None:
        self.written[int(layer_id)] = True
        self.seq_lens[int(layer_id)] = [int(x) for x in seq_lens]


def block_count(seq_len: int, sink_len: int, obs_len: int, block_size: int = 16) -> int:
    """N middle blocks scored for a sequence of ``seq_len`` tokens (0 when too short)."""
    return int(_ext.load().ukv_snapkv_block_count(int(seq_len), int(sink_len), int(obs_len), int(block_size)))


def _run(q, q_strides, k, k_strides, table, max_blocks, num_pages, layers, seqs, seq_len, sink_len, obs_len,
         num_q_heads, num_kv_heads, head_dim, n_rep, block_size, scale, out, stats=None):
    lib = _ext.load()
    ws_bytes = int(lib.ukv_snapkv_workspace_bytes(layers, seqs, seq_len, sink_len, obs_len, num_q_heads,
                                                  num_kv_heads, head_dim, n_rep, block_size))
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=q.device)
    args = [q.data_ptr(), _ext.i64_array(q_strides), k.data_ptr(), _ext.i64_array(k_strides),
            table.data_ptr() if table is not None else None, int(max_blocks), int(num_pages),
            layers, seqs, seq_len, sink_len, obs_len, num_q_heads, num_kv_heads, head_dim, n_rep, block_size,
            float(scale), _DTYPES[q.dtype]]
    tail = [out.data_ptr(), int(out.stride(0)), ws.data_ptr(), ws.numel(), torch.cuda.current_stream(q.device).cuda_stream]
    if stats is None:
        code = lib.ukv_snapkv_scores(*args, *tail)
        _ext.check(code, "ukv_snapkv_scores")
    else:
        code = lib.ukv_snapkv_scores_from_stats(*args, stats.data_ptr(), *tail)
        _ext.check(code, "ukv_snapkv_scores_from_stats")
    return out


def score_layer_blocks(K: torch.Tensor, Q_obs: torch.Tensor, *, sink_len: int, obs_len: int, n_rep: int,
                       block_size: int = 16, softmax_scale: Optional[float] = None) -> torch.Tensor:
    """Block scores of one layer of one sequence (core/scheduler.py:565-592).

    K [H_kv, L, D], Q_obs [H_q, obs_len, D] (fp16/bf16, one GPU). Returns fp32 [N]."""
    if K.dim() != 3 or Q_obs.dim() != 3:
        raise RuntimeError("selected_writeback_bad_score_shape")
    h_kv, L, D = (int(x) for x in K.shape)
    h_q = int(Q_obs.shape[0])
    n = block_count(L, sink_len, obs_len, block_size)
    if n == 0:
        return torch.empty((0,), dtype=torch.float32, device=K.device)
    if int(Q_obs.shape[1]) != int(obs_len) or int(Q_obs.shape[2]) != D:
        raise RuntimeError("selected_writeback_bad_score_shape")
    if K.dtype not in _DTYPES or Q_obs.dtype != K.dtype or K.device != Q_obs.device or K.device.type != "cuda":
        raise RuntimeError("selected_writeback_bad_score_shape")
    if K.stride(2) != 1:
        K = K.contiguous()
    if Q_obs.stride(2) != 1:
        Q_obs = Q_obs.contiguous()
    out = torch.empty((1, n), dtype=torch.float32, device=K.device)
    scale = float(D) ** -0.5 if softmax_scale is None else float(softmax_scale)
    # one item: layer stride 0, sequence stride 0; token and head strides of K
    _run(Q_obs, (0, Q_obs.stride(0), Q_obs.stride(1)), K, (0, 0, K.stride(1), K.stride(0)), None, 0, 0, 1, 1, L,
         sink_len, obs_len, h_q, h_kv, D, int(n_rep), block_size, scale, out)
    return out[0]


def _check_obs_stats(st: "ObsStats", seqs, layers, h_q, seq_len, sink_len, obs_len, scale, dev) -> torch.Tensor:
    if not isinstance(st, ObsStats):
        raise TypeError("obs_stats must be an ObsStats")
    if (st.seqs, st.layers, st.num_q_heads, st.obs_len, st.sink_len) != (seqs, layers, h_q, obs_len, sink_len):
        raise RuntimeError("selected_writeback_bad_score_shape:obs_stats")
    if st.data.device != dev:
        raise RuntimeError("selected_writeback_bad_score_device")
    if not st.same_scale(scale):
        raise RuntimeError("selected_writeback_bad_score_stats:softmax_scale")
    if not all(st.written):
        raise RuntimeError("selected_writeback_bad_score_stats:layer_missing")
    if any(lens != [int(seq_len)] * seqs for lens in st.seq_lens):
        raise RuntimeError("selected_writeback_bad_score_stats:seq_len")
    return st.data


def score_blocks(q_obs: torch.Tensor, k_pool: torch.Tensor, block_table: torch.Tensor, *, seq_len: int,
                 sink_len: int, obs_len: int, n_rep: int, block_size: int = 16,
                 softmax_scale: Optional[float] = None, obs_stats: Optional[ObsStats] = None) -> torch.Tensor:
    """Block scores of every (sequence, layer) item, K read from the paged pool.

    q_obs [seqs, layers, H_q, obs_len, D]; k_pool [layers, N, 16, H_kv, D] (a pool's k_cache);
    block_table int32 [seqs, max_blocks] (page lists shared by all layers); every sequence holds
    ``seq_len`` tokens. Returns fp32 [seqs * layers, N], row b * layers + l.

    ``obs_stats``: the normalisers the prefill of these sequences' final chunk produced for
    every layer (same sink_len, obs_len and softmax scale, chunk ending at seq_len): the
    scores then take one pass over the keys instead of two."""
    seqs, layers, h_q, obs, D = (int(x) for x in q_obs.shape)
    if obs != int(obs_len) or k_pool.dim() != 5 or int(k_pool.shape[0]) != layers or int(k_pool.shape[4]) != D:
        raise RuntimeError("selected_writeback_bad_score_shape")
    if int(k_pool.shape[2]) != 16:
        raise RuntimeError("selected_writeback_bad_score_shape")
    if int(k_pool.stride(4)) != 1:  # the kernel reads 16-byte runs of a key row; the ABI carries no dim stride
        raise RuntimeError("selected_writeback_bad_score_shape:k_pool_stride")
    n = block_count(seq_len, sink_len, obs_len, block_size)
    out = torch.empty((seqs * layers, n), dtype=torch.float32, device=q_obs.device)
    if n == 0:
        return out
    if q_obs.dtype not in _DTYPES or k_pool.dtype != q_obs.dtype:
        raise RuntimeError("selected_writeback_bad_score_shape")
    # The kernel reads table rows 0 .. seqs-1 on q_obs's device: check both before any launch.
    if k_pool.device != q_obs.device or block_table.device != q_obs.device:
        raise RuntimeError("selected_writeback_bad_score_device")
    if block_table.dim() != 2 or int(block_table.shape[0]) < seqs:
        raise RuntimeError("selected_writeback_bad_score_shape")
    if q_obs.device.type != "cuda":
        raise RuntimeError("selected_writeback_bad_score_device")
    if q_obs.stride(4) != 1 or q_obs.stride(0) != layers * q_obs.stride(1):
        q_obs = q_obs.contiguous()
    if block_table.dtype != torch.int32:
        block_table = block_table.to(torch.int32)
    block_table = block_table.contiguous()
    scale = float(D) ** -0.5 if softmax_scale is None else float(softmax_scale)
    stats = None
    if obs_stats is not None:
        stats = _check_obs_stats(obs_stats, seqs, layers, h_q, int(seq_len), int(sink_len), int(obs_len), scale,
                                 q_obs.device)
    ks = k_pool.stride()
    _run(q_obs, (q_obs.stride(1), q_obs.stride(2), q_obs.stride(3)), k_pool, (ks[0], ks[1], ks[2], ks[3]),
         block_table, int(block_table.shape[1]), int(k_pool.shape[1]), layers, seqs, int(seq_len), sink_len,
         obs_len, h_q, int(k_pool.shape[3]), D, int(n_rep), block_size, scale, out, stats)
    return out


__all__ = ["ObsStats", "block_count", "score_layer_blocks", "score_blocks"]
