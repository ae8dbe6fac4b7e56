"""TEST INFRASTRUCTURE ONLY - CPU restatement of SnapKV's observation-window block scores.

Only tests/ (and bench.py's CPU baseline) may import this module. It follows
core/scheduler.py:565-592 (``_score_layer_blocks_for_selection``) of BP-KV step by step,
in float64 on host arrays:

* ``mid_keys``            :577-582  K_mid = K[:, sink : L - obs], zero-padded to a block multiple
* ``repeat_kv``           core/compress.py:7-20 (q head h reads KV head h // n_rep)
* ``score_layer_blocks``  :583-591  softmax(Q_obs K_mid^T * scale) -> mean over queries ->
                                    max over heads -> sum per block -> maxpool(3, 1, 1) if N >= 3
* ``score_layer_blocks_loops``      the same with explicit loops (tiny shapes; cross-check)
* ``maxpool3``            torch.nn.functional.max_pool1d(kernel_size=3, stride=1, padding=1)
* ``obs_row_stats``       :586-587  the softmax's normaliser per (q head, query): log2 of
                          sum_j exp(Q_obs K_mid_j^T * scale) over the padded K_mid, the row statistics
                          ukv_paged_prefill_obs_stats produces during the prefill
* ``score_heads_f32``     the dense fp32 formulation (matmul, softmax, mean) for a subset of heads:
                          the CPU baseline's sample
* ``score_layer_blocks_model_dtype``  the same steps with the reference's rounding points: every
                          torch op of :586-588 runs in the model dtype there, so its output is
                          rounded to bf16 / fp16 (matmul, * scale, softmax, mean, block sum);
                          bounds how far exact scores sit from the reference's own arithmetic
"""
from __future__ import annotations

import math

import numpy as np

from . import oracle as _bits


def mid_keys(K: np.ndarray, sink_len: int, obs_len: int, block_size: int):
    """K [H_kv, L, D] -> (zero-padded K_mid [H_kv, aligned, D], N); N = 0 when too short."""
    L = K.shape[1]
    if L < sink_len + obs_len + block_size:
        return None, 0
    K_mid = K[:, sink_len:L - obs_len, :]
    L_mid = K_mid.shape[1]
    aligned = int(math.ceil(max(1, L_mid) / block_size) * block_size)
    if aligned > L_mid:
        K_mid = np.concatenate([K_mid, np.zeros((K.shape[0], aligned - L_mid, K.shape[2]), K.dtype)], axis=1)
    return K_mid, aligned // block_size


def repeat_kv(x: np.ndarray, n_rep: int) -> np.ndarray:
    """[H_kv, S, D] -> [H_kv * n_rep, S, D], head h = kv h // n_rep."""
    return np.repeat(x, n_rep, axis=0)


def maxpool3(x: np.ndarray) -> np.ndarray:
    left = np.concatenate([[-np.inf], x[:-1]])
    right = np.concatenate([x[1:], [-np.inf]])
    return np.maximum(np.maximum(left, x), right)


def score_layer_blocks(K, Q_obs, *, sink_len: int, obs_len: int, n_rep: int, block_size: int = 16,
                       scale: float = None) -> np.ndarray:
    """K [H_kv, L, D], Q_obs [H_q, obs, D] (any float dtype) -> float64 [N] block scores."""
    K = np.asarray(K, dtype=np.float64)
    Q = np.asarray(Q_obs, dtype=np.float64)
    scale = K.shape[2] ** -0.5 if scale is None else scale
    K_mid, N = mid_keys(K, sink_len, obs_len, block_size)
    if N == 0:
        return np.empty(0)
    Ke = repeat_kv(K_mid, n_rep)                       # [H_q, aligned, D]
    S = np.matmul(Q, Ke.transpose(0, 2, 1)) * scale    # [H_q, obs, aligned]
    S -= S.max(axis=-1, keepdims=True)
    A = np.exp(S)
    A /= A.sum(axis=-1, keepdims=True)
    s = A.mean(axis=1).max(axis=0)                      # [aligned]
    blocks = s.reshape(N, block_size).sum(axis=-1)
    return maxpool3(blocks) if N >= 3 else blocks


def obs_row_stats(K, Q_obs, *, sink_len: int, obs_len: int, n_rep: int, block_size: int = 16,
                  scale: float = None) -> np.ndarray:
    """K [H_kv, L, D], Q_obs [H_q, obs, D] -> float64 [H_q, obs]: log2 sum_j 2^(s_j * scale * log2 e)
    over the zero-padded middle keys j (the softmax normaliser of :586-587 in log2 units)."""
    K = np.asarray(K, dtype=np.float64)
    Q = np.asarray(Q_obs, dtype=np.float64)
    scale = K.shape[2] ** -0.5 if scale is None else scale
    K_mid, N = mid_keys(K, sink_len, obs_len, block_size)
    if N == 0:
        return np.empty((Q.shape[0], 0))
    S = np.matmul(Q, repeat_kv(K_mid, n_rep).transpose(0, 2, 1)) * scale  # natural-log units
    m = S.max(axis=-1, keepdims=True)
    return (m[..., 0] + np.log(np.exp(S - m).sum(axis=-1))) / math.log(2.0)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Values of x rounded to "bf16" or "fp16" (nearest-even, via fp32), returned as float64."""
    x32 = np.asarray(x, dtype=np.float32)
    if dtype == "bf16":
        r = _bits.bf16_bits_to_f32(_bits.f32_to_bf16_bits(x32))
    elif dtype == "fp16":
        r = x32.astype(np.float16).astype(np.float32)
    elif dtype == "exact":
        return np.asarray(x, dtype=np.float64)
    else:
        raise ValueError(dtype)
    return r.astype(np.float64)


def score_layer_blocks_model_dtype(K, Q_obs, *, sink_len: int, obs_len: int, n_rep: int, dtype: str,
                                   block_size: int = 16, scale: float = None) -> np.ndarray:
    """core/scheduler.py:583-591 with each torch op's output rounded to the model dtype.

    torch computes matmul, softmax, mean and sum in fp32 internally and rounds their outputs
    to the tensor dtype; ``* scale`` rounds too; max and max_pool1d are exact. dtype "exact"
    reduces this to score_layer_blocks.
    """
    K = np.asarray(K, dtype=np.float64)
    Q = np.asarray(Q_obs, dtype=np.float64)
    scale = K.shape[2] ** -0.5 if scale is None else scale
    K_mid, N = mid_keys(K, sink_len, obs_len, block_size)
    if N == 0:
        return np.empty(0)
    Ke = repeat_kv(K_mid, n_rep)
    S = round_to(np.matmul(Q, Ke.transpose(0, 2, 1)), dtype)
    S = round_to(S * scale, dtype)
    S = S - S.max(axis=-1, keepdims=True)
    A = np.exp(S)
    A = round_to(A / A.sum(axis=-1, keepdims=True), dtype)
    s = round_to(A.mean(axis=1), dtype).max(axis=0)
    blocks = round_to(s.reshape(N, block_size).sum(axis=-1), dtype)
    return maxpool3(blocks) if N >= 3 else blocks


def score_layer_blocks_loops(K, Q_obs, *, sink_len: int, obs_len: int, n_rep: int, block_size: int = 16,
                             scale: float = None) -> np.ndarray:
    K = np.asarray(K, dtype=np.float64)
    Q = np.asarray(Q_obs, dtype=np.float64)
    H_kv, L, D = K.shape
    H_q, obs, _ = Q.shape
    scale = D ** -0.5 if scale is None else scale
    if L < sink_len + obs_len + block_size:
        return np.empty(0)
    L_mid = L - sink_len - obs_len
    N = -(-max(1, L_mid) // block_size)
    aligned = N * block_size
    col = [[0.0] * aligned for _ in range(H_q)]
    for h in range(H_q):
        g = h // n_rep
        for i in range(obs):
            logits = []
            for j in range(aligned):
                krow = K[g, sink_len + j] if j < L_mid else np.zeros(D)
                logits.append(sum(Q[h, i, d] * krow[d] for d in range(D)) * scale)
            mx = max(logits)
            ex = [math.exp(x - mx) for x in logits]
            tot = sum(ex)
            for j in range(aligned):
                col[h][j] += ex[j] / tot / obs
    s = [max(col[h][j] for h in range(H_q)) for j in range(aligned)]
    raw = [sum(s[n * block_size:(n + 1) * block_size]) for n in range(N)]
    if N < 3:
        return np.array(raw)
    return np.array([max(raw[max(0, n - 1):n + 2]) for n in range(N)])


def score_heads_f32(K_mid: np.ndarray, Q: np.ndarray, scale: float) -> np.ndarray:
    """K_mid [aligned, D] (one KV head, padded), Q [heads, obs, D] of its group, float32:
    the per-key max over these heads of the mean softmax weight (core/scheduler.py:587-588)."""
    S = np.matmul(Q, K_mid.T) * np.float32(scale)
    S -= S.max(axis=-1, keepdims=True)
    np.exp(S, out=S)
    S /= S.sum(axis=-1, keepdims=True)
    return S.mean(axis=1).max(axis=0)
