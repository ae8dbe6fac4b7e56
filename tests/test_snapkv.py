"""SnapKV observation-window block scores (the importance scores of retain-set selection).

Oracle: oracle/snapkv_oracle.py, a float64 restatement of core/scheduler.py:565-592, pinned
below by an explicit-loop version, closed forms (all-zero keys give uniform weights over the
padded keys; one dominant key gives ~1 at its block and its pooled neighbours), the
max-pool's definition, and the reference tests' shapes (benchmarks/tests.py:36-54,
test_block_alignment_regression.py:15-47). The reference computes these steps in the model
dtype; the kernels compute in fp32, so GPU results are compared with the float64 oracle:
|gpu - oracle| <= 1e-4 * max|oracle| + 1e-3 * |oracle| per item. The paged path must equal the
dense path on the same keys to the same bound.
"""
import math

import numpy as np
import pytest

from oracle import oracle as dec_oracle
from oracle import snapkv_oracle as so
from unifiedkv_amd import workloads

ATOL_REL_MAX, RTOL = 1e-4, 1e-3


# ------------------------------------------------------------------ CPU: the oracle, pinned
def test_loops_equal_vectorised_on_tiny_shapes():
    rng = np.random.default_rng(0)
    for (h_kv, n_rep, D, L, sink, obs) in [(2, 2, 8, 70, 8, 16), (1, 3, 4, 45, 0, 8), (2, 1, 4, 60, 4, 4),
                                           (1, 2, 4, 41, 8, 16)]:
        K = rng.standard_normal((h_kv, L, D))
        Q = rng.standard_normal((h_kv * n_rep, obs, D))
        a = so.score_layer_blocks(K, Q, sink_len=sink, obs_len=obs, n_rep=n_rep)
        b = so.score_layer_blocks_loops(K, Q, sink_len=sink, obs_len=obs, n_rep=n_rep)
        assert a.shape == b.shape and np.allclose(a, b, rtol=1e-12, atol=1e-15)


MODEL_DTYPE_CASES = [(2, 4, 64, 600, 16, 32), (4, 2, 128, 1000, 64, 64), (1, 8, 128, 333, 4, 16)]


def _model_dtype_inputs(rng, case, dtype):
    h_kv, n_rep, D, L, sink, obs = case
    code = workloads.DTYPE_CODES[dtype]
    K = dec_oracle.bits_to_f32(_bits(rng, (h_kv, L, D), dtype), code)
    Q = dec_oracle.bits_to_f32(_bits(rng, (h_kv * n_rep, obs, D), dtype), code)
    return K, Q


def test_model_dtype_exact_mode_is_the_fp64_oracle():
    rng = np.random.default_rng(1)
    K, Q = rng.standard_normal((2, 300, 64)), rng.standard_normal((8, 32, 64))
    a = so.score_layer_blocks(K, Q, sink_len=16, obs_len=32, n_rep=4)
    b = so.score_layer_blocks_model_dtype(K, Q, sink_len=16, obs_len=32, n_rep=4, dtype="exact")
    np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("case", MODEL_DTYPE_CASES)
def test_model_dtype_rounding_matches_torch_cpu_kernels(dtype, case):
    """torch's own CPU kernels running core/scheduler.py:583-591's op sequence in the model dtype
    (an implementation independent of the numpy emulation) give the same block scores."""
    import torch

    h_kv, n_rep, D, L, sink, obs = case
    rng = np.random.default_rng(L + D)
    K, Q = _model_dtype_inputs(rng, case, dtype)
    emu = so.score_layer_blocks_model_dtype(K, Q, sink_len=sink, obs_len=obs, n_rep=n_rep, dtype=dtype)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    Kt, Qt = torch.tensor(K, dtype=tdt), torch.tensor(Q, dtype=tdt)
    Km = Kt[:, sink:L - obs, :]
    aligned = math.ceil(Km.shape[1] / 16) * 16
    Km = torch.nn.functional.pad(Km, (0, 0, 0, aligned - Km.shape[1]))
    Ke = Km.repeat_interleave(n_rep, dim=0)
    attn = torch.softmax(torch.matmul(Qt, Ke.transpose(-2, -1)) * (D ** -0.5), dim=-1)
    blocks = attn.mean(dim=1).max(dim=0).values.view(aligned // 16, 16).sum(dim=-1).float()
    ref = torch.nn.functional.max_pool1d(blocks.view(1, 1, -1), kernel_size=3, stride=1, padding=1).view(-1)
    np.testing.assert_allclose(emu, ref.numpy().astype(np.float64), rtol=2.0 ** -10, atol=0)
    exact = so.score_layer_blocks(K, Q, sink_len=sink, obs_len=obs, n_rep=n_rep)
    assert np.max(np.abs(emu - exact) / exact) < 2.0 ** -6  # the model dtype's own rounding stays small


def test_maxpool_definition():
    assert so.maxpool3(np.array([1.0, 5.0, 2.0, 0.0, 3.0])).tolist() == [5.0, 5.0, 5.0, 3.0, 3.0]
    assert so.maxpool3(np.array([2.0, 1.0, 0.5])).tolist() == [2.0, 2.0, 1.0]


def test_zero_keys_give_uniform_weights_over_the_padded_keys():
    # L_mid = 50 -> 64 aligned keys (14 zero pad rows): every logit is 0, every weight 1/64,
    # every block 16/64 (and the pool keeps it).
    K = np.zeros((2, 16 + 50 + 8, 8))
    Q = np.random.default_rng(1).standard_normal((4, 8, 8))
    got = so.score_layer_blocks(K, Q, sink_len=16, obs_len=8, n_rep=2)
    assert got.shape == (4,) and np.allclose(got, 16 / 64, rtol=0, atol=1e-15)


def test_dominant_key_marks_its_block_and_pooled_neighbours():
    rng = np.random.default_rng(2)
    D, sink, obs, L = 16, 16, 16, 16 + 160 + 16
    K = rng.standard_normal((1, L, D)) * 0.01
    Q = np.zeros((2, obs, D))
    Q[..., 0] = 1.0
    j = 75  # mid key 75 -> block 4
    K[0, sink + j, 0] = 400.0
    got = so.score_layer_blocks(K, Q, sink_len=sink, obs_len=obs, n_rep=2)
    assert got.shape == (10,)
    assert np.all(got[3:6] > 0.999) and np.all(np.delete(got, [3, 4, 5]) < 1e-3)


@pytest.mark.parametrize("n_rep,obs,L", [(1, 8, 16 + 70 + 8), (4, 16, 16 + 96 + 16), (2, 5, 16 + 33 + 5)])
def test_score_heads_f32_matches_the_fp64_steps(n_rep, obs, L):
    """The scores CPU baseline's fp32 formulation, per KV group, equals the per-key head maximum of
    the fp64 steps: weights rebuilt from the pinned row normalisers (obs_row_stats), averaged over
    the queries and maximised over the group's heads; block sums and maxpool3 of the maximum over
    groups then give score_layer_blocks."""
    rng = np.random.default_rng(obs + L)
    H_kv, D, sink = 2, 16, 16
    K = rng.standard_normal((H_kv, L, D)).astype(np.float32)
    Q = rng.standard_normal((H_kv * n_rep, obs, D)).astype(np.float32) * 2
    scale = D ** -0.5
    K_mid, N = so.mid_keys(K.astype(np.float64), sink, obs, 16)
    lse2 = so.obs_row_stats(K, Q, sink_len=sink, obs_len=obs, n_rep=n_rep, scale=scale)  # [H_q, obs]
    per_group = []
    for g in range(H_kv):
        heads = slice(g * n_rep, (g + 1) * n_rep)
        got = so.score_heads_f32(K_mid[g].astype(np.float32), Q[heads], scale)
        s2 = np.matmul(Q[heads].astype(np.float64), K_mid[g].T) * scale / math.log(2.0)
        exp = np.exp2(s2 - lse2[heads][..., None]).mean(axis=1).max(axis=0)
        assert got.shape == (N * 16,)
        np.testing.assert_allclose(got, exp, rtol=0, atol=1e-6 * exp.max())
        per_group.append(got.astype(np.float64))
    s = np.max(per_group, axis=0)
    blocks = s.reshape(N, 16).sum(axis=-1)
    pooled = so.maxpool3(blocks) if N >= 3 else blocks
    ref = so.score_layer_blocks(K, Q, sink_len=sink, obs_len=obs, n_rep=n_rep, scale=scale)
    np.testing.assert_allclose(pooled, ref, rtol=1e-5, atol=0)


def test_too_short_and_block_counts_of_the_reference_tests():
    K = np.zeros((1, 16 + 16 + 15, 4))
    assert so.score_layer_blocks(K, np.zeros((1, 16, 4)), sink_len=16, obs_len=16, n_rep=1).size == 0
    # benchmarks/test_block_alignment_regression.py: L=2795, sink 16, obs 16 -> 2763 mid tokens -> 173 blocks
    assert so.mid_keys(np.zeros((1, 2795, 1)), 16, 16, 16)[1] == 173
    # benchmarks/tests.py test_2_compress: L=16500, sink 64, obs 64 -> 16372 mid tokens -> 1024 blocks
    assert so.mid_keys(np.zeros((1, 16500, 1)), 64, 64, 16)[1] == 1024


def test_block_count_entry_point_matches_the_oracle():
    from unifiedkv_amd import snapkv

    for L, sink, obs in [(2795, 16, 16), (16500, 64, 64), (47, 16, 16), (48, 16, 16), (32768, 64, 128)]:
        want = so.mid_keys(np.zeros((1, L, 1)), sink, obs, 16)[1]
        assert snapkv.block_count(L, sink, obs) == want


def test_entry_point_rejects_bad_shapes_before_any_launch():
    import ctypes

    from unifiedkv_amd import _ext

    lib = _ext.load()
    s3 = _ext.i64_array((0, 8, 8))
    s4 = _ext.i64_array((0, 0, 8, 8))
    p = 1 << 20

    def call(**kw):
        a = dict(layers=1, seqs=1, L=200, sink=16, obs=16, hq=4, hkv=2, d=64, n_rep=2, bs=16, stride=64)
        a.update(kw)
        return lib.ukv_snapkv_scores(p, s3, p, s4, None, 0, 0, a["layers"], a["seqs"], a["L"], a["sink"], a["obs"],
                                     a["hq"], a["hkv"], a["d"], a["n_rep"], a["bs"], ctypes.c_float(0.125),
                                     _ext.UKV_DTYPE_BF16, p, a["stride"], p, 1 << 30, None)

    assert call(bs=32) == _ext.UKV_ERR_INVALID_ARGUMENT          # blocks are 16-token pages
    assert call(hq=6) == _ext.UKV_ERR_INVALID_ARGUMENT           # H_q != H_kv * n_rep
    assert call(layers=300, seqs=300) == _ext.UKV_ERR_INVALID_ARGUMENT
    assert call(stride=5) == _ext.UKV_ERR_INVALID_ARGUMENT       # row stride below N
    assert call(L=16 + 16 + 15) == _ext.UKV_OK                   # too short: nothing to do
    assert lib.ukv_snapkv_workspace_bytes(1, 1, 200, 16, 16, 4, 2, 64, 2, 32) == 0


def test_copy_2d_rejects_bad_pitches():
    from unifiedkv_amd import _ext

    lib = _ext.load()
    assert lib.ukv_copy_2d(None, 0, None, 0, 0, 5, None) == _ext.UKV_OK       # empty
    assert lib.ukv_copy_2d(None, 64, 1 << 20, 64, 64, 1, None) == _ext.UKV_ERR_INVALID_ARGUMENT
    assert lib.ukv_copy_2d(1 << 20, 32, 1 << 21, 64, 64, 2, None) == _ext.UKV_ERR_INVALID_ARGUMENT


# ------------------------------------------------------------------------------ GPU
def _bits(rng, shape, dtype):
    return workloads._round_bits(rng.standard_normal(shape, dtype=np.float32), dtype)


def _dev(bits, dtype):
    import torch

    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to("cuda").view(tdt)


def _f(bits, dtype):
    return dec_oracle.bits_to_f32(bits, workloads.DTYPE_CODES[dtype])


def _assert_scores(got, want, what):
    assert got.shape == want.shape, f"{what}: shape {got.shape} vs {want.shape}"
    if want.size == 0:
        return
    err = np.abs(got - want)
    bound = ATOL_REL_MAX * np.abs(want).max() + RTOL * np.abs(want)
    assert np.all(err <= bound), f"{what}: max err {err.max():.3e}, worst excess {(err - bound).max():.3e}"


DENSE_CASES = [
    # h_kv, n_rep, D, L, sink, obs      path
    (8, 4, 128, 1000, 64, 64),        # tiled, 2 row tiles per wave
    (8, 4, 128, 1100, 64, 128),       # tiled, 4 row tiles per wave (512 rows)
    (2, 8, 128, 700, 16, 128),        # tiled, heads split into 2 units per group
    (4, 4, 64, 500, 16, 32),          # tiled, D=64
    (4, 4, 128, 900, 32, 48),         # tiled, 3 tiles per head: 1 row tile per wave, 2 heads per unit
    (2, 4, 64, 777, 16, 80),          # tiled, 5 tiles per head: 1 row tile per wave, 1 head per unit
    (2, 4, 128, 1234, 0, 96),         # tiled, 6 tiles per head: 2 row tiles per wave, 2 heads per unit
    (2, 8, 128, 640, 16, 16),         # tiled, 1 tile per head: 8 heads per unit
    (8, 4, 32, 2795, 16, 16),         # scalar (D=32): the reference's block-alignment test shape
    (2, 2, 64, 300, 8, 24),           # scalar (obs not a multiple of 16)
    (4, 2, 128, 64 + 64 + 16, 64, 64),  # N = 1
    (4, 2, 128, 64 + 64 + 20, 64, 64),  # N = 2 (12 zero pad keys)
    (4, 2, 128, 64 + 64 + 40, 64, 64),  # N = 3 (pool on)
]


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("case", DENSE_CASES)
def test_dense_scores_match_oracle(cuda, dtype, case):
    from unifiedkv_amd import snapkv

    h_kv, n_rep, D, L, sink, obs = case
    rng = np.random.default_rng(L + D)
    K = _bits(rng, (h_kv, L, D), dtype)
    Q = _bits(rng, (h_kv * n_rep, obs, D), dtype)
    got = snapkv.score_layer_blocks(_dev(K, dtype), _dev(Q, dtype), sink_len=sink, obs_len=obs, n_rep=n_rep)
    want = so.score_layer_blocks(_f(K, dtype), _f(Q, dtype), sink_len=sink, obs_len=obs, n_rep=n_rep)
    _assert_scores(got.cpu().numpy(), want, f"{case} {dtype}")


@pytest.mark.gpu
def test_too_short_gives_empty_and_views_are_accepted(cuda):
    import torch

    from unifiedkv_amd import snapkv

    rng = np.random.default_rng(9)
    K = _dev(_bits(rng, (4, 100, 128), "bf16"), "bf16")
    Q = _dev(_bits(rng, (16, 64, 128), "bf16"), "bf16")
    assert snapkv.score_layer_blocks(K[:, :64 + 64 + 15], Q, sink_len=64, obs_len=64, n_rep=4).numel() == 0
    with pytest.raises(RuntimeError, match="selected_writeback_bad_score_shape"):
        snapkv.score_layer_blocks(K[0], Q, sink_len=64, obs_len=64, n_rep=4)
    # a [H_kv, L, D] view of a [L, H_kv, D] buffer (token-major, as the pool stores rows)
    Kt = K.transpose(0, 1).contiguous().transpose(0, 1)
    a = snapkv.score_layer_blocks(K, Q, sink_len=16, obs_len=64, n_rep=4)
    b = snapkv.score_layer_blocks(Kt, Q, sink_len=16, obs_len=64, n_rep=4)
    assert torch.equal(a, b)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_paged_multi_item_scores_match_oracle(cuda, dtype):
    import torch

    from unifiedkv_amd import snapkv

    rng = np.random.default_rng(21)
    layers, seqs, h_kv, n_rep, D, L, sink, obs = 3, 2, 4, 4, 128, 1500, 64, 64
    pages = -(-L // 16)
    N = seqs * pages + 7
    pool = _bits(rng, (layers, N, 16, h_kv, D), dtype)
    perm = rng.permutation(N)[: seqs * pages].astype(np.int32).reshape(seqs, pages)
    table = np.zeros((seqs, pages + 3), np.int32)
    table[:, :pages] = perm
    q = _bits(rng, (seqs, layers, h_kv * n_rep, obs, D), dtype)
    got = snapkv.score_blocks(_dev(q, dtype), _dev(pool, dtype), torch.from_numpy(table).cuda(), seq_len=L,
                              sink_len=sink, obs_len=obs, n_rep=n_rep).cpu().numpy()
    assert got.shape == (seqs * layers, snapkv.block_count(L, sink, obs))
    pf = _f(pool, dtype)
    for b in range(seqs):
        for l in range(layers):
            dense = pf[l][perm[b]].reshape(pages * 16, h_kv, D)[:L].transpose(1, 0, 2)  # [H_kv, L, D]
            want = so.score_layer_blocks(dense, _f(q[b, l], dtype), sink_len=sink, obs_len=obs, n_rep=n_rep)
            _assert_scores(got[b * layers + l], want, f"paged item seq {b} layer {l}")


@pytest.mark.gpu
def test_config5_shape_sampled_items(cuda):
    # 32K-token sequences with sink 64 / obs 128 (config 5): 4 layers x 2 sequences scored in
    # one call; two items are checked against the oracle, every item for shape, finiteness
    # and non-negativity.
    import torch

    from unifiedkv_amd import snapkv

    rng = np.random.default_rng(5)
    layers, seqs, h_kv, n_rep, D, L, sink, obs = 4, 2, 8, 4, 128, 32768, 64, 128
    pages = L // 16
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    pool = torch.randn((layers, seqs * pages + 16, 16, h_kv, D), generator=g, device="cuda").to(torch.bfloat16)
    perm = torch.from_numpy(rng.permutation(seqs * pages + 16)[: seqs * pages].astype(np.int32).reshape(seqs, pages))
    q = torch.randn((seqs, layers, h_kv * n_rep, obs, D), generator=g, device="cuda").to(torch.bfloat16)
    got = snapkv.score_blocks(q, pool, perm.cuda(), seq_len=L, sink_len=sink, obs_len=obs, n_rep=n_rep)
    got = got.cpu().numpy()
    assert got.shape == (seqs * layers, (L - sink - obs) // 16) and np.isfinite(got).all() and (got >= 0).all()
    for b, l in [(0, 0), (1, 3)]:
        dense = pool[l][perm[b].long().cuda()].reshape(pages * 16, h_kv, D).transpose(0, 1).float().cpu().numpy()
        want = so.score_layer_blocks(dense, q[b, l].float().cpu().numpy(), sink_len=sink, obs_len=obs, n_rep=n_rep)
        _assert_scores(got[b * layers + l], want, f"config-5 item seq {b} layer {l}")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_scores_and_selection_against_the_reference_dtype_arithmetic(cuda, dtype):
    """The kernel computes exact fp32 scores; the reference rounds every step to the model dtype
    (core/scheduler.py:586-588). Bound the gap: scores within 1 % of the model-dtype emulation,
    and the 20 % top-k blocks chosen from either agree except for blocks whose reference score
    lies within that 1 % of the k-th largest."""
    from unifiedkv_amd import compaction, snapkv
    import torch

    h_kv, n_rep, D, L, sink, obs = 8, 4, 128, 8192, 64, 128
    rng = np.random.default_rng(77)
    Kb, Qb = _bits(rng, (h_kv, L, D), dtype), _bits(rng, (h_kv * n_rep, obs, D), dtype)
    got = snapkv.score_layer_blocks(_dev(Kb, dtype), _dev(Qb, dtype), sink_len=sink, obs_len=obs, n_rep=n_rep)
    emu = so.score_layer_blocks_model_dtype(_f(Kb, dtype), _f(Qb, dtype), sink_len=sink, obs_len=obs, n_rep=n_rep,
                                            dtype=dtype)
    g = got.cpu().numpy().astype(np.float64)
    assert np.max(np.abs(g - emu) / emu) < 1e-2
    k = int(0.2 * emu.size)
    mine = set(compaction.select_blocks(got.view(1, -1).float().contiguous(), k).cpu().numpy()[0].tolist())
    ref = set(np.argsort(-emu, kind="stable")[:k].tolist())
    kth = np.sort(emu)[::-1][k - 1]
    for i in mine ^ ref:
        assert abs(emu[i] - kth) <= 1e-2 * kth, f"block {i}: {emu[i]} vs k-th {kth}"
