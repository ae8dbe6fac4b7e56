"""Retain-set selection and compaction (rows a6 / a7), bit-exact.

Known answers from the reference's own tests:
* benchmarks/test_block_alignment_regression.py:15-47 - L=2795, sink=obs=16, budget 2048:
  mid 2763 tokens, aligned 2768, 173 blocks, output exactly 2048 tokens, max index < 173;
* benchmarks/tests.py:36-54 with core/compress.py:37-42 - L=16500, sink=obs=64, r=0.2:
  1024 blocks (ceil alignment), k=204, L_final=3392, ratio in (0.10, 0.40).
L=32768, sink 64, window 128, r=0.2 -> 2036 middle blocks, k=407, 419 pages.
The selection oracle is pinned against a brute-force definition of the tie rule.
"""
import itertools

import numpy as np
import pytest
import torch

from oracle import compaction_oracle as co
from oracle import pool_oracle
from unifiedkv_amd import compaction


# ---------------------------------------------------------------- CPU: arithmetic
def test_kat_block_alignment_regression():
    d = co.snapkv_arithmetic(2795, block_size=16, sink_len=16, obs_len=16, retain_budget_tokens=2048)
    assert d["mid_tokens_before_align"] == 2795 - 16 - 16 == 2763
    assert d["mid_tokens_aligned"] == 2768 and d["mid_block_count"] == 173
    assert d["effective_retained_tokens"] == 2048
    k, eff, mode = compaction.selection_budget_blocks(2795, block_size=16, sink_len=16, obs_len=16,
                                                      retain_budget_tokens=2048)
    assert (k, eff, mode) == (126, 2048, "fixed_budget") and k < 173


def test_kat_tests_py_compress_ratio():
    d = co.snapkv_arithmetic(16500, block_size=16, sink_len=64, obs_len=64, retain_ratio=0.20)
    assert d["mid_block_count"] == 1024 and d["retained_block_count"] == 204
    assert d["effective_retained_tokens"] == 3392
    assert 0.10 < 3392 / 16500 < 0.40
    k, eff, mode = compaction.selection_budget_blocks(16500, block_size=16, sink_len=64, obs_len=64,
                                                      retain_ratio=0.20)
    assert (k, eff, mode) == (204, 3392, "ratio")


def test_config5_budget():
    k, eff, mode = compaction.selection_budget_blocks(32768, block_size=16, sink_len=64, obs_len=128,
                                                      retain_ratio=0.20)
    assert (k, eff, mode) == (407, 6704, "ratio") and eff // 16 == 419


@pytest.mark.parametrize("L,Ls,Lo,r,budget", itertools.product(
    [0, 15, 47, 48, 49, 300, 2795, 16500, 32768], [0, 16, 64], [16, 128], [0.1, 0.2, 1.0], [0, 1024, 2048]))
def test_budget_invariants(L, Ls, Lo, r, budget):
    k, eff, mode = compaction.selection_budget_blocks(L, block_size=16, sink_len=Ls, obs_len=Lo, retain_ratio=r,
                                                      retain_budget_tokens=budget)
    assert (k, eff, mode) == co.selection_budget(L, 16, Ls, Lo, r, budget)
    if mode in ("input_le_budget", "too_short"):
        assert (k, eff) == (0, L)
        return
    mid_blocks = -(-(L - Ls - Lo) // 16)
    assert 0 <= k <= mid_blocks and eff == Ls + 16 * k + Lo
    if mode == "fixed_budget":
        assert eff <= max(budget, Ls + Lo)
    else:
        assert k >= 1


def _brute_topk(row, k):
    """i wins iff fewer than k elements beat it; j beats i iff it ranks higher (NaN > numbers),
    or ties with i and has the lower index."""
    n = len(row)

    def rank_key(x):
        return (1, 0.0) if np.isnan(x) else (0, float(x))

    sel = []
    for i in range(n):
        beats = sum(1 for j in range(n) if rank_key(row[j]) > rank_key(row[i])
                    or (rank_key(row[j]) == rank_key(row[i]) and j < i))
        if beats < k:
            sel.append(i)
    return sel


@pytest.mark.parametrize("seed", range(6))
def test_selection_oracle_matches_brute_force(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 40))
    row = rng.integers(0, 5, n).astype(np.float32)  # many ties
    if seed % 2:
        row[rng.integers(0, n)] = np.nan
    for k in range(0, n + 1):
        assert co.select_topk(row[None], k)[0].tolist() == _brute_topk(row, k)


def test_retained_pages_layout_config5():
    sel = np.sort(np.random.default_rng(0).permutation(2036)[:407]).astype(np.int32)[None]
    keep = co.retained_pages(32768, sel, 16, 64, 128)
    assert keep.shape == (1, 419)
    assert keep[0, :4].tolist() == [0, 1, 2, 3] and keep[0, -8:].tolist() == list(range(2040, 2048))
    assert (np.diff(keep[0]) > 0).all()


# ------------------------------------------------------------------- GPU kernels
@pytest.mark.gpu
@pytest.mark.parametrize("n,k", [(2036, 407), (1, 1), (300, 0), (300, 300), (257, 100), (5000, 1234), (64, 63)])
def test_select_kernel_matches_oracle(cuda, n, k):
    rng = np.random.default_rng(n + k)
    scores = rng.random((12, n), dtype=np.float32)
    scores[3] = np.round(scores[3] * 4) / 4  # heavy ties
    scores[4] = 0.5  # all equal
    scores[5, ::7] = np.nan
    scores[6] = -scores[6]
    got = compaction.select_blocks(torch.from_numpy(scores).to(cuda), k).cpu().numpy()
    np.testing.assert_array_equal(got, co.select_topk(scores, k))


@pytest.mark.gpu
def test_select_kernel_ragged_rows(cuda):
    rng = np.random.default_rng(9)
    scores = rng.random((8, 600), dtype=np.float32)
    n_valid = np.array([600, 1, 0, 17, 599, 256, 300, 42], dtype=np.int32)
    k_row = np.array([100, 5, 3, 17, 0, 256, 150, 40], dtype=np.int32)
    got = compaction.select_blocks(torch.from_numpy(scores).to(cuda), 200, torch.from_numpy(n_valid),
                                   torch.from_numpy(k_row)).cpu().numpy()
    for r in range(8):
        kk = min(int(k_row[r]), int(n_valid[r]), 200)
        exp = co.select_topk(scores[r:r + 1, : n_valid[r]], kk)[0] if kk > 0 else np.zeros(0, np.int32)
        np.testing.assert_array_equal(got[r, :kk], exp)
        assert (got[r, kk:] == -1).all()


@pytest.mark.gpu
def test_config5_selection_full_size(cuda):
    """32 layers x 8 sequences, 2036 middle blocks, U(0,1) scores, k=407 per row."""
    rng = np.random.default_rng(55)
    scores = rng.random((32 * 8, 2036), dtype=np.float32)
    got = compaction.select_blocks(torch.from_numpy(scores).to(cuda), 407).cpu().numpy()
    np.testing.assert_array_equal(got, co.select_topk(scores, 407))


@pytest.mark.gpu
def test_compaction_bit_exact(cuda):
    from unifiedkv_amd.pool import PagedKVPool

    L, seqs, pages_per_seq, N = 4, 3, 40, 200
    pool = PagedKVPool(16, L, 8, 128, torch.bfloat16, num_blocks=N, device=cuda)
    g = torch.Generator().manual_seed(3)
    pool.k_cache.copy_(torch.randn(pool.k_cache.shape, generator=g).to(torch.bfloat16).to(cuda))
    pool.v_cache.copy_(torch.randn(pool.v_cache.shape, generator=g).to(torch.bfloat16).to(cuda))
    ref_alloc = pool_oracle.FifoAllocator(N)
    lists = []
    rng = np.random.default_rng(4)
    for _ in range(seqs):  # interleave allocations so page lists are fragmented
        ids = pool.allocate_blocks(pages_per_seq)
        assert ids == ref_alloc.allocate_blocks(pages_per_seq)
        lists.append(ids)
    freed = lists[1][::3]
    pool.free_blocks_by_ids(freed)
    ref_alloc.free_blocks_by_ids(freed)
    T = pages_per_seq * 16
    k_blocks, eff, _ = compaction.selection_budget_blocks(T, sink_len=32, obs_len=48, retain_ratio=0.25)
    scores = rng.random((L * seqs, pages_per_seq - 5), dtype=np.float32)
    sel = compaction.select_blocks(torch.from_numpy(scores).to(cuda), k_blocks)
    retained = [compaction.retained_pages(T, sel[s * L:(s + 1) * L], sink_len=32, obs_len=48) for s in range(seqs)]
    k_np = pool.k_cache.view(torch.int16).cpu().numpy()
    v_np = pool.v_cache.view(torch.int16).cpu().numpy()
    res = compaction.compact(pool, lists, retained, [eff] * seqs)
    sel_np = co.select_topk(scores, k_blocks)
    ret_np = [co.retained_pages(T, sel_np[s * L:(s + 1) * L], 16, 32, 48) for s in range(seqs)]
    for a, b in zip(retained, ret_np):
        np.testing.assert_array_equal(a.cpu().numpy(), b)
    exp_lists = co.compact(k_np, v_np, ref_alloc, lists, ret_np)
    assert res.page_lists == exp_lists
    np.testing.assert_array_equal(pool.k_cache.view(torch.int16).cpu().numpy(), k_np)
    np.testing.assert_array_equal(pool.v_cache.view(torch.int16).cpu().numpy(), v_np)
    np.testing.assert_array_equal(res.block_table.cpu().numpy(), pool_oracle.build_block_table(exp_lists))
    assert pool.free_blocks == ref_alloc.free_blocks


@pytest.mark.gpu
def test_compaction_rolls_back_when_the_pool_is_short(cuda):
    from unifiedkv_amd.pool import PagedKVPool

    pool = PagedKVPool(16, 2, 2, 64, torch.float16, num_blocks=30, device=cuda)
    lists = [pool.allocate_blocks(10), pool.allocate_blocks(10)]
    before = pool.free_blocks
    keep = [torch.arange(6, dtype=torch.int32).expand(2, -1), torch.arange(8, dtype=torch.int32).expand(2, -1)]
    with pytest.raises(MemoryError):
        compaction.compact(pool, lists, [k.to(cuda) for k in keep], [96, 128])  # needs 14 of 10 free
    assert sorted(pool.free_blocks) == sorted(before)
