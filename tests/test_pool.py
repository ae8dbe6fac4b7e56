"""Drop-in PagedKVPool (core/pool.py) and the page-movement kernels, checked bit-exact.

The oracle is oracle/pool_oracle.py, a restatement of core/pool.py:36-189 and
core/scheduler.py:401-408 on host arrays. CPU tests cover the host logic (FIFO
allocation order, watermarks, sizing, table packing); tests marked gpu cover
the kernels (token scatter/gather, page copy, decode append) and the device
block tables.
"""
import numpy as np
import pytest
import torch

from oracle import pool_oracle
from unifiedkv_amd.pool import PagedKVPool, pack_block_table


# ----------------------------------------------------------------- CPU: host logic
def test_fifo_allocation_matches_reference_under_random_ops():
    rng = np.random.default_rng(0)
    N = 200
    pool = PagedKVPool(16, 2, 8, 64, num_blocks=N)
    ref = pool_oracle.FifoAllocator(N)
    held = []
    for step in range(2000):
        op = rng.integers(0, 4)
        if op < 2:
            n = int(rng.integers(0, 40))
            a, b = pool.allocate_blocks(n), ref.allocate_blocks(n)
            assert a == b
            held.extend(a)
        elif op == 2 and held:
            k = int(rng.integers(1, len(held) + 1))
            idx = rng.choice(len(held), size=k, replace=False)
            ids = [held[i] for i in idx]
            held = [h for i, h in enumerate(held) if i not in set(idx.tolist())]
            pool.free_blocks_by_ids(ids)
            ref.free_blocks_by_ids(ids)
        else:
            n_req = int(rng.integers(0, N))
            assert pool.check_watermark(n_req) == ref.check_watermark(n_req)
        assert pool.n_free == ref.n_free
        assert pool.free_blocks == ref.free_blocks
        assert pool.used_blocks == ref.used_blocks


def test_allocation_edge_semantics():
    pool, ref = PagedKVPool(16, 1, 1, 8, num_blocks=10), pool_oracle.FifoAllocator(10)
    assert pool.allocate_blocks(11) == ref.allocate_blocks(11) == []
    assert pool.allocate_blocks(0) == ref.allocate_blocks(0) == []
    assert pool.allocate_blocks(-3) == ref.allocate_blocks(-3)  # list-slice semantics free[:n]
    assert pool.free_blocks == ref.free_blocks
    pool.free_blocks_by_ids([4, 4])  # freeing twice appends twice, as the reference does
    ref.free_blocks_by_ids([4, 4])
    assert pool.free_blocks == ref.free_blocks
    assert (pool.N_wm_low, pool.N_wm_high) == (ref.N_wm_low, ref.N_wm_high)


def test_pool_sizing_formula(monkeypatch):
    class Props:
        total_memory = 288 * 1024**3

    monkeypatch.setattr(torch.cuda, "get_device_properties", lambda dev=None: Props())
    monkeypatch.setattr(torch.cuda, "memory_allocated", lambda dev=None: 16 * 1024**3)
    # Known answers of core/pool.py:36-45 worked by hand: 288 GiB total, 16 GiB in use, a 10 %
    # reserve of 28.8 GiB leaves 243.2 GiB; one block of 32 layers x 16 tokens x 8 heads x 128
    # x 2 B x (K, V) is 2 MiB, i.e. 512 blocks per GiB: 243.2 * 512 * frac blocks, floored.
    # frac 0.2 -> 24903.68 -> 24903; frac 0.75 -> 93388.8 -> 93388.
    for frac, n_total in ((0.2, 24903), (0.75, 93388)):
        pool = PagedKVPool(16, 32, 8, 128, torch.float16, frac, 48.0)
        assert pool.N_total == n_total
        assert pool_oracle.pool_size(288 * 1024**3, 16 * 1024**3, frac, 32, 16, 8, 128) == n_total
        assert (pool.N_wm_low, pool.N_wm_high) == (int(0.15 * n_total), int(0.40 * n_total))
        assert pool.cpu_budget == int(48.0 * 1024**3) and pool.cpu_used_bytes == 0
        assert not pool.is_allocated
    # Less free memory than one block still yields one block (the max(1, .) of :45).
    monkeypatch.setattr(torch.cuda, "memory_allocated", lambda dev=None: 288 * 1024**3 - 2 * 1024**2)
    assert PagedKVPool(16, 32, 8, 128, torch.float16, 0.75, 48.0).N_total == 1
    assert pool_oracle.pool_size(288 * 1024**3, 288 * 1024**3 - 2 * 1024**2, 0.75, 32, 16, 8, 128) == 1


@pytest.mark.parametrize("lens", [[3, 0, 7], [1], [2048] * 4, [5, 128, 33]])
def test_block_table_packing(lens):
    rng = np.random.default_rng(sum(lens))
    lists = [rng.integers(0, 10_000, n).tolist() for n in lens]
    got = pack_block_table(lists)
    exp = pool_oracle.build_block_table(lists)
    assert got.dtype == np.int32 and got.shape == exp.shape
    np.testing.assert_array_equal(got, exp)


# -------------------------------------------------------------- GPU: the kernels
def _rand16(shape, dtype, g):
    return torch.randn(shape, generator=g, dtype=torch.float32).to(dtype)


def _np(t):
    return t.view(torch.int16).cpu().numpy()


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("T", [800, 1, 15, 16, 17, 500])
def test_write_read_tokens_bit_exact(cuda, dtype, T):
    g = torch.Generator().manual_seed(T)
    pool = PagedKVPool(16, 3, 8, 128, dtype, num_blocks=300, device=cuda)
    pool.k_cache.copy_(_rand16(pool.k_cache.shape, dtype, g).to(cuda))
    pool.v_cache.copy_(_rand16(pool.v_cache.shape, dtype, g).to(cuda))
    before_k = _np(pool.k_cache[1]).copy()
    before_v = _np(pool.v_cache[1]).copy()
    n_ids = (T + 15) // 16 + 2  # extra ids beyond the data are ignored
    ids = pool.allocate_blocks(n_ids)
    ids = list(np.random.default_rng(T).permutation(ids))
    K = _rand16((8, T, 128), dtype, g)
    V = _rand16((8, T, 128), dtype, g)
    pool.write_kv_to_blocks(1, ids, K.to(cuda), V.to(cuda))
    pool_oracle.write_kv_to_blocks(before_k, ids, _np(K))
    pool_oracle.write_kv_to_blocks(before_v, ids, _np(V))
    np.testing.assert_array_equal(_np(pool.k_cache[1]), before_k)  # includes untouched slots and pages
    np.testing.assert_array_equal(_np(pool.v_cache[1]), before_v)
    for seq_len in (T, T - 1, 16 * n_ids + 5, 0):
        Kr, Vr = pool.read_kv_from_blocks(1, ids, seq_len)
        np.testing.assert_array_equal(_np(Kr), pool_oracle.read_kv_from_blocks(before_k, ids, seq_len))
        np.testing.assert_array_equal(_np(Vr), pool_oracle.read_kv_from_blocks(before_v, ids, seq_len))
    assert pool.k_cache.shape == (3, 300, 16, 8, 128)


@pytest.mark.gpu
def test_write_from_cpu_fp32_source_converts_like_torch(cuda):
    pool = PagedKVPool(16, 1, 2, 64, torch.bfloat16, num_blocks=8, device=cuda)
    ids = pool.allocate_blocks(2)
    K = torch.randn(2, 20, 64)
    V = torch.randn(2, 20, 64)
    pool.write_kv_to_blocks(0, ids, K, V)
    Kr, _ = pool.read_kv_from_blocks(0, ids, 20)
    assert torch.equal(Kr.cpu(), K.to(torch.bfloat16))


@pytest.mark.gpu
def test_reference_pool_round_trip(cuda):
    """benchmarks/tests.py:12-33 (test_1_pool): 50 blocks, 8 heads, 800 tokens, fp16 round trip."""
    pool = PagedKVPool(16, 4, 8, 128, torch.float16, num_blocks=1000, device=cuda)
    ids = pool.allocate_blocks(50)
    assert len(ids) == 50
    K = torch.randn(8, 50 * 16, 128, device=cuda, dtype=torch.float16)
    V = torch.randn_like(K)
    pool.write_kv_to_blocks(0, ids, K, V)
    K_r, V_r = pool.read_kv_from_blocks(0, ids, 50 * 16)
    assert torch.equal(K, K_r) and torch.equal(V, V_r)
    pool.free_blocks_by_ids(ids)
    assert pool.n_free == pool.N_total


@pytest.mark.gpu
@pytest.mark.parametrize("per_layer_src", [True, False])
def test_page_copy_bit_exact(cuda, per_layer_src):
    g = torch.Generator().manual_seed(5)
    pool = PagedKVPool(16, 4, 8, 128, torch.bfloat16, num_blocks=64, device=cuda)
    pool.k_cache.copy_(_rand16(pool.k_cache.shape, torch.bfloat16, g).to(cuda))
    pool.v_cache.copy_(_rand16(pool.v_cache.shape, torch.bfloat16, g).to(cuda))
    rng = np.random.default_rng(1)
    src_pages = rng.permutation(32)[:10]  # sources in 0..31, destinations in 32..63
    dst = rng.permutation(np.arange(32, 64))[:10].astype(np.int32)
    if per_layer_src:
        src = np.stack([rng.permutation(src_pages) for _ in range(4)]).astype(np.int32)
    else:
        src = src_pages.astype(np.int32)
    k0, v0 = _np(pool.k_cache).copy(), _np(pool.v_cache).copy()
    pool.copy_pages(torch.from_numpy(src), torch.from_numpy(dst))
    for l in range(4):
        s = src[l] if per_layer_src else src
        k0[l, dst] = k0[l, s]
        v0[l, dst] = v0[l, s]
    np.testing.assert_array_equal(_np(pool.k_cache), k0)
    np.testing.assert_array_equal(_np(pool.v_cache), v0)


@pytest.mark.gpu
@pytest.mark.parametrize("bs", [16, 8])
def test_decode_append_matches_scheduler_scatter(cuda, bs):
    g = torch.Generator().manual_seed(bs)
    B, H, D, N = 6, 8, 128, 80
    pool = PagedKVPool(bs, 2, H, D, torch.float16, num_blocks=N, device=cuda)
    pool.k_cache.copy_(_rand16(pool.k_cache.shape, torch.float16, g).to(cuda))
    pool.v_cache.copy_(_rand16(pool.v_cache.shape, torch.float16, g).to(cuda))
    rng = np.random.default_rng(bs)
    old = np.array([0, bs - 1, bs, 3 * bs + 2, 5 * bs - 1, 7], dtype=np.int32)
    lists = [pool.allocate_blocks(int(L) // bs + 1) for L in old]
    bt = pack_block_table(lists)
    k_new = _rand16((B, 1, H, D), torch.float16, g)
    v_new = _rand16((B, 1, H, D), torch.float16, g)
    k0, v0 = _np(pool.k_cache[1]).copy(), _np(pool.v_cache[1]).copy()
    exp_lens = pool_oracle.kv_append(k0, v0, bt, old, _np(k_new)[:, 0], _np(v_new)[:, 0], block_size=bs)
    lens = pool.append_decode_tokens(1, torch.from_numpy(bt).to(cuda), torch.from_numpy(old).to(cuda),
                                     k_new.to(cuda), v_new.to(cuda))
    np.testing.assert_array_equal(lens.cpu().numpy(), exp_lens)
    np.testing.assert_array_equal(_np(pool.k_cache[1]), k0)
    np.testing.assert_array_equal(_np(pool.v_cache[1]), v0)


@pytest.mark.gpu
def test_build_block_table_contents_and_reuse(cuda):
    pool = PagedKVPool(16, 3, 8, 128, num_blocks=500, device=cuda)
    lists = [pool.allocate_blocks(n) for n in (5, 17, 1)]
    k0, v0, t0 = pool.build_block_table(0, [list(x) for x in lists])
    np.testing.assert_array_equal(t0.cpu().numpy(), pool_oracle.build_block_table(lists))
    assert t0.dtype == torch.int32 and t0.device == cuda
    assert k0.data_ptr() == pool.k_cache[0].data_ptr() and v0.shape == (500, 16, 8, 128)
    _, _, t1 = pool.build_block_table(1, [list(x) for x in lists])  # same lists, next layer
    assert t1 is t0
    old_table = pool_oracle.build_block_table(lists)
    lists[1].append(pool.allocate_blocks(1)[0])  # a decode step crossed a page boundary
    _, _, t2 = pool.build_block_table(0, [list(x) for x in lists])
    assert t2 is not t0
    np.testing.assert_array_equal(t2.cpu().numpy(), pool_oracle.build_block_table(lists))
    np.testing.assert_array_equal(t0.cpu().numpy(), old_table)  # an earlier table is never rewritten
