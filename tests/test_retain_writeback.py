"""Token-granular retain-set writeback and pool->pool compaction (row a7), bit-exact.

The oracle restates the reference's writeback step by step (core/scheduler.py:666-799,
805-878; core/offload.py:1236-1262). It is pinned here, on the CPU, by:
* the compressor's own tensor result (core/compress.py:99-175, restated as pad / gather / cat in
  ``compress_tensors``): the pages the piecewise writeback fills, read back in order, must hold
  exactly that token sequence, whatever the alignment of L, the sink and the window;
* the reference's regression shape (benchmarks/test_block_alignment_regression.py:15-47):
  L=2795, sink=window=16, budget 2048 -> 126 blocks, 2048 tokens, 128 pages;
* the aligned fast path (block-indexed) and the piecewise path agreeing byte for byte;
* brute force for the prune copy (the kept spans concatenated) and its free-list order;
* planted mistakes in the oracle (padding before the piece, a window shifted by one, a
  dropped pad) that the compressor check must catch.
GPU tests then compare whole pools (every slot, written or not) and free lists with the oracle.
"""
import math

import numpy as np
import pytest
import torch

from oracle import compaction_oracle as co
from oracle import pool_oracle
from unifiedkv_amd import compaction


def _rand_kv(rng, H, L, D):
    K = rng.integers(-30000, 30000, size=(H, L, D), dtype=np.int64).astype(np.int16)
    V = rng.integers(-30000, 30000, size=(H, L, D), dtype=np.int64).astype(np.int16)
    return K, V


def _pool(rng, layers, N, H, D):
    return (rng.integers(-30000, 30000, size=(layers, N, 16, H, D), dtype=np.int64).astype(np.int16),
            rng.integers(-30000, 30000, size=(layers, N, 16, H, D), dtype=np.int64).astype(np.int16))


def _case(rng, L=None, Ls=None, Lo=None):
    L = int(rng.integers(60, 700)) if L is None else L
    Ls = int(rng.integers(0, 40)) if Ls is None else Ls
    Lo = int(rng.integers(1, 40)) if Lo is None else Lo
    n_mid = -(-(L - Ls - Lo) // 16)
    k = int(rng.integers(1, n_mid + 1))
    return L, Ls, Lo, n_mid, k


# ------------------------------------------------------------------------ CPU: the oracle
@pytest.mark.parametrize("seed", range(12))
def test_oracle_pages_hold_the_compressor_output(seed):
    rng = np.random.default_rng(seed)
    H, D = int(rng.integers(1, 4)), 8 * int(rng.integers(1, 5))
    L, Ls, Lo, n_mid, k = _case(rng)
    K, V = _rand_kv(rng, H, L, D)
    sel = np.sort(rng.permutation(n_mid)[:k])
    eff = Ls + 16 * k + Lo
    kc, vc = _pool(rng, 1, 4 * (eff // 16 + 2), H, D)
    ids = list(rng.permutation(kc.shape[1])[: -(-eff // 16)])
    co.write_selected_layer(kc[0], vc[0], ids, K, V, list(sel), eff, "ratio", Ls, Lo)
    Kf, Vf = co.compress_tensors(K, V, sel, Ls, Lo)
    assert Kf.shape[1] == eff
    np.testing.assert_array_equal(co.pool_read(kc[0], ids, eff), Kf)
    np.testing.assert_array_equal(co.pool_read(vc[0], ids, eff), Vf)


def test_oracle_regression_shape_budget_2048():
    """benchmarks/test_block_alignment_regression.py: 2795 tokens, sink = window = 16, budget 2048."""
    rng = np.random.default_rng(7)
    L, Ls, Lo = 2795, 16, 16
    k, eff, mode = co.selection_budget(L, 16, Ls, Lo, 0.2, 2048)
    assert (k, eff, mode) == (126, 2048, "fixed_budget")
    n_mid = -(-(L - Ls - Lo) // 16)
    assert n_mid == 173
    K, V = _rand_kv(rng, 8, L, 32)
    sel = np.sort(rng.permutation(n_mid)[:k])
    sel[-1] = n_mid - 1  # the partial (zero-padded) last middle block is kept
    kc, vc = _pool(rng, 1, 200, 8, 32)
    alloc = pool_oracle.FifoAllocator(200)
    ids = co.selected_writeback(kc, vc, alloc, [(K, V)], [list(sel)], eff, mode, Ls, Lo)
    assert len(ids) == 128
    Kf, _ = co.compress_tensors(K, V, sel, Ls, Lo)
    assert Kf.shape[1] == 2048
    np.testing.assert_array_equal(co.pool_read(kc[0], ids, eff), Kf)
    # the padded block: 2763 middle tokens = 172 whole blocks + 11, so 5 zero rows
    tail = co.pool_read(kc[0], ids, eff)[:, Ls + 16 * (k - 1):Ls + 16 * k]
    assert (tail[:, 11:] == 0).all() and not (tail[:, :11] == 0).all()


@pytest.mark.parametrize("seed", range(6))
def test_oracle_fast_path_equals_piecewise_path(seed):
    rng = np.random.default_rng(100 + seed)
    H, D = 2, 16
    Ls, Lo = 16 * int(rng.integers(0, 3)), 16 * int(rng.integers(1, 3))
    L = Ls + Lo + 16 * int(rng.integers(3, 30))
    n_mid = (L - Ls - Lo) // 16
    k = int(rng.integers(1, n_mid + 1))
    sel = list(np.sort(rng.permutation(n_mid)[:k]))
    K, V = _rand_kv(rng, H, L, D)
    eff = Ls + 16 * k + Lo
    a = _pool(rng, 1, 64, H, D)
    b = (a[0].copy(), a[1].copy())
    ids = list(rng.permutation(64)[: eff // 16])
    co.write_selected_layer(a[0][0], a[1][0], ids, K, V, sel, eff, "ratio", Ls, Lo, allow_fast=True)
    co.write_selected_layer(b[0][0], b[1][0], ids, K, V, sel, eff, "ratio", Ls, Lo, allow_fast=False)
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1], b[1])


def test_oracle_pass_through_modes_keep_the_prefix():
    rng = np.random.default_rng(3)
    for L, mode in ((37, "too_short"), (1000, "input_le_budget"), (64, "input_le_budget")):
        K, V = _rand_kv(rng, 2, L, 8)
        kc, vc = _pool(rng, 1, 80, 2, 8)
        ids = list(rng.permutation(80)[: -(-L // 16)])
        co.write_selected_layer(kc[0], vc[0], ids, K, V, [], L, mode, 16, 16)
        np.testing.assert_array_equal(co.pool_read(kc[0], ids, L), K)
        np.testing.assert_array_equal(co.pool_read(vc[0], ids, L), V)


def test_oracle_block_indexed_bail_outs():
    rng = np.random.default_rng(4)
    K, V = _rand_kv(rng, 2, 64, 8)
    kc, vc = _pool(rng, 1, 10, 2, 8)
    assert not co.write_block_indexed_layer(kc[0], vc[0], [1, 2], K, V, [0])       # length mismatch
    assert not co.write_block_indexed_layer(kc[0], vc[0], [1], K[:, :60], V[:, :60], [0])  # unaligned
    assert not co.write_block_indexed_layer(kc[0], vc[0], [1], K, V, [4])          # past the end
    assert not co.write_block_indexed_layer(kc[0], vc[0], [], K, V, [])
    assert co.write_block_indexed_layer(kc[0], vc[0], [5, 2], K, V, [3, 0])
    np.testing.assert_array_equal(kc[0, 5], K[:, 48:64].transpose(1, 0, 2))
    np.testing.assert_array_equal(vc[0, 2], V[:, 0:16].transpose(1, 0, 2))


def test_oracle_prune_copy_brute_force():
    rng = np.random.default_rng(5)
    layers, H, D, N = 2, 2, 8, 40
    kc, vc = _pool(rng, layers, N, H, D)
    alloc = pool_oracle.FifoAllocator(N)
    old = alloc.allocate_blocks(9)
    alloc.free_blocks_by_ids(alloc.allocate_blocks(3))  # rotate the free list
    old_len = 16 * 8 + 5  # last block partial
    kept = [0, 2, 3, 7, 8]
    before_k = kc.copy()
    free_before = list(alloc.free_blocks)
    new = co.prune_copy(kc, vc, alloc, old, old_len, kept)
    keep_len = 4 * 16 + 5
    assert new == free_before[:5]
    assert alloc.free_blocks == free_before[5:] + old
    for layer in range(layers):
        full = co.pool_read(before_k[layer], old, old_len)
        exp = np.concatenate([full[:, 16 * b:min(old_len, 16 * b + 16)] for b in kept], axis=1)
        assert exp.shape[1] == keep_len
        np.testing.assert_array_equal(co.pool_read(kc[layer], new, keep_len), exp)


_MUTATIONS = {
    # (original text in write_selected_layer, planted mistake)
    "window_shift": ("obs_start = max(0, L - Lo)", "obs_start = max(0, L - Lo - 1)"),
    "mid_off_by_one": ("start = mid_start + int(mid_idx) * B", "start = mid_start + int(mid_idx) * B + 1"),
    "mid_end_from_L": ("mid_start, mid_end = Ls, max(Ls, L - Lo)", "mid_start, mid_end = Ls, L"),
    "sink_dropped": ("pos = write_piece_to_blocks(k_cache, v_cache, block_ids, 0, K[:, :Ls], V[:, :Ls], B)",
                     "pos = 0"),
}


def _mutated_write_selected_layer(mistake):
    import inspect
    import textwrap

    src = textwrap.dedent(inspect.getsource(co.write_selected_layer))
    old, new = _MUTATIONS[mistake]
    assert old in src
    ns = dict(vars(co))
    exec(compile(src.replace(old, new), "<mutated oracle>", "exec"), ns)
    return ns["write_selected_layer"]


@pytest.mark.parametrize("mistake", ["pad_before", "no_pad", *_MUTATIONS])
def test_oracle_check_catches_planted_mistakes(monkeypatch, mistake):
    """The compressor comparison (or the writeback's own length check) fails when the piecewise
    writeback is wrong in a plausible way."""
    rng = np.random.default_rng(11)
    L, Ls, Lo = 16 * 20 + 7, 5, 9  # every boundary unaligned, last middle block partial
    K, V = _rand_kv(rng, 2, L, 8)
    n_mid = -(-(L - Ls - Lo) // 16)
    sel = np.array([0, 4, n_mid - 1])
    eff = Ls + 16 * 3 + Lo
    write = co.write_selected_layer
    if mistake == "pad_before":
        def bad_pad(Kp, Vp, B=16):
            miss = B - Kp.shape[1]
            if miss <= 0:
                return Kp, Vp
            z = np.zeros((Kp.shape[0], miss, Kp.shape[2]), dtype=Kp.dtype)
            return np.concatenate([z, Kp], axis=1), np.concatenate([z, Vp], axis=1)
        monkeypatch.setattr(co, "pad_piece_to_block", bad_pad)
    elif mistake == "no_pad":
        monkeypatch.setattr(co, "pad_piece_to_block", lambda Kp, Vp, B=16: (Kp, Vp))
    else:
        write = _mutated_write_selected_layer(mistake)
    kc, vc = _pool(rng, 1, 40, 2, 8)
    ids = list(range(-(-eff // 16)))
    try:
        write(kc[0], vc[0], ids, K, V, list(sel), eff, "ratio", Ls, Lo)
    except RuntimeError:
        return  # the length check caught it
    Kf, _ = co.compress_tensors(K, V, sel, Ls, Lo)
    assert not np.array_equal(co.pool_read(kc[0], ids, eff), Kf)


def test_retained_pages_rejects_padded_selections():
    with pytest.raises(ValueError, match="outside"):
        compaction.retained_pages(256, torch.tensor([[0, -1]], dtype=torch.int32), sink_len=16, obs_len=16)
    with pytest.raises(ValueError, match="outside"):
        compaction.retained_pages(256, torch.tensor([[0, 14]], dtype=torch.int32), sink_len=16, obs_len=16)


# -------------------------------------------------------------------------------- GPU
def _dev_pool(cuda, layers, N, H, D, rng, dtype=torch.bfloat16):
    from unifiedkv_amd.pool import PagedKVPool

    pool = PagedKVPool(16, layers, H, D, dtype, num_blocks=N, device=cuda)
    kn, vn = _pool(rng, layers, N, H, D)
    pool.k_cache.view(torch.int16).copy_(torch.from_numpy(kn))
    pool.v_cache.view(torch.int16).copy_(torch.from_numpy(vn))
    return pool, kn, vn


def _assert_pool(pool, kn, vn):
    torch.cuda.synchronize()
    np.testing.assert_array_equal(pool.k_cache.view(torch.int16).cpu().numpy(), kn)
    np.testing.assert_array_equal(pool.v_cache.view(torch.int16).cpu().numpy(), vn)


def _raw_layers(rng, layers, H, L, D, cuda, strided=False):
    host, dev = [], []
    for _ in range(layers):
        K, V = _rand_kv(rng, H, L, D)
        host.append((K, V))
        if strided:  # rows of a wider buffer: [H, L, D] views with a padded token stride
            Kw = torch.zeros((H, L, D + 8), dtype=torch.int16)
            Vw = torch.zeros((H, L, D + 8), dtype=torch.int16)
            Kw[..., :D], Vw[..., :D] = torch.from_numpy(K), torch.from_numpy(V)
            dev.append((Kw.to(cuda).view(torch.bfloat16)[..., :D], Vw.to(cuda).view(torch.bfloat16)[..., :D]))
        else:
            dev.append((torch.from_numpy(K).to(cuda).view(torch.bfloat16),
                        torch.from_numpy(V).to(cuda).view(torch.bfloat16)))
    return host, dev


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(10))
def test_selected_writeback_random_unaligned(cuda, seed):
    rng = np.random.default_rng(1000 + seed)
    layers, H, D = int(rng.integers(1, 5)), int(rng.choice([1, 2, 8])), int(rng.choice([32, 64, 128]))
    L, Ls, Lo, n_mid, k = _case(rng)
    eff = Ls + 16 * k + Lo
    N = -(-eff // 16) + 30
    pool, kn, vn = _dev_pool(cuda, layers, N, H, D, rng)
    alloc = pool_oracle.FifoAllocator(N)
    taken = pool.allocate_blocks(7)
    assert taken == alloc.allocate_blocks(7)
    host, dev = _raw_layers(rng, layers, H, L, D, cuda, strided=seed % 3 == 0)
    sels = [list(np.sort(rng.permutation(n_mid)[:k])) for _ in range(layers)]
    as_tensor = seed % 2 == 0
    arg = torch.tensor(sels, dtype=torch.int32, device=cuda) if as_tensor else {i: s for i, s in enumerate(sels)}
    print(f"[retain] seed={seed} layers={layers} H={H} D={D} L={L} sink={Ls} window={Lo} k={k}", flush=True)
    got = compaction.selected_writeback(pool, dev, arg, eff, "ratio", sink_len=Ls, obs_len=Lo)
    exp = co.selected_writeback(kn, vn, alloc, host, sels, eff, "ratio", Ls, Lo)
    assert got == exp
    _assert_pool(pool, kn, vn)
    assert pool.free_blocks == alloc.free_blocks


@pytest.mark.gpu
def test_selected_writeback_regression_shape(cuda):
    """2795 tokens, sink = window = 16, budget 2048 (the reference's regression test shape, D=32)."""
    rng = np.random.default_rng(2795)
    L, Ls, Lo, layers, H, D = 2795, 16, 16, 4, 8, 32
    k, eff, mode = compaction.selection_budget_blocks(L, sink_len=Ls, obs_len=Lo, retain_budget_tokens=2048)
    assert (k, eff) == (126, 2048)
    pool, kn, vn = _dev_pool(cuda, layers, 300, H, D, rng)
    alloc = pool_oracle.FifoAllocator(300)
    host, dev = _raw_layers(rng, layers, H, L, D, cuda)
    sels = [list(np.sort(rng.permutation(173)[:k])) for _ in range(layers)]
    sels[0][-1] = 172  # the zero-padded partial block
    got = compaction.selected_writeback(pool, dev, sels, eff, mode, sink_len=Ls, obs_len=Lo)
    exp = co.selected_writeback(kn, vn, alloc, host, sels, eff, mode, Ls, Lo)
    assert got == exp and len(got) == 128
    _assert_pool(pool, kn, vn)


@pytest.mark.gpu
@pytest.mark.parametrize("L,mode", [(37, "too_short"), (1000, "input_le_budget"), (64, "input_le_budget")])
def test_selected_writeback_pass_through(cuda, L, mode):
    rng = np.random.default_rng(L)
    pool, kn, vn = _dev_pool(cuda, 2, 90, 2, 64, rng)
    alloc = pool_oracle.FifoAllocator(90)
    host, dev = _raw_layers(rng, 2, 2, L, 64, cuda)
    got = compaction.selected_writeback(pool, dev, [], L, mode, sink_len=16, obs_len=16)
    exp = co.selected_writeback(kn, vn, alloc, host, [[], []], L, mode, 16, 16)
    assert got == exp
    _assert_pool(pool, kn, vn)


@pytest.mark.gpu
def test_selected_writeback_refusals_free_their_pages(cuda):
    rng = np.random.default_rng(8)
    pool, kn, vn = _dev_pool(cuda, 2, 60, 2, 64, rng)
    host, dev = _raw_layers(rng, 2, 2, 300, 64, cuda)
    before = pool.free_blocks
    with pytest.raises(RuntimeError, match="selected_writeback_len_mismatch"):
        compaction.selected_writeback(pool, dev, [1, 2], 500, "ratio", sink_len=16, obs_len=16)
    with pytest.raises(RuntimeError, match="len_mismatch"):  # layers keep different block counts
        compaction.selected_writeback(pool, dev, {0: [1, 2], 1: [3]}, 16 + 32 + 16, "ratio", sink_len=16, obs_len=16)
    with pytest.raises(ValueError, match="negative"):
        compaction.selected_writeback(pool, dev, [1, -2], 16 + 32 + 16, "ratio", sink_len=16, obs_len=16)
    # device selections (select_blocks' form): a -1 pad or an index past the 17 middle blocks of
    # L = 300 (sink 16, window 16) is refused on the device before any page is taken
    order = pool.free_blocks
    for bad in ([[1, -1], [2, 3]], [[1, 2], [3, 17]]):
        sel = torch.tensor(bad, dtype=torch.int32, device=cuda)
        with pytest.raises(ValueError, match="outside the middle blocks"):
            compaction.selected_writeback(pool, dev, sel, 16 + 32 + 16, "ratio", sink_len=16, obs_len=16)
    assert pool.free_blocks == order
    assert sorted(pool.free_blocks) == sorted(before)
    with pytest.raises(MemoryError):
        compaction.selected_writeback(pool, dev, [], 61 * 16, "too_short", sink_len=16, obs_len=16)
    _assert_pool(pool, kn, vn)


@pytest.mark.gpu
def test_write_block_indexed_layer_matches_oracle(cuda):
    rng = np.random.default_rng(12)
    pool, kn, vn = _dev_pool(cuda, 3, 50, 8, 128, rng)
    K, V = _rand_kv(rng, 8, 160, 128)
    Kd = torch.from_numpy(K).to(cuda).view(torch.bfloat16)
    Vd = torch.from_numpy(V).to(cuda).view(torch.bfloat16)
    ids, src = [4, 9, 2, 33], [9, 0, 0, 5]
    assert compaction.write_block_indexed_layer(pool, 1, ids, Kd, Vd, src)
    assert co.write_block_indexed_layer(kn[1], vn[1], ids, K, V, src)
    assert not compaction.write_block_indexed_layer(pool, 1, ids, Kd, Vd, [0, 1, 10, 2])
    assert not compaction.write_block_indexed_layer(pool, 1, ids, Kd[:, :150], Vd[:, :150], src)
    assert not compaction.write_block_indexed_layer(pool, 1, ids[:3], Kd, Vd, src)
    _assert_pool(pool, kn, vn)


def _oracle_compact_selected(kn, vn, alloc, lists, lens, sels, Ls, Lo, free_sources):
    out = []
    for pages, L, sel in zip(lists, lens, sels):
        if sel is None:
            mode, k, eff = "too_short", 0, L
        else:
            mode, k = "ratio", len(sel[0])
            eff = Ls + 16 * k + (L - max(0, L - Lo))
        ids = alloc.allocate_blocks(-(-max(1, eff) // 16))
        for layer in range(kn.shape[0]):
            K = co.pool_read(kn[layer], pages, L)
            V = co.pool_read(vn[layer], pages, L)
            co.write_selected_layer(kn[layer], vn[layer], ids, K, V, [] if sel is None else list(sel[layer]), eff,
                                    mode, Ls, Lo)
        if free_sources:
            alloc.free_blocks_by_ids(pages)
        out.append((ids, eff))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("free_sources", [False, True])
@pytest.mark.parametrize("seed", range(4))
def test_compact_selected_pool_to_pool(cuda, seed, free_sources):
    rng = np.random.default_rng(2000 + seed)
    layers, H, D = 3, 8, 64
    Ls, Lo = int(rng.integers(0, 33)), int(rng.integers(1, 40))
    lens = [2795 if seed == 0 else int(rng.integers(Ls + Lo + 16, 900)) for _ in range(3)] + [40]
    total = sum(-(-L // 16) for L in lens)
    # free_sources: room for the largest result only, so later sequences receive freed pages
    N = total + (-(-max(lens) // 16) + 2 if free_sources else total + 20)
    pool, kn, vn = _dev_pool(cuda, layers, N, H, D, rng)
    alloc = pool_oracle.FifoAllocator(N)
    order = [int(x) for x in rng.permutation(N)]  # a shuffled free list: fragmented page lists
    assert pool.allocate_blocks(N) == alloc.allocate_blocks(N)
    pool.free_blocks_by_ids(order)
    alloc.free_blocks_by_ids(order)
    lists = []
    for L in lens:
        n = -(-L // 16)
        ids = pool.allocate_blocks(n)
        assert ids == alloc.allocate_blocks(n)
        lists.append(ids)
    sels = []
    for L in lens[:3]:
        n_mid = -(-(L - Ls - Lo) // 16)
        k = int(rng.integers(1, n_mid + 1)) if seed else 126
        rows = [np.sort(rng.permutation(n_mid)[:k]) for _ in range(layers)]
        rows[0][-1] = n_mid - 1
        rows[0] = np.sort(np.unique(rows[0]))
        if len(rows[0]) < k:
            rows[0] = np.sort(rng.permutation(n_mid)[:k])
        sels.append(np.stack(rows).astype(np.int32))
    sels.append(None)  # a short sequence kept whole
    print(f"[compact_selected] seed={seed} free={free_sources} lens={lens} sink={Ls} window={Lo}", flush=True)
    res = compaction.compact_selected(pool, lists, lens, [None if s is None else torch.from_numpy(s).to(cuda)
                                                          for s in sels], sink_len=Ls, obs_len=Lo,
                                      free_sources=free_sources)
    exp = _oracle_compact_selected(kn, vn, alloc, lists, lens, sels, Ls, Lo, free_sources)
    assert res.page_lists == [e[0] for e in exp]
    assert res.seq_lens == [e[1] for e in exp]
    _assert_pool(pool, kn, vn)
    assert pool.free_blocks == alloc.free_blocks
    np.testing.assert_array_equal(res.block_table.cpu().numpy(), pool_oracle.build_block_table(res.page_lists))


@pytest.mark.gpu
def test_compact_selected_rejects_out_of_range_selections(cuda):
    rng = np.random.default_rng(1)
    pool, _, _ = _dev_pool(cuda, 2, 60, 2, 64, rng)
    ids = pool.allocate_blocks(20)
    before = pool.free_blocks
    n_mid = -(-(300 - 16 - 16) // 16)  # 17
    for bad in ([[0, n_mid], [1, 2]], [[0, -1], [1, 2]]):
        with pytest.raises(ValueError, match="outside the middle"):
            compaction.compact_selected(pool, [ids], [300], [torch.tensor(bad, dtype=torch.int32, device=cuda)],
                                        sink_len=16, obs_len=16)
    assert pool.free_blocks == before


@pytest.mark.gpu
def test_compact_selected_refuses_before_taking_pages(cuda):
    """A later sequence's invalid input is refused before the earlier ones are copied: the free list
    and the pool bytes stay as they were."""
    rng = np.random.default_rng(2)
    pool, kn, vn = _dev_pool(cuda, 2, 80, 2, 64, rng)
    a, b = pool.allocate_blocks(20), pool.allocate_blocks(10)
    before = pool.free_blocks
    good = torch.tensor([[0, 3], [1, 2]], dtype=torch.int32, device=cuda)
    for lens, sels, what in (([300, 161], [good, None], "holds 10 pages"),  # 161 tokens in 10 pages
                             ([300, 8], [good, good], "shorter than its sink"),
                             ([300, 150], [good, torch.tensor([[0, 99], [1, 2]], dtype=torch.int32, device=cuda)],
                              "outside the middle")):
        with pytest.raises(ValueError, match=what):
            compaction.compact_selected(pool, [a, b], lens, sels, sink_len=16, obs_len=16)
        assert pool.free_blocks == before
    torch.cuda.synchronize()
    np.testing.assert_array_equal(pool.k_cache.view(torch.int16).cpu().numpy(), kn)
    np.testing.assert_array_equal(pool.v_cache.view(torch.int16).cpu().numpy(), vn)


@pytest.mark.gpu
@pytest.mark.parametrize("old_len,kept", [(16 * 8 + 5, [0, 2, 3, 7, 8]), (16 * 9, [1, 4, 8]), (100, [0, 6, 9, 12])])
def test_prune_window_matches_oracle(cuda, old_len, kept):
    rng = np.random.default_rng(old_len)
    pool, kn, vn = _dev_pool(cuda, 3, 40, 8, 128, rng)
    alloc = pool_oracle.FifoAllocator(40)
    old = pool.allocate_blocks(-(-old_len // 16))
    assert old == alloc.allocate_blocks(-(-old_len // 16))
    x = pool.allocate_blocks(4)
    assert x == alloc.allocate_blocks(4)
    pool.free_blocks_by_ids(x)
    alloc.free_blocks_by_ids(x)
    got = compaction.prune_window(pool, old, old_len, kept)
    exp = co.prune_copy(kn, vn, alloc, old, old_len, [b for b in kept if 16 * b < old_len])
    assert got == exp
    _assert_pool(pool, kn, vn)
    assert pool.free_blocks == alloc.free_blocks


@pytest.mark.gpu
def test_compact_free_sources_matches_per_sequence_order(cuda):
    """Aligned compaction with the old pages freed after each sequence; the pool is tight enough
    that the second sequence receives pages the first one gave back."""
    rng = np.random.default_rng(21)
    layers, N = 2, 52  # 12 free pages after the two lists: the second sequence reuses the first's
    pool, kn, vn = _dev_pool(cuda, layers, N, 2, 64, rng)
    alloc = pool_oracle.FifoAllocator(N)
    lists = [pool.allocate_blocks(20), pool.allocate_blocks(20)]
    assert lists == [alloc.allocate_blocks(20), alloc.allocate_blocks(20)]
    keeps = [np.stack([np.sort(rng.permutation(20)[:12]) for _ in range(layers)]).astype(np.int32) for _ in lists]
    res = compaction.compact(pool, lists, [torch.from_numpy(k).to(cuda) for k in keeps], [192, 192],
                             free_sources=True)
    exp_lists = []
    for pages, keep in zip(lists, keeps):
        exp_lists += co.compact(kn, vn, alloc, [pages], [keep])
        alloc.free_blocks_by_ids(pages)
    assert res.page_lists == exp_lists
    assert set(res.page_lists[1]) & set(lists[0])  # reuse of freed pages happened
    _assert_pool(pool, kn, vn)
    assert pool.free_blocks == alloc.free_blocks
