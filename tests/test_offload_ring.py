"""Per-sequence offload / prefetch over the pinned page arena (offload policy integration).

Oracle: oracle/offload_oracle.py restates core/offload.py:547-691 and 362-449 (maps, states, FIFO
allocation, freed ids, CPU bytes); pinned by hand-derived cases below. GPU tests check the
SequenceOffloader's bookkeeping against it step by step and every moved byte bit-exact: pages
read back through the published maps equal the originals, whatever happened to the freed pages
in between.
"""
import numpy as np
import pytest

from oracle import offload_oracle, pool_oracle
from unifiedkv_amd.offload import ExtentAllocator, runs_of


# ---------------------------------------------------------------------------------- CPU
def test_extent_allocator_first_fit_and_coalescing():
    a = ExtentAllocator(10)
    assert a.alloc(3) == [(0, 3)] and a.alloc(4) == [(3, 4)]
    a.free([(0, 3)])
    assert a.free_extents == [(0, 3), (7, 3)]
    assert a.alloc(5) == [(0, 3), (7, 2)]          # lowest addresses first, split over extents
    assert a.free_extents == [(9, 1)] and a.alloc(2) is None
    a.free([(3, 4), (0, 3), (7, 2)])
    assert a.free_extents == [(0, 10)] and a.n_free == 10
    with pytest.raises(ValueError):
        a.free([(2, 1)])


def test_extent_allocator_matches_a_slot_bitmap():
    rng = np.random.default_rng(0)
    cap = 64
    a = ExtentAllocator(cap)
    used = np.zeros(cap, bool)
    held = []
    for _ in range(3000):
        if held and rng.random() < 0.45:
            ext = held.pop(int(rng.integers(0, len(held))))
            a.free(ext)
            for s, c in ext:
                assert used[s:s + c].all()
                used[s:s + c] = False
        else:
            n = int(rng.integers(1, 12))
            ext = a.alloc(n)
            if (~used).sum() < n:
                assert ext is None
                continue
            free_slots = np.flatnonzero(~used)[:n]   # first fit = the n lowest free slots
            got = [s for st, c in ext for s in range(st, st + c)]
            assert got == free_slots.tolist()
            used[got] = True
            held.append(ext)
        assert a.n_free == int((~used).sum())


def test_runs_of():
    assert runs_of([4, 5, 6, 9, 10, 2]) == [(0, 4, 3), (3, 9, 2), (5, 2, 1)]
    assert runs_of([]) == []


def test_oracle_hand_case():
    # 10 pages, FIFO; sequence 7 holds pages [2, 5, 8] of 40 tokens (last block 8 tokens).
    alloc = pool_oracle.FifoAllocator(10)
    alloc.free_blocks = [0, 1, 3]                     # pages 2, 4..9 are in use elsewhere
    o = offload_oracle.OffloadOracle(alloc, num_layers=2, block_size=16, heads=1, dim=4, cpu_budget=10**9)
    o.add(7, [[2, 5, 8], [2, 5, 8]], seq_len=40)
    assert o.offload_blocks(7, [2, 0, 9]) is True      # blocks 0 and 2; 9 is out of range
    assert o.seqs[7]["state"] == "OFFLOAD_INFLIGHT"
    assert o.cpu_used == 2 * (2 * 1 * 16 * 4 * 2 + 2 * 1 * 8 * 4 * 2)
    o.finalize_offload(7)
    assert o.seqs[7]["maps"] == [[-1, 5, -1], [-1, 5, -1]] and o.seqs[7]["state"] == "MIXED"
    assert alloc.free_blocks == [0, 1, 3, 2, 8]        # freed pages appended in ascending order
    assert o.offload_blocks(7, [0]) is False            # no page there any more
    assert o.prefetch_blocks(7, [0, 1, 2]) is False     # issued: blocks 0 and 2 get pages 0 and 1
    o.finalize_prefetch(7)
    assert o.seqs[7]["maps"] == [[0, 5, 1], [0, 5, 1]] and o.seqs[7]["state"] == "ON_GPU"
    assert alloc.free_blocks == [3, 2, 8] and o.cpu_used == 0
    assert o.prefetch_blocks(7, [0]) is True            # resident: nothing to do


# ---------------------------------------------------------------------------------- GPU
def _setup(cuda, L=3, N=96, H=4, D=64, arena=48, chunk=8, cpu_budget_gb=48.0, seed=0):
    import torch

    from unifiedkv_amd.offload import SequenceOffloader
    from unifiedkv_amd.pool import PagedKVPool

    pool = PagedKVPool(16, L, H, D, torch.bfloat16, cpu_mem_gb=cpu_budget_gb, num_blocks=N, device=cuda)
    g = torch.Generator(device=cuda)
    g.manual_seed(seed)
    pool.k_cache.copy_(torch.randn(pool.k_cache.shape, generator=g, device=cuda).to(torch.bfloat16))
    pool.v_cache.copy_(torch.randn(pool.v_cache.shape, generator=g, device=cuda).to(torch.bfloat16))
    off = SequenceOffloader(pool, arena_pages=arena, chunk_pages=chunk)
    ref_alloc = pool_oracle.FifoAllocator(N)
    ref = offload_oracle.OffloadOracle(ref_alloc, L, 16, H, D, pool.cpu_budget)
    return pool, off, ref, ref_alloc


def _seq_pages(pool, maps):
    """Per layer, the K and V pages of every logical block (None where on the host)."""
    out = []
    for l, m in enumerate(maps):
        out.append([None if b < 0 else (pool.k_cache[l, b].clone(), pool.v_cache[l, b].clone()) for b in m])
    return out


def _same_pages(a, b):
    import torch

    for la, lb in zip(a, b):
        for x, y in zip(la, lb):
            assert torch.equal(x[0].view(torch.int16), y[0].view(torch.int16))
            assert torch.equal(x[1].view(torch.int16), y[1].view(torch.int16))


def _check(off, ref, pool, ref_alloc, seq):
    st, rs = off.seqs[seq], ref.seqs[seq]
    assert st.maps == rs["maps"] and st.state == rs["state"]
    assert pool.free_blocks == ref_alloc.free_blocks
    assert pool.cpu_used_bytes == ref.cpu_used


@pytest.mark.gpu
def test_round_trip_bit_exact_with_freed_pages_overwritten(cuda):
    import torch

    pool, off, ref, ref_alloc = _setup(cuda)
    rng = np.random.default_rng(1)
    lens = {3: 16 * 9 + 5, 8: 16 * 12}
    for sid, L_tok in lens.items():
        n = -(-L_tok // 16)
        ids, rid = pool.allocate_blocks(n), ref_alloc.allocate_blocks(n)
        assert ids == rid
        perm = [ids[i] for i in rng.permutation(n)]
        off.add_sequence(sid, perm, L_tok)
        ref.add(sid, [perm] * pool.num_layers, L_tok)
    before = {sid: _seq_pages(pool, off.seqs[sid].maps) for sid in lens}

    sel = [0, 2, 3, 4, 7, 9]
    assert off.offload_sequence_blocks(3, sel) is True and ref.offload_blocks(3, sel) is True
    assert off.state(3) == "OFFLOAD_INFLIGHT"
    assert off.finalize_offload(3, force_sync=True)
    ref.finalize_offload(3)
    _check(off, ref, pool, ref_alloc, 3)
    # the freed pages are reused and overwritten
    reused = pool.allocate_blocks(len(sel))
    ref_alloc.allocate_blocks(len(sel))
    for b in reused:
        pool.k_cache[:, b].fill_(7.0)
        pool.v_cache[:, b].fill_(-7.0)
    pool.free_blocks_by_ids(reused)
    ref_alloc.free_blocks_by_ids(reused)

    assert off.prefetch_sequence_blocks(3, [9, 2, 0]) is False     # issued (a subset: 3 of 6)
    ref.prefetch_blocks(3, [9, 2, 0])
    assert off.state(3) == "PREFETCH_INFLIGHT"
    assert off.finalize_prefetch(3, force_sync=True)
    ref.finalize_prefetch(3)
    _check(off, ref, pool, ref_alloc, 3)
    assert off.prefetch_sequence(3) is False                        # the other three
    ref.prefetch_blocks(3, range(10))
    assert off.finalize_prefetch(3, force_sync=True)
    ref.finalize_prefetch(3)
    _check(off, ref, pool, ref_alloc, 3)
    assert off.state(3) == "ON_GPU" and off.arena.slots.n_free == off.arena.capacity
    _same_pages(_seq_pages(pool, off.seqs[3].maps), before[3])
    _same_pages(_seq_pages(pool, off.seqs[8].maps), before[8])
    torch.cuda.synchronize()


@pytest.mark.gpu
def test_offload_sees_pending_compute_stream_writes(cuda):
    import torch

    pool, off, ref, _ = _setup(cuda, N=64, arena=32)
    ids = pool.allocate_blocks(8)
    off.add_sequence(1, ids, 8 * 16)
    # A long chain of compute-stream writes to the pages, then offload at once: the side stream
    # must wait for it (the reference's transfer stream does not, core/offload.py:578).
    for i in range(20):
        for b in ids:
            pool.k_cache[:, b].fill_(float(i))
    assert off.offload_sequence(1)
    assert off.finalize_offload(1, force_sync=True)
    a = off.arena
    slots = [off.seqs[1].slot_of[i] for i in range(8)]
    got = a.k[:, slots].float()
    assert bool((got == 19.0).all())


@pytest.mark.gpu
def test_per_layer_maps_and_slot_reuse_across_sequences(cuda):
    import torch

    pool, off, ref, ref_alloc = _setup(cuda, L=3, N=120, arena=20, chunk=4)
    rng = np.random.default_rng(4)
    maps = {}
    for sid in (10, 11):
        per_layer = [pool.allocate_blocks(6) for _ in range(3)]        # different pages per layer
        for m in per_layer:
            ref_alloc.allocate_blocks(6)
        maps[sid] = per_layer
        off.add_sequence(sid, per_layer, 6 * 16)
        ref.add(sid, per_layer, 6 * 16)
    before = {sid: _seq_pages(pool, maps[sid]) for sid in maps}
    for step in range(6):
        for sid in (10, 11):
            idx = sorted(rng.choice(6, size=int(rng.integers(1, 7)), replace=False).tolist())
            st = off.state(sid)
            if st in ("ON_GPU", "MIXED") and rng.random() < 0.6:
                r1 = off.offload_sequence_blocks(sid, idx)
                r2 = ref.offload_blocks(sid, idx)
                assert r1 == r2
                off.finalize_offload(sid, force_sync=True)
                ref.finalize_offload(sid)
            else:
                r1 = off.prefetch_sequence_blocks(sid, idx)
                r2 = ref.prefetch_blocks(sid, idx)
                assert r1 == r2, (step, sid, idx)
                off.finalize_prefetch(sid, force_sync=True)
                ref.finalize_prefetch(sid)
            _check(off, ref, pool, ref_alloc, sid)
    for sid in (10, 11):
        off.prefetch_sequence(sid)
        ref.prefetch_blocks(sid, range(6))
        off.finalize_prefetch(sid, force_sync=True)
        ref.finalize_prefetch(sid)
        _check(off, ref, pool, ref_alloc, sid)
        _same_pages(_seq_pages(pool, off.seqs[sid].maps), before[sid])
    torch.cuda.synchronize()


@pytest.mark.gpu
def test_refusals_leave_no_state_behind(cuda):
    pool, off, ref, ref_alloc = _setup(cuda, N=16, arena=4, chunk=4, cpu_budget_gb=48.0)
    ids = pool.allocate_blocks(6)
    off.add_sequence(5, ids, 6 * 16)
    assert off.offload_sequence_blocks(5, range(6)) is False        # 6 pages, 4 arena slots
    assert off.state(5) == "ON_GPU" and off.arena.slots.n_free == 4 and pool.cpu_used_bytes == 0
    assert off.offload_sequence_blocks(5, [0, 1, 2]) and off.finalize_offload(5, force_sync=True)
    others = pool.allocate_blocks(pool.n_free)                       # pool is now full
    assert off.prefetch_sequence_blocks(5, [0, 1, 2]) is False       # no pages: refused
    assert off.state(5) == "MIXED" and pool.n_free == 0 and off.stats.get("prefetch_fail") == 1
    pool.free_blocks_by_ids(others)
    assert off.prefetch_sequence_blocks(5, [0, 1, 2]) is False and off.finalize_prefetch(5, force_sync=True)
    assert off.prefetch_sequence_blocks(5, [0]) is True              # resident: nothing to do
    # CPU budget (core/offload.py:572-574)
    pool.cpu_used_bytes = pool.cpu_budget
    assert off.offload_sequence_blocks(5, [0]) is False and off.state(5) == "ON_GPU"
    held = [b for b in off.seqs[5].maps[0] if b >= 0]
    assert sorted(pool.free_blocks + held) == list(range(16)) and len(held) == 6
