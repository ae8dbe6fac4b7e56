"""The fused decode prologue: device block table + lengths per step, fused append + decode.

Oracle: oracle/pool_oracle.py ``reserve_decode_slots`` (core/offload.py:838-866 in batch
order) and ``decode_steps`` (the reference's step: reserve, per-layer table, append at
old_len, attention over old_len + 1, commit), with the fp64 dense attention of
oracle/oracle.py. Bars: page lists, block tables, lengths and pool bytes bit-exact;
attention |gpu - oracle| <= 2e-3 + 1e-2 * |oracle|. The fused call must equal
``kv_append`` followed by ``page16_decode_attention`` bit for bit (same values, same
reduction order).
"""
import ctypes
import math

import numpy as np
import pytest
import torch

from oracle import oracle, pool_oracle
from unifiedkv_amd import _ext, workloads
from unifiedkv_amd.decode_step import plan_decode_pages
from unifiedkv_amd.pool import PagedKVPool

ATOL, RTOL = 2e-3, 1e-2


# ------------------------------------------------------------- CPU: the oracle, pinned
def test_reserve_oracle_known_answers():
    # Hand-derived from core/offload.py:838-866: only lengths that are multiples of 16 take
    # a page, FIFO from the head of the free list, in batch order; a zero length also takes
    # one (0 % 16 == 0) even though its first page is still empty.
    alloc = pool_oracle.FifoAllocator(10)
    alloc.free_blocks = [7, 3, 9]
    lists = [[5], [6, 2], [8]]
    got = pool_oracle.reserve_decode_slots(alloc, lists, [16, 20, 0])
    assert got == [7, None, 3]
    assert lists == [[5, 7], [6, 2], [8, 3]]
    assert alloc.free_blocks == [9]
    got = pool_oracle.reserve_decode_slots(alloc, lists, [17, 21, 1])
    assert got == [None, None, None] and alloc.free_blocks == [9]


def test_reserve_oracle_exhaustion_keeps_earlier_pages():
    alloc = pool_oracle.FifoAllocator(4)
    alloc.free_blocks = [2]
    lists = [[0], [1]]
    with pytest.raises(RuntimeError, match="direct_decode_expand_evict_failed"):
        pool_oracle.reserve_decode_slots(alloc, lists, [16, 32])
    assert lists == [[0, 2], [1]]


def test_decode_steps_oracle_on_a_hand_case():
    # One sequence, one layer, H=1, D=1: the attention of step s is the softmax-weighted
    # mean of the values written so far; with equal keys it is the plain mean.
    alloc = pool_oracle.FifoAllocator(4)
    k = [np.zeros((4, 16, 1, 1))]
    v = [np.zeros((4, 16, 1, 1))]
    lists = [[alloc.allocate_blocks(1)[0]]]
    tokens = [[(None, np.ones((1, 1, 1)), np.full((1, 1, 1), float(s + 1)))] for s in range(20)]

    def attend(layer, q, bt, lens):
        vals = [v[layer][bt[0, t // 16], t % 16, 0, 0] for t in range(int(lens[0]))]
        return float(np.mean(vals))

    outs, lens = pool_oracle.decode_steps(alloc, k, v, lists, [0], tokens, attend)
    assert [o[0] for o in outs] == [float(np.mean(np.arange(1, s + 2))) for s in range(20)]
    assert int(lens[0]) == 20
    # length 0 took a page at step 0 (0 % 16 == 0), length 16 another one
    assert lists == [[0, 1, 2]]


# --------------------------------------------------------------- CPU: the host planner
def test_planner_matches_reference_over_random_steps():
    rng = np.random.default_rng(3)
    N = 400
    pool = PagedKVPool(16, 2, 8, 64, num_blocks=N)
    ref = pool_oracle.FifoAllocator(N)
    B = 12
    lens = [int(x) for x in rng.integers(0, 100, B)]
    lists_a, lists_b = [], []
    for L in lens:
        n = max(1, -(-L // 16))
        a, b = pool.allocate_blocks(n), ref.allocate_blocks(n)
        assert a == b
        lists_a.append(list(a))
        lists_b.append(list(b))
    for step in range(300):
        trip = plan_decode_pages(pool.allocate_blocks, lists_a, lens, 16)
        got = pool_oracle.reserve_decode_slots(ref, lists_b, lens)
        assert lists_a == lists_b
        assert trip == [(i, len(lists_a[i]) - 1, g) for i, g in enumerate(got) if g is not None]
        lens = [L + 1 for L in lens]
        if step % 50 == 49:  # a sequence finishes and its pages go back
            i = int(rng.integers(0, B))
            pool.free_blocks_by_ids(lists_a[i])
            ref.free_blocks_by_ids(lists_b[i])
            lists_a[i], lists_b[i] = pool.allocate_blocks(1), ref.allocate_blocks(1)
            lens[i] = 0
    assert pool.free_blocks == ref.free_blocks


def test_planner_errors_and_eviction_hook():
    pool = PagedKVPool(16, 1, 1, 8, num_blocks=3)
    lists = [pool.allocate_blocks(1), pool.allocate_blocks(1)]
    with pytest.raises(RuntimeError, match="^page16_native_blocked:direct_decode_expand_evict_failed$") as ei:
        plan_decode_pages(pool.allocate_blocks, lists, [16, 16], 16)
    assert ei.value.triples == [(0, 1, 2)] and lists == [[0, 2], [1]]

    calls = []
    with pytest.raises(RuntimeError, match="^page16_native_blocked:direct_decode_expand_alloc_failed$"):
        plan_decode_pages(pool.allocate_blocks, lists, [32, 16], 16, seq_ids=[70, 71],
                          on_pool_full=lambda sid: calls.append(sid) or True)
    assert calls == [70]

    pool = PagedKVPool(16, 1, 1, 8, num_blocks=4)
    lists = [pool.allocate_blocks(1), pool.allocate_blocks(1)]
    victim = pool.allocate_blocks(1)  # another sequence's page; free list is now [3]

    def evict(sid):
        pool.free_blocks_by_ids(victim)
        return True

    trip = plan_decode_pages(pool.allocate_blocks, lists, [16, 16], 16, on_pool_full=evict)
    assert trip == [(0, 1, 3), (1, 1, 2)] and lists == [[0, 3], [1, 2]]


def test_prologue_rejects_bad_triples_before_any_launch():
    lib = _ext.load()
    bad = [(2, 0, 5), (-1, 0, 5), (0, 4, 5), (0, -1, 5)]
    for t in bad:
        arr = (ctypes.c_int32 * 3)(*t)
        assert lib.ukv_decode_prologue(None, 4, 2, None, None, arr, 1, None) == _ext.UKV_ERR_INVALID_ARGUMENT
    assert lib.ukv_decode_prologue(None, 4, 2, None, None, None, 1, None) == _ext.UKV_ERR_INVALID_ARGUMENT
    assert lib.ukv_decode_prologue(None, 4, -1, None, None, None, 0, None) == _ext.UKV_ERR_INVALID_ARGUMENT
    # nothing to do: no triples, no lengths -> no launch, OK
    assert lib.ukv_decode_prologue(None, 4, 2, None, None, None, 0, None) == _ext.UKV_OK


def test_fused_entry_point_rejects_missing_token_rows():
    # Every other argument is present (never dereferenced: the call returns before any launch).
    lib = _ext.load()
    s = _ext.i64_array((8, 8, 8))
    p = 1 << 20
    for k_new, v_new, strides in ((None, p, s), (p, None, s), (p, p, None)):
        rc = lib.ukv_page16_decode_append(p, p, p, p, p, k_new, v_new, strides, p, 1, 8, 8, 8, 1, 1, 1,
                                          s, s, s, ctypes.c_float(1.0), _ext.UKV_DTYPE_BF16, p, 1 << 20, None)
        assert rc == _ext.UKV_ERR_INVALID_ARGUMENT


# ------------------------------------------------------------------------ GPU
def _tdt(dtype):
    return torch.bfloat16 if dtype == "bf16" else torch.float16


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _rand_bits(rng, shape, dtype):
    return workloads._round_bits(rng.standard_normal(shape, dtype=np.float32), dtype)


def _dev(bits, dtype, device):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(device).view(_tdt(dtype))


def _assert_close(actual, expected, what):
    ok, max_err, excess = oracle.allclose_report(actual, expected, ATOL, RTOL)
    assert ok, f"{what}: max_abs_err={max_err:.3e} worst_excess={excess:.3e}"


@pytest.mark.gpu
@pytest.mark.parametrize("fused_append", [False, True])
@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_multi_step_multi_layer_matches_reference_flow(cuda, dtype, fused_append):
    from unifiedkv_amd.decode_step import DecodeBatch

    rng = np.random.default_rng(11)
    n_layers, Hq, Hkv, D, N = 3, 16, 4, 128, 160
    dt = workloads.DTYPE_CODES[dtype]
    lens0 = [15, 16, 31, 1, 47, 0, 200]
    B = len(lens0)
    pool = PagedKVPool(16, n_layers, Hkv, D, _tdt(dtype), num_blocks=N, device=cuda)
    k0 = _rand_bits(rng, (n_layers, N, 16, Hkv, D), dtype)
    v0 = _rand_bits(rng, (n_layers, N, 16, Hkv, D), dtype)
    pool.k_cache.copy_(_dev(k0, dtype, cuda))
    pool.v_cache.copy_(_dev(v0, dtype, cuda))
    ref = pool_oracle.FifoAllocator(N)
    lists, ref_lists = [], []
    for L in lens0:
        n = max(1, -(-L // 16))
        a, b = pool.allocate_blocks(n), ref.allocate_blocks(n)
        assert a == b
        lists.append(a)
        ref_lists.append(list(b))
    steps = 40
    scale = 1.0 / math.sqrt(D)
    tokens = [[(_rand_bits(rng, (B, Hq, D), dtype), _rand_bits(rng, (B, Hkv, D), dtype),
                _rand_bits(rng, (B, Hkv, D), dtype)) for _ in range(n_layers)] for _ in range(steps)]

    batch = DecodeBatch(pool, lists, lens0, capacity_blocks=1,  # width 64: no growth needed here
                        fused_append=fused_append)
    got = []
    for s in range(steps):
        batch.begin_step()
        row = []
        for layer in range(n_layers):
            q, kn, vn = (_dev(x, dtype, cuda) for x in tokens[s][layer])
            row.append(batch.attention(layer, q, kn, vn, softmax_scale=scale, n_rep=Hq // Hkv).float().cpu().numpy())
        batch.end_step()
        got.append(row)

    kref = [k0[l].copy() for l in range(n_layers)]
    vref = [v0[l].copy() for l in range(n_layers)]
    f = lambda a: oracle.bits_to_f32(a, dt)

    def attend(layer, q, bt, attn_lens):
        return oracle.page16_decode_dense(f(q), f(kref[layer]), f(vref[layer]), bt, attn_lens, softmax_scale=scale,
                                          n_rep=Hq // Hkv)

    want, lens_end = pool_oracle.decode_steps(ref, kref, vref, ref_lists, lens0, tokens, attend)
    for s in range(steps):
        for layer in range(n_layers):
            _assert_close(got[s][layer], want[s][layer], f"{dtype} step {s} layer {layer}")
    assert batch.page_lists == ref_lists
    assert batch.seq_lens == [int(x) for x in lens_end]
    assert pool.free_blocks == ref.free_blocks
    bt = batch.block_table.cpu().numpy()
    want_bt = pool_oracle.build_block_table(ref_lists)
    assert np.array_equal(bt[:, : want_bt.shape[1]], want_bt) and not bt[:, want_bt.shape[1]:].any()
    assert np.array_equal(batch.cache_seqlens.cpu().numpy(), lens_end)
    torch.cuda.synchronize()
    for layer in range(n_layers):
        assert np.array_equal(_bits(pool.k_cache[layer]), kref[layer]), f"K pool layer {layer}"
        assert np.array_equal(_bits(pool.v_cache[layer]), vref[layer]), f"V pool layer {layer}"


def _fused_vs_unfused(cuda, seed, B, Hq, Hkv, D, lens, dtype="bf16", n_rep=None, max_blocks=None, bad_tail=None,
                      new_layout="contig"):
    from unifiedkv_amd import page_ops
    from unifiedkv_amd.page16_native import page16_decode_append_attention, page16_decode_attention

    rng = np.random.default_rng(seed)
    pages = [max(1, -(-int(L) // 16)) for L in lens]
    N = int(sum(pages) * 1.3) + 4
    draw = rng.permutation(N)[: sum(pages)].astype(np.int32)
    lists, o = [], 0
    for n in pages:
        lists.append(draw[o:o + n])
        o += n
    mb = max_blocks or max(pages)
    bt = workloads.tables_from_pages([x[:mb] for x in lists], mb)
    if bad_tail is not None:  # an invalid page id where sequence bad_tail's token goes
        L = int(lens[bad_tail])
        bt[bad_tail, (L - 1) // 16] = N + 5
    k = _dev(_rand_bits(rng, (N, 16, Hkv, D), dtype), dtype, cuda)
    v = _dev(_rand_bits(rng, (N, 16, Hkv, D), dtype), dtype, cuda)
    q = _dev(_rand_bits(rng, (B, Hq, D), dtype), dtype, cuda)
    if new_layout == "contig":
        kn = _dev(_rand_bits(rng, (B, Hkv, D), dtype), dtype, cuda)
        vn = _dev(_rand_bits(rng, (B, Hkv, D), dtype), dtype, cuda)
    else:  # rows of a wider projection output: [B, Hkv, D] views with a padded batch stride
        kn = _dev(_rand_bits(rng, (B, Hkv + 1, D), dtype), dtype, cuda)[:, 1:]
        vn = _dev(_rand_bits(rng, (B, Hkv + 1, D), dtype), dtype, cuda)[:, 1:]
    bt_d = torch.from_numpy(bt).to(cuda)
    lens_d = torch.tensor(lens, dtype=torch.int32, device=cuda)
    n_rep = n_rep or Hq // Hkv
    scale = 1.0 / math.sqrt(D)

    k1, v1 = k.clone(), v.clone()
    page_ops.kv_append(k1, v1, bt_d, (lens_d - 1).clamp_min(-1), kn, vn, return_new_lens=False)
    out1 = page16_decode_attention(q, k1, v1, bt_d, lens_d, softmax_scale=scale, n_rep=n_rep)
    k2, v2 = k.clone(), v.clone()
    out2 = page16_decode_append_attention(q, k2, v2, bt_d, lens_d, kn, vn, softmax_scale=scale, n_rep=n_rep)
    torch.cuda.synchronize()
    assert torch.equal(k1.view(torch.int16), k2.view(torch.int16)), "K pool differs"
    assert torch.equal(v1.view(torch.int16), v2.view(torch.int16)), "V pool differs"
    o1, o2 = out1.float().cpu().numpy(), out2.float().cpu().numpy()
    assert np.array_equal(np.isnan(o1), np.isnan(o2))
    assert np.array_equal(np.nan_to_num(o1), np.nan_to_num(o2)), "outputs differ"
    return k, v, k2, v2, bt, lens


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("Hq,Hkv,D", [(32, 8, 128), (16, 2, 64), (8, 2, 256), (32, 32, 128), (48, 4, 128)])
def test_fused_equals_append_then_decode(cuda, dtype, Hq, Hkv, D):
    lens = [1, 16, 17, 31, 32, 33, 255, 256, 1000, 47]
    _fused_vs_unfused(cuda, 5, len(lens), Hq, Hkv, D, lens, dtype)


@pytest.mark.gpu
def test_fused_edge_lengths_and_ids(cuda):
    # zero length: nothing written, NaN output; beyond the table: clamped, nothing written;
    # an invalid page id at the token's page: nothing written, its tokens masked.
    lens = [0, 20, 64 * 16 + 5, 40, 1]
    k, v, k2, v2, bt, _ = _fused_vs_unfused(cuda, 6, len(lens), 32, 8, 128, lens, max_blocks=64, bad_tail=3)
    changed = torch.nonzero((k.view(torch.int16) != k2.view(torch.int16)).any(-1).any(-1))
    rows = {(int(p), int(t)) for p, t in changed.cpu().numpy()}
    assert rows == {(int(bt[1, 19 // 16]), 19 % 16), (int(bt[4, 0]), 0)}


@pytest.mark.gpu
def test_fused_strided_rows_and_unfused_shapes(cuda):
    lens = [5, 16, 300, 17]
    _fused_vs_unfused(cuda, 7, len(lens), 32, 8, 128, lens, new_layout="strided")
    # fewer q-head groups than KV heads: heads past the last group are appended but not read
    _fused_vs_unfused(cuda, 8, len(lens), 8, 8, 128, lens, n_rep=2)
    # head_dim without a split-kernel instance: the append kernel, then the scalar kernel
    _fused_vs_unfused(cuda, 9, len(lens), 8, 2, 96, lens)


@pytest.mark.gpu
def test_prologue_many_pages_in_place_lens_and_table_growth(cuda):
    from unifiedkv_amd.decode_step import DecodeBatch

    B = 300  # more new pages in one step than one prologue launch carries
    pool = PagedKVPool(16, 1, 1, 64, torch.bfloat16, num_blocks=4 * B, device=cuda)
    lists = [pool.allocate_blocks(1) for _ in range(B)]
    batch = DecodeBatch(pool, lists, [16] * B)
    assert batch.block_table.shape[1] == 64
    batch.begin_step()
    batch.end_step()
    bt = batch.block_table.cpu().numpy()
    assert [r[:2].tolist() for r in bt] == batch.page_lists
    assert all(len(x) == 2 for x in batch.page_lists)

    lib = _ext.load()
    lens = torch.arange(B, dtype=torch.int32, device=cuda)
    rc = lib.ukv_decode_prologue(None, 0, B, lens.data_ptr(), lens.data_ptr(), None, 0,
                                 torch.cuda.current_stream().cuda_stream)
    assert rc == _ext.UKV_OK
    assert torch.equal(lens.cpu(), torch.arange(1, B + 1, dtype=torch.int32))

    # a table that must widen: 63 pages fit a 64-wide table; length 1024 needs column 64
    pool2 = PagedKVPool(16, 1, 1, 64, torch.bfloat16, num_blocks=80, device=cuda)
    ids = pool2.allocate_blocks(63)
    batch2 = DecodeBatch(pool2, [ids], [63 * 16 - 1])
    assert batch2.block_table.shape[1] == 64
    versions = []
    for _ in range(18):
        batch2.begin_step()
        batch2.end_step()
        versions.append(batch2.table_version)
    assert batch2.block_table.shape[1] == 128
    # one reallocation, at the step whose new page (column 64) lay past the width
    assert versions[0] == 0 and versions[-1] == 1 and sorted(versions) == versions
    assert len(batch2.page_lists[0]) == 65
    assert batch2.block_table[0, :65].cpu().tolist() == batch2.page_lists[0]


@pytest.mark.gpu
def test_exhaustion_keeps_earlier_pages_in_the_device_table(cuda):
    from unifiedkv_amd.decode_step import DecodeBatch

    pool = PagedKVPool(16, 1, 1, 64, torch.bfloat16, num_blocks=3, device=cuda)
    lists = [pool.allocate_blocks(1), pool.allocate_blocks(1)]
    batch = DecodeBatch(pool, lists, [16, 16])
    with pytest.raises(RuntimeError, match="^page16_native_blocked:direct_decode_expand_evict_failed$"):
        batch.begin_step()
    assert batch.page_lists == [[0, 2], [1]]
    assert batch.block_table[:, :2].cpu().tolist() == [[0, 2], [1, 0]]
    assert batch.seq_lens == [16, 16] and batch.cache_seqlens.cpu().tolist() == [16, 16]


@pytest.mark.gpu
@pytest.mark.parametrize("fused_append", [False, True])
def test_layer_calls_replay_from_a_captured_graph(cuda, fused_append):
    # The per-layer fused append + decode calls of a step hold no host synchronisation and
    # no memset, so a serving loop can capture them. Capture one step's layers, then replay
    # the graph several times with eager work in between: every replay must equal the eager
    # result bit for bit (the appends rewrite the same rows with the same values).
    from unifiedkv_amd.decode_step import DecodeBatch

    rng = np.random.default_rng(21)
    n_layers, Hq, Hkv, D, N, dtype = 3, 32, 8, 128, 96, "bf16"
    lens0 = [40, 16, 100, 5]
    B = len(lens0)
    pool = PagedKVPool(16, n_layers, Hkv, D, _tdt(dtype), num_blocks=N, device=cuda)
    pool.k_cache.copy_(_dev(_rand_bits(rng, (n_layers, N, 16, Hkv, D), dtype), dtype, cuda))
    pool.v_cache.copy_(_dev(_rand_bits(rng, (n_layers, N, 16, Hkv, D), dtype), dtype, cuda))
    lists = [pool.allocate_blocks(max(1, -(-L // 16))) for L in lens0]
    batch = DecodeBatch(pool, lists, lens0, fused_append=fused_append)
    scale = 1.0 / math.sqrt(D)
    ins = [tuple(_dev(_rand_bits(rng, shape, dtype), dtype, cuda) for shape in ((B, Hq, D), (B, Hkv, D), (B, Hkv, D)))
           for _ in range(n_layers)]
    batch.begin_step()
    eager = [batch.attention(layer, *ins[layer], softmax_scale=scale, n_rep=Hq // Hkv).clone()
             for layer in range(n_layers)]
    torch.cuda.synchronize()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm the allocator on the capture stream
        for layer in range(n_layers):
            batch.attention(layer, *ins[layer], softmax_scale=scale, n_rep=Hq // Hkv)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = [batch.attention(layer, *ins[layer], softmax_scale=scale, n_rep=Hq // Hkv)
                for layer in range(n_layers)]
    for rep in range(4):
        for o in outs:
            o.fill_(0)
        graph.replay()
        torch.cuda.synchronize()
        for layer in range(n_layers):
            assert torch.equal(outs[layer].view(torch.int16), eager[layer].view(torch.int16)), (rep, layer)
        # eager work of the program between replays
        again = batch.attention(1, *ins[1], softmax_scale=scale, n_rep=Hq // Hkv)
        torch.cuda.synchronize()
        assert torch.equal(again.view(torch.int16), eager[1].view(torch.int16))
    batch.end_step()


@pytest.mark.gpu
@pytest.mark.parametrize("fused_append", [False, True])
def test_per_parity_graphs_replay_a_run_of_steps(cuda, fused_append):
    # One graph of the per-layer calls per parity of the step (the attention lengths alternate
    # between two device buffers), replayed after each step's eager prologue for 20 steps that
    # cross page boundaries and take new pages: every step's outputs and, at the end, every pool
    # byte, the page lists and the free list equal an eager run of the same steps on a twin pool.
    from unifiedkv_amd.decode_step import DecodeBatch

    rng = np.random.default_rng(33)
    n_layers, Hq, Hkv, D, N, dtype = 3, 32, 8, 128, 96, "bf16"
    lens0 = [40, 16, 100, 5, 31]
    B = len(lens0)
    kc = _dev(_rand_bits(rng, (n_layers, N, 16, Hkv, D), dtype), dtype, cuda)
    vc = _dev(_rand_bits(rng, (n_layers, N, 16, Hkv, D), dtype), dtype, cuda)
    pools, batches = [], []
    for _ in range(2):
        pool = PagedKVPool(16, n_layers, Hkv, D, _tdt(dtype), num_blocks=N, device=cuda)
        pool.k_cache.copy_(kc)
        pool.v_cache.copy_(vc)
        lists = [pool.allocate_blocks(max(1, -(-L // 16))) for L in lens0]
        pools.append(pool)
        batches.append(DecodeBatch(pool, lists, lens0, capacity_blocks=16, fused_append=fused_append))
    eager_b, graph_b = batches
    scale = 1.0 / math.sqrt(D)
    steps = 20
    ins = [[tuple(_dev(_rand_bits(rng, s, dtype), dtype, cuda) for s in ((B, Hq, D), (B, Hkv, D), (B, Hkv, D)))
            for _ in range(n_layers)] for _ in range(steps)]
    # static inputs the graphs read; each step's inputs are copied in before its replay
    static = [tuple(t.clone() for t in ins[0][layer]) for layer in range(n_layers)]

    def run_layers(batch, src):
        return [batch.attention(layer, *src[layer], softmax_scale=scale, n_rep=Hq // Hkv) for layer in range(n_layers)]

    graphs, outs = {}, {}
    for step in range(steps):
        eager_b.begin_step()
        exp = [o.clone() for o in run_layers(eager_b, ins[step])]
        eager_b.end_step()
        for layer in range(n_layers):
            for dst, src in zip(static[layer], ins[step][layer]):
                dst.copy_(src)
        graph_b.begin_step()
        par = graph_b.step_parity
        if par not in graphs:
            torch.cuda.synchronize()
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                outs[par] = run_layers(graph_b, static)
            graphs[par] = gr
        graphs[par].replay()
        graph_b.end_step()
        torch.cuda.synchronize()
        for layer in range(n_layers):
            assert torch.equal(outs[par][layer].view(torch.int16), exp[layer].view(torch.int16)), (step, layer)
    assert graph_b.page_lists == eager_b.page_lists and graph_b.seq_lens == eager_b.seq_lens
    assert pools[0].free_blocks == pools[1].free_blocks
    assert torch.equal(pools[0].k_cache.view(torch.int16), pools[1].k_cache.view(torch.int16))
    assert torch.equal(pools[0].v_cache.view(torch.int16), pools[1].v_cache.view(torch.int16))
