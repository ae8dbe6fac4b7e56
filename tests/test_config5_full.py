"""BASELINE config 5 at its full size on the GPU: 32 layers x 8 sequences x 2048 fragmented pages.

(a) compaction: select_blocks -> retained_pages -> compact. The page lists equal the oracle's
    FIFO lists replayed on a FifoAllocator, the device table equals build_block_table of them,
    and for every layer pool[l, dst] equals pool[l, src] with the sources of the oracle's
    selection (core/scheduler.py:805-878). The token-granular kernel (compact_selected) then
    produces the same bytes in other pages, and the free list matches the oracle's throughout.
(b) offload / prefetch: the 27.3 GB of evicted pages (1629 per layer and sequence) through
    pinned host memory onto newly allocated ids, bit-exact per layer (core/offload.py:547-691).
(c) decode at B=8, L=6704 on the compacted tables: two sampled sequences of two layers against
    the fp64 oracle (|gpu - oracle| <= 2e-3 + 1e-2 |oracle|), and bit-identical output after a
    random relabelling of every physical page.
(0) first, on the uncompacted pool: the SnapKV scores from the row statistics of the sequences'
    final prefill chunk against the two-pass scores and fp64 row sums.
"""
import gc

import numpy as np
import pytest
import torch

from oracle import compaction_oracle as co
from oracle import oracle, pool_oracle
from unifiedkv_amd import compaction, page16_native
from unifiedkv_amd.pool import PagedKVPool
from unifiedkv_amd.staging import PageStager

pytestmark = pytest.mark.gpu

LAYERS, SEQS, CTX, HKV, HQ, D, SINK, OBS, RATIO = 32, 8, 32768, 8, 32, 128, 64, 128, 0.20
PER = CTX // 16  # 2048 pages per sequence
SEED = 5


def log(msg):
    print(f"[config5] {msg}", flush=True)


@pytest.fixture(scope="module")
def c5(cuda):
    k_blocks, eff, mode = compaction.selection_budget_blocks(CTX, sink_len=SINK, obs_len=OBS, retain_ratio=RATIO)
    assert (k_blocks, eff, mode) == (407, 6704, "ratio")
    keep = eff // 16
    evict = PER - keep
    # sources + two compactions + the prefetch targets
    N = SEQS * PER + 2 * SEQS * keep + SEQS * evict
    log(f"pool {N} pages x {LAYERS} layers ({2 * N * LAYERS * 16 * HKV * D * 2 / 1e9:.1f} GB)")
    pool = PagedKVPool(16, LAYERS, HKV, D, torch.bfloat16, num_blocks=N, device=cuda)
    alloc = pool_oracle.FifoAllocator(N)
    rng = np.random.default_rng(SEED)
    # a shuffled free list, so that every sequence's pages are fragmented
    order = [int(x) for x in rng.permutation(N)]
    assert pool.allocate_blocks(N) == alloc.allocate_blocks(N)
    pool.free_blocks_by_ids(order)
    alloc.free_blocks_by_ids(order)
    lists = [pool.allocate_blocks(PER) for _ in range(SEQS)]
    assert lists == [alloc.allocate_blocks(PER) for _ in range(SEQS)]
    g = torch.Generator(device=cuda)
    g.manual_seed(SEED)
    used = torch.tensor(sorted(p for ids in lists for p in ids), dtype=torch.long, device=cuda)
    for layer in range(LAYERS):
        for lo in range(0, used.numel(), 2048):
            idx = used[lo:lo + 2048]
            for cache in (pool.k_cache, pool.v_cache):
                cache[layer, idx] = torch.randn((idx.numel(), 16, HKV, D), generator=g, device=cuda).to(torch.bfloat16)
    scores = rng.random((SEQS * LAYERS, PER - (SINK + OBS) // 16), dtype=np.float32)
    torch.cuda.synchronize()
    log("pool filled")
    state = dict(pool=pool, alloc=alloc, lists=lists, scores=scores, k=k_blocks, eff=eff, keep=keep, evict=evict)
    yield state
    state.clear()
    del pool
    gc.collect()
    torch.cuda.empty_cache()


def _src_ids(lists, ret):
    """Physical source ids per sequence: [layers, keep] from the oracle's retained logical pages."""
    return [np.asarray(pages)[r] for pages, r in zip(lists, ret)]


def test_0_scores_from_final_chunk_statistics_full_size(c5, cuda):
    """(0) SnapKV scores with the row statistics of each sequence's final 2048-token chunk (layers 0
    and 31 through a strided two-layer view of the pool): equal to the two-pass scores within the
    two-pass path's own fp16 rounding, and sampled rows within 5e-6 (log2 units) of fp64 sums."""
    import math

    from oracle import snapkv_oracle as so
    from unifiedkv_amd import prefill, snapkv
    from unifiedkv_amd.pool import pack_block_table

    pool, lists = c5["pool"], c5["lists"]
    C, scale, n_rep = 2048, D ** -0.5, HQ // HKV
    layers = (0, LAYERS - 1)
    table = torch.from_numpy(pack_block_table(lists)).to(cuda)
    g = torch.Generator(device=cuda)
    g.manual_seed(SEED + 3)
    qc = torch.randn((SEQS * C, HQ, D), generator=g, device=cuda).to(torch.bfloat16)
    cu = torch.arange(0, SEQS * C + 1, C, dtype=torch.int32, device=cuda)
    lens = torch.full((SEQS,), CTX, dtype=torch.int32, device=cuda)
    st = snapkv.ObsStats(SEQS, len(layers), HQ, sink_len=SINK, obs_len=OBS, softmax_scale=scale, device=cuda)
    for j, layer in enumerate(layers):
        prefill.paged_prefill_attention(qc, pool.k_cache[layer], pool.v_cache[layer], table, cu, lens,
                                        softmax_scale=scale, n_rep=n_rep, max_chunk=C, obs_stats=st, layer_id=j,
                                        host_lens=([C] * SEQS, [CTX] * SEQS))
    q_obs = qc.view(SEQS, C, HQ, D)[:, C - OBS:].permute(0, 2, 1, 3).unsqueeze(1)
    q_obs = q_obs.expand(SEQS, len(layers), HQ, OBS, D).contiguous()
    kview = pool.k_cache[0::LAYERS - 1]                      # layers 0 and 31, no copy
    assert kview.shape[0] == 2 and kview.data_ptr() == pool.k_cache[0].data_ptr()
    one = snapkv.score_blocks(q_obs, kview, table, seq_len=CTX, sink_len=SINK, obs_len=OBS, n_rep=n_rep,
                              obs_stats=st).cpu().numpy()
    two = snapkv.score_blocks(q_obs, kview, table, seq_len=CTX, sink_len=SINK, obs_len=OBS,
                              n_rep=n_rep).cpu().numpy()
    rel = np.abs(one - two) / np.maximum(np.abs(two), 1e-30)
    log(f"scores from statistics against two passes: max rel diff {rel.max():.2e}")
    assert np.all(np.abs(one - two) <= 2.0 ** -9 * np.abs(two) + 1e-7)
    data = st.data.cpu().numpy()
    assert np.all(data[..., 1] == 0)
    rng = np.random.default_rng(SEED + 13)
    worst = 0.0
    for b in sorted(rng.choice(SEQS, 2, replace=False)):
        for j, layer in enumerate(layers):
            ids = torch.tensor(lists[b], dtype=torch.long, device=cuda)
            for h in sorted(rng.choice(HQ, 2, replace=False)):
                kg = pool.k_cache[layer, ids][:, :, h // n_rep].reshape(-1, D).float().cpu().numpy()
                rows = sorted(rng.choice(OBS, 3, replace=False))
                qr = q_obs[b, j, h, rows].float().cpu().numpy()
                want = so.obs_row_stats(kg[None], qr[None], sink_len=SINK, obs_len=OBS, n_rep=1, scale=scale)[0]
                err = np.abs(data[b, j, h, rows, 0] - want).max()
                worst = max(worst, err)
                assert err <= 5e-6, (b, layer, h, err)
    log(f"final-chunk row statistics within {worst:.2e} of fp64 (log2 units)")
    assert math.isfinite(worst)


def test_a_compaction_full_size(c5, cuda):
    pool, alloc, lists = c5["pool"], c5["alloc"], c5["lists"]
    scores = torch.from_numpy(c5["scores"]).to(cuda)
    sel = compaction.select_blocks(scores, c5["k"])
    retained = [compaction.retained_pages(CTX, sel[b * LAYERS:(b + 1) * LAYERS], sink_len=SINK, obs_len=OBS)
                for b in range(SEQS)]
    res = compaction.compact(pool, lists, retained, [c5["eff"]] * SEQS)
    log("compact done")
    sel_np = co.select_topk(c5["scores"], c5["k"])
    ret_np = [co.retained_pages(CTX, sel_np[b * LAYERS:(b + 1) * LAYERS], 16, SINK, OBS) for b in range(SEQS)]
    for a, b in zip(retained, ret_np):
        np.testing.assert_array_equal(a.cpu().numpy(), b)
    # the oracle's compaction on a stand-in pool of one byte per page: same FIFO lists
    tiny = np.zeros((LAYERS, pool.N_total, 1), dtype=np.int8)
    exp_lists = co.compact(tiny, tiny.copy(), alloc, lists, ret_np)
    assert res.page_lists == exp_lists
    assert pool.free_blocks == alloc.free_blocks
    np.testing.assert_array_equal(res.block_table.cpu().numpy(), pool_oracle.build_block_table(exp_lists))
    srcs = _src_ids(lists, ret_np)
    dst = torch.tensor([p for ids in exp_lists for p in ids], dtype=torch.long, device=cuda)
    for layer in range(LAYERS):
        src = torch.from_numpy(np.concatenate([s[layer] for s in srcs])).to(cuda).long()
        assert torch.equal(pool.k_cache[layer, dst], pool.k_cache[layer, src]), f"K layer {layer}"
        assert torch.equal(pool.v_cache[layer, dst], pool.v_cache[layer, src]), f"V layer {layer}"
    log("compact bit-exact on every layer")
    # the token-granular kernel on the same selection: the same bytes in a second set of pages
    mids = [sel[b * LAYERS:(b + 1) * LAYERS] for b in range(SEQS)]
    res2 = compaction.compact_selected(pool, lists, [CTX] * SEQS, mids, sink_len=SINK, obs_len=OBS)
    exp2 = [alloc.allocate_blocks(c5["keep"]) for _ in range(SEQS)]
    assert res2.page_lists == exp2 and res2.seq_lens == [c5["eff"]] * SEQS
    assert pool.free_blocks == alloc.free_blocks
    dst2 = torch.tensor([p for ids in exp2 for p in ids], dtype=torch.long, device=cuda)
    for layer in range(LAYERS):
        assert torch.equal(pool.k_cache[layer, dst2], pool.k_cache[layer, dst]), f"K layer {layer}"
        assert torch.equal(pool.v_cache[layer, dst2], pool.v_cache[layer, dst]), f"V layer {layer}"
    log("compact_selected equals compact on every layer")
    c5.update(res=res, ret_np=ret_np)


def test_b_offload_round_trip_full_size(c5, cuda):
    if "ret_np" not in c5:
        pytest.skip("needs the compaction of test_a_compaction_full_size")
    pool, alloc, lists = c5["pool"], c5["alloc"], c5["lists"]
    ret_np = c5["ret_np"]
    evicted = []
    for b in range(SEQS):
        table = np.asarray(lists[b])
        evicted.append(np.stack([table[np.setdiff1d(np.arange(PER), ret_np[b][l])] for l in range(LAYERS)]))
    ev = np.concatenate(evicted, axis=1).astype(np.int32)  # [layers, 8 * 1629]
    n = ev.shape[1]
    assert n == SEQS * c5["evict"] == 13032
    new = pool.allocate_blocks(n)
    assert new == alloc.allocate_blocks(n)
    stager = PageStager(pool, chunk_pages=512)
    log(f"offload {2 * LAYERS * n * 16 * HKV * D * 2 / 1e9:.2f} GB")
    host = stager.offload(torch.from_numpy(ev))
    event = stager.prefetch(host, torch.tensor(new, dtype=torch.int32))
    stager.wait(event)
    torch.cuda.synchronize()
    log("round trip done")
    ev_d = torch.from_numpy(ev).to(cuda).long()
    new_d = torch.tensor(new, dtype=torch.long, device=cuda)
    for layer in range(LAYERS):
        assert torch.equal(pool.k_cache[layer, new_d], pool.k_cache[layer, ev_d[layer]]), f"K layer {layer}"
        assert torch.equal(pool.v_cache[layer, new_d], pool.v_cache[layer, ev_d[layer]]), f"V layer {layer}"
    del host, stager
    gc.collect()
    if hasattr(torch._C, "_host_emptyCache"):  # give the 27 GB of pinned host memory back
        torch._C._host_emptyCache()
    log("round trip bit-exact on every layer")


def test_c_decode_on_compacted_tables(c5, cuda):
    if "res" not in c5:
        pytest.skip("needs the compaction of test_a_compaction_full_size")
    pool, res = c5["pool"], c5["res"]
    eff = c5["eff"]
    g = torch.Generator(device=cuda)
    g.manual_seed(SEED + 7)
    q = torch.randn((SEQS, HQ, D), generator=g, device=cuda).to(torch.bfloat16)
    lens = torch.full((SEQS,), eff, dtype=torch.int32, device=cuda)
    table = res.block_table
    assert tuple(table.shape) == (SEQS, eff // 16)
    scale = D ** -0.5
    rng = np.random.default_rng(SEED + 11)
    for layer in (0, LAYERS - 1):
        out = page16_native.page16_decode_attention(q, pool.k_cache[layer], pool.v_cache[layer], table, lens,
                                                    softmax_scale=scale, n_rep=HQ // HKV)
        got = out.float().cpu().numpy()
        for b in sorted(rng.choice(SEQS, 2, replace=False)):
            ids = torch.tensor(res.page_lists[b], dtype=torch.long, device=cuda)
            kb = pool.k_cache[layer, ids].float().cpu().numpy()
            vb = pool.v_cache[layer, ids].float().cpu().numpy()
            exp = oracle.page16_decode_dense(q[b:b + 1].float().cpu().numpy(), kb, vb,
                                             np.arange(eff // 16, dtype=np.int32)[None], np.array([eff], np.int32),
                                             softmax_scale=scale, n_rep=HQ // HKV)
            ok, err, excess = oracle.allclose_report(got[b:b + 1], exp, 2e-3, 1e-2)
            assert ok, f"layer {layer} seq {b}: max abs err {err:.3e}"
            log(f"layer {layer} seq {b}: max abs err {err:.2e}")
        # relabel every page of the batch: a new one-layer pool holding the same pages elsewhere
        flat = torch.tensor([p for ids in res.page_lists for p in ids], dtype=torch.long, device=cuda)
        M = flat.numel() + 97
        dest = torch.from_numpy(rng.permutation(M)[:flat.numel()]).to(cuda)
        k2 = torch.zeros((M, 16, HKV, D), dtype=torch.bfloat16, device=cuda)
        v2 = torch.zeros_like(k2)
        k2[dest] = pool.k_cache[layer, flat]
        v2[dest] = pool.v_cache[layer, flat]
        remap = torch.full((pool.N_total,), -1, dtype=torch.long, device=cuda)
        remap[flat] = dest
        table2 = remap[table.long()].to(torch.int32)
        out2 = page16_native.page16_decode_attention(q, k2, v2, table2, lens, softmax_scale=scale, n_rep=HQ // HKV)
        assert torch.equal(out.view(torch.int16), out2.view(torch.int16)), f"layer {layer}: relabelling changed it"
        del k2, v2
    log("decode on compacted tables matches")


def test_d_selected_writeback_from_dense_raw_kv_full_size(c5, cuda):
    """The unchanged scheduler's selected writeback at config 5's shape: two sequences of 32768
    tokens, each layer's raw K/V dense [8, 32768, 128] (core/scheduler.py:509, 541, 702-733), the
    top-k of the config's scores per layer, 4 sink + 407 selected + 8 window pages written into
    FIFO pages of a second pool by ukv_retain_writeback_dense (one launch per sequence), against
    the oracle's writeback of the same bytes (core/scheduler.py:735-799, 805-878): page ids, free
    list and every byte of the pool."""
    k, eff = c5["k"], c5["eff"]
    keep = c5["keep"]
    N2 = 2 * keep + 5
    pool2 = PagedKVPool(16, LAYERS, HKV, D, torch.bfloat16, num_blocks=N2, device=cuda)
    pool2.k_cache.zero_()
    pool2.v_cache.zero_()
    alloc2 = pool_oracle.FifoAllocator(N2)
    assert pool2.allocate_blocks(3) == alloc2.allocate_blocks(3)  # the FIFO head is not page 0
    kn = np.zeros((LAYERS, N2, 16, HKV, D), dtype=np.int16)
    vn = np.zeros_like(kn)
    sel_np = co.select_topk(c5["scores"], k)
    sel_dev = compaction.select_blocks(torch.from_numpy(c5["scores"]).to(cuda), k)
    g = torch.Generator(device=cuda)
    g.manual_seed(SEED + 23)
    for b in (0, 5):
        raw_dev = [(torch.randn((HKV, CTX, D), generator=g, device=cuda).to(torch.bfloat16),
                    torch.randn((HKV, CTX, D), generator=g, device=cuda).to(torch.bfloat16)) for _ in range(LAYERS)]
        log(f"selected writeback of sequence {b}: {2 * LAYERS * HKV * CTX * D * 2 / 1e9:.1f} GB of dense raw KV")
        got = compaction.selected_writeback(pool2, raw_dev, sel_dev[b * LAYERS:(b + 1) * LAYERS], eff, "ratio",
                                            sink_len=SINK, obs_len=OBS)
        raw_host = [(K.view(torch.int16).cpu().numpy(), V.view(torch.int16).cpu().numpy()) for K, V in raw_dev]
        del raw_dev
        sels = [list(sel_np[b * LAYERS + layer]) for layer in range(LAYERS)]
        exp = co.selected_writeback(kn, vn, alloc2, raw_host, sels, eff, "ratio", SINK, OBS)
        del raw_host
        assert got == exp and len(got) == keep
        assert pool2.free_blocks == alloc2.free_blocks
    torch.cuda.synchronize()
    np.testing.assert_array_equal(pool2.k_cache.view(torch.int16).cpu().numpy(), kn)
    np.testing.assert_array_equal(pool2.v_cache.view(torch.int16).cpu().numpy(), vn)
    log("selected writeback bit-exact: page ids, free list, every pool byte")
    del pool2
    torch.cuda.empty_cache()
