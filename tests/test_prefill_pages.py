"""Prefill written straight into the pool (PrefillPages), then decode and scores from those pages.

The reference keeps the prefill's past in a DynamicCache and writes the pool only after
compression (core/engine.py:1826-1882, core/pool.py:127-141). Checked here against the
oracles: every chunk's attention (prefill_oracle, fp64, |err| <= 2e-3 + 1e-2 |ref|), the pool
bytes of every sequence (token t of layer l at page list[t // 16], slot t % 16, bit-exact with
the dense concatenation of all chunks - what write_kv_to_blocks would have written), the page
lists (pool_oracle.prefill_chunk_pages: FIFO, batch order), a decode step on the prefilled
pages (oracle.page16_decode_dense) and SnapKV scores from them (snapkv_oracle).
"""
import math

import numpy as np
import pytest

from oracle import oracle, pool_oracle, prefill_oracle
from oracle import snapkv_oracle as so
from unifiedkv_amd import workloads

ATOL, RTOL = 2e-3, 1e-2


def test_prefill_chunk_pages_oracle_hand_case():
    alloc = pool_oracle.FifoAllocator(8)
    alloc.free_blocks = [6, 2, 7, 0, 5]
    lists = [[], [3], []]
    took = pool_oracle.prefill_chunk_pages(alloc, lists, [0, 10, 0], [17, 6, 0])
    # seq 0: 17 tokens -> 2 pages; seq 1: 10 + 6 = 16 tokens fit its one page; seq 2: nothing
    assert took == [[6, 2], [], []] and lists == [[6, 2], [3], []]
    took = pool_oracle.prefill_chunk_pages(alloc, lists, [17, 16, 0], [15, 1, 1])
    assert took == [[], [7], [0]] and alloc.free_blocks == [5]
    with pytest.raises(RuntimeError, match="prefill_pages_alloc_failed"):
        pool_oracle.prefill_chunk_pages(alloc, lists, [32, 17, 1], [33, 0, 0])
    assert alloc.free_blocks == [5]                 # nothing taken on failure


def _bits(rng, shape, dtype="bf16"):
    return workloads._round_bits(rng.standard_normal(shape, dtype=np.float32), dtype)


def _dev(bits):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to("cuda").view(torch.bfloat16)


def _f(bits):
    return oracle.bits_to_f32(bits, workloads.DTYPE_CODES["bf16"])


@pytest.mark.gpu
def test_chunked_prefill_into_pages_then_decode_and_scores(cuda):
    import torch

    from unifiedkv_amd import snapkv
    from unifiedkv_amd.decode_step import DecodeBatch
    from unifiedkv_amd.pool import PagedKVPool
    from unifiedkv_amd.prefill import PrefillPages

    rng = np.random.default_rng(12)
    L, Hq, Hkv, D, N = 2, 16, 4, 128, 400
    scale, n_rep = 1.0 / math.sqrt(D), Hq // Hkv
    pool = PagedKVPool(16, L, Hkv, D, torch.bfloat16, num_blocks=N, device=cuda)
    ref_alloc = pool_oracle.FifoAllocator(N)
    # an unrelated allocation first, so the prefill's pages are not 0, 1, 2, ...
    assert pool.allocate_blocks(5) == ref_alloc.allocate_blocks(5)
    chunks = [[40, 17, 0], [16, 33, 5], [1, 0, 70], [300, 250, 230]]
    B = 3
    pp = PrefillPages(pool, B)
    ref_lists = [[] for _ in range(B)]
    dense_k = [[np.zeros((0, Hkv, D), np.uint16) for _ in range(B)] for _ in range(L)]
    dense_v = [[np.zeros((0, Hkv, D), np.uint16) for _ in range(B)] for _ in range(L)]
    lens = [0] * B
    for ci, cl in enumerate(chunks):
        pool_oracle.prefill_chunk_pages(ref_alloc, ref_lists, lens, cl)
        bt, cu, kv, mc = pp.begin_chunk(cl)
        assert pp.page_lists == ref_lists and pool.free_blocks == ref_alloc.free_blocks
        total = sum(cl)
        cu_h = np.concatenate([[0], np.cumsum(cl)]).astype(np.int32)
        kv_h = np.array([a + c for a, c in zip(lens, cl)], np.int32)
        for layer in range(L):
            q, k, v = _bits(rng, (total, Hq, D)), _bits(rng, (total, Hkv, D)), _bits(rng, (total, Hkv, D))
            out = pp.attention(layer, _dev(q), _dev(k), _dev(v), softmax_scale=scale, n_rep=n_rep).float().cpu().numpy()
            for b in range(B):
                dense_k[layer][b] = np.concatenate([dense_k[layer][b], k[cu_h[b]:cu_h[b + 1]]])
                dense_v[layer][b] = np.concatenate([dense_v[layer][b], v[cu_h[b]:cu_h[b + 1]]])
            # oracle: a compact pool holding each sequence's dense keys in order
            width = max(1, max(-(-int(x) // 16) for x in kv_h))
            kp = np.zeros((B * width, 16, Hkv, D), np.uint16)
            vp = np.zeros_like(kp)
            table = np.zeros((B, width), np.int32)
            for b in range(B):
                n = int(kv_h[b])
                table[b] = np.arange(b * width, (b + 1) * width)
                kp.reshape(B, width * 16, Hkv, D)[b, :n] = dense_k[layer][b]
                vp.reshape(B, width * 16, Hkv, D)[b, :n] = dense_v[layer][b]
            want = prefill_oracle.prefill_dense(_f(q), _f(kp), _f(vp), table, cu_h, kv_h, softmax_scale=scale,
                                                n_rep=n_rep)
            ok, err, exc = oracle.allclose_report(out, want, ATOL, RTOL)
            assert ok, f"chunk {ci} layer {layer}: max err {err:.3e} excess {exc:.3e}"
        pp.end_chunk()
        lens = list(kv_h)
    assert pp.seq_lens == lens
    # pool bytes = the dense concatenation, token t at page[t // 16], slot t % 16
    torch.cuda.synchronize()
    for layer in range(L):
        kc = pool.k_cache[layer].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
        vc = pool.v_cache[layer].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
        for b in range(B):
            ids = np.asarray(pp.page_lists[b])
            n = lens[b]
            assert np.array_equal(kc[ids].reshape(-1, Hkv, D)[:n], dense_k[layer][b])
            assert np.array_equal(vc[ids].reshape(-1, Hkv, D)[:n], dense_v[layer][b])

    # one decode step on the prefilled pages
    batch = DecodeBatch(pool, pp.page_lists, pp.seq_lens)
    batch.begin_step()
    q, k, v = _bits(rng, (B, Hq, D)), _bits(rng, (B, Hkv, D)), _bits(rng, (B, Hkv, D))
    out = batch.attention(1, _dev(q), _dev(k), _dev(v), softmax_scale=scale, n_rep=n_rep).float().cpu().numpy()
    batch.end_step()
    bt = batch.block_table.cpu().numpy()
    kc = pool.k_cache[1].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    vc = pool.v_cache[1].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    want = oracle.page16_decode_dense(_f(q), _f(kc), _f(vc), bt, np.array(lens) + 1, softmax_scale=scale, n_rep=n_rep)
    ok, err, exc = oracle.allclose_report(out, want, ATOL, RTOL)
    assert ok, f"decode after prefill: max err {err:.3e}"

    # SnapKV scores of sequence 0 straight from its pages (layer 0), obs = the last 64 positions
    sink, obs = 16, 64
    L0 = lens[0] + 1
    qo = _bits(rng, (1, 1, Hq, obs, D))
    table = torch.from_numpy(bt[:1].copy()).to(cuda)
    got = snapkv.score_blocks(_dev(qo)[:, :1].expand(1, 2, Hq, obs, D).contiguous(), pool.k_cache, table,
                              seq_len=L0, sink_len=sink, obs_len=obs, n_rep=n_rep).cpu().numpy()
    kc0 = pool.k_cache[0].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    dense0 = kc0[np.asarray(bt[0][: -(-L0 // 16)])].reshape(-1, Hkv, D)[:L0].transpose(1, 0, 2)
    want = so.score_layer_blocks(_f(dense0), _f(qo[0, 0]), sink_len=sink, obs_len=obs, n_rep=n_rep)
    err = np.abs(got[0] - want)
    assert np.all(err <= 1e-4 * np.abs(want).max() + 1e-3 * np.abs(want))


@pytest.mark.gpu
def test_prefill_pages_refuses_a_chunk_the_pool_cannot_hold(cuda):
    import torch

    from unifiedkv_amd.pool import PagedKVPool
    from unifiedkv_amd.prefill import PrefillPages

    pool = PagedKVPool(16, 1, 2, 64, torch.bfloat16, num_blocks=6, device=cuda)
    pp = PrefillPages(pool, 2)
    pp.begin_chunk([33, 20])          # 3 + 2 pages
    pp.end_chunk()
    with pytest.raises(RuntimeError, match="^prefill_pages_alloc_failed$"):
        pp.begin_chunk([40, 0])       # needs 3 more, 1 free
    assert pool.n_free == 1 and [len(x) for x in pp.page_lists] == [3, 2]
    with pytest.raises(RuntimeError, match="prefill_chunk_not_open"):
        pp.end_chunk()


@pytest.mark.gpu
def test_prefill_pages_chunk_tensors_outlive_a_side_stream(cuda):
    """The chunk's table and lengths, uploaded on the default stream and read by attention on a
    side stream that is still busy when end_chunk drops them, are not handed to the default
    stream's next allocations (which are overwritten with zeros at once): the side stream's
    output equals the same chunk's on one stream, bit for bit."""
    import torch

    from unifiedkv_amd.pool import PagedKVPool
    from unifiedkv_amd.prefill import PrefillPages

    rng = np.random.default_rng(5)
    Hq, Hkv, D = 8, 2, 128
    cl = [96, 40]
    total = sum(cl)
    q, k, v = _bits(rng, (total, Hq, D)), _bits(rng, (total, Hkv, D)), _bits(rng, (total, Hkv, D))
    outs = []
    for side in (False, True):
        pool = PagedKVPool(16, 1, Hkv, D, torch.bfloat16, num_blocks=64, device=cuda)
        pp = PrefillPages(pool, 2)
        pp.begin_chunk(cl)
        qd, kd, vd = _dev(q), _dev(k), _dev(v)
        if not side:
            out = pp.attention(0, qd, kd, vd, softmax_scale=D ** -0.5, n_rep=Hq // Hkv)
            pp.end_chunk()
        else:
            s = torch.cuda.Stream(device=cuda)
            s.wait_stream(torch.cuda.current_stream(cuda))
            with torch.cuda.stream(s):
                torch.cuda._sleep(50_000_000)  # the side stream is still busy after end_chunk
                out = pp.attention(0, qd, kd, vd, softmax_scale=D ** -0.5, n_rep=Hq // Hkv)
            pp.end_chunk()
            # allocations of the chunk tensors' sizes on the default stream, zeroed at once (zero
            # lengths and page 0: a kernel that read them would attend nothing, never out of bounds)
            junk = [torch.zeros(n, dtype=torch.int32, device=cuda) for n in (12, 5, 12, 5)]
            s.synchronize()
            del junk
        torch.cuda.synchronize()
        outs.append(out.view(torch.int16).cpu())
    assert torch.equal(outs[0], outs[1])
