"""Offload / prefetch staging (row a8): bit-exact round trips through pinned host memory.

The reference's own round-trip check is benchmarks/tests.py:78-99 (test_4_offload:
register, offload, prefetch, read back, compare); it asserts ON_CPU right after an
asynchronous offload and is stale. The intent - contents survive, page ids change
- is what these tests pin, bit-exact.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _pool(cuda, N=300, L=3, dtype=torch.bfloat16, seed=0):
    from unifiedkv_amd.pool import PagedKVPool

    pool = PagedKVPool(16, L, 8, 128, dtype, num_blocks=N, device=cuda)
    g = torch.Generator().manual_seed(seed)
    pool.k_cache.copy_(torch.randn(pool.k_cache.shape, generator=g).to(dtype).to(cuda))
    pool.v_cache.copy_(torch.randn(pool.v_cache.shape, generator=g).to(dtype).to(cuda))
    return pool


@pytest.mark.parametrize("n,chunk", [(150, 64), (1, 512), (64, 64), (200, 512)])
def test_round_trip_to_new_pages_bit_exact(cuda, n, chunk):
    from unifiedkv_amd.staging import PageStager

    pool = _pool(cuda, N=450)
    rng = np.random.default_rng(n)
    perm = rng.permutation(450)
    src, dst = perm[:n].tolist(), perm[n:2 * n].tolist()
    k0 = pool.k_cache[:, src].clone()
    v0 = pool.v_cache[:, src].clone()
    st = PageStager(pool, chunk_pages=chunk)
    host = st.offload(src)
    st.wait(host.event)  # pages may be reused only after the offload event
    pool.k_cache[:, src] = 0
    assert host.nbytes == 2 * 3 * n * 16 * 8 * 128 * 2
    ev = st.prefetch(host, dst)
    st.wait(ev)
    assert torch.equal(pool.k_cache[:, dst], k0)
    assert torch.equal(pool.v_cache[:, dst], v0)


def test_offload_sees_compute_stream_writes(cuda):
    from unifiedkv_amd.staging import PageStager

    pool = _pool(cuda, seed=1)
    pages = [5, 17, 42]
    st = PageStager(pool, chunk_pages=2)
    for _ in range(3):
        val = float(np.random.default_rng().integers(1, 100))
        pool.k_cache[:, pages] = val  # enqueued on the compute stream, no host sync
        host = st.offload(pages)
        host.event.synchronize()
        for c in host.k_chunks:
            assert bool((c.float() == val).all())


def test_decode_after_relabelled_prefetch_is_identical(cuda):
    """Offload a sequence's pages, prefetch them to other ids, rewrite the table: Page16 output unchanged."""
    from unifiedkv_amd.page16_native import page16_decode_attention
    from unifiedkv_amd.staging import PageStager

    pool = _pool(cuda, N=400, L=2, seed=2)
    rng = np.random.default_rng(3)
    perm = rng.permutation(400)
    pages = [perm[0:50].tolist(), perm[50:80].tolist()]
    lens = torch.tensor([50 * 16 - 3, 30 * 16], dtype=torch.int32, device=cuda)
    q = torch.randn(2, 32, 128, device=cuda).to(torch.bfloat16)
    layer = 1
    bt = pool.block_table_for(pages)
    out0 = page16_decode_attention(q, pool.k_cache[layer], pool.v_cache[layer], bt, lens,
                                   softmax_scale=128 ** -0.5, n_rep=4)
    st = PageStager(pool, chunk_pages=32)
    new_pages = [perm[100:150].tolist(), perm[150:180].tolist()]
    for old, new in zip(pages, new_pages):
        host = st.offload(old)
        st.wait(st.prefetch(host, new))
    bt2 = pool.block_table_for(new_pages)
    out1 = page16_decode_attention(q, pool.k_cache[layer], pool.v_cache[layer], bt2, lens,
                                   softmax_scale=128 ** -0.5, n_rep=4)
    assert torch.equal(out0.view(torch.int16), out1.view(torch.int16))


def test_per_layer_page_lists_round_trip(cuda):
    """Config 5b evicts a different page set per layer: [layers, n] id lists."""
    from unifiedkv_amd.staging import PageStager

    pool = _pool(cuda, N=500, L=3, seed=4)
    rng = np.random.default_rng(5)
    src = np.stack([rng.permutation(250)[:70] for _ in range(3)]).astype(np.int32)
    dst = np.stack([250 + rng.permutation(250)[:70] for _ in range(3)]).astype(np.int32)
    k0 = [pool.k_cache[l, src[l]].clone() for l in range(3)]
    v0 = [pool.v_cache[l, src[l]].clone() for l in range(3)]
    st = PageStager(pool, chunk_pages=32)
    host = st.offload(torch.from_numpy(src))
    st.wait(st.prefetch(host, torch.from_numpy(dst)))
    for l in range(3):
        assert torch.equal(pool.k_cache[l, dst[l]], k0[l])
        assert torch.equal(pool.v_cache[l, dst[l]], v0[l])


def test_offload_keeps_callers_device_ids_alive(cuda):
    """A caller's int32 device id tensor, dropped right after offload() returns, is not handed to
    the compute stream's next allocation while the side stream's copies still read it: the pages
    that reach the host are the ones asked for, not those of whatever reuses the freed block."""
    from unifiedkv_amd.staging import PageStager

    pool = _pool(cuda, N=450, seed=2)
    rng = np.random.default_rng(7)
    busy = rng.permutation(450)[:400].tolist()
    sel = rng.permutation(np.arange(1, 450))[:64].tolist()
    k0 = pool.k_cache[:, sel].clone()
    st = PageStager(pool, chunk_pages=8)
    for _ in range(3):
        st.offload(busy)  # queues many small copies on the side stream ahead of the next offload
        ids = torch.tensor(sel, dtype=torch.int32, device=cuda)
        host = st.offload(ids)
        del ids
        junk = torch.empty(len(sel), dtype=torch.int32, device=cuda)  # the allocator's next block of that size
        junk.fill_(0)  # page 0 (never selected) on the compute stream
        host.event.synchronize()
        got = torch.cat([c for c in host.k_chunks], dim=1).to(cuda)
        assert torch.equal(got, k0)
