"""Host-side argument checks that must fire before any kernel launch (no GPU needed).

Tensors on the ``meta`` device carry shapes, dtypes and strides but no memory, so each
rejected case below proves that the wrapper raised before it could hand a pointer to
libukv.so; the accepted shapes then stop at the "must be on a GPU" check.
"""
import pytest
import torch

from unifiedkv_amd import page_ops, snapkv
from unifiedkv_amd.decode_step import DecodeBatch
from unifiedkv_amd.pool import PagedKVPool
from unifiedkv_amd.prefill import PrefillPages

META = torch.device("meta")


def _pool_layer(N=8, bs=16, H=2, D=64, dtype=torch.float16, dev=META):
    return torch.empty((N, bs, H, D), dtype=dtype, device=dev)


def _append_args(B=3, H=2, D=64, **over):
    args = dict(k_layer=_pool_layer(H=H, D=D), v_layer=_pool_layer(H=H, D=D),
                block_table=torch.empty((B, 4), dtype=torch.int32, device=META),
                old_lens=torch.empty((B,), dtype=torch.int32, device=META),
                k_new=torch.empty((B, H, D), dtype=torch.float16, device=META),
                v_new=torch.empty((B, H, D), dtype=torch.float16, device=META))
    args.update(over)
    return args


def test_kv_append_accepts_good_shapes_up_to_the_device_check():
    with pytest.raises(RuntimeError, match="must be on a GPU"):
        page_ops.kv_append(**_append_args())
    four_d = _append_args(k_new=torch.empty((3, 1, 2, 64), dtype=torch.float16, device=META),
                          v_new=torch.empty((3, 1, 2, 64), dtype=torch.float16, device=META))
    with pytest.raises(RuntimeError, match="must be on a GPU"):
        page_ops.kv_append(**four_d)


@pytest.mark.parametrize("bad, match", [
    (dict(old_lens=torch.empty((2,), dtype=torch.int32, device=META)), "old_lens has 2 entries"),
    (dict(k_new=torch.empty((2, 2, 64), dtype=torch.float16, device=META)), "k_new / v_new must be"),
    (dict(v_new=torch.empty((3, 4, 64), dtype=torch.float16, device=META)), "k_new / v_new must be"),
    (dict(k_new=torch.empty((3, 2, 32), dtype=torch.float16, device=META)), "k_new / v_new must be"),
    (dict(k_new=torch.empty((3, 2, 2, 64), dtype=torch.float16, device=META),
          v_new=torch.empty((3, 2, 2, 64), dtype=torch.float16, device=META)), r"\[batch, 1, H, D\]"),
    (dict(k_new=torch.empty((3, 2, 64), dtype=torch.bfloat16, device=META),
          v_new=torch.empty((3, 2, 64), dtype=torch.bfloat16, device=META)), "pool's dtype"),
    (dict(old_lens=torch.zeros((3,), dtype=torch.int32)), "old_lens is on cpu"),
    (dict(block_table=torch.zeros((3, 4), dtype=torch.int32)), "block_table is on cpu"),
    (dict(k_new=torch.zeros((3, 2, 64), dtype=torch.float16)), "k_new is on cpu"),
    (dict(v_layer=_pool_layer(N=9)), "equal"),
    (dict(block_table=torch.empty((3,), dtype=torch.int32, device=META)), r"\[batch, max_blocks\]"),
])
def test_kv_append_rejects_before_launch(bad, match):
    with pytest.raises(RuntimeError, match=match):
        page_ops.kv_append(**_append_args(**bad))


def test_kv_append_rejects_cpu_tensors():
    cpu = dict(k_layer=_pool_layer(dev="cpu"), v_layer=_pool_layer(dev="cpu"),
               block_table=torch.zeros((3, 4), dtype=torch.int32), old_lens=torch.zeros((3,), dtype=torch.int32),
               k_new=torch.zeros((3, 2, 64), dtype=torch.float16), v_new=torch.zeros((3, 2, 64), dtype=torch.float16))
    with pytest.raises(RuntimeError, match="must be on a GPU"):
        page_ops.kv_append(**cpu)


def _score_args(seqs=2, layers=2, Hq=8, Hkv=2, obs=16, D=64, table_rows=2, table_dev=META, dev=META):
    q = torch.empty((seqs, layers, Hq, obs, D), dtype=torch.float16, device=dev)
    k = torch.empty((layers, 64, 16, Hkv, D), dtype=torch.float16, device=dev)
    bt = torch.empty((table_rows, 40), dtype=torch.int32, device=table_dev)
    return q, k, bt


def test_score_blocks_rejects_short_or_foreign_tables():
    q, k, bt = _score_args(table_rows=1)
    with pytest.raises(RuntimeError, match="bad_score_shape"):
        snapkv.score_blocks(q, k, bt, seq_len=512, sink_len=16, obs_len=16, n_rep=4)
    q, k, bt = _score_args(table_dev="cpu")
    with pytest.raises(RuntimeError, match="bad_score_device"):
        snapkv.score_blocks(q, k, bt, seq_len=512, sink_len=16, obs_len=16, n_rep=4)
    q, k, bt = _score_args()
    with pytest.raises(RuntimeError, match="bad_score_device"):  # meta is not a GPU
        snapkv.score_blocks(q, k, bt, seq_len=512, sink_len=16, obs_len=16, n_rep=4)
    # a pool view whose key rows are not contiguous (the C entry point has no stride for D)
    k_t = torch.empty((2, 64, 16, 64, 2), dtype=torch.float16, device=META).transpose(3, 4)
    with pytest.raises(RuntimeError, match="k_pool_stride"):
        snapkv.score_blocks(q, k_t, bt, seq_len=512, sink_len=16, obs_len=16, n_rep=4)


class _FakePool:
    """The attributes DecodeBatch / PrefillPages read before they touch the device."""

    def __init__(self, N=64, B=16, layers=2):
        self.N_total, self.B, self.num_layers = N, B, layers


def test_decode_batch_rejects_lists_shorter_than_their_lengths():
    pool = _FakePool()
    with pytest.raises(ValueError, match="length 33 needs 3 pages"):
        DecodeBatch(pool, [[1, 2], [3, 4, 5]], [33, 33])
    with pytest.raises(ValueError, match="length 17 needs 2 pages"):
        DecodeBatch(pool, [[1]], [17])


def test_prefill_write_rejects_out_of_range_layers():
    pp = PrefillPages.__new__(PrefillPages)
    pp.pool = _FakePool(layers=2)
    pp._chunk = dict(total=4)
    for bad in (-1, 2, 7):
        with pytest.raises(IndexError, match="outside the pool"):
            pp.write(bad, None, None)


def test_decode_batch_rejects_pages_shared_between_sequences():
    with pytest.raises(ValueError, match="more than one sequence"):
        DecodeBatch(_FakePool(), [[1, 2], [3, 2]], [20, 20])


def test_token_io_and_page_copy_refuse_mismatched_or_host_tensors():
    pool = _pool_layer(H=2, D=64)
    with pytest.raises(ValueError, match="does not hold the pool's 2 heads x 64 dims"):
        page_ops.scatter_tokens(pool, [0, 1], torch.empty((1, 20, 64), dtype=torch.float16, device=META))
    with pytest.raises(ValueError, match="does not hold"):
        page_ops.scatter_tokens(pool, [0, 1], torch.empty((2, 20, 32), dtype=torch.float16, device=META))
    with pytest.raises(ValueError, match="one dtype"):
        page_ops.scatter_tokens(pool, [0, 1], torch.empty((2, 20, 64), dtype=torch.bfloat16, device=META))
    with pytest.raises(RuntimeError, match="must be on a GPU"):
        page_ops.scatter_tokens(pool, [0, 1], torch.empty((2, 20, 64), dtype=torch.float16, device=META))
    with pytest.raises(RuntimeError, match="must be on a GPU"):
        page_ops.gather_tokens(_pool_layer(dev="cpu"), [0], 4)
    stacked = torch.empty((2, 8, 16, 2, 64), dtype=torch.float16)
    with pytest.raises(RuntimeError, match="must be on a GPU"):
        page_ops.page_copy([stacked], [stacked], [0], [1])


def test_select_blocks_refuses_host_scores():
    from unifiedkv_amd import compaction

    with pytest.raises(RuntimeError, match="must be on a GPU"):
        compaction.select_blocks(torch.rand((2, 10)), 3)


def test_write_chunk_kv_refuses_rows_that_do_not_match_the_pool():
    from unifiedkv_amd import prefill

    pool = _pool_layer(H=2, D=64)
    bt = torch.empty((2, 4), dtype=torch.int32, device=META)
    lens = torch.empty((2,), dtype=torch.int32, device=META)
    rows = lambda n, h=2, d=64: torch.empty((n, h, d), dtype=torch.float16, device=META)  # noqa: E731
    with pytest.raises(ValueError, match=r"must be \[total, 2, 64\]"):
        prefill.write_chunk_kv(pool, pool, rows(10, h=1), rows(10, h=1), bt, [0, 4, 10], lens)
    with pytest.raises(ValueError, match=r"must be \[total, 2, 64\]"):
        prefill.write_chunk_kv(pool, pool, rows(10), rows(9), bt, [0, 4, 10], lens)
    with pytest.raises(RuntimeError, match="paged_prefill_unavailable:device"):  # meta is not a GPU
        prefill.write_chunk_kv(pool, pool, rows(10), rows(10), bt, [0, 4, 10], lens)
    cpu_pool = _pool_layer(H=2, D=64, dev="cpu")
    cpu_rows = torch.empty((8, 2, 64), dtype=torch.float16)
    with pytest.raises(RuntimeError, match="paged_prefill_unavailable:device"):
        prefill.write_chunk_kv(cpu_pool, cpu_pool, cpu_rows, cpu_rows, torch.zeros((2, 4), dtype=torch.int32),
                               [0, 4, 8], torch.zeros((2,), dtype=torch.int32))
