"""Chunked prefill over the paged pool (row a9).

CPU: the fp64 prefill oracle is pinned by closed forms - its last chunk query
equals the Page16 decode closed form over the same keys, a single key returns
V_0, and perturbing keys after a query's position leaves that query unchanged.
GPU (marked gpu): the chunk K/V write is bit-exact against the restatement and
the attention matches the oracle to |err| <= 2e-3 + 1e-2 |ref| (NaN-aligned),
including BASELINE config 4 at full size on sampled (query, head) pairs.
"""
import math

import numpy as np
import pytest

from oracle import oracle, prefill_oracle
from unifiedkv_amd import workloads

ATOL, RTOL = 2e-3, 1e-2
LSE_TOL_JUMP = 5e-6  # log2 units, on top of the fp32 dot-product bound


def make_case(seed, prefix, chunk, Hq=32, Hkv=8, D=128, dtype="bf16", extra_pages=7):
    """Pages hold prefix + chunk tokens; q/k_new/v_new are the chunk's packed rows."""
    rng = np.random.default_rng(seed)
    B = len(prefix)
    kv = [p + c for p, c in zip(prefix, chunk)]
    pages = [(L + 15) // 16 for L in kv]
    N = sum(pages) + extra_pages
    perm = rng.permutation(N).astype(np.int32)
    lists, o = [], 0
    for n in pages:
        lists.append(perm[o:o + n])
        o += n
    bt = workloads.tables_from_pages(lists)
    rnd = lambda shape: workloads._round_bits(rng.standard_normal(shape, dtype=np.float32), dtype)
    total = sum(chunk)
    case = dict(k_cache=rnd((N, 16, Hkv, D)), v_cache=rnd((N, 16, Hkv, D)), q=rnd((total, Hq, D)),
                k_new=rnd((total, Hkv, D)), v_new=rnd((total, Hkv, D)), block_table=bt,
                cu=np.concatenate([[0], np.cumsum(chunk)]).astype(np.int32), kv_lens=np.array(kv, dtype=np.int32),
                dtype=dtype, scale=1.0 / math.sqrt(D), n_rep=Hq // Hkv, chunk=list(chunk))
    return case


def written_pool(case):
    """The pool after the chunk write (bit patterns), by the restatement."""
    k, v = case["k_cache"].copy(), case["v_cache"].copy()
    for b in range(len(case["kv_lens"])):
        rows = slice(case["cu"][b], case["cu"][b + 1])
        start = int(case["kv_lens"][b]) - (case["cu"][b + 1] - case["cu"][b])
        prefill_oracle.write_chunk(k, case["block_table"][b], start, case["k_new"][rows])
        prefill_oracle.write_chunk(v, case["block_table"][b], start, case["v_new"][rows])
    return k, v


def expected(case, rows=None, n_rep=None):
    dt = workloads.DTYPE_CODES[case["dtype"]]
    k, v = written_pool(case)
    f = lambda a: oracle.bits_to_f32(a, dt)
    return prefill_oracle.prefill_dense(f(case["q"]), f(k), f(v), case["block_table"], case["cu"], case["kv_lens"],
                                        softmax_scale=case["scale"], n_rep=n_rep or case["n_rep"], rows=rows)


# ------------------------------------------------------------------ CPU pinning
def test_last_chunk_query_equals_decode_closed_form():
    case = make_case(1, [40, 3], [9, 20], Hq=8, Hkv=2, D=16)
    out = expected(case)
    k, v = written_pool(case)
    f = lambda a: oracle.bits_to_f32(a, oracle.DT_BF16)
    last_rows = [int(case["cu"][b + 1]) - 1 for b in range(2)]
    dec = oracle.page16_decode_dense(f(case["q"][last_rows]), f(k), f(v), case["block_table"], case["kv_lens"],
                                     softmax_scale=case["scale"], n_rep=4)
    np.testing.assert_allclose(out[last_rows], dec, rtol=1e-12, atol=1e-12)


def test_single_key_returns_v0_and_causality():
    case = make_case(2, [0], [5], Hq=4, Hkv=1, D=16)
    out = expected(case)
    f = lambda a: oracle.bits_to_f32(a, oracle.DT_BF16)
    np.testing.assert_array_equal(out[0], np.broadcast_to(f(case["v_new"][0, 0]), (4, 16)))
    # keys after a query's position must not matter: change the last chunk row's K/V
    mod = dict(case)
    mod["k_new"] = case["k_new"].copy()
    mod["v_new"] = case["v_new"].copy()
    mod["k_new"][4] ^= 0x1234
    mod["v_new"][4] ^= 0x0F0F
    out2 = expected(mod)
    np.testing.assert_array_equal(out[:4], out2[:4])
    assert not np.allclose(out[4], out2[4])


def test_oracle_matches_torch_sdpa_with_a_bottom_right_causal_mask():
    """torch.nn.functional.scaled_dot_product_attention (CPU, fp32) is the dense attention HF
    falls back to without flash-attn; with an explicit bottom-right causal mask over
    prefix + chunk it must give the oracle's values."""
    import torch

    case = make_case(5, [37, 0, 90], [20, 9, 33], Hq=8, Hkv=2, D=32)
    out = expected(case)
    k, v = written_pool(case)
    f = lambda a: oracle.bits_to_f32(a, oracle.DT_BF16)
    for b in range(3):
        L = int(case["kv_lens"][b])
        C = int(case["cu"][b + 1] - case["cu"][b])
        if C == 0:
            continue
        pages = case["block_table"][b][: (L + 15) // 16]
        K = torch.tensor(f(k)[pages].reshape(-1, 2, 32)[:L]).transpose(0, 1).repeat_interleave(4, dim=0)
        V = torch.tensor(f(v)[pages].reshape(-1, 2, 32)[:L]).transpose(0, 1).repeat_interleave(4, dim=0)
        Q = torch.tensor(f(case["q"])[case["cu"][b]:case["cu"][b + 1]]).transpose(0, 1)
        mask = torch.arange(L)[None, :] <= (L - C + torch.arange(C))[:, None]
        ref = torch.nn.functional.scaled_dot_product_attention(Q, K, V, attn_mask=mask, scale=case["scale"])
        np.testing.assert_allclose(out[case["cu"][b]:case["cu"][b + 1]], ref.transpose(0, 1).numpy(),
                                   rtol=1e-5, atol=1e-6)


def _logical_kv(case, b):
    """Sequence b's keys and values [L, H_kv, D] (fp32) in logical order, from the written pool."""
    k, v = written_pool(case)
    f = lambda a: oracle.bits_to_f32(a, workloads.DTYPE_CODES[case["dtype"]])
    L = int(case["kv_lens"][b])
    pages = case["block_table"][b][: (L + 15) // 16]
    Hkv, D = k.shape[2], k.shape[3]
    return f(k)[pages].reshape(-1, Hkv, D)[:L], f(v)[pages].reshape(-1, Hkv, D)[:L]


@pytest.mark.parametrize("Hq,Hkv", [(4, 4), (8, 2), (8, 1)])
@pytest.mark.parametrize("prefix", [0, 37])
def test_prefill_rows_f32_matches_the_fp64_oracle(Hq, Hkv, prefix):
    """The config-4 CPU baseline's formulation (dense fp32 matmul-softmax-matmul of sampled chunk
    rows) equals the pinned fp64 prefill at n_rep 1, 4 and 8, with and without a prefix."""
    chunk = 23
    case = make_case(40 + Hq + Hkv + prefix, [prefix], [chunk], Hq=Hq, Hkv=Hkv, D=32)
    exp = expected(case)
    K, V = _logical_kv(case, 0)
    f = lambda a: oracle.bits_to_f32(a, oracle.DT_BF16)
    rows = np.array([0, 5, chunk - 1])
    got = prefill_oracle.prefill_rows_f32(f(case["q"])[rows], K, V, prefix + rows, softmax_scale=case["scale"],
                                          n_rep=Hq // Hkv)
    np.testing.assert_allclose(got, exp[rows], rtol=1e-5, atol=1e-5)
    # A causal mask one key too wide is caught at this tolerance.
    wide = prefill_oracle.prefill_rows_f32(f(case["q"])[rows[:2]], K, V, prefix + rows[:2] + 1,
                                           softmax_scale=case["scale"], n_rep=Hq // Hkv)
    assert np.abs(wide - exp[rows[:2]]).max() > 1e-3


# ---------------------------------------------------------------------- GPU
def to_dev(case, cuda):
    import torch

    tdt = torch.bfloat16 if case["dtype"] == "bf16" else torch.float16
    up = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(cuda).view(tdt)
    return dict(q=up(case["q"]), k_new=up(case["k_new"]), v_new=up(case["v_new"]), k_cache=up(case["k_cache"]),
                v_cache=up(case["v_cache"]), block_table=torch.from_numpy(case["block_table"]).to(cuda),
                cu=torch.from_numpy(case["cu"]).to(cuda), kv_lens=torch.from_numpy(case["kv_lens"]).to(cuda))


def run_gpu(case, cuda, n_rep=None):
    from unifiedkv_amd import prefill

    t = to_dev(case, cuda)
    out = prefill.chunked_prefill(t["q"], t["k_new"], t["v_new"], t["k_cache"], t["v_cache"], t["block_table"],
                                  t["cu"], t["kv_lens"], softmax_scale=case["scale"], n_rep=n_rep or case["n_rep"],
                                  max_chunk=max(case["chunk"]))
    return out, t


def check(actual, exp, what):
    ok, err, exc = oracle.allclose_report(actual, exp, ATOL, RTOL)
    assert ok, f"{what}: max_abs_err={err:.3e} excess={exc:.3e}"


@pytest.mark.gpu
@pytest.mark.parametrize("prefix,chunk", [([0], [37]), ([100, 16], [64, 16]), ([333, 0, 48], [5, 70, 1]),
                                          ([2000], [300]), ([17], [129]), ([50, 20], [0, 9]), ([15], [1]),
                                          ([31], [33]), ([64, 1], [64, 63]), ([4000], [17])])
@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_prefill_matches_oracle(cuda, prefix, chunk, dtype):
    case = make_case(sum(prefix) + sum(chunk), prefix, chunk, dtype=dtype)
    out, t = run_gpu(case, cuda)
    import torch

    k_dev = t["k_cache"].view(torch.int16).cpu().numpy().view(np.uint16)
    k_exp, _ = written_pool(case)
    np.testing.assert_array_equal(k_dev, k_exp)  # the chunk write, bit-exact
    check(out.float().cpu().numpy(), expected(case), f"prefix={prefix} chunk={chunk} {dtype}")


@pytest.mark.gpu
@pytest.mark.parametrize("Hq,Hkv,D", [(32, 32, 128), (16, 8, 128), (64, 8, 128), (16, 1, 128), (32, 8, 64),
                                      (24, 8, 128), (32, 8, 96)])
def test_prefill_head_shapes(cuda, Hq, Hkv, D):
    case = make_case(Hq + D, [50, 7], [40, 33], Hq=Hq, Hkv=Hkv, D=D)
    out, _ = run_gpu(case, cuda)
    check(out.float().cpu().numpy(), expected(case), f"Hq={Hq} Hkv={Hkv} D={D}")


@pytest.mark.gpu
@pytest.mark.parametrize("big", [70000.0, 3.0e38])
def test_prefill_bf16_v_beyond_fp16_range(cuda, big):
    """bf16 V values that fp16 cannot hold take the fp32 fallback and still match."""
    case = make_case(77, [300, 40], [64, 25])
    bits = workloads._round_bits(np.array([big, -big / 3], dtype=np.float32), "bf16")
    case["v_cache"][case["block_table"][0][3], 5, 2, 7] = bits[0]  # a prefix key of sequence 0
    case["v_new"][70, 1, 100] = bits[1]  # a chunk key of sequence 1
    out, _ = run_gpu(case, cuda)
    got = out.float().cpu().numpy()
    exp = expected(case)
    fin = np.isfinite(exp)
    assert np.array_equal(np.isfinite(got), fin)
    check(np.where(fin, got, 0.0), np.where(fin, exp, 0.0), f"bf16 V with |v| = {big}")


@pytest.mark.gpu
def test_prefill_bf16_v_beyond_fp16_range_under_a_vanishing_weight(cuda):
    """A bf16 V of 3e38 at a key whose weight (below 2^-30 of the running max's even when that
    lags the largest score by the whole 2^8 allowance) rounds to zero in fp16: its true share,
    ~1e-13 x 3e38, dominates those outputs, so the workgroup must still take the fp32 fallback
    however small the key's fp16 weight is."""
    case = make_case(78, [300, 40], [64, 25])
    f = lambda a: oracle.bits_to_f32(a, oracle.DT_BF16)
    u = f(case["q"][0, 0])
    case["q"][:] = case["q"][0, 0]
    low = workloads._round_bits((-24.0 / (case["scale"] * float(u @ u)) * u).astype(np.float32), "bf16")
    page = case["block_table"][0][5]
    case["k_cache"][page, 3] = low                       # prefix key 83 of sequence 0, every head
    case["v_cache"][page, 3, 2, 7] = workloads._round_bits(np.array([3.0e38], np.float32), "bf16")[0]
    exp = expected(case)
    assert np.isfinite(exp).all() and np.abs(exp).max() > 1e20   # the vanishing weight's share shows
    out, _ = run_gpu(case, cuda)
    check(out.float().cpu().numpy(), exp, "bf16 V of 3e38 under a weight fp16 rounds to zero")


@pytest.mark.gpu
@pytest.mark.parametrize("Hq,Hkv,chunk", [
    (32, 8, [640] * 8),                              # 4 + 4 blocks of 96 / 64 queries per pair
    (32, 8, [640, 600, 37, 640, 1, 640, 333, 0]),    # the same plan over ragged chunks
    (32, 2, [600] * 8),                              # n_rep 16: 16 + 14 blocks of 24 / 16 queries
    (16, 1, [1024, 1000, 512, 1024, 7, 1024, 900, 1024]),  # n_rep 16, one KV head: 32 + 16
])
def test_prefill_block_plans_of_both_widths_sampled(cuda, Hq, Hkv, chunk):
    """Multi-round launches whose block plan (on a 256-CU device) mixes blocks of three and two
    column blocks per wave, anchored at each chunk's end, so shorter chunks leave partial and
    empty blocks at their start. Sampled (query, head) pairs - both ends of every chunk, the
    queries either side of the block boundaries, random ones - against the fp64 oracle."""
    prefix = [300, 0, 1000, 64, 17, 500, 2000, 5]
    case = make_case(sum(chunk) + Hq, prefix, chunk, Hq=Hq, Hkv=Hkv)
    out, t = run_gpu(case, cuda)
    got = out.float().cpu().numpy()
    qpb = 16 // (Hq // Hkv)
    rng = np.random.default_rng(3)
    rows = set()
    for b, C in enumerate(chunk):
        if C == 0:
            continue
        base = int(case["cu"][b])
        edges = {0, C - 1}
        for w in (8 * 3 * qpb, 8 * 2 * qpb):  # boundaries of either block width below the chunk's end
            for k in range(1, C // w + 1):
                if k % 3 == 1:
                    edges |= {C - k * w, C - k * w - 1}
        for i in edges | set(rng.integers(0, C, 6).tolist()):
            if 0 <= i < C:
                rows.add((base + int(i), int(rng.integers(0, Hq))))
    rows = sorted(rows)
    exp = expected(case, rows=rows)
    for r, h in rows:
        check(got[r, h], exp[(r, h)], f"Hq={Hq} Hkv={Hkv} chunks {chunk}: row {r} head {h}")


@pytest.mark.gpu
def test_prefill_last_row_matches_page16_decode(cuda):
    """The last query of a chunk sees exactly the decode step's keys."""
    import torch

    from unifiedkv_amd.page16_native import page16_decode_attention

    case = make_case(9, [500, 260], [64, 40])
    out, t = run_gpu(case, cuda)
    last = (t["cu"][1:] - 1).long()
    dec = page16_decode_attention(t["q"][last].contiguous(), t["k_cache"], t["v_cache"], t["block_table"],
                                  t["kv_lens"], softmax_scale=case["scale"], n_rep=4)
    check(out[last].float().cpu().numpy(), dec.float().cpu().numpy(), "prefill last row vs decode")


def test_max_chunk_is_derived_or_checked_on_the_host():
    """As core/varlen.py:28-29 derives max_seqlen from the lengths: with host lengths an
    understated max_chunk is refused before any launch, and a missing one is derived."""
    import torch

    from unifiedkv_amd import prefill

    assert prefill._max_chunk([0, 5, 12, 12], None) == 7
    assert prefill._max_chunk(torch.tensor([0, 5, 12], dtype=torch.int32), 9) == 9
    assert prefill._max_chunk([0, 5, 12], 7) == 7
    assert prefill._max_chunk(None, 3, chunk_lens=[3, 1]) == 3
    for cu, mc, lens in (([0, 5, 12], 6, None), (torch.tensor([0, 5, 12]), 6, None), (None, 2, [3, 1]),
                         ([0, 1], -1, None)):
        with pytest.raises(RuntimeError, match="paged_prefill_shape_unsupported:max_chunk"):
            prefill._max_chunk(cu, mc, chunk_lens=lens)
    # through the public entry point, on CPU tensors: refused in the host checks, before the library
    z = lambda *s: torch.zeros(s, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="max_chunk"):
        prefill.chunked_prefill(z(12, 4, 128), z(12, 1, 128), z(12, 1, 128), z(4, 16, 1, 128), z(4, 16, 1, 128),
                                torch.zeros((2, 2), dtype=torch.int32), [0, 5, 12], [5, 7], softmax_scale=0.1,
                                n_rep=4, max_chunk=6)


@pytest.mark.gpu
@pytest.mark.parametrize("path", ["tiled", "scalar", "stats"])
def test_understated_max_chunk_on_device_lengths_gives_nan_rows(cuda, path):
    """Lengths only on the device cannot be checked without a synchronisation: a chunk longer than
    the declared max_chunk comes out NaN in every row of its output (loud), not as stale memory;
    chunks within it are unaffected. "stats" is the call that also writes SnapKV row statistics
    (through the C entry point: the Python wrapper reads those lengths back to check the window);
    the over-long chunk's statistics rows are NaN and flagged for the scorer to recompute."""
    import torch

    from unifiedkv_amd import _ext, prefill, snapkv

    D = 128 if path != "scalar" else 64
    case = make_case(61, [300, 40, 10], [150, 90, 20], Hq=8, Hkv=2, D=D)
    mc = 100  # sequence 0's chunk (150 queries) is longer
    t = to_dev(case, cuda)
    prefill.write_chunk_kv(t["k_cache"], t["v_cache"], t["k_new"], t["v_new"], t["block_table"], t["cu"], t["kv_lens"],
                           max(case["chunk"]))
    st = snapkv.ObsStats(3, 1, 8, sink_len=16, obs_len=16, softmax_scale=case["scale"], device=cuda)
    exp = expected(case, n_rep=4)
    for _ in range(2):  # the second call's output memory held the first call's values
        if path != "stats":
            out = prefill.paged_prefill_attention(t["q"], t["k_cache"], t["v_cache"], t["block_table"], t["cu"],
                                                  t["kv_lens"], softmax_scale=case["scale"], n_rep=4, max_chunk=mc)
        else:
            out = torch.empty_like(t["q"])
            code = _ext.load().ukv_paged_prefill_obs_stats(
                t["q"].data_ptr(), t["k_cache"].data_ptr(), t["v_cache"].data_ptr(), t["block_table"].data_ptr(),
                t["cu"].data_ptr(), t["kv_lens"].data_ptr(), out.data_ptr(), 3, int(t["q"].shape[0]), mc, 8, 2, D, 4,
                int(t["block_table"].shape[1]), int(t["k_cache"].shape[0]), _ext.i64_array(t["q"].stride()[:2]),
                _ext.i64_array(t["k_cache"].stride()[:3]), _ext.i64_array(t["v_cache"].stride()[:3]),
                float(case["scale"]), _ext.UKV_DTYPE_BF16, 16, 16, *st.layer_view(0),
                torch.cuda.current_stream().cuda_stream)
            assert code == _ext.UKV_OK
        torch.cuda.synchronize()
        got = out.float().cpu().numpy()
        assert np.isnan(got[:150]).all(), f"{path}: rows of the over-long chunk must all be NaN"
        check(got[150:], exp[150:], f"{path}: chunks within max_chunk")
    if path == "stats":
        rows = st.data[0, 0].cpu().numpy()  # sequence 0, layer 0: [H_q, obs, 2]
        assert np.isnan(rows[..., 0]).all() and (rows[..., 1] == 1).all()
        assert np.isfinite(st.data[1:, 0, ..., 0].cpu().numpy()).all()


@pytest.mark.gpu
def test_statistics_rows_of_chunks_shorter_than_the_window_are_left_alone(cuda):
    """Through the C entry point (the Python wrapper refuses such chunks): a sequence whose chunk
    holds fewer than obs_len queries has window rows only for the queries it holds (none for an
    empty chunk); the other slots keep what they held. A sequence whose keys all lie in the sink
    has an empty middle: its rows are flagged. The attention output is the plain prefill's."""
    import torch

    from unifiedkv_amd import _ext, prefill, snapkv

    case = make_case(62, [300, 40, 10], [150, 0, 5], Hq=8, Hkv=2, D=128)
    t = to_dev(case, cuda)
    prefill.write_chunk_kv(t["k_cache"], t["v_cache"], t["k_new"], t["v_new"], t["block_table"], t["cu"], t["kv_lens"],
                           max(case["chunk"]))
    st = snapkv.ObsStats(3, 1, 8, sink_len=16, obs_len=16, softmax_scale=case["scale"], device=cuda)
    st.data.fill_(-7.0)
    out = torch.empty_like(t["q"])
    code = _ext.load().ukv_paged_prefill_obs_stats(
        t["q"].data_ptr(), t["k_cache"].data_ptr(), t["v_cache"].data_ptr(), t["block_table"].data_ptr(),
        t["cu"].data_ptr(), t["kv_lens"].data_ptr(), out.data_ptr(), 3, int(t["q"].shape[0]), 150, 8, 2, 128, 4,
        int(t["block_table"].shape[1]), int(t["k_cache"].shape[0]), _ext.i64_array(t["q"].stride()[:2]),
        _ext.i64_array(t["k_cache"].stride()[:3]), _ext.i64_array(t["v_cache"].stride()[:3]),
        float(case["scale"]), _ext.UKV_DTYPE_BF16, 16, 16, *st.layer_view(0), torch.cuda.current_stream().cuda_stream)
    assert code == _ext.UKV_OK
    torch.cuda.synchronize()
    check(out.float().cpu().numpy(), expected(case, n_rep=4), "attention output with statistics")
    rows = st.data[:, 0].cpu().numpy()  # [seq, H_q, obs, (value, flag)]
    assert np.isfinite(rows[0, ..., 0]).all() and (rows[0, ..., 1] == 0).all()  # 450 keys, middle [16, 434)
    assert (rows[1] == -7.0).all()                                               # an empty chunk
    assert (rows[2, :, :11] == -7.0).all()                                       # 5 queries: rows 11 .. 15
    assert (rows[2, :, 11:, 1] == 1.0).all()                                     # 15 keys, all in the sink


@pytest.mark.gpu
def test_config4_full_size_sampled(cuda):
    """4 sequences x (16384-token prefix + 2048-token chunk), H_q=32, H_kv=8, D=128, bf16."""
    import torch

    from unifiedkv_amd import prefill

    rng = np.random.default_rng(44)
    B, P, C, Hq, Hkv, D = 4, 16384, 2048, 32, 8, 128
    per = (P + C) // 16
    N = B * per + 1000
    perm = rng.permutation(N).astype(np.int32)
    bt = perm[: B * per].reshape(B, per)
    g = torch.Generator(device=cuda)
    g.manual_seed(4)
    mk = lambda *s: torch.randn(s, generator=g, device=cuda).to(torch.bfloat16)
    k_cache, v_cache = mk(N, 16, Hkv, D), mk(N, 16, Hkv, D)
    q, k_new, v_new = mk(B * C, Hq, D), mk(B * C, Hkv, D), mk(B * C, Hkv, D)
    cu = torch.arange(0, B * C + 1, C, dtype=torch.int32, device=cuda)
    lens = torch.full((B,), P + C, dtype=torch.int32, device=cuda)
    btd = torch.from_numpy(bt).to(cuda)
    out = prefill.chunked_prefill(q, k_new, v_new, k_cache, v_cache, btd, cu, lens, softmax_scale=D ** -0.5,
                                  n_rep=4, max_chunk=C)
    torch.cuda.synchronize()
    samples = [(int(b * C + i), int(h)) for b, i, h in zip(rng.integers(0, B, 24), rng.integers(0, C, 24),
                                                          rng.integers(0, Hq, 24))]
    samples += [(0, 0), (C - 1, 31), (B * C - 1, 5), (2 * C, 17)]
    # host copies of only the pages the sampled sequences use
    seqs = sorted({r // C for r, _ in samples})
    ids = torch.from_numpy(bt[seqs].reshape(-1).astype(np.int64)).to(cuda)
    kk = k_cache.index_select(0, ids).float().cpu().numpy()
    vv = v_cache.index_select(0, ids).float().cpu().numpy()
    sub_bt = np.arange(len(seqs) * per, dtype=np.int32).reshape(len(seqs), per)
    qf = q.float().cpu().numpy()
    rows = []
    for r, h in samples:
        s = seqs.index(r // C)
        rows.append((s * C + r % C, h))
    sub_q = np.concatenate([qf[b * C:(b + 1) * C] for b in seqs])
    exp = prefill_oracle.prefill_dense(sub_q, kk, vv, sub_bt, np.arange(0, len(seqs) * C + 1, C),
                                       np.full(len(seqs), P + C), softmax_scale=D ** -0.5, n_rep=4, rows=rows)
    got = out.float().cpu().numpy()
    for (r, h), (rr, hh) in zip(samples, rows):
        check(got[r, h], exp[(rr, hh)], f"config4 row {r} head {h}")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_prefill_score_jump_at_a_tiles_later_key(cuda, dtype):
    """A key whose score is 16 (natural units), far above every earlier key's, at a key of its
    32-key tile other than the first ones: the running max has to move to it, or its weight
    (beyond 2^16 under the old max) overflows fp16. Every query row is the same vector u and a
    jump key is gamma * u with gamma * scale * |u|^2 = 16, so it dominates each query that sees it. Sequence 0's jump key is prefix key
    126 (tile 3, offset 30), sequence 1's chunk key 231 (tile 7, offset 7: seen from chunk
    query 31 on). Both the plain and the statistics instance are checked against the oracle."""
    import torch

    from oracle import snapkv_oracle as so
    from unifiedkv_amd import prefill, snapkv

    case = make_case(11, [300, 200], [40, 96], dtype=dtype)
    f = lambda a: oracle.bits_to_f32(a, workloads.DTYPE_CODES[dtype])
    u = f(case["q"][0, 0])
    case["q"][:] = case["q"][0, 0]
    gamma = 16.0 / (case["scale"] * float(u @ u))
    jump = workloads._round_bits((gamma * u).astype(np.float32), dtype)
    case["k_cache"][case["block_table"][0][126 // 16], 126 % 16] = jump   # every KV head
    case["k_new"][int(case["cu"][1]) + 31] = jump
    k, _ = written_pool(case)
    assert float(f(k[case["block_table"][0][7], 14, 0]) @ u) * case["scale"] > 15.5
    exp = expected(case)
    out, t = run_gpu(case, cuda)
    got = out.float().cpu().numpy()
    assert np.all(np.isfinite(got))
    check(got, exp, f"score jump {dtype}")

    # the statistics instance over the same pool (the chunk is written): output and rows
    sink, obs = 4, 32
    Hq, D = case["q"].shape[1], case["q"].shape[2]
    st = snapkv.ObsStats(2, 1, Hq, sink_len=sink, obs_len=obs, softmax_scale=case["scale"], device=cuda)
    out2 = prefill.paged_prefill_attention(t["q"], t["k_cache"], t["v_cache"], t["block_table"], t["cu"],
                                           t["kv_lens"], softmax_scale=case["scale"], n_rep=case["n_rep"],
                                           obs_stats=st, layer_id=0)
    check(out2.float().cpu().numpy(), exp, f"score jump {dtype}, statistics instance")
    rows = st.data.cpu().numpy()
    for b in range(2):
        L = int(case["kv_lens"][b])
        Kd = f(k[case["block_table"][b]]).reshape(-1, k.shape[2], D)[:L].transpose(1, 0, 2)
        Qo = f(case["q"][int(case["cu"][b + 1]) - obs:int(case["cu"][b + 1])]).transpose(1, 0, 2)
        want = so.obs_row_stats(Kd, Qo, sink_len=sink, obs_len=obs, n_rep=case["n_rep"], scale=case["scale"])
        assert np.all(rows[b, 0, :, :, 1] == 0)
        # fp32 dot products of 128 terms summing to ~180 before scaling: the row's error bound
        # is D * 2^-24 * sum|q_d k_d| * scale * log2(e), about 2e-4 here
        bound = D * 2.0 ** -24 * float(np.abs(u * f(jump)).sum()) * case["scale"] / math.log(2) + LSE_TOL_JUMP
        err = np.abs(rows[b, 0, :, :, 0] - want).max()
        assert err <= bound, f"seq {b}: normaliser off by {err:.3e} > {bound:.3e}"
