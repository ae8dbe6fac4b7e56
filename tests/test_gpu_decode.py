"""Parity of the gfx950 Page16 decode kernels with the CPU oracle.

Tolerance (fp16/bf16 with fp32 accumulation on both sides):
|gpu - oracle| <= 2e-3 + 1e-2 * |oracle|, NaN where the oracle is NaN.
The oracle is the fp64 closed form (dense softmax over the gathered pages); the
C page loop that restates core/page16_native.py:34-80 is checked against the
same bound on the small cases.

Full-size configs 2 and 3 are checked on sampled sequences (their pages are
gathered into a compact pool and the oracle runs on that), plus two
size-independent properties: bit-identical output under a random permutation of
the physical pages, and run-to-run determinism. Closed forms: one attended token
returns its V row bit for bit, equal keys return the mean of V, and extra table
columns change nothing (bit-identical).
"""
import math

import numpy as np
import pytest

from oracle import oracle
from unifiedkv_amd import workloads

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def _torch():
    import torch

    return torch


def decode_gpu(tc, n_rep=None, scale=None):
    from unifiedkv_amd.page16_native import page16_decode_attention

    return page16_decode_attention(tc["q"], tc["k_cache"], tc["v_cache"], tc["block_table"], tc["seqlens"],
                                   softmax_scale=tc["scale"] if scale is None else scale,
                                   n_rep=tc["n_rep"] if n_rep is None else n_rep)


def to_f32(t):
    torch = _torch()
    return t.float().cpu().numpy() if t.dtype in (torch.float16, torch.bfloat16) else t.cpu().numpy()


def expected_dense(case, n_rep=None, scale=None):
    dt = workloads.DTYPE_CODES[case["dtype"]]
    f = lambda a: oracle.bits_to_f32(a, dt)
    return oracle.page16_decode_dense(f(case["q"]), f(case["k_cache"]), f(case["v_cache"]), case["block_table"],
                                      case["seqlens"], softmax_scale=case["scale"] if scale is None else scale,
                                      n_rep=case["n_rep"] if n_rep is None else n_rep)


def assert_close(actual, expected, what):
    ok, max_err, excess = oracle.allclose_report(actual, expected, ATOL, RTOL)
    assert ok, f"{what}: max_abs_err={max_err:.3e} worst_excess={excess:.3e}"


def custom_case(seed, B, Hq, Hkv, D, lens, dtype="bf16", N=None, max_blocks=None):
    rng = np.random.default_rng(seed)
    pages = [(int(L) + 15) // 16 for L in lens]
    N = N or max(8, int(sum(pages) * 1.25) + 3)
    draw = rng.permutation(N)[: sum(pages)].astype(np.int32)
    lists, o = [], 0
    for n in pages:
        lists.append(draw[o:o + n])
        o += n
    mb = max_blocks or max(1, max(pages))
    layout = dict(B=B, Hq=Hq, Hkv=Hkv, D=D, dtype=dtype, N=N, seqlens=np.array(lens, dtype=np.int32),
                  block_table=workloads.tables_from_pages(lists, mb))
    return workloads.numpy_decode_case(layout, seed)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_config1_tiny_fp16(cuda, seed):
    case = workloads.numpy_case("tiny", seed)
    out = to_f32(decode_gpu(workloads.to_torch(case)))
    assert_close(out, expected_dense(case), f"config1 seed {seed}")


def test_config1_matches_reference_order_pageloop(cuda):
    case = workloads.numpy_case("tiny", 1234)
    out = to_f32(decode_gpu(workloads.to_torch(case)))
    loop = oracle.page16_decode_pageloop(case["q"], case["k_cache"], case["v_cache"], case["block_table"],
                                         case["seqlens"], softmax_scale=case["scale"], n_rep=case["n_rep"],
                                         dtype=oracle.DT_F16)
    assert_close(out, loop, "config1 vs page loop")
    fx = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "page16_tiny.npz")
    assert_close(out, fx["out_f64"], "config1 vs golden fixture")


@pytest.mark.parametrize("Hq,Hkv,D", [
    (32, 8, 128), (32, 32, 128), (16, 8, 128), (64, 8, 128), (8, 8, 64), (32, 8, 64),
    (32, 4, 256), (32, 8, 256), (16, 1, 128), (28, 4, 128), (20, 4, 128), (32, 16, 64),
    (32, 8, 96), (32, 8, 80), (24, 8, 72),
])
@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_head_shapes(cuda, Hq, Hkv, D, dtype):
    case = custom_case(Hq * 1000 + D, 3, Hq, Hkv, D, [300, 1, 77], dtype=dtype)
    out = to_f32(decode_gpu(workloads.to_torch(case)))
    assert_close(out, expected_dense(case), f"Hq={Hq} Hkv={Hkv} D={D} {dtype}")


def test_page_boundary_lengths(cuda):
    lens = [1, 2, 15, 16, 17, 31, 32, 33, 255, 256, 257, 1000]
    case = custom_case(21, len(lens), 32, 8, 128, lens)
    out = to_f32(decode_gpu(workloads.to_torch(case)))
    assert_close(out, expected_dense(case), "boundary lengths")


def test_long_and_short_mix_many_chunks(cuda):
    lens = [5000, 16, 4097, 3, 2048]
    case = custom_case(22, len(lens), 32, 8, 128, lens)
    out = to_f32(decode_gpu(workloads.to_torch(case)))
    assert_close(out, expected_dense(case), "mixed lengths")


def test_zero_length_gives_nan_and_overlong_is_clamped(cuda):
    case = custom_case(23, 3, 32, 8, 128, [40, 64, 64], max_blocks=4)
    case["seqlens"] = np.array([0, 64, 10_000], dtype=np.int32)  # 10000 > 16*max_blocks=64
    out = to_f32(decode_gpu(workloads.to_torch(case)))
    exp = expected_dense(case)
    assert np.isnan(out[0]).all() and np.isnan(exp[0]).all()
    assert_close(out, exp, "zero / clamped lengths")


def test_stale_workspace_with_fewer_pages_than_workgroups(cuda):
    # A wide table with short sequences: B * max_blocks / 8 split workgroups but only 10
    # pages, so most workgroups own no page and write no partial. The workspace is
    # pre-filled with garbage (huge finite values, NaN, zeros) that must never be read.
    from unifiedkv_amd import _ext

    torch = _torch()
    lens = [20, 30, 16, 17, 1, 0, 33]
    B, Hq, Hkv, D, mb = len(lens), 32, 8, 128, 256
    case = custom_case(41, B, Hq, Hkv, D, lens, max_blocks=mb)
    tc = workloads.to_torch(case)
    exp = expected_dense(case)
    lib = _ext.load()
    ws_bytes = int(lib.ukv_page16_workspace_bytes(B, Hq, D, mb))
    for fill in (0x7F, 0xFF, 0x00):
        ws = torch.full((ws_bytes,), fill, dtype=torch.uint8, device=cuda)
        out = torch.empty_like(tc["q"])
        rc = lib.ukv_page16_decode(
            tc["q"].data_ptr(), tc["k_cache"].data_ptr(), tc["v_cache"].data_ptr(), tc["block_table"].data_ptr(),
            tc["seqlens"].data_ptr(), out.data_ptr(), B, Hq, Hkv, D, Hq // Hkv, mb, case["N"],
            _ext.i64_array(tc["q"].stride()[:2]), _ext.i64_array(tc["k_cache"].stride()[:3]),
            _ext.i64_array(tc["v_cache"].stride()[:3]), case["scale"], _ext.UKV_DTYPE_BF16, ws.data_ptr(), ws_bytes,
            torch.cuda.current_stream().cuda_stream)
        assert rc == _ext.UKV_OK
        got = to_f32(out)
        assert np.isnan(got[5]).all()
        assert_close(got, exp, f"stale workspace filled with {fill:#x}")


def test_one_workspace_serves_shapes_back_to_back(cuda):
    # One workspace serves calls of different shapes back to back (long, ragged, single-page
    # and empty sequences, several q-head groupings), each reading the partials the previous
    # call left behind as garbage; each call must match the oracle.
    from unifiedkv_amd import _ext

    torch = _torch()
    lib = _ext.load()
    ws = torch.full((64 << 20,), 0x7F, dtype=torch.uint8, device=cuda)
    shapes = [(4, 32, 8, 128, [3000, 17, 1, 2048], 200), (9, 16, 2, 64, [0, 700, 5000, 33, 64, 1, 900, 12, 3], 320),
              (2, 64, 8, 128, [40000, 1], 2500), (5, 8, 8, 256, [600, 0, 1200, 48, 16], 80)]
    for i, (B, Hq, Hkv, D, lens, mb) in enumerate(shapes):
        case = custom_case(300 + i, B, Hq, Hkv, D, lens, max_blocks=mb)
        tc = workloads.to_torch(case)
        out = torch.empty_like(tc["q"])
        rc = lib.ukv_page16_decode(
            tc["q"].data_ptr(), tc["k_cache"].data_ptr(), tc["v_cache"].data_ptr(), tc["block_table"].data_ptr(),
            tc["seqlens"].data_ptr(), out.data_ptr(), B, Hq, Hkv, D, Hq // Hkv, mb, case["N"],
            _ext.i64_array(tc["q"].stride()[:2]), _ext.i64_array(tc["k_cache"].stride()[:3]),
            _ext.i64_array(tc["v_cache"].stride()[:3]), case["scale"], _ext.UKV_DTYPE_BF16, ws.data_ptr(),
            ws.numel(), torch.cuda.current_stream().cuda_stream)
        assert rc == _ext.UKV_OK
        assert_close(to_f32(out), expected_dense(case), f"shape {i}")


def test_batch_of_4200_short_sequences(cuda):
    # 4200 sequences of 0..48 tokens: every workgroup holds many whole and split sequences,
    # and the combine walks 4200 x 32 (sequence, head) merges. Empty sequences give NaN.
    torch = _torch()
    B = 4200
    rng = np.random.default_rng(77)
    lens = rng.integers(0, 49, B)
    case = custom_case(78, B, 32, 8, 128, [int(x) for x in lens], max_blocks=3)
    out = to_f32(decode_gpu(workloads.to_torch(case)))
    exp = expected_dense(case)
    assert np.isnan(out[lens == 0]).all()
    assert_close(out, exp, "4200-sequence batch")
    torch.cuda.synchronize()


def test_invalid_page_ids_are_masked(cuda):
    case = custom_case(24, 2, 32, 8, 128, [64, 48])
    case["block_table"] = case["block_table"].copy()
    case["block_table"][0, 1] = case["N"] + 5
    case["block_table"][1, 0] = -3
    out = to_f32(decode_gpu(workloads.to_torch(case)))
    assert_close(out, expected_dense(case), "invalid page ids")


def test_nan_in_unused_slots_does_not_leak(cuda):
    case = custom_case(25, 2, 32, 8, 128, [37, 20])
    for b, L in enumerate(case["seqlens"]):
        last = case["block_table"][b, (L - 1) // 16]
        case["k_cache"][last, L % 16:] = 0x7FC0
        case["v_cache"][last, L % 16:] = 0x7FC0
    out = to_f32(decode_gpu(workloads.to_torch(case)))
    assert np.isfinite(out).all()
    assert_close(out, expected_dense(case), "NaN rows past the length")


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_closed_form_invariants(cuda, dtype):
    # One attended token: the output is that token's V row, bit for bit.
    case = custom_case(31, 4, 32, 8, 128, [1, 1, 1, 1], dtype=dtype)
    out = decode_gpu(workloads.to_torch(case)).view(_torch().int16).cpu().numpy().view(np.uint16)
    for b in range(4):
        page = case["block_table"][b, 0]
        for h in range(32):
            assert np.array_equal(out[b, h], case["v_cache"][page, 0, h // 4]), (b, h)
    # Every key of a head equal: uniform weights, the output is the mean of the head's V rows.
    lens = [300, 17, 1024]
    case = custom_case(32, 3, 32, 8, 128, lens, dtype=dtype)
    case["k_cache"] = case["k_cache"].copy()
    case["k_cache"][:, :] = case["k_cache"][0, 0]
    got = to_f32(decode_gpu(workloads.to_torch(case)))
    v = oracle.bits_to_f32(case["v_cache"], workloads.DTYPE_CODES[dtype]).astype(np.float64)
    for b, L in enumerate(lens):
        rows = np.concatenate([v[case["block_table"][b, p]] for p in range((L + 15) // 16)])[:L]  # [L, Hkv, D]
        mean = rows.mean(axis=0)
        for h in range(32):
            assert np.all(np.abs(got[b, h] - mean[h // 4]) <= ATOL + RTOL * np.abs(mean[h // 4])), (b, h)
    # Extra table columns holding other pages change nothing (bit-identical). The batch is
    # long enough (3 x 688 pages) that both tables split over one workgroup per CU.
    lens = [200, 33, 11000]
    case = custom_case(33, 3, 32, 8, 128, lens, dtype=dtype)
    base = decode_gpu(workloads.to_torch(case)).view(_torch().int16).cpu().numpy()
    wide = case["block_table"]
    extra = np.random.default_rng(5).integers(0, case["N"], size=(3, 9)).astype(np.int32)
    case["block_table"] = np.concatenate([wide, extra], axis=1)
    for b, L in enumerate(lens):  # and past each sequence's pages within its row
        case["block_table"][b, (L + 15) // 16:wide.shape[1]] = extra[b, 0]
    again = decode_gpu(workloads.to_torch(case)).view(_torch().int16).cpu().numpy()
    assert np.array_equal(base, again)


def test_explicit_n_rep_and_scale(cuda):
    # q head h reads KV head h // n_rep with n_rep passed by the caller (core/page16_native.py:36)
    case = custom_case(26, 2, 16, 8, 128, [90, 33])
    tc = workloads.to_torch(case)
    out = to_f32(decode_gpu(tc, n_rep=4, scale=0.05))
    assert_close(out, expected_dense(case, n_rep=4, scale=0.05), "n_rep=4 on 8 kv heads")


def test_int64_table_and_strided_cache_views(cuda):
    torch = _torch()
    case = custom_case(27, 2, 32, 8, 128, [70, 130], dtype="bf16")
    tc = workloads.to_torch(case)
    exp = expected_dense(case)
    tc64 = dict(tc)
    tc64["block_table"] = tc["block_table"].to(torch.int64)
    assert_close(to_f32(decode_gpu(tc64)), exp, "int64 table")
    # a layer of a 5-D pool [layers, N, 16, Hkv, D] (core/pool.py:67-71)
    for key in ("k_cache", "v_cache"):
        pool = torch.zeros((3,) + tuple(tc[key].shape), dtype=tc[key].dtype, device=tc[key].device)
        pool[1] = tc[key]
        tc64[key] = pool[1]
    assert_close(to_f32(decode_gpu(tc64)), exp, "pool layer view")
    # rows padded in memory (token stride 8*128+8 elements: 16-byte aligned, fast path)
    # and rows misaligned (token stride +4 elements: scalar path)
    for pad in (8, 4):
        sv = dict(tc)
        for key in ("k_cache", "v_cache"):
            N, P, H, D = tc[key].shape
            buf = torch.zeros((N, P, H * D + pad), dtype=tc[key].dtype, device=tc[key].device)
            buf[:, :, : H * D] = tc[key].reshape(N, P, H * D)
            sv[key] = buf.as_strided((N, P, H, D), (P * (H * D + pad), H * D + pad, D, 1))
        assert_close(to_f32(decode_gpu(sv)), exp, f"strided rows pad={pad}")


def test_runs_on_current_stream_without_sync(cuda):
    torch = _torch()
    case = custom_case(28, 4, 32, 8, 128, [500, 600, 700, 800])
    tc = workloads.to_torch(case)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        out = decode_gpu(tc)
    s.synchronize()
    assert_close(to_f32(out), expected_dense(case), "side stream")


# ---------------------------------------------------------------------------
# Full-size BASELINE configs
# ---------------------------------------------------------------------------
def _sample_check(tc, layout, seqs, what):
    """Oracle on sequences `seqs`: gather their pages into a compact host pool."""
    torch = _torch()
    out = decode_gpu(tc)
    torch.cuda.synchronize()
    bt = layout["block_table"]
    lens = layout["seqlens"]
    sub_pages, sub_rows = [], []
    o = 0
    for b in seqs:
        n = (int(lens[b]) + 15) // 16
        sub_pages.append(bt[b, :n])
        sub_rows.append(np.arange(o, o + n, dtype=np.int32))
        o += n
    ids = torch.from_numpy(np.concatenate(sub_pages).astype(np.int64)).to(tc["k_cache"].device)
    k = tc["k_cache"].index_select(0, ids).view(torch.int16).cpu().numpy().view(np.uint16)
    v = tc["v_cache"].index_select(0, ids).view(torch.int16).cpu().numpy().view(np.uint16)
    q = tc["q"][list(seqs)].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    case = dict(q=q, k_cache=k, v_cache=v, block_table=workloads.tables_from_pages(sub_rows),
                seqlens=lens[list(seqs)], dtype=layout["dtype"], scale=tc["scale"], n_rep=tc["n_rep"])
    exp = expected_dense(case)
    assert_close(to_f32(out[list(seqs)]), exp, what)
    return out


def _permutation_property(tc, out_ref, seed):
    """Relabel physical pages with a random permutation: output must be bit-identical."""
    torch = _torch()
    N = tc["k_cache"].shape[0]
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    perm = torch.randperm(N, generator=g).to(tc["k_cache"].device)  # new page i holds old page perm[i]
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(N, device=perm.device)
    moved = dict(tc)
    moved["k_cache"] = tc["k_cache"].index_select(0, perm)
    moved["v_cache"] = tc["v_cache"].index_select(0, perm)
    moved["block_table"] = inv[tc["block_table"].long()].to(torch.int32)
    out2 = decode_gpu(moved)
    out3 = decode_gpu(tc)
    torch.cuda.synchronize()
    assert torch.equal(out2.view(torch.int16), out_ref.view(torch.int16)), "page permutation changed the output"
    assert torch.equal(out3.view(torch.int16), out_ref.view(torch.int16)), "non-deterministic output"
    del moved


def test_config2_longctx_full_size(cuda):
    layout = workloads.layout_longctx(np.random.default_rng(2024))
    tc = workloads.torch_decode_case(layout, 2024)
    out = _sample_check(tc, layout, [0, 11], "config2 sampled sequences")
    assert np.isfinite(to_f32(out)).all()
    _permutation_property(tc, out, 7)


def test_config3_ragged_full_size(cuda):
    layout = workloads.layout_ragged(np.random.default_rng(3))
    tc = workloads.torch_decode_case(layout, 3)
    lens = layout["seqlens"]
    seqs = [int(np.argmax(lens)), int(np.argmin(lens)), 5, 40]
    out = _sample_check(tc, layout, seqs, "config3 sampled sequences")
    _permutation_property(tc, out, 8)
