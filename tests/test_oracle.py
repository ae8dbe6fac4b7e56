"""Pins the CPU oracle of the Page16 decode path (no GPU needed).

The oracle restates core/page16_native.py:34-80 (C page loop, fp32) and the
dense-rebuild formulation core/engine.py:4021-4115 (numpy fp64). The reference
ships no Page16 golden vectors, so the checks are: agreement of three
independent formulations, closed-form special cases, invariants, the committed
config-1 fixture, and planted mistakes that the checks must catch.
"""
import hashlib
import math
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle
from unifiedkv_amd import workloads

GOLDEN = Path(__file__).resolve().parent / "golden"


def small_case(seed, B=2, Hq=4, Hkv=2, D=8, N=12, lens=(37, 20), max_blocks=4, dtype=oracle.DT_BF16):
    rng = np.random.default_rng(seed)
    q = oracle.f32_to_bits(rng.standard_normal((B, Hq, D)).astype(np.float32), dtype)
    k = oracle.f32_to_bits(rng.standard_normal((N, 16, Hkv, D)).astype(np.float32), dtype)
    v = oracle.f32_to_bits(rng.standard_normal((N, 16, Hkv, D)).astype(np.float32), dtype)
    perm = rng.permutation(N).astype(np.int32)
    bt = np.zeros((B, max_blocks), dtype=np.int32)
    o = 0
    for b, L in enumerate(lens):
        n = (L + 15) // 16
        bt[b, :n] = perm[o:o + n]
        o += n
    return dict(q=q, k=k, v=v, bt=bt, lens=np.array(lens, dtype=np.int32), dtype=dtype,
                scale=1.0 / math.sqrt(D), n_rep=Hq // Hkv)


def run_loop(c, **kw):
    args = dict(softmax_scale=c["scale"], n_rep=c["n_rep"], dtype=c["dtype"])
    args.update(kw)
    return oracle.page16_decode_pageloop(c["q"], c["k"], c["v"], c["bt"], c["lens"], **args)


def run_dense(c, **kw):
    f = lambda a: oracle.bits_to_f32(a, c["dtype"])
    args = dict(softmax_scale=c["scale"], n_rep=c["n_rep"])
    args.update(kw)
    return oracle.page16_decode_dense(f(c["q"]), f(c["k"]), f(c["v"]), c["bt"], c["lens"], **args)


@pytest.mark.parametrize("dtype", [oracle.DT_F16, oracle.DT_BF16])
def test_three_formulations_agree(dtype):
    c = small_case(3, dtype=dtype)
    f = lambda a: oracle.bits_to_f32(a, dtype)
    brute = oracle.page16_decode_bruteforce(f(c["q"]).tolist(), f(c["k"]).tolist(), f(c["v"]).tolist(),
                                            c["bt"].tolist(), c["lens"].tolist(),
                                            softmax_scale=c["scale"], n_rep=c["n_rep"])
    dense = run_dense(c)
    loop = run_loop(c)
    np.testing.assert_allclose(dense, brute, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(loop, dense, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dtype", [oracle.DT_F16, oracle.DT_BF16])
def test_torch_cpu_dense_form_matches_the_closed_form(dtype):
    # The CPU baseline's second form (page gather + eager fp32 attention, as _rebuild_pkv).
    c = small_case(5, dtype=dtype)
    got = oracle.page16_decode_torch_dense(c["q"], c["k"], c["v"], c["bt"], c["lens"], softmax_scale=c["scale"],
                                           n_rep=c["n_rep"], dtype=dtype)
    np.testing.assert_allclose(got, run_dense(c), rtol=1e-5, atol=1e-6)


def test_pageloop_is_the_same_with_one_thread():
    c = small_case(6, dtype=oracle.DT_BF16)
    oracle.set_threads(1)
    one = run_loop(c)
    oracle.set_threads(4)
    many = run_loop(c)
    np.testing.assert_array_equal(one, many)  # each (sequence, head) is computed by one thread


def test_config1_pageloop_matches_dense():
    case = workloads.numpy_case("tiny", 7)
    c = dict(q=case["q"], k=case["k_cache"], v=case["v_cache"], bt=case["block_table"], lens=case["seqlens"],
             dtype=oracle.DT_F16, scale=case["scale"], n_rep=case["n_rep"])
    np.testing.assert_allclose(run_loop(c), run_dense(c), rtol=1e-4, atol=2e-6)


def test_golden_fixture_config1():
    fx = np.load(GOLDEN / "page16_tiny.npz")
    case = workloads.numpy_case("tiny", int(fx["seed"]))
    sha = lambda a: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
    assert sha(case["q"]) == str(fx["q_sha"])
    assert sha(case["k_cache"]) == str(fx["k_sha"])
    assert sha(case["v_cache"]) == str(fx["v_sha"])
    np.testing.assert_array_equal(case["block_table"], fx["block_table"])
    np.testing.assert_array_equal(case["seqlens"], fx["seqlens"])
    c = dict(q=case["q"], k=case["k_cache"], v=case["v_cache"], bt=case["block_table"], lens=case["seqlens"],
             dtype=oracle.DT_F16, scale=case["scale"], n_rep=case["n_rep"])
    np.testing.assert_allclose(run_dense(c), fx["out_f64"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(run_loop(c), fx["out_f64"], rtol=1e-4, atol=2e-6)
    # config 1 shape facts from the workload definition
    assert case["q"].shape == (4, 32, 128) and case["k_cache"].shape == (1024, 16, 8, 128)
    assert ((case["seqlens"] >= 256) & (case["seqlens"] <= 2048)).all()
    used = np.concatenate([case["block_table"][b, :(int(L) + 15) // 16] for b, L in enumerate(case["seqlens"])])
    assert len(np.unique(used)) == len(used)  # one draw without replacement


def test_single_token_returns_v0():
    c = small_case(5, lens=(1, 1))
    out = run_loop(c)
    f = lambda a: oracle.bits_to_f32(a, c["dtype"])
    V = f(c["v"])
    for b in range(2):
        for h in range(4):
            np.testing.assert_array_equal(out[b, h], V[c["bt"][b, 0], 0, h // c["n_rep"]])


def test_constant_keys_and_zero_scale_give_mean_of_v():
    c = small_case(6, lens=(40, 33))
    c["k"][:] = c["k"][0, 0, 0, 0]
    f = lambda a: oracle.bits_to_f32(a, c["dtype"]).astype(np.float64)
    V = f(c["v"])
    for run in (run_loop(c), run_loop(small_case(6, lens=(40, 33)), softmax_scale=0.0)):
        for b, L in enumerate(c["lens"]):
            rows = np.stack([V[c["bt"][b, t // 16], t % 16] for t in range(L)])  # [L, Hkv, D]
            for h in range(4):
                np.testing.assert_allclose(run[b, h], rows[:, h // 2].mean(0), rtol=1e-5, atol=1e-6)


def test_gqa_equals_mha_over_repeat_kv():
    c = small_case(8, Hq=8, Hkv=2, lens=(50, 17))
    rep = dict(c)
    rep["k"] = np.repeat(c["k"], 4, axis=2)  # repeat_kv: head g -> heads 4g..4g+3
    rep["v"] = np.repeat(c["v"], 4, axis=2)
    rep["n_rep"] = 1
    np.testing.assert_array_equal(run_loop(c), run_loop(rep))


def test_physical_page_permutation_is_invisible():
    c = small_case(9, N=16, lens=(49, 31))
    rng = np.random.default_rng(0)
    perm = rng.permutation(16)
    inv = np.argsort(perm)
    moved = dict(c)
    moved["k"] = c["k"][perm]  # new page i holds old page perm[i]
    moved["v"] = c["v"][perm]
    moved["bt"] = inv[c["bt"]].astype(np.int32)
    np.testing.assert_array_equal(run_loop(c), run_loop(moved))


def test_garbage_past_length_is_ignored():
    c = small_case(10, N=16, lens=(37, 20), max_blocks=6)
    base = run_loop(c)
    g = dict(c)
    rng = np.random.default_rng(1)
    g["k"] = c["k"].copy()
    g["v"] = c["v"].copy()
    for b, L in enumerate(c["lens"]):
        last = c["bt"][b, (L - 1) // 16]
        g["k"][last, L % 16 or 16:] = 0x7FC0  # NaN pattern in unused slots
        g["v"][last, L % 16 or 16:] = 0x7FC0
    g["bt"] = c["bt"].copy()
    g["bt"][0, 3:] = rng.integers(0, 16, 3)  # spare columns hold real page ids
    np.testing.assert_array_equal(base, run_loop(g))


def test_zero_length_is_nan_and_long_length_is_clamped():
    c = small_case(11, lens=(0, 64), max_blocks=4)
    out = run_loop(c)
    assert np.isnan(out[0]).all()
    clamp = dict(c)
    clamp["lens"] = np.array([0, 10_000], dtype=np.int32)
    np.testing.assert_array_equal(run_loop(clamp)[1], out[1])
    assert np.isnan(run_dense(c)[0]).all()


def test_invalid_page_ids_are_masked():
    c = small_case(12, N=12, lens=(48, 20))
    bad = dict(c)
    bad["bt"] = c["bt"].copy()
    bad["bt"][0, 1] = 9999  # tokens 16..31 of sequence 0 dropped
    out = run_loop(bad)
    ref = run_dense(bad)
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-6)
    assert not np.allclose(out[0], run_loop(c)[0])


@pytest.mark.parametrize("mutation", [1, 2, 3, 4, 5])
def test_planted_mistakes_are_caught(mutation):
    """Each planted mistake in the C restatement must disagree with the closed form."""
    c = small_case(13, B=2, Hq=8, Hkv=2, D=16, N=16, lens=(45, 29), max_blocks=4)
    # slot L holds a real finite row so an off-by-one mask changes the result
    dense = run_dense(c)
    ok, _, _ = oracle.allclose_report(run_loop(c, mutation=mutation), dense, atol=2e-3, rtol=1e-2)
    assert not ok, f"mutation {mutation} slipped through"
    ok0, _, _ = oracle.allclose_report(run_loop(c), dense, atol=2e-3, rtol=1e-2)
    assert ok0


def test_rounding_helpers():
    x = np.array([1.0, 1.00390625, 1.005859375, -2.5, 65504.0, np.inf, np.nan], dtype=np.float32)
    b = oracle.f32_to_bf16_bits(x)
    # 1.00390625 is the bf16 midpoint between 1.0 and 1.0078125 -> ties to even (1.0)
    assert b[0] == 0x3F80 and b[1] == 0x3F80 and b[2] == 0x3F81 and b[3] == 0xC020
    assert b[5] == 0x7F80 and (b[6] & 0x7FC0) == 0x7FC0
    np.testing.assert_array_equal(oracle.bf16_bits_to_f32(b[:5]), [1.0, 1.0, 1.0078125, -2.5, 65536.0])
    h = oracle.f32_to_f16_bits(np.array([1.0, 0.5, -3.0, 65504.0], dtype=np.float32))
    np.testing.assert_array_equal(oracle.f16_bits_to_f32(h), [1.0, 0.5, -3.0, 65504.0])
