"""Seeded random-shape parity sweep of the attention kernels against the oracle.

Each case draws its own shape from its seed: head layout (H_kv, n_rep, D), dtype,
batch, ragged lengths (including empty sequences, one-page sequences and, for the
plain decode, a length beyond its table row), zero-padded tables with a few
out-of-range page ids. The kernels must match the fp64 oracle to
|err| <= 2e-3 + 1e-2 |ref| (NaN-aligned); pool writes (the fused decode append and
the prefill chunk write) must match the restatement bit for bit. SnapKV block
scores use the bound of tests/test_snapkv.py (1e-4 of the row maximum + 1e-3 rel).

The fused append is drawn without lengths beyond the table row: such a length
attends the row's zero padding (page 0), which may be another sequence's append
target, and the header states that case as outside the fused call's contract.
"""
import math

import numpy as np
import pytest

from oracle import oracle, prefill_oracle
from oracle import snapkv_oracle as so
from unifiedkv_amd import workloads

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def _bits(rng, shape, dt):
    return workloads._round_bits(rng.standard_normal(shape, dtype=np.float32), dt)


def _up(a, dt):
    import torch

    tdt = torch.bfloat16 if dt == "bf16" else torch.float16
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda().view(tdt)


def _i32(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).cuda()


def _down(t):
    import torch

    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def _f(a, dt):
    return oracle.bits_to_f32(a, workloads.DTYPE_CODES[dt])


def _check(got, want, what):
    ok, err, exc = oracle.allclose_report(got, want, ATOL, RTOL)
    assert ok, f"{what}: max_abs_err={err:.3e} worst_excess={exc:.3e}"


def _decode_layout(rng, append):
    dt = str(rng.choice(["bf16", "fp16"]))
    Hkv = int(rng.choice([1, 2, 4, 8]))
    n_rep = int(rng.choice([1, 2, 3, 4, 5, 8, 16]))
    D = int(rng.choice([64, 128, 256]))
    B = int(rng.integers(1, 40))
    lens = rng.integers(0, 3000, size=B)
    lens[rng.random(B) < 0.1] = 0
    lens[rng.random(B) < 0.1] = rng.integers(1, 17)
    pages = [(int(L) + 15) // 16 for L in lens]
    mb = max(1, max(pages) + int(rng.integers(0, 4)))
    N = max(8, sum(pages) + int(rng.integers(1, 20)))
    perm = rng.permutation(N).astype(np.int32)
    bt = np.zeros((B, mb), np.int32)
    o = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[o:o + n]
        o += n
    if rng.random() < 0.3:
        bt[rng.random(bt.shape) < 0.02] = rng.choice([-1, N, N + 5, -100])
    if not append and rng.random() < 0.15:
        lens[0] = 16 * mb + int(rng.integers(1, 40))
    return dt, Hkv, n_rep, D, B, lens.astype(np.int32), bt, N


@pytest.mark.parametrize("seed", range(24))
def test_random_decode(cuda, seed):
    from unifiedkv_amd.page16_native import page16_decode_attention

    rng = np.random.default_rng(1000 + seed)
    dt, Hkv, n_rep, D, B, lens, bt, N = _decode_layout(rng, append=False)
    Hq = Hkv * n_rep
    q, k, v = _bits(rng, (B, Hq, D), dt), _bits(rng, (N, 16, Hkv, D), dt), _bits(rng, (N, 16, Hkv, D), dt)
    scale = 1.0 / math.sqrt(D)
    out = page16_decode_attention(_up(q, dt), _up(k, dt), _up(v, dt), _i32(bt), _i32(lens), softmax_scale=scale,
                                  n_rep=n_rep)
    want = oracle.page16_decode_dense(_f(q, dt), _f(k, dt), _f(v, dt), bt, lens, softmax_scale=scale, n_rep=n_rep)
    _check(out.float().cpu().numpy(), want, f"seed {seed} {dt} B={B} Hq={Hq} Hkv={Hkv} D={D}")


@pytest.mark.parametrize("seed", range(24))
def test_random_decode_append(cuda, seed):
    from unifiedkv_amd.page16_native import page16_decode_append_attention

    rng = np.random.default_rng(2000 + seed)
    dt, Hkv, n_rep, D, B, lens, bt, N = _decode_layout(rng, append=True)
    Hq = Hkv * n_rep
    q, k, v = _bits(rng, (B, Hq, D), dt), _bits(rng, (N, 16, Hkv, D), dt), _bits(rng, (N, 16, Hkv, D), dt)
    kn, vn = _bits(rng, (B, Hkv, D), dt), _bits(rng, (B, Hkv, D), dt)
    scale = 1.0 / math.sqrt(D)
    kd, vd = _up(k, dt), _up(v, dt)
    out = page16_decode_append_attention(_up(q, dt), kd, vd, _i32(bt), _i32(lens), _up(kn, dt), _up(vn, dt),
                                         softmax_scale=scale, n_rep=n_rep)
    mb = bt.shape[1]
    for b in range(B):  # the restatement of the append (core/scheduler.py:401-408) on valid slots
        L = int(lens[b])
        if 0 < L <= 16 * mb and 0 <= bt[b, (L - 1) // 16] < N:
            k[bt[b, (L - 1) // 16], (L - 1) % 16] = kn[b]
            v[bt[b, (L - 1) // 16], (L - 1) % 16] = vn[b]
    what = f"seed {seed} {dt} B={B} Hq={Hq} Hkv={Hkv} D={D}"
    np.testing.assert_array_equal(_down(kd), k, err_msg=what)
    np.testing.assert_array_equal(_down(vd), v, err_msg=what)
    want = oracle.page16_decode_dense(_f(q, dt), _f(k, dt), _f(v, dt), bt, lens, softmax_scale=scale, n_rep=n_rep)
    _check(out.float().cpu().numpy(), want, what)


@pytest.mark.parametrize("seed", range(16))
def test_random_prefill(cuda, seed):
    from unifiedkv_amd import prefill

    rng = np.random.default_rng(3000 + seed)
    dt = str(rng.choice(["bf16", "fp16"]))
    Hkv = int(rng.choice([1, 2, 4, 8]))
    n_rep = int(rng.choice([1, 2, 4, 8]))
    D = int(rng.choice([64, 96, 128, 128]))
    B = int(rng.integers(1, 5))
    prefix = [int(x) for x in rng.integers(0, 700, size=B)]
    chunk = [int(x) for x in rng.integers(0, 200, size=B)]
    chunk[0] = max(chunk[0], 1)
    kv = [p + c for p, c in zip(prefix, chunk)]
    pages = [(L + 15) // 16 for L in kv]
    N = sum(pages) + 5
    perm = rng.permutation(N).astype(np.int32)
    lists = np.split(perm[: sum(pages)], np.cumsum(pages)[:-1])
    bt = workloads.tables_from_pages(lists)
    Hq, total = Hkv * n_rep, sum(chunk)
    k, v = _bits(rng, (N, 16, Hkv, D), dt), _bits(rng, (N, 16, Hkv, D), dt)
    q, kn, vn = _bits(rng, (total, Hq, D), dt), _bits(rng, (total, Hkv, D), dt), _bits(rng, (total, Hkv, D), dt)
    cu = np.concatenate([[0], np.cumsum(chunk)]).astype(np.int32)
    kvl = np.array(kv, np.int32)
    scale = 1.0 / math.sqrt(D)
    kd, vd = _up(k, dt), _up(v, dt)
    out = prefill.chunked_prefill(_up(q, dt), _up(kn, dt), _up(vn, dt), kd, vd, _i32(bt), _i32(cu), _i32(kvl),
                                  softmax_scale=scale, n_rep=n_rep, max_chunk=max(chunk))
    for b in range(B):
        rows = slice(cu[b], cu[b + 1])
        prefill_oracle.write_chunk(k, bt[b], prefix[b], kn[rows])
        prefill_oracle.write_chunk(v, bt[b], prefix[b], vn[rows])
    what = f"seed {seed} {dt} Hq={Hq} Hkv={Hkv} D={D} prefix={prefix} chunk={chunk}"
    np.testing.assert_array_equal(_down(kd), k, err_msg=what)
    np.testing.assert_array_equal(_down(vd), v, err_msg=what)
    want = prefill_oracle.prefill_dense(_f(q, dt), _f(k, dt), _f(v, dt), bt, cu, kvl, softmax_scale=scale,
                                        n_rep=n_rep)
    _check(out.float().cpu().numpy(), want, what)


@pytest.mark.parametrize("seed", range(24))
def test_random_snapkv_scores(cuda, seed):
    from unifiedkv_amd import snapkv

    rng = np.random.default_rng(4000 + seed)
    dt = str(rng.choice(["bf16", "fp16"]))
    h_kv = int(rng.choice([1, 2, 4, 8]))
    n_rep = int(rng.choice([1, 2, 4, 8]))
    D = int(rng.choice([32, 64, 128]))
    obs = int(rng.choice([16, 24, 32, 40, 48, 64, 80, 96, 128]))
    sink = int(rng.choice([0, 4, 16, 32, 64]))
    L = int(rng.integers(sink + obs + 1, sink + obs + 2500))
    K, Q = _bits(rng, (h_kv, L, D), dt), _bits(rng, (h_kv * n_rep, obs, D), dt)
    got = snapkv.score_layer_blocks(_up(K, dt), _up(Q, dt), sink_len=sink, obs_len=obs, n_rep=n_rep).cpu().numpy()
    want = so.score_layer_blocks(_f(K, dt), _f(Q, dt), sink_len=sink, obs_len=obs, n_rep=n_rep)
    what = f"seed {seed} {dt} h_kv={h_kv} n_rep={n_rep} D={D} L={L} sink={sink} obs={obs}"
    assert got.shape == want.shape, what
    if want.size:
        err = np.abs(got - want)
        bound = 1e-4 * np.abs(want).max() + 1e-3 * np.abs(want)
        assert np.all(err <= bound), f"{what}: max err {err.max():.3e}"



PROFILES = ("jump", "sink", "sharp", "bigv")


def _scaled(a, factor, dt):
    return workloads._round_bits(_f(a, dt) * np.float32(factor), dt)


def _sink_row(q, dt, D):
    """A key along the queries' mean direction, 3 sqrt(D) long: it dominates every row."""
    qm = _f(q, dt).reshape(-1, D).mean(axis=0)
    return workloads._round_bits(qm / max(float(np.linalg.norm(qm)), 1e-6) * 3.0 * np.sqrt(D), dt)


@pytest.mark.parametrize("seed", range(16))
def test_random_decode_hard_scores(cuda, seed):
    """test_random_decode's layouts under the profiles of the hard prefill sweep below: jump
    (1 in 200 key rows x8), sink (each sequence's first key along the queries' mean
    direction), sharp (queries x4), bigv (values x1000; compared in units of that scale)."""
    from unifiedkv_amd.page16_native import page16_decode_attention

    rng = np.random.default_rng(7000 + seed)
    kind = PROFILES[seed % len(PROFILES)]
    dt, Hkv, n_rep, D, B, lens, bt, N = _decode_layout(rng, append=False)
    Hq = Hkv * n_rep
    q, k, v = _bits(rng, (B, Hq, D), dt), _bits(rng, (N, 16, Hkv, D), dt), _bits(rng, (N, 16, Hkv, D), dt)
    if kind == "jump":
        flat = k.reshape(-1, D)
        idx = rng.choice(flat.shape[0], size=max(1, flat.shape[0] // 200), replace=False)
        flat[idx] = _scaled(flat[idx], 8.0, dt)
    elif kind == "sink":
        row = _sink_row(q, dt, D)
        for b in range(B):
            if lens[b] > 0 and 0 <= bt[b, 0] < N:
                k[bt[b, 0], 0] = row
    elif kind == "sharp":
        q = _scaled(q, 4.0, dt)
    else:
        v = _scaled(v, 1000.0, dt)
    scale = 1.0 / math.sqrt(D)
    out = page16_decode_attention(_up(q, dt), _up(k, dt), _up(v, dt), _i32(bt), _i32(lens), softmax_scale=scale,
                                  n_rep=n_rep)
    want = oracle.page16_decode_dense(_f(q, dt), _f(k, dt), _f(v, dt), bt, lens, softmax_scale=scale, n_rep=n_rep)
    vscale = 1000.0 if kind == "bigv" else 1.0
    _check(out.float().cpu().numpy() / vscale, want / vscale, f"seed {seed} {kind} {dt} B={B} Hq={Hq} Hkv={Hkv} D={D}")


@pytest.mark.parametrize("seed", range(16))
def test_random_prefill_hard_scores(cuda, seed):
    """test_random_prefill's layouts at D = 128 (the tiled kernel) under harder score profiles,
    chunks long enough for several tiles and both block widths:
    jump  - 1 in 200 key rows x8: scores tens of log2 units above the rest at random keys, so
            the running max moves inside tiles, at any key of a tile;
    sink  - each sequence's first key along the queries' mean direction: it dominates;
    sharp - every query x4: peaked rows;
    bigv  - values x1000 (within fp16's range); the outputs are compared in units of that
            scale, since the weights' fp16 rounding (2^-11 each) bounds the error by
            2^-11 max|v|, and the north star's 2e-3 absolute bound is for unit-scale values."""
    from unifiedkv_amd import prefill

    rng = np.random.default_rng(5000 + seed)
    kind = PROFILES[seed % len(PROFILES)]
    dt = str(rng.choice(["bf16", "fp16"]))
    Hkv = int(rng.choice([1, 2, 4, 8]))
    n_rep = int(rng.choice([1, 2, 4, 8, 16]))
    D = 128
    B = int(rng.integers(1, 5))
    prefix = [int(x) for x in rng.integers(0, 900, size=B)]
    chunk = [int(x) for x in rng.integers(1, 400, size=B)]
    kv = [p + c for p, c in zip(prefix, chunk)]
    pages = [(L + 15) // 16 for L in kv]
    N = sum(pages) + 5
    perm = rng.permutation(N).astype(np.int32)
    lists = np.split(perm[: sum(pages)], np.cumsum(pages)[:-1])
    bt = workloads.tables_from_pages(lists)
    Hq, total = Hkv * n_rep, sum(chunk)
    k, v = _bits(rng, (N, 16, Hkv, D), dt), _bits(rng, (N, 16, Hkv, D), dt)
    q, kn, vn = _bits(rng, (total, Hq, D), dt), _bits(rng, (total, Hkv, D), dt), _bits(rng, (total, Hkv, D), dt)
    cu = np.concatenate([[0], np.cumsum(chunk)]).astype(np.int32)
    if kind == "jump":
        for arr in (k.reshape(-1, D), kn.reshape(-1, D)):
            idx = rng.choice(arr.shape[0], size=max(1, arr.shape[0] // 200), replace=False)
            arr[idx] = _scaled(arr[idx], 8.0, dt)
    elif kind == "sink":
        row = _sink_row(q, dt, D)
        for b in range(B):
            if prefix[b] > 0:
                k[bt[b][0], 0] = row
            else:
                kn[cu[b]] = row
    elif kind == "sharp":
        q = _scaled(q, 4.0, dt)
    else:
        v, vn = _scaled(v, 1000.0, dt), _scaled(vn, 1000.0, dt)
    kvl = np.array(kv, np.int32)
    scale = 1.0 / math.sqrt(D)
    kd, vd = _up(k, dt), _up(v, dt)
    out = prefill.chunked_prefill(_up(q, dt), _up(kn, dt), _up(vn, dt), kd, vd, _i32(bt), _i32(cu), _i32(kvl),
                                  softmax_scale=scale, n_rep=n_rep, max_chunk=max(chunk))
    for b in range(B):
        rows = slice(cu[b], cu[b + 1])
        prefill_oracle.write_chunk(k, bt[b], prefix[b], kn[rows])
        prefill_oracle.write_chunk(v, bt[b], prefix[b], vn[rows])
    what = f"seed {seed} {kind} {dt} Hq={Hq} Hkv={Hkv} prefix={prefix} chunk={chunk}"
    want = prefill_oracle.prefill_dense(_f(q, dt), _f(k, dt), _f(v, dt), bt, cu, kvl, softmax_scale=scale,
                                        n_rep=n_rep)
    got = out.float().cpu().numpy()
    assert np.all(np.isfinite(got)), what
    vscale = 1000.0 if kind == "bigv" else 1.0
    _check(got / vscale, want / vscale, what)


@pytest.mark.parametrize("seed", range(16))
def test_random_snapkv_scores_hard(cuda, seed):
    """test_random_snapkv_scores under the profiles jump (1 in 200 key rows x8), sink (the first
    key and the first middle key along the queries' mean direction) and sharp (queries x4)."""
    from unifiedkv_amd import snapkv

    rng = np.random.default_rng(6000 + seed)
    kind = PROFILES[seed % 3]
    dt = str(rng.choice(["bf16", "fp16"]))
    h_kv = int(rng.choice([1, 2, 4, 8]))
    n_rep = int(rng.choice([1, 2, 4, 8]))
    D = int(rng.choice([64, 128]))
    obs = int(rng.choice([16, 32, 48, 64, 128]))
    sink = int(rng.choice([0, 4, 16, 64]))
    L = int(rng.integers(sink + obs + 1, sink + obs + 2500))
    K, Q = _bits(rng, (h_kv, L, D), dt), _bits(rng, (h_kv * n_rep, obs, D), dt)
    if kind == "jump":
        flat = K.reshape(-1, D)
        idx = rng.choice(flat.shape[0], size=max(1, flat.shape[0] // 200), replace=False)
        flat[idx] = _scaled(flat[idx], 8.0, dt)
    elif kind == "sink":
        row = _sink_row(Q, dt, D)
        K[:, 0] = row
        K[:, sink] = row
    else:
        Q = _scaled(Q, 4.0, dt)
    got = snapkv.score_layer_blocks(_up(K, dt), _up(Q, dt), sink_len=sink, obs_len=obs, n_rep=n_rep).cpu().numpy()
    want = so.score_layer_blocks(_f(K, dt), _f(Q, dt), sink_len=sink, obs_len=obs, n_rep=n_rep)
    what = f"seed {seed} {kind} {dt} h_kv={h_kv} n_rep={n_rep} D={D} L={L} sink={sink} obs={obs}"
    assert got.shape == want.shape, what
    if want.size:
        err = np.abs(got - want)
        bound = 1e-4 * np.abs(want).max() + 1e-3 * np.abs(want)
        assert np.all(err <= bound), f"{what}: max err {err.max():.3e}"
