"""Seeded random-shape sweep of the integer and copy kernels, bit-exact against the oracle.

* Retain-set top-k (a6): rows of random length and k, optional ragged per-row n and k,
  scores mixing uniform values, heavy ties, +0 / -0, +-inf, NaN of both signs and other
  payloads, subnormals and +-FLT_MAX, against compaction_oracle.select_topk (score
  descending, lower index on ties, -0 equal to +0, every NaN above every number).
* Token scatter / gather (a5): random head count, head dim, token count and page ids,
  token-major dense views, against pool_oracle.write_kv_to_blocks / read_kv_from_blocks.
* Page copy (a7/a8): random layer counts, one or two pools, shared or per-layer source and
  destination ids; every byte of the destination pools compared.
"""
import numpy as np
import pytest

from oracle import compaction_oracle as co
from oracle import pool_oracle

pytestmark = pytest.mark.gpu

SPECIALS = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, -np.nan, 1e-45, -1e-45, 1e-40, 3.4028235e38,
                     -3.4028235e38, 0.5, -0.5], dtype=np.float32)


def _scores(rng, rows, n):
    s = rng.random((rows, n), dtype=np.float32)
    mode = rng.integers(0, 4)
    if mode == 1:
        s = np.round(s * 8) / 8  # heavy ties
    elif mode == 2:
        s = rng.choice(SPECIALS, size=(rows, n))  # mostly special values
    mask = rng.random((rows, n)) < 0.05
    s[mask] = rng.choice(SPECIALS, size=int(mask.sum()))
    bits = s.view(np.uint32)
    nan_mask = rng.random((rows, n)) < 0.01  # NaN with other payloads and signs
    bits[nan_mask] = rng.choice(np.array([0x7F800001, 0xFFC00000, 0x7FFFFFFF, 0xFF800123], dtype=np.uint32),
                                size=int(nan_mask.sum()))
    return bits.view(np.float32)


@pytest.mark.parametrize("seed", range(20))
def test_random_select(cuda, seed):
    import torch

    from unifiedkv_amd import compaction

    rng = np.random.default_rng(5000 + seed)
    rows = int(rng.integers(1, 20))
    n = int(rng.integers(1, 3000))
    k = int(rng.integers(0, n + 1))
    s = _scores(rng, rows, n)
    what = f"seed {seed} rows={rows} n={n} k={k}"
    if rng.random() < 0.5:
        got = compaction.select_blocks(torch.from_numpy(s).to(cuda), k).cpu().numpy()
        np.testing.assert_array_equal(got, co.select_topk(s, k), err_msg=what)
        return
    n_valid = rng.integers(0, n + 1, size=rows).astype(np.int32)
    k_row = rng.integers(0, n + 1, size=rows).astype(np.int32)
    kmax = max(1, k)
    got = compaction.select_blocks(torch.from_numpy(s).to(cuda), kmax, torch.from_numpy(n_valid),
                                   torch.from_numpy(k_row)).cpu().numpy()
    for r in range(rows):
        kk = min(int(k_row[r]), int(n_valid[r]), kmax)
        exp = co.select_topk(s[r:r + 1, : n_valid[r]], kk)[0] if kk > 0 else np.zeros(0, np.int32)
        np.testing.assert_array_equal(got[r, :kk], exp, err_msg=f"{what} row {r}")
        assert (got[r, kk:] == -1).all(), f"{what} row {r}: padding"


def test_select_signed_zeros_tie_to_the_lower_index(cuda):
    import torch

    from unifiedkv_amd import compaction

    s = np.array([[-0.0, 0.0, -1.0, 0.0], [0.0, -0.0, -0.0, 1.0], [-2.0, -0.0, -0.0, 0.0]], dtype=np.float32)
    got = compaction.select_blocks(torch.from_numpy(s).to(cuda), 2).cpu().numpy()
    np.testing.assert_array_equal(got, [[0, 1], [0, 3], [1, 2]])
    np.testing.assert_array_equal(got, co.select_topk(s, 2))


def _rand16(rng, shape):
    return rng.integers(0, 1 << 16, size=shape, dtype=np.uint16)


def _dev(a, cuda):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(cuda).view(torch.bfloat16)


def _host(t):
    import torch

    return t.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("seed", range(12))
def test_random_token_io(cuda, seed):
    from unifiedkv_amd import page_ops

    rng = np.random.default_rng(6000 + seed)
    H = int(rng.choice([1, 2, 3, 8]))
    D = int(rng.choice([16, 64, 96, 128, 256]))
    T = int(rng.integers(1, 700))
    n_ids = (T + 15) // 16 + int(rng.integers(0, 3))  # ids beyond the data are ignored
    N = n_ids + int(rng.integers(0, 30))
    ids = rng.permutation(N)[:n_ids].astype(np.int32)
    pool = _rand16(rng, (N, 16, H, D))
    dense = _rand16(rng, (T, H, D))  # token-major buffer; the kernels see its [H, T, D] view
    what = f"seed {seed} H={H} D={D} T={T} N={N}"
    pool_d = _dev(pool, cuda)
    page_ops.scatter_tokens(pool_d, ids, _dev(dense, cuda).transpose(0, 1))
    exp = pool.copy()
    pool_oracle.write_kv_to_blocks(exp, ids, dense.transpose(1, 0, 2))
    np.testing.assert_array_equal(_host(pool_d), exp, err_msg=what)
    for n_tok in (T, int(rng.integers(0, T + 1)), 16 * n_ids + 3):
        got = page_ops.gather_tokens(pool_d, ids, n_tok)
        np.testing.assert_array_equal(_host(got), pool_oracle.read_kv_from_blocks(exp, ids, n_tok),
                                      err_msg=f"{what} gather {n_tok}")


@pytest.mark.parametrize("seed", range(12))
def test_random_page_copy(cuda, seed):
    from unifiedkv_amd import page_ops

    rng = np.random.default_rng(7000 + seed)
    L = int(rng.integers(1, 6))
    H, D = int(rng.choice([1, 4, 8])), int(rng.choice([64, 128]))
    n = int(rng.integers(1, 40))
    N = 2 * n + int(rng.integers(0, 20))
    two = bool(rng.random() < 0.5)
    pools = [_rand16(rng, (L, N, 16, H, D)) for _ in range(2 if two else 1)]
    half = rng.permutation(N)
    src_pages, dst_pages = half[:n], half[n:2 * n]  # disjoint sources and destinations
    per_layer_src, per_layer_dst = bool(rng.random() < 0.5), bool(rng.random() < 0.5)
    src = np.stack([rng.permutation(src_pages) for _ in range(L)]) if per_layer_src else src_pages
    dst = np.stack([rng.permutation(dst_pages) for _ in range(L)]) if per_layer_dst else dst_pages
    src, dst = src.astype(np.int32), dst.astype(np.int32)
    dev = [_dev(p, cuda) for p in pools]
    import torch

    page_ops.page_copy(dev, dev, torch.from_numpy(src), torch.from_numpy(dst))
    what = f"seed {seed} L={L} H={H} D={D} n={n} N={N} two={two} per_layer={per_layer_src, per_layer_dst}"
    for p, d in zip(pools, dev):
        exp = p.copy()
        for l in range(L):
            exp[l, dst[l] if per_layer_dst else dst] = p[l, src[l] if per_layer_src else src]
        np.testing.assert_array_equal(_host(d), exp, err_msg=what)
