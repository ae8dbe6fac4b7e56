"""SnapKV's softmax normalisers taken during the prefill, and the scores that start from them.

The reference captures the observation window's queries in its q_proj hook during the prefill
(core/scheduler.py:269-341) and, at selection time, normalises their softmax over the middle
keys K_mid (core/scheduler.py:565-592). ``ukv_paged_prefill_obs_stats`` takes that
normaliser (log2 sum_j 2^(s_j * scale * log2 e) over the zero-padded K_mid) while the prefill
kernel streams the keys, and ``ukv_snapkv_scores_from_stats`` skips its own pass over the keys.

Checked here:
* the oracle's normaliser (snapkv_oracle.obs_row_stats) against scipy's logsumexp, against
  the closed form for all-zero keys (log2 of the padded key count) and against the oracle's
  own scores (weights 2^(s - lse) sum to 1 per row, and rebuild score_layer_blocks);
* on the GPU, the prefill's rows against that oracle (fp64) within LSE_TOL in log2 units
  (the prefill's denominators sum fp16-rounded weights, less the sink and window keys' weights
  rounded the same way), its attention output
  against the plain prefill's, the scores from these rows against the two-pass scores
  (within the two-pass first pass's own rounding: each weight enters its sum as fp16,
  2^-11 relative) and against the fp64 oracle with the bound the other score tests use;
* rows the kernels flag (a sum that underflowed because the sink dominates, a window that
  holds most of the weight) and rows that are flagged or non-finite in the given statistics: those items are recomputed by the
  first pass and then equal the two-pass scores bit for bit;
* the host-side refusals (chunk shorter than the window, a layer not written, another
  length or softmax scale);
* seeded random shapes through the whole path (dtype, n_rep 1-8, sink, windows of 16-128 queries
  including one not a multiple of 16, each sequence's own chunk split, sequences too short to
  score), with the checks above.
"""
import math

import numpy as np
import pytest

from oracle import oracle
from oracle import snapkv_oracle as so
from unifiedkv_amd import workloads

# log2 units. The prefill's softmax denominators sum the weights rounded to fp16 (each within
# 2^-11 relative, of random sign, as in the two-pass scorer's first pass); the middle keys' sum is
# that less the sink and window keys' weights, rounded the same way, which cancel where the
# running max did not move after them. A row of a few dominant keys can carry the full 2^-11
# (7.0e-4 in log2 units); a row whose sink and window hold half its weight or more is flagged.
LSE_TOL = 7.1e-4


def _middle_share(K, Q, *, sink, obs, n_rep, scale):
    """K [H_kv, L, D], Q [H_q, obs, D] (the window's queries, at positions L - obs ..) -> float64
    [H_q, obs]: the share of each query's softmax weight, over every key it sees, that falls on
    the middle keys [sink, L - obs)."""
    K = np.asarray(K, np.float64)
    Q = np.asarray(Q, np.float64)
    L = K.shape[1]
    S = np.matmul(Q, np.repeat(K, n_rep, axis=0).transpose(0, 2, 1)) * scale  # [H_q, obs, L]
    seen = np.arange(L)[None, :] <= (L - obs + np.arange(obs))[:, None]
    S = np.where(seen[None], S, -np.inf)
    w = np.exp(S - S.max(axis=-1, keepdims=True))
    return w[..., sink:max(sink, L - obs)].sum(axis=-1) / w.sum(axis=-1)


def _rand(rng, shape):
    return rng.standard_normal(shape)


def test_oracle_normaliser_matches_scipy_logsumexp():
    from scipy.special import logsumexp

    rng = np.random.default_rng(3)
    Hkv, n_rep, L, D, sink, obs = 2, 3, 203, 32, 5, 24
    K, Q = _rand(rng, (Hkv, L, D)), _rand(rng, (Hkv * n_rep, obs, D))
    scale = 0.37
    got = so.obs_row_stats(K, Q, sink_len=sink, obs_len=obs, n_rep=n_rep, scale=scale)
    L_mid = L - sink - obs
    aligned = -(-L_mid // 16) * 16
    for h in range(Hkv * n_rep):
        Km = np.concatenate([K[h // n_rep, sink:L - obs], np.zeros((aligned - L_mid, D))])
        want = logsumexp(Q[h] @ Km.T * scale, axis=-1) / math.log(2.0)
        np.testing.assert_allclose(got[h], want, rtol=0, atol=1e-12)


def test_oracle_normaliser_of_zero_keys_is_log2_of_the_padded_count():
    K = np.zeros((1, 101, 8))
    Q = np.ones((2, 16, 8))
    got = so.obs_row_stats(K, Q, sink_len=4, obs_len=16, n_rep=2)
    np.testing.assert_allclose(got, math.log2(96), rtol=1e-15)  # 81 middle keys padded to 96, scores 0


def test_oracle_normaliser_rebuilds_the_oracle_scores():
    rng = np.random.default_rng(4)
    Hkv, n_rep, L, D, sink, obs = 2, 2, 330, 16, 16, 32
    K, Q = _rand(rng, (Hkv, L, D)), _rand(rng, (Hkv * n_rep, obs, D))
    lse = so.obs_row_stats(K, Q, sink_len=sink, obs_len=obs, n_rep=n_rep)
    K_mid, N = so.mid_keys(K, sink, obs, 16)
    S = Q @ so.repeat_kv(K_mid, n_rep).transpose(0, 2, 1) * (D ** -0.5) / math.log(2.0)
    A = np.exp2(S - lse[..., None])
    np.testing.assert_allclose(A.sum(-1), 1.0, rtol=0, atol=1e-12)
    blocks = A.mean(axis=1).max(axis=0).reshape(N, 16).sum(-1)
    want = so.score_layer_blocks(K, Q, sink_len=sink, obs_len=obs, n_rep=n_rep)
    np.testing.assert_allclose(so.maxpool3(blocks), want, rtol=1e-12, atol=0)


def test_obs_stats_host_checks():
    import torch

    from unifiedkv_amd import snapkv
    from unifiedkv_amd.prefill import paged_prefill_attention

    st = snapkv.ObsStats(2, 3, 8, sink_len=4, obs_len=32, softmax_scale=0.125, device="meta")
    assert st.layer_view(2)[1] == 3 * 8 * 32
    with pytest.raises(IndexError):
        st.layer_view(3)
    meta = torch.device("meta")
    q = torch.empty((100, 8, 128), dtype=torch.bfloat16, device=meta)
    kc = torch.empty((40, 16, 2, 128), dtype=torch.bfloat16, device=meta)
    bt = torch.empty((2, 10), dtype=torch.int32, device=meta)
    call = dict(softmax_scale=0.125, n_rep=4, obs_stats=st, layer_id=0)
    with pytest.raises(RuntimeError, match="obs_window_spans_chunks"):
        paged_prefill_attention(q, kc, kc, bt, [0, 80, 100], [150, 120], **call)
    with pytest.raises(RuntimeError, match="obs_stats_scale"):
        paged_prefill_attention(q, kc, kc, bt, [0, 50, 100], [150, 120], **dict(call, softmax_scale=0.1))
    with pytest.raises(ValueError, match="needs layer_id"):
        paged_prefill_attention(q, kc, kc, bt, [0, 50, 100], [150, 120], **dict(call, layer_id=None))
    with pytest.raises(RuntimeError, match="paged_prefill_unavailable:device"):
        paged_prefill_attention(q, kc, kc, bt, [0, 50, 100], [150, 120], **call)
    # score side: every layer written at the scored length, same window and scale
    check = dict(seqs=2, layers=3, h_q=8, seq_len=150, sink_len=4, obs_len=32, scale=0.125, dev=meta)
    with pytest.raises(RuntimeError, match="layer_missing"):
        snapkv._check_obs_stats(st, **check)
    for layer in range(3):
        st.mark(layer, [150, 150])
    assert snapkv._check_obs_stats(st, **check) is st.data
    with pytest.raises(RuntimeError, match="seq_len"):
        snapkv._check_obs_stats(st, **dict(check, seq_len=151))
    with pytest.raises(RuntimeError, match="softmax_scale"):
        snapkv._check_obs_stats(st, **dict(check, scale=0.1))
    with pytest.raises(RuntimeError, match="bad_score_shape:obs_stats"):
        snapkv._check_obs_stats(st, **dict(check, obs_len=16))


# --------------------------------------------------------------------------- GPU


def _bits(rng, shape, dtype):
    return workloads._round_bits(rng.standard_normal(shape, dtype=np.float32), dtype)


def _dev(bits, dtype):
    import torch

    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to("cuda").view(tdt)


def _f(bits, dtype):
    return oracle.bits_to_f32(bits, workloads.DTYPE_CODES[dtype])


def _prefill(cuda, dtype, chunks, *, Hq, Hkv, layers, sink, obs, seed, q_fill=None, k_sink_fill=None,
             k_window_fill=None):
    """Chunked prefill through PrefillPages, the final chunk with ObsStats; returns what the
    checks need: pool, pages, statistics, the final chunk's outputs with and without them,
    the window's queries and the dense keys."""
    import torch

    from unifiedkv_amd import snapkv
    from unifiedkv_amd.pool import PagedKVPool
    from unifiedkv_amd.prefill import PrefillPages, paged_prefill_attention

    rng = np.random.default_rng(seed)
    D = 128
    n_rep = Hq // Hkv
    scale = 1.0 / math.sqrt(D)
    B = len(chunks[0])
    total_len = [sum(c[b] for c in chunks) for b in range(B)]
    pool = PagedKVPool(16, layers, Hkv, D, torch.bfloat16 if dtype == "bf16" else torch.float16,
                       num_blocks=sum(-(-n // 16) for n in total_len) + 8, device=cuda)
    pool.allocate_blocks(3)                      # pages of the prefill do not start at 0
    pp = PrefillPages(pool, B)
    st = snapkv.ObsStats(B, layers, Hq, sink_len=sink, obs_len=obs, softmax_scale=scale, device=cuda)
    q_obs = np.zeros((B, layers, Hq, obs, D), np.uint16)
    outs = {}
    for ci, cl in enumerate(chunks):
        last = ci == len(chunks) - 1
        pp.begin_chunk(cl)
        total = sum(cl)
        cu = np.concatenate([[0], np.cumsum(cl)]).astype(np.int64)
        for layer in range(layers):
            q, k, v = (_bits(rng, (total, Hq, D), dtype), _bits(rng, (total, Hkv, D), dtype),
                       _bits(rng, (total, Hkv, D), dtype))
            if q_fill is not None:
                q[:] = workloads._round_bits(np.full(q.shape, q_fill, np.float32), dtype)
            if k_sink_fill is not None and ci == 0:
                k[cu[:-1]] = workloads._round_bits(np.full((B, Hkv, D), k_sink_fill, np.float32), dtype)
            if k_window_fill is not None and last:
                for b in range(B):
                    k[cu[b + 1] - obs:cu[b + 1]] = workloads._round_bits(
                        np.full((obs, Hkv, D), k_window_fill, np.float32), dtype)
            if last:
                out = pp.attention(layer, _dev(q, dtype), _dev(k, dtype), _dev(v, dtype), softmax_scale=scale,
                                   n_rep=n_rep, obs_stats=st)
                c = pp._chunk
                plain = paged_prefill_attention(_dev(q, dtype), pool.k_cache[layer], pool.v_cache[layer], c["bt"],
                                                c["cu"], c["kv"], softmax_scale=scale, n_rep=n_rep,
                                                max_chunk=c["max_chunk"])
                outs[layer] = (out.float().cpu().numpy(), plain.float().cpu().numpy())
                for b in range(B):
                    q_obs[b, layer] = q[cu[b + 1] - obs:cu[b + 1]].transpose(1, 0, 2)
            else:
                pp.attention(layer, _dev(q, dtype), _dev(k, dtype), _dev(v, dtype), softmax_scale=scale,
                             n_rep=n_rep)
        pp.end_chunk()
    torch.cuda.synchronize()
    dense = []
    for layer in range(layers):
        kc = pool.k_cache[layer].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
        dense.append([kc[np.asarray(pp.page_lists[b])].reshape(-1, Hkv, D)[:total_len[b]].transpose(1, 0, 2)
                      for b in range(B)])
    return dict(pool=pool, pp=pp, st=st, outs=outs, q_obs=q_obs, dense=dense, scale=scale, n_rep=n_rep,
                lens=total_len, D=D)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype, Hq, Hkv, sink, obs, chunks", [
    ("bf16", 16, 4, 4, 32, [[700, 650], [400, 517]]),
    ("fp16", 16, 2, 64, 128, [[900, 300], [300, 901]]),
    ("bf16", 8, 8, 0, 48, [[1000, 500], [300, 48]]),  # n_rep 1, obs not a multiple of 16, no sink,
                                                      # a final chunk of exactly the window
    ("bf16", 32, 8, 16, 128, [[300, 2000]]),          # one chunk each
    ("bf16", 32, 8, 64, 128, [[1280] * 8]),           # 8 x 8 groups: 96- and 64-query blocks
    ("bf16", 8, 8, 16, 64, [[1536] * 8]),             # n_rep 1: 384- and 256-query blocks
    ("fp16", 32, 4, 32, 64, [[512] * 8]),             # n_rep 8: 48- and 32-query blocks
    # n_rep 16: windows that span blocks of both widths (three-column ones, then two-column ones)
    ("bf16", 128, 8, 16, 64, [[128] * 14]),
    ("fp16", 128, 8, 0, 32, [[96] * 13]),
    # a final chunk of exactly the window's 128 queries
    ("bf16", 32, 8, 16, 128, [[1000, 800], [128, 128]]),
])
def test_prefill_rows_match_oracle_and_outputs_match_plain_prefill(cuda, dtype, Hq, Hkv, sink, obs, chunks):
    layers = 2
    r = _prefill(cuda, dtype, chunks, Hq=Hq, Hkv=Hkv, layers=layers, sink=sink, obs=obs, seed=7)
    data = r["st"].data.cpu().numpy()
    worst = 0.0
    for layer in range(layers):
        out, plain = r["outs"][layer]
        ok, err, exc = oracle.allclose_report(out, plain, 2e-3, 1e-2)
        assert ok, f"layer {layer}: output differs from the plain prefill by {err:.3e}"
        for b in range(len(chunks[0])):
            want = so.obs_row_stats(_f(r["dense"][layer][b], dtype), _f(r["q_obs"][b, layer], dtype), sink_len=sink,
                                    obs_len=obs, n_rep=r["n_rep"], scale=r["scale"])
            got, flags = data[b, layer, :, :, 0], data[b, layer, :, :, 1]
            # rows whose sink and window keys hold half of the weight or more are flagged (the
            # middle sum would be a difference of nearby values); the rest carry their sum
            share = _middle_share(_f(r["dense"][layer][b], dtype), _f(r["q_obs"][b, layer], dtype), sink=sink,
                                  obs=obs, n_rep=r["n_rep"], scale=r["scale"])
            assert np.all(flags[share > 0.55] == 0), f"layer {layer} seq {b}: a row of middle share > 0.55 flagged"
            assert np.all(flags[share < 0.45] == 1), f"layer {layer} seq {b}: a row of middle share < 0.45 kept"
            if not np.any(flags == 0):
                continue
            err = np.abs(got - want)[flags == 0].max()
            worst = max(worst, err)
            assert err <= LSE_TOL, f"layer {layer} seq {b}: normaliser off by {err:.3e} (log2 units)"
    print(f"max |lse - oracle| = {worst:.3e}")


def _scores(r, *, sink, obs, stats):
    import torch

    from unifiedkv_amd import snapkv

    pp = r["pp"]
    width = max(len(x) for x in pp.page_lists)
    table = torch.tensor([x + [0] * (width - len(x)) for x in pp.page_lists], dtype=torch.int32, device="cuda")
    q_obs = r["q_dev"]
    return snapkv.score_blocks(q_obs, r["pool"].k_cache, table, seq_len=r["lens"][0], sink_len=sink, obs_len=obs,
                               n_rep=r["n_rep"], obs_stats=r["st"] if stats else None)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_scores_from_prefill_rows_match_two_pass_and_oracle(cuda, dtype):
    sink, obs, layers = 16, 64, 3
    r = _prefill(cuda, dtype, [[1500, 1500], [613, 613]], Hq=16, Hkv=4, layers=layers, sink=sink, obs=obs, seed=11)
    r["q_dev"] = _dev(r["q_obs"], dtype)
    one = _scores(r, sink=sink, obs=obs, stats=True).cpu().numpy()
    two = _scores(r, sink=sink, obs=obs, stats=False).cpu().numpy()
    # the first pass's weights enter its normaliser as fp16 (2^-11 relative each), and the
    # second pass rounds its weights to fp16 under either normaliser
    np.testing.assert_allclose(one, two, rtol=2.0 ** -9, atol=1e-7)
    for b in range(2):
        for layer in range(layers):
            want = so.score_layer_blocks(_f(r["dense"][layer][b], dtype), _f(r["q_obs"][b, layer], dtype),
                                         sink_len=sink, obs_len=obs, n_rep=r["n_rep"])
            got = one[b * layers + layer]
            err = np.abs(got - want)
            assert np.all(err <= 1e-4 * np.abs(want).max() + 1e-3 * np.abs(want)), (b, layer, err.max())


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(12))
def test_random_shapes_through_the_statistics_path(cuda, seed):
    """Seeded random shapes: dtype, head layout (n_rep 1-8), sink, window (including one that
    is not a multiple of 16), batch and each sequence's own chunk split (empty earlier chunks,
    a final chunk from exactly the window up to the whole sequence). The final chunk's outputs
    equal the plain prefill's, kept rows match the fp64 normalisers, and the scores from the
    rows match the two-pass scores and the fp64 oracle."""
    rng = np.random.default_rng(90000 + seed)
    dtype = ("bf16", "fp16")[int(rng.integers(2))]
    Hkv = int(rng.choice([1, 2, 4, 8]))
    n_rep = int(rng.choice([1, 2, 4, 8]))
    obs = int(rng.choice([16, 24, 32, 48, 64, 128]))
    sink = int(rng.choice([0, 4, 16, 64]))
    B = int(rng.integers(1, 4))
    total = int(rng.integers(sink + obs + 1, 2600))  # at least one middle key
    n_chunks = int(rng.integers(1, 4))
    per_seq = []
    for _ in range(B):
        # n_chunks - 1 earlier chunks (some possibly empty) split what the final chunk leaves
        final = int(rng.integers(obs, total + 1)) if n_chunks > 1 else total
        cuts = np.sort(rng.integers(0, total - final + 1, size=max(0, n_chunks - 2)))
        parts = np.diff(np.concatenate([[0], cuts, [total - final]])).tolist() if n_chunks > 1 else []
        per_seq.append(parts + [final])
    chunks = [[per_seq[b][i] for b in range(B)] for i in range(n_chunks)]
    chunks = [c for c in chunks[:-1] if sum(c) > 0] + [chunks[-1]]
    layers = 2
    r = _prefill(cuda, dtype, chunks, Hq=Hkv * n_rep, Hkv=Hkv, layers=layers, sink=sink, obs=obs, seed=seed)
    what = f"seed {seed}: {dtype} Hkv {Hkv} n_rep {n_rep} sink {sink} obs {obs} chunks {chunks}"
    data = r["st"].data.cpu().numpy()
    for layer in range(layers):
        out, plain = r["outs"][layer]
        ok, err, _ = oracle.allclose_report(out, plain, 2e-3, 1e-2)
        assert ok, f"{what}: layer {layer} output differs from the plain prefill by {err:.3e}"
        for b in range(B):
            want = so.obs_row_stats(_f(r["dense"][layer][b], dtype), _f(r["q_obs"][b, layer], dtype), sink_len=sink,
                                    obs_len=obs, n_rep=n_rep, scale=r["scale"])
            got, flags = data[b, layer, :, :, 0], data[b, layer, :, :, 1]
            # (a sequence shorter than sink + window + one block has no middle blocks to score)
            if want.size and np.any(flags == 0):
                err = np.abs(got - want)[flags == 0].max()
                assert err <= LSE_TOL, f"{what}: layer {layer} seq {b} normaliser off by {err:.3e}"
    r["q_dev"] = _dev(r["q_obs"], dtype)
    one = _scores(r, sink=sink, obs=obs, stats=True).cpu().numpy()
    two = _scores(r, sink=sink, obs=obs, stats=False).cpu().numpy()
    if total < sink + obs + 16:
        assert one.shape == (B * layers, 0) and two.shape == (B * layers, 0), what
    np.testing.assert_allclose(one, two, rtol=2.0 ** -9, atol=1e-7, err_msg=what)
    for b in range(B):
        for layer in range(layers):
            want = so.score_layer_blocks(_f(r["dense"][layer][b], dtype), _f(r["q_obs"][b, layer], dtype),
                                         sink_len=sink, obs_len=obs, n_rep=n_rep)
            assert want.shape == one[b * layers + layer].shape, what
            if want.size:
                err = np.abs(one[b * layers + layer] - want)
                assert np.all(err <= 1e-4 * np.abs(want).max() + 1e-3 * np.abs(want)), (what, b, layer, err.max())


def _statistics_case(cuda):
    """A final chunk with statistics: the prefill kernel, which leaves the rows' (max, denominator)
    pairs, and the kernel that turns them into the rows, on the caller's stream."""
    import torch

    from unifiedkv_amd import snapkv
    from unifiedkv_amd.prefill import paged_prefill_attention

    B, P, C, Hq, Hkv, D, sink, obs = 4, 1500, 700, 32, 8, 128, 16, 128
    g = torch.Generator(device=cuda)
    g.manual_seed(5)
    per = -(-(P + C) // 16)
    N = B * per + 8
    bt = torch.randperm(N, generator=g, device=cuda)[:B * per].view(B, per).to(torch.int32)
    mk = lambda *shape: torch.randn(shape, generator=g, device=cuda).to(torch.bfloat16)  # noqa: E731
    kc, vc = mk(N, 16, Hkv, D), mk(N, 16, Hkv, D)
    qs = [mk(B * C, Hq, D) for _ in range(4)]
    cu = torch.arange(0, B * C + 1, C, dtype=torch.int32, device=cuda)
    lens = torch.full((B,), P + C, dtype=torch.int32, device=cuda)
    stats = lambda: snapkv.ObsStats(B, 1, Hq, sink_len=sink, obs_len=obs, softmax_scale=D ** -0.5,  # noqa: E731
                                    device=cuda)

    def call(q, st):
        return paged_prefill_attention(q, kc, vc, bt, cu, lens, softmax_scale=D ** -0.5, n_rep=Hq // Hkv,
                                       max_chunk=C, obs_stats=st, layer_id=0, host_lens=([C] * B, [P + C] * B))
    return qs, stats, call


@pytest.mark.gpu
def test_prefill_with_statistics_replays_from_a_captured_graph(cuda):
    """A captured graph holds both launches, and each replay (new queries copied in, eager calls
    and synchronisations between replays) equals the eager call bit for bit."""
    import torch

    qs, stats, call = _statistics_case(cuda)
    st_g, st_e = stats(), stats()
    q = qs[0].clone()
    call(q, st_g)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_g = call(q, st_g)
    for i in (1, 2, 3):
        q.copy_(qs[i])
        graph.replay()
        torch.cuda.synchronize()
        want = call(qs[i], st_e)
        torch.cuda.synchronize()
        assert torch.equal(out_g, want), f"replay {i}: attention output"
        assert torch.equal(st_g.data, st_e.data), f"replay {i}: statistics"


@pytest.mark.gpu
def test_prefill_with_statistics_orders_the_callers_stream(cuda):
    """On a caller's own stream, work queued after the call sees both kernels' results."""
    import torch

    qs, stats, call = _statistics_case(cuda)
    st_e, st_s = stats(), stats()
    want = call(qs[1], st_e)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        st_s.data.fill_(float("nan"))
        out = call(qs[1], st_s)
        got_out, got_st = out.clone(), st_s.data.clone()  # queued right behind the call
    s.synchronize()
    assert torch.equal(got_out, want)
    assert torch.equal(got_st, st_e.data)


@pytest.mark.gpu
def test_flagged_or_non_finite_rows_make_the_first_pass_redo_their_items(cuda):
    sink, obs, layers = 4, 32, 2
    r = _prefill(cuda, "bf16", [[800, 800], [300, 300]], Hq=16, Hkv=4, layers=layers, sink=sink, obs=obs, seed=5)
    r["q_dev"] = _dev(r["q_obs"], "bf16")
    clean = _scores(r, sink=sink, obs=obs, stats=True).cpu().numpy()
    two = _scores(r, sink=sink, obs=obs, stats=False).cpu().numpy()
    data = r["st"].data
    data[1, 0, 3, 5, 0] = 1e30                    # a wrong value, flagged: item (seq 1, layer 0)
    data[1, 0, 3, 5, 1] = 1.0
    data[0, 1, 0, 0, 0] = float("nan")            # non-finite, unflagged: item (seq 0, layer 1)
    got = _scores(r, sink=sink, obs=obs, stats=True).cpu().numpy()
    redone = [1 * layers + 0, 0 * layers + 1]
    for item in range(2 * layers):
        want = two[item] if item in redone else clean[item]
        assert np.array_equal(got[item], want), item


@pytest.mark.gpu
def test_a_dominant_sink_flags_the_rows_and_the_scores_stay_exact(cuda):
    # every query is (1, ..., 1) and the first key of each sequence is (16, ..., 16): its score
    # 2048 / sqrt(128) = 181 sits 261 log2 units above the middle keys', whose weights under
    # that max underflow fp32 - the kernel flags every window row, and the scores recompute them
    sink, obs, layers = 4, 32, 1
    r = _prefill(cuda, "bf16", [[600, 600]], Hq=8, Hkv=2, layers=layers, sink=sink, obs=obs, seed=9, q_fill=1.0,
                 k_sink_fill=16.0)
    flags = r["st"].data[..., 1].cpu().numpy()
    assert np.all(flags == 1.0)
    r["q_dev"] = _dev(r["q_obs"], "bf16")
    one = _scores(r, sink=sink, obs=obs, stats=True).cpu().numpy()
    two = _scores(r, sink=sink, obs=obs, stats=False).cpu().numpy()
    assert np.array_equal(one, two)


@pytest.mark.gpu
def test_a_dominant_window_flags_the_rows_and_the_scores_stay_exact(cuda):
    # every query is (1, ..., 1) and the window's keys are (2, ..., 2): their scores (256 / sqrt(128)
    # = 22.6) hold nearly all of each row's weight, so the middle sum would be the small difference
    # of two large ones - the rows are flagged (not underflowed: the middle weights stay far above
    # 2^-100 of the max) and the scores recompute them
    sink, obs, layers = 4, 32, 1
    r = _prefill(cuda, "bf16", [[600, 600]], Hq=8, Hkv=2, layers=layers, sink=sink, obs=obs, seed=13, q_fill=1.0,
                 k_window_fill=2.0)
    flags = r["st"].data[..., 1].cpu().numpy()
    assert np.all(flags == 1.0)
    r["q_dev"] = _dev(r["q_obs"], "bf16")
    one = _scores(r, sink=sink, obs=obs, stats=True).cpu().numpy()
    two = _scores(r, sink=sink, obs=obs, stats=False).cpu().numpy()
    assert np.array_equal(one, two)


@pytest.mark.gpu
def test_scores_from_prefill_rows_on_the_scalar_scoring_path(cuda):
    # obs_len 40 is not a multiple of 16: the scores run the scalar kernel pair, which takes the
    # imported rows the same way (and recomputes a flagged item's rows from the keys)
    sink, obs, layers = 5, 40, 2
    r = _prefill(cuda, "bf16", [[300, 300], [200, 200]], Hq=8, Hkv=2, layers=layers, sink=sink, obs=obs, seed=21)
    r["q_dev"] = _dev(r["q_obs"], "bf16")
    one = _scores(r, sink=sink, obs=obs, stats=True).cpu().numpy()
    two = _scores(r, sink=sink, obs=obs, stats=False).cpu().numpy()
    np.testing.assert_allclose(one, two, rtol=1e-5, atol=1e-8)   # both sides sum fp32 weights here
    for b in range(2):
        for layer in range(layers):
            want = so.score_layer_blocks(_f(r["dense"][layer][b], "bf16"), _f(r["q_obs"][b, layer], "bf16"),
                                         sink_len=sink, obs_len=obs, n_rep=r["n_rep"])
            err = np.abs(one[b * layers + layer] - want)
            assert np.all(err <= 1e-4 * np.abs(want).max() + 1e-3 * np.abs(want)), (b, layer, err.max())
    r["st"].data[0, 1, 2, 7, 1] = 1.0                          # flag one row of item (seq 0, layer 1)
    r["st"].data[0, 1, 2, 7, 0] = -1e30
    got = _scores(r, sink=sink, obs=obs, stats=True).cpu().numpy()
    for item in range(2 * layers):
        assert np.array_equal(got[item], two[item] if item == 1 else one[item]), item


def test_c_entry_points_refuse_bad_statistics_arguments_before_any_launch():
    # every refusal below returns before the library touches a device
    from unifiedkv_amd import _ext

    lib = _ext.load()
    i64 = _ext.i64_array
    q_st, kv_st = i64((32 * 128, 128)), i64((16 * 8 * 128, 8 * 128, 128))

    def prefill_stats(sink, obs, stats, stride):
        return lib.ukv_paged_prefill_obs_stats(None, None, None, None, None, None, None, 2, 64, 32, 32, 8, 128, 4,
                                               4, 16, q_st, kv_st, kv_st, 0.088, _ext.UKV_DTYPE_BF16, sink, obs,
                                               stats, stride, None)

    assert prefill_stats(4, 16, None, 32 * 16) == _ext.UKV_ERR_INVALID_ARGUMENT        # no buffer
    assert prefill_stats(4, 16, 0x1004, 32 * 16) == _ext.UKV_ERR_INVALID_ARGUMENT      # not 8-byte aligned
    assert prefill_stats(4, 16, 0x1000, 32 * 16 - 1) == _ext.UKV_ERR_INVALID_ARGUMENT  # rows overlap
    assert prefill_stats(-1, 16, 0x1000, 32 * 16) == _ext.UKV_ERR_INVALID_ARGUMENT     # negative sink
    assert prefill_stats(4, 0, 0x1000, 32 * 16) == _ext.UKV_ERR_INVALID_ARGUMENT       # empty window

    def scores_from(stats):
        return lib.ukv_snapkv_scores_from_stats(None, i64((0, 0, 0)), None, i64((0, 0, 0, 0)), None, 0, 0, 1, 1,
                                                4096, 64, 128, 32, 8, 128, 4, 16, 0.088, _ext.UKV_DTYPE_BF16, stats,
                                                None, 0, None, 0, None)

    assert scores_from(None) == _ext.UKV_ERR_INVALID_ARGUMENT
    assert scores_from(0x1004) == _ext.UKV_ERR_INVALID_ARGUMENT


@pytest.mark.gpu
def test_shapes_off_the_tiled_prefill_flag_every_row(cuda):
    # head_dim 64 runs the scalar prefill: it writes every row flagged, and the scores then equal
    # the two-pass scores bit for bit (every item recomputed)
    import torch

    from unifiedkv_amd import snapkv
    from unifiedkv_amd.pool import PagedKVPool
    from unifiedkv_amd.prefill import PrefillPages

    rng = np.random.default_rng(31)
    B, L, Hq, Hkv, D, sink, obs, C = 2, 2, 8, 2, 64, 4, 32, 300
    scale = D ** -0.5
    pool = PagedKVPool(16, L, Hkv, D, torch.bfloat16, num_blocks=64, device=cuda)
    pp = PrefillPages(pool, B)
    st = snapkv.ObsStats(B, L, Hq, sink_len=sink, obs_len=obs, softmax_scale=scale, device=cuda)
    st.data.fill_(7.0)
    pp.begin_chunk([C] * B)
    q_obs = np.zeros((B, L, Hq, obs, D), np.uint16)
    for layer in range(L):
        q, k, v = _bits(rng, (B * C, Hq, D), "bf16"), _bits(rng, (B * C, Hkv, D), "bf16"), _bits(rng, (B * C, Hkv, D), "bf16")
        pp.attention(layer, _dev(q, "bf16"), _dev(k, "bf16"), _dev(v, "bf16"), softmax_scale=scale, n_rep=Hq // Hkv,
                     obs_stats=st)
        for b in range(B):
            q_obs[b, layer] = q[(b + 1) * C - obs:(b + 1) * C].transpose(1, 0, 2)
    pp.end_chunk()
    data = st.data.cpu().numpy()
    assert np.all(data[..., 1] == 1.0) and np.all(data[..., 0] == 0.0)
    width = max(len(x) for x in pp.page_lists)
    table = torch.tensor([x + [0] * (width - len(x)) for x in pp.page_lists], dtype=torch.int32, device=cuda)
    qd = _dev(q_obs, "bf16")
    one = snapkv.score_blocks(qd, pool.k_cache, table, seq_len=C, sink_len=sink, obs_len=obs, n_rep=Hq // Hkv,
                              obs_stats=st).cpu().numpy()
    two = snapkv.score_blocks(qd, pool.k_cache, table, seq_len=C, sink_len=sink, obs_len=obs,
                              n_rep=Hq // Hkv).cpu().numpy()
    assert np.array_equal(one, two)
