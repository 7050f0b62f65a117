"""GPU token-aware clustering (tac_cluster_flat) against the oracle's
restatement of src/tac/tac.zig, bit for bit: centroids, assignments,
kappa per token and wcss_total, and the same error for the same input."""
import numpy as np
import pytest

from oracle import binding as orc
from tac_gpu import errors, synth, tac

pytestmark = pytest.mark.gpu


def _params(kappa, seed, **kw):
    return tac.ClusteringParams(kappa_total=kappa, seed=seed, **kw)


def _check(ids, v, dim, kappa, seed, **kw):
    ref = orc.tac_cluster_flat(ids, v, dim, orc.tac_params(kappa, seed, **kw))
    assert ref.status == 0, ref.status
    got = tac.cluster_flat(ids, v, dim, _params(kappa, seed, **kw))
    assert np.array_equal(got.kappa_per_token, ref.kappa_per_token)
    assert got.centroids.tobytes() == ref.centroids.tobytes()
    assert np.array_equal(got.assignments, ref.assignments)
    assert np.float32(got.wcss_total).tobytes() == np.float32(ref.wcss_total).tobytes()
    return got


def _feasible_kappa(ids, frac=0.6, mu=128, tau=256, theta=39):
    f = np.bincount(ids)
    tail = int(((f > 0) & (f < mu)).sum() + 2 * ((f >= mu) & (f < tau)).sum())
    return tail + int(frac * (f[f >= tau] // theta).sum())


def _themes(counts, themes, sigma, seed):
    rng = np.random.default_rng(seed)
    ids, vec = [], []
    for tid, (c, t) in enumerate(zip(counts, themes)):
        for _ in range(c):
            ids.append(tid)
            vec.append(np.asarray(t, np.float32) + rng.standard_normal(len(t)).astype(np.float32) * sigma)
    return np.array(ids, np.uint32), np.array(vec, np.float32)


def test_reference_test_inputs(gpu):
    # The shapes of the reference's clusterFlat tests (tac.zig:1131-1306).
    ids, v = _themes([10, 10, 6, 4], [(1, 0), (0, 1), (-1, 0), (0, -1)], 0.05, 7)
    _check(ids, v, 2, 14, 42, mu=3, tau=5, epsilon=1, theta=1)
    rng = np.random.default_rng(1)
    _check((np.arange(40) % 5).astype(np.uint32), rng.standard_normal((40, 3)).astype(np.float32),
           3, 18, 12345, mu=3, tau=5, epsilon=1, theta=1)
    r = _check(np.array([1, 1, 1, 1, 2, 2, 2, 2, 3, 3, 3, 3], np.uint32),
               np.arange(1, 13, dtype=np.float32) / 10, 1, 6, 0, mu=3, tau=5, epsilon=1, theta=1)
    assert r.kappa_per_token.tolist() == [0, 2, 2, 2]
    ids, v = _themes([6, 6, 6], [(10, 0), (0, 10), (-10, 0)], 0.05, 99)
    r = _check(ids, v, 2, 3, 0, mu=2, tau=5, epsilon=1, theta=1)
    assert np.array_equal(r.assignments, ids)


@pytest.mark.parametrize("n,vocab,dim,seed", [(60_000, 2048, 64, 3), (30_000, 1024, 128, 4)])
def test_synthetic_token_dumps(gpu, n, vocab, dim, seed):
    ids, v = synth.tac_vectors(n, dim, vocab, 1.05, 0.15, seed)
    _check(ids, v, dim, _feasible_kappa(ids), 5)


def test_synthetic_200k(gpu):
    """200,000 x 64 over 4,096 tokens: ~80 active tokens with up to ~500
    centroids each, next to thousands of micro tokens."""
    ids, v = synth.tac_vectors(200_000, 64, 4096, 1.05, 0.15, 3)
    _check(ids, v, 64, _feasible_kappa(ids), 5)


@pytest.mark.parametrize("dim", [3, 16, 33, 95, 96, 100, 191, 192, 256, 257, 384, 448, 512])
def test_generic_dims(gpu, dim):
    # generic 16-lane distances; 95 / 96 straddle the 128 / 64-row tiles, 191 /
    # 192 the 64 KB and the wide-row LDS budgets; 4 to 8 dimensions per lane
    # in the spread and fold waves past 192
    ids, v = synth.tac_vectors(6000, dim, 300, 1.0, 0.2, dim)
    _check(ids, v, dim, _feasible_kappa(ids, mu=20, tau=40, theta=8), 9, mu=20, tau=40,
           epsilon=4, theta=8)


@pytest.mark.parametrize("dim", [64, 96, 191, 320, 512])
def test_spread_batch_edges(gpu, dim):
    # token sizes on either side of one, two and three 32-row spread batches
    # (16 rows at 4 to 6 dimensions per lane, 8 rows beyond)
    # and of the 64-row batches of the dim-64 kernel, up to past its ring of
    # four (the last, partial batch is the only one with a row test), in
    # shuffled input order, with spreads that decide the budgets of tokens >=
    # mu rows
    sizes = [1, 31, 32, 33, 40, 63, 64, 65, 95, 96, 97, 128, 129, 191, 192, 193, 255, 256,
             257, 319, 320, 321, 449, 512, 577]
    rng = np.random.default_rng(dim)
    ids = np.concatenate([np.full(c, t, np.uint32) for t, c in enumerate(sizes)])
    ids = ids[rng.permutation(ids.size)]
    scale = (1.0 + np.arange(len(sizes), dtype=np.float32))[ids, None]
    v = (rng.standard_normal((ids.size, dim)).astype(np.float32) * scale).astype(np.float32)
    _check(ids, v, dim, _feasible_kappa(ids, frac=0.9, mu=20, tau=40, theta=8), 4, mu=20,
           tau=40, epsilon=4, theta=8)


def test_thread_grouping_and_exact_draws(gpu, monkeypatch):
    ids, v = synth.tac_vectors(60_000, 64, 2048, 1.05, 0.15, 8)
    kap = _feasible_kappa(ids)
    for nt in (3, 10):
        _check(ids, v, 64, kap, 21, n_threads=nt)
    # Draws sent to the exact sequential evaluation: every draw ("1"), and
    # the draws of round c of problem q with (c + q) % 7 == 0 ("7"), so that
    # tokens stall at different rounds and are replayed beside tokens that
    # finished, some stalling again while they replay.
    for every in ("1", "7"):
        monkeypatch.setenv("TAC_GPU_KPP_EXACT", every)
        _check(ids, v, 64, kap, 21)
        _check(ids, v, 64, kap, 21, n_threads=3)


def test_degenerate_and_tiny_tokens(gpu):
    # mu=2: tokens with one row are micro (k = 1 >= n = 1, the degenerate
    # branch of kmeans.fit); small tokens of 2-3 rows get k = 2.
    rng = np.random.default_rng(5)
    ids = np.array([0, 1, 1, 2, 2, 2, 3, 4, 4, 4, 4, 4, 4, 4, 4] + [5] * 40, np.uint32)
    v = rng.standard_normal((ids.size, 4)).astype(np.float32)
    _check(ids, v, 4, 20, 3, mu=2, tau=4, epsilon=2, theta=2)


def test_token_id_past_2_pow_26(gpu):
    # One row carries token id 70,000,000, so the vocabulary holds 70M ids:
    # one spread wave per id is 4.5e9 work-items, more than one dispatch's
    # grid, and the spreads run in slices of ids.
    rng = np.random.default_rng(5)
    ids = (np.arange(3000) % 7).astype(np.uint32)
    ids[-1] = 70_000_000
    v = rng.standard_normal((3000, 8)).astype(np.float32)
    r = _check(ids, v, 8, 12, 3, mu=3, tau=5, epsilon=1, theta=1)
    assert r.kappa_per_token.size == 70_000_001 and r.kappa_per_token[-1] == 1


@pytest.mark.parametrize("case", ["dump", "ties", "untame"])
def test_matrix_core_assignment(gpu, monkeypatch, case):
    """64-float rows: the MFMA-screened assignment on every problem (a k
    threshold of 1) gives the oracle's bits, also with exact ties between
    centroids (rows the screen cannot settle) and with subnormal or huge
    components (blocks that fall back to the exact search)."""
    monkeypatch.setenv("TAC_GPU_TAC_MFMA_KMIN", "1")
    if case == "dump":
        ids, v = synth.tac_vectors(60_000, 64, 2048, 1.05, 0.15, 8)
        _check(ids, v, 64, _feasible_kappa(ids), 5)
        return
    rng = np.random.default_rng(11 if case == "ties" else 12)
    ids = (np.arange(6000) % 3).astype(np.uint32)
    if case == "ties":
        # small-integer rows: the first assignment (centroids are seeded rows)
        # has exact distance ties, some of them inside one lane's centroids
        v = rng.integers(0, 3, (ids.size, 64)).astype(np.float32)
    else:
        v = rng.standard_normal((ids.size, 64)).astype(np.float32)
        v[::97, 5] = np.float32(1e-40)  # subnormal
        v[::389, 9] = np.float32(3e18)  # beyond the screen's bound
    _check(ids, v.astype(np.float32), 64, 60, 21, mu=3, tau=5, epsilon=1, theta=1)


def test_token_beyond_the_lds_code_counters(gpu):
    """A token with 12,600 centroids (more than the 12,288 per-code LDS
    counters of the grouping kernels) groups its rows by counting and
    ranking codes within each tile instead; same bits as the oracle."""
    rng = np.random.default_rng(31)
    ids = np.zeros(40000, np.uint32)
    ids[:500] = 1
    v = rng.standard_normal((40000, 2)).astype(np.float32)
    r = _check(ids, v, 2, 13100, 5, mu=3, tau=5, epsilon=1, theta=1, max_iters=3)
    assert r.kappa_per_token[0] > 12288


@pytest.mark.parametrize("n,dim", [(40_000, 64), (70_000, 320)])
def test_device_resident_vectors(gpu, n, dim):
    """tac_cluster_flat_device: the same token dump resident on the device
    gives the oracle's bits, as the host entry point does (70,000 rows: the
    grouping runs on several host threads; dim 320: wide-row tiles)."""
    from tac_gpu import device
    ids, v = synth.tac_vectors(n, dim, 1024, 1.05, 0.15, 6)
    kap = _feasible_kappa(ids)
    ref = orc.tac_cluster_flat(ids, v, dim, orc.tac_params(kap, 9))
    assert ref.status == 0
    dv = device.DeviceArray.from_host(np.ascontiguousarray(v))
    try:
        got = tac.cluster_flat(ids, dv, dim, _params(kap, 9))
    finally:
        dv.free()
    assert np.array_equal(got.kappa_per_token, ref.kappa_per_token)
    assert got.centroids.tobytes() == ref.centroids.tobytes()
    assert np.array_equal(got.assignments, ref.assignments)
    assert np.float32(got.wcss_total).tobytes() == np.float32(ref.wcss_total).tobytes()


@pytest.mark.parametrize("resident", [False, True])
def test_early_spreads(gpu, monkeypatch, resident):
    """The spreads of the largest tokens advanced while the rows arrive: each
    8 MB staged chunk of the 51 MB host upload, or all rows at once when they
    are resident on the device.  TAC_GPU_TAC_PRESPREAD_MIN=500 gives all 8
    slots a token (chunks end inside their runs of rows).  Both that path and
    the one with it off (TAC_GPU_TAC_PRESPREAD=0) give the oracle's bits."""
    from tac_gpu import device
    ids, v = synth.tac_vectors(200_000, 64, 4096, 1.05, 0.15, 3)
    assert np.sort(np.bincount(ids))[-8] >= 500
    kap = _feasible_kappa(ids)
    ref = orc.tac_cluster_flat(ids, v, 64, orc.tac_params(kap, 5))
    assert ref.status == 0
    monkeypatch.setenv("TAC_GPU_TAC_PRESPREAD_MIN", "500")
    dv = device.DeviceArray.from_host(np.ascontiguousarray(v)) if resident else None
    try:
        for on in ("1", "0"):
            monkeypatch.setenv("TAC_GPU_TAC_PRESPREAD", on)
            got = tac.cluster_flat(ids, dv if resident else v, 64, _params(kap, 5))
            assert np.array_equal(got.kappa_per_token, ref.kappa_per_token), on
            assert got.centroids.tobytes() == ref.centroids.tobytes(), on
            assert np.array_equal(got.assignments, ref.assignments), on
            assert np.float32(got.wcss_total).tobytes() == np.float32(ref.wcss_total).tobytes()
    finally:
        if dv is not None:
            dv.free()


def _expect(ids, v, dim, p_kw, exc):
    ref = orc.tac_cluster_flat(ids, v, dim, orc.tac_params(**p_kw))
    assert ref.status == exc.status
    kw = dict(p_kw)
    with pytest.raises(exc):
        tac.cluster_flat(ids, v, dim, _params(kw.pop("kappa_total"), kw.pop("seed"), **kw))


def test_errors_match_the_reference(gpu):
    v2 = np.array([[1, 0], [0, 1]], np.float32)
    _expect(np.zeros(0, np.uint32), np.zeros(0, np.float32), 2, dict(kappa_total=1, seed=0),
            errors.EmptyTokenDump)
    _expect([0, 0], v2, 2, dict(kappa_total=0, seed=0), errors.BudgetTooSmall)
    _expect([0, 0, 0], v2, 2, dict(kappa_total=4, seed=0), errors.InvalidThresholds)
    _expect([0, 0], v2, 2, dict(kappa_total=4, seed=0, mu=5, tau=5), errors.InvalidThresholds)
    _expect([0, 1, 2], np.zeros((3, 2), np.float32), 2, dict(kappa_total=2, seed=0),
            errors.BudgetTooSmall)
    ids = np.zeros(300, np.uint32)
    _expect(ids, np.random.default_rng(0).standard_normal((300, 2)).astype(np.float32), 2,
            dict(kappa_total=50, seed=0), errors.BudgetTooLarge)
    # k-means++ failures of small tokens (k = 2 from the tail tier, spreads
    # unused): identical rows (AllZero) and a NaN row (NonFinite); the lowest
    # failing token id decides.  An active token's NaN spread fails earlier,
    # in phase 2 (InvalidThresholds).
    same = np.tile(np.array([[0.5, 0.25]], np.float32), (4, 1))
    nan = np.random.default_rng(1).standard_normal((4, 2)).astype(np.float32)
    nan[2, 1] = np.nan
    p = dict(kappa_total=4, seed=0, mu=3, tau=5, epsilon=1, theta=1)
    _expect(np.array([0] * 4 + [1] * 4, np.uint32), np.vstack([same, nan]), 2, p, errors.AllZero)
    _expect(np.array([1] * 4 + [0] * 4, np.uint32), np.vstack([same, nan]), 2, p,
            errors.NonFinite)
    nan6 = np.vstack([nan, nan[:2]])
    _expect(np.zeros(6, np.uint32), nan6, 2, dict(kappa_total=2, seed=0, mu=3, tau=5, epsilon=1,
                                                  theta=1), errors.InvalidThresholds)
    with pytest.raises(errors.Unsupported):
        tac.cluster_flat(np.zeros(4, np.uint32), np.zeros((4, 513), np.float32), 513,
                         _params(1, 0))
    # a clean call after the errors
    ids, v = synth.tac_vectors(3000, 8, 100, 1.0, 0.2, 1)
    _check(ids, v, 8, _feasible_kappa(ids, mu=5, tau=20, theta=4), 2, mu=5, tau=20, epsilon=4,
           theta=4)


def test_full_corpus_scale_properties(gpu):
    """1,521,797 x 64 over a 30,522-id vocabulary, kappa_total 40,960, through
    properties the reference fixes at any size: kappa sums to the budget,
    every token's assignments lie in its own centroid range, and every
    non-empty centroid is the serial fp32 fold of its final members times
    fl(1 / fl(count)) (kmeans.zig:177-198: centroids are updated from the
    assignments that fit returns)."""
    d, ids, v = synth.tac_workload("tac-1.52m")
    r = tac.cluster_flat(ids, v, d["dim"], _params(d["kappa_total"], 0))
    k = r.kappa_per_token
    assert int(k.sum()) == d["kappa_total"]
    goff = np.concatenate([[0], np.cumsum(k.astype(np.int64))])
    a = r.assignments.astype(np.int64)
    assert np.all(a >= goff[ids]) and np.all(a < goff[ids + 1])
    # serial member folds, all clusters at once, one member rank at a time
    order = np.lexsort((np.arange(ids.size), a))
    cnt = np.bincount(a, minlength=d["kappa_total"])
    first = np.concatenate([[0], np.cumsum(cnt)[:-1]])
    s = np.zeros((d["kappa_total"], d["dim"]), np.float32)
    live = np.nonzero(cnt)[0]
    for rank in range(int(cnt.max())):
        live = live[cnt[live] > rank]
        s[live] = (s[live] + v[order[first[live] + rank]]).astype(np.float32)
    nz = cnt > 0
    inv = (np.float32(1.0) / cnt[nz].astype(np.float32)).astype(np.float32)
    want = (s[nz] * inv[:, None]).astype(np.float32)
    assert want.tobytes() == r.centroids[nz].tobytes()
    assert np.isfinite(r.wcss_total) and r.wcss_total > 0


@pytest.mark.parametrize("tol,dim", [(1e-2, 64), (2e-3, 64), (5e-4, 8)])
def test_problems_converging_around_the_readbacks(gpu, tol, dim):
    """Loose tolerances make tokens of different k converge at different
    iterations, on both sides of the points where the Lloyd loop reads the
    done flags back and shrinks its launches to the unfinished problems
    (iterations 3, 6, 10, 15 and 21), and let the loop end early through
    the all-converged exit: centroids, assignments, kappa and wcss_total
    equal the oracle's (kmeans.zig:214-223 per token)."""
    ids, v = synth.tac_vectors(60_000, dim, 2048, 1.05, 0.15, 17)
    _check(ids, v, dim, _feasible_kappa(ids), 23, max_iters=25, tol=tol)
