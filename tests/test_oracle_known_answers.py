"""Pins the CPU oracle against the reference's own known answers, invariants
and closed forms (the reference ships no golden-vector files; its tests hold
hand-checked values inline).  Each test names the reference test it
restates.  No GPU needed.
"""
import math

import numpy as np
import pytest

from oracle import binding as orc

ST_OK, ST_DIM_NOT_DIV, ST_DIM, ST_EMPTY_CORPUS = 0, 1, 2, 3
ST_BUDGET, ST_EMPTY_SET = 6, 7
ST_EMPTY_DIST, ST_NONFINITE, ST_ALLZERO = 8, 9, 10
NEVER = float("-inf")


def f32(*v):
    return np.array(v, dtype=np.float32)


# ---- vec primitives: src/util/vec.zig tests ---------------------------------

def test_l2sq_hand_checked():  # vec.zig:367-372
    assert orc.l2sq(f32(1, 2, 3), f32(4, 6, 3)) == 25.0


def test_l2sq_identical_is_zero():  # vec.zig:374-377
    a = f32(0.5, -0.5, 0.25, -0.25, 1.0)
    assert orc.l2sq(a, a) == 0.0


def test_l2sq_tail_beyond_lane():  # vec.zig:379-388
    a = np.arange(9, dtype=np.float32)
    assert orc.l2sq(a, a + 1) == 9.0


def _np_generic(a, b, lanes, dot=False):
    """vec.l2sqGeneric / dotGeneric (vec.zig:90-103, :159-175) in numpy
    float32, every operation rounded: lane j adds the products of elements
    j, j + lanes, ... of the whole chunks to 0.0, the lanes are added in
    order, then the tail elements one by one."""
    a, b = f32(*a), f32(*b)
    p = a * b if dot else (a - b) * (a - b)
    acc = np.zeros(lanes, np.float32)
    i = 0
    while i + lanes <= a.size:
        acc = acc + p[i:i + lanes]
        i += lanes
    s = acc[0]
    for j in range(1, lanes):
        s = np.float32(s + acc[j])
    for k in range(i, a.size):
        s = np.float32(s + p[k])
    return s


@pytest.mark.parametrize("lanes", [4, 8, 16])
@pytest.mark.parametrize("dim", [3, 8, 9, 16, 20, 33, 100])
def test_generic_vec_lane_count(lanes, dim):
    """The generic path at each host lane count (vec.zig:16), pinned three
    ways: against the chunked form above; at 8 and 16 lanes for dims below
    two lane widths against the plain sequential fold (a different
    formula); and, at 4 lanes and dim 8, against the pairing of element j
    with j + 4, while a planted pairing of neighbours (j with j + 1) and the
    sequential fold both disagree on some of the same inputs."""
    rng = np.random.default_rng(dim * 31 + lanes)
    seq_diff = adj_diff = 0
    with orc.lane_count(lanes):
        for _ in range(400):
            a = rng.standard_normal(dim).astype(np.float32)
            b = rng.standard_normal(dim).astype(np.float32)
            got = orc.l2sq(a, b)
            if dim not in (2, 4, 64, 128):
                assert got == _np_generic(a, b, lanes), (a, b)
                assert orc.dot(a, b) == _np_generic(a, b, lanes, dot=True)
            sq = ((a - b) * (a - b)).astype(np.float32)
            seq = np.float32(0.0)
            for v in sq:
                seq = np.float32(seq + v)
            if dim < 2 * lanes:
                assert got == seq
            if lanes == 4 and dim == 8:
                lane = (sq[:4] + sq[4:]).astype(np.float32)
                assert got == np.float32(np.float32(np.float32(lane[0] + lane[1]) + lane[2]) + lane[3])
                adj = (sq[0::2] + sq[1::2]).astype(np.float32)
                planted = np.float32(np.float32(np.float32(adj[0] + adj[1]) + adj[2]) + adj[3])
                seq_diff += int(got != seq)
                adj_diff += int(got != planted)
    if lanes == 4 and dim == 8:
        assert seq_diff > 0 and adj_diff > 0


def test_lane_count_rejects_other_values():
    assert orc.lib.orc_set_lane_count(5) != 0
    assert orc.lib.orc_set_lane_count(32) != 0
    assert orc.lib.orc_lane_count() == 16


@pytest.mark.parametrize("lanes", [4, 16])
def test_vectorized_dsub8_matches_per_pair_path(lanes):
    """PQ at sub-dimension 8: the oracle's vectorized all-codeword distance
    form (the 4-lane pairing at 4 lanes) against its per-pair orc_l2sq
    path, on the train trace and the codes."""
    rng = np.random.default_rng(lanes)
    x = rng.standard_normal((3000, 64)).astype(np.float32) * np.float32(0.3)
    init = x[rng.permutation(3000)[:64]].reshape(64, 8, 8).transpose(1, 0, 2).copy()
    with orc.lane_count(lanes):
        fast = orc.pq_train(x, 64, 8, 64, init=init, max_iters=4, tol=NEVER, trace=True)
        fcodes = orc.pq_encode(x, 64, 8, 64, fast.codebooks)
        with orc.scalar_distances():
            slow = orc.pq_train(x, 64, 8, 64, init=init, max_iters=4, tol=NEVER, trace=True)
            scodes = orc.pq_encode(x, 64, 8, 64, fast.codebooks)
    assert fast.trace.tobytes() == slow.trace.tobytes()
    assert np.array_equal(fcodes, scodes)


def test_l2sq_dim4_hand_checked():  # vec.zig:513-519
    assert orc.l2sq(f32(1, 2, 3, 4), f32(5, 6, 7, 8)) == 64.0


def test_l2sq_batch_values():  # vec.zig:440-452 (l2sqBatch = l2sq per row)
    q = f32(0, 0)
    assert [orc.l2sq(q, p) for p in (f32(1, 0), f32(0, 2), f32(3, 4))] == [1.0, 4.0, 25.0]


def test_dot_hand_checked():  # vec.zig:334-339, :497-511
    assert orc.dot(f32(1, 2, 3), f32(4, -5, 6)) == 12.0
    assert orc.dot(f32(1, 2), f32(3, 4)) == 11.0
    assert orc.dot(f32(1, 2, 3, 4), f32(5, 6, 7, 8)) == 70.0
    a = np.arange(1, 18, dtype=np.float32)
    assert orc.dot(a, np.full(17, 2, np.float32)) == 306.0  # vec.zig:341-353


def _seq_l2sq(a, b):
    s = np.float32(0.0)
    for x, y in zip(a, b):
        d = np.float32(x) - np.float32(y)
        s = np.float32(s + np.float32(d * d))
    return s


@pytest.mark.parametrize("d", [1, 2, 3, 4, 5, 6, 7, 8, 16])
def test_l2sq_is_sequential_fold_below_host_lanes(d):
    # src/util/vec.zig:109-175: dims 2 and 4 are explicit left folds; other
    # dims below the host lane count reduce an all-zero vector and then fold
    # the tail left to right — the same value as a sequential fold.
    rng = np.random.default_rng(d)
    for _ in range(200):
        a = rng.standard_normal(d).astype(np.float32)
        b = rng.standard_normal(d).astype(np.float32)
        assert orc.l2sq(a, b) == _seq_l2sq(a, b)


@pytest.mark.parametrize("d", [64, 128])
def test_l2sq_four_lane_grouping(d):
    # src/util/vec.zig:142-155: four accumulators over chunks of 4, then an
    # ordered reduce.  Differs from the sequential fold in the last bits; a
    # transposed chunk/lane index would change it again.
    rng = np.random.default_rng(d)
    a = rng.standard_normal(d).astype(np.float32)
    b = rng.standard_normal(d).astype(np.float32)
    acc = np.zeros(4, np.float32)
    for c in range(0, d, 4):
        t = (a[c:c + 4] - b[c:c + 4]).astype(np.float32)
        acc = (acc + (t * t).astype(np.float32)).astype(np.float32)
    want = np.float32(np.float32(np.float32(acc[0] + acc[1]) + acc[2]) + acc[3])
    assert orc.l2sq(a, b) == want
    assert abs(float(orc.l2sq(a, b)) - float(np.sum((a.astype(np.float64) - b) ** 2))) < 1e-4


def test_argmin_argmax():  # vec.zig:420-438
    assert orc.argmin(f32(3.0, 1.5, 4.0, -2.0, 7.0)) == 3
    assert orc.argmin(f32(1.0, 1.0, 2.0)) == 0  # ties pick first
    assert orc.argmax(f32(-3.0, 1.5, 4.0, -2.0, 7.0)) == 4
    assert orc.argmax(f32(7.0, 1.0, 7.0)) == 0


# ---- rng: src/util/rng.zig tests (stream unpinned; properties only) ---------

def test_prng_same_seed_same_stream():  # rng.zig:104-111
    a, b = orc.ZigPrng(42), orc.ZigPrng(42)
    assert [a.uint_less_than(1000) for _ in range(32)] == [b.uint_less_than(1000) for _ in range(32)]


def test_prng_splitmix_xoshiro_published_vector():
    # Xoshiro256++ reference implementation (Blackman & Vigna) seeded with
    # SplitMix64(0): first outputs of the published C code.
    r = orc.ZigPrng(0)
    sm = 0
    state = []
    for _ in range(4):
        sm = (sm + 0x9E3779B97F4A7C15) & (2**64 - 1)
        z = sm
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & (2**64 - 1)
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & (2**64 - 1)
        state.append(z ^ (z >> 31))
    s = state

    def rotl(x, k):
        return ((x << k) | (x >> (64 - k))) & (2**64 - 1)

    for _ in range(16):
        want = (rotl((s[0] + s[3]) & (2**64 - 1), 23) + s[0]) & (2**64 - 1)
        t = (s[1] << 17) & (2**64 - 1)
        s[2] ^= s[0]
        s[3] ^= s[1]
        s[1] ^= s[2]
        s[0] ^= s[3]
        s[2] ^= t
        s[3] = rotl(s[3], 45)
        assert r.next() == want


def test_prng_float_in_unit_interval():  # rng.zig:122-129
    r = orc.ZigPrng(7)
    xs = [r.float_f64() for _ in range(4096)]
    assert all(0.0 <= x < 1.0 for x in xs)
    assert 0.45 < sum(xs) / len(xs) < 0.55


def test_uint_less_than_is_uniform_and_bounded():
    r = orc.ZigPrng(123)
    xs = [r.uint_less_than(10) for _ in range(20000)]
    assert min(xs) == 0 and max(xs) == 9
    counts = np.bincount(xs, minlength=10)
    assert counts.min() > 1800 and counts.max() < 2200


def test_weighted_sample_rules():  # rng.zig:131-170, :57-82
    r = orc.ZigPrng(99)
    for _ in range(256):
        st, idx = r.weighted_sample(f32(0.0, 1.0, 0.0, 0.0, 2.0))
        assert st == ST_OK and idx in (1, 4)
    assert orc.ZigPrng(1).weighted_sample(np.zeros(0, np.float32))[0] == ST_EMPTY_DIST
    assert orc.ZigPrng(1).weighted_sample(f32(1.0, float("nan")))[0] == ST_NONFINITE
    assert orc.ZigPrng(1).weighted_sample(f32(1.0, -1.0))[0] == ST_NONFINITE
    assert orc.ZigPrng(1).weighted_sample(f32(0.0, 0.0))[0] == ST_ALLZERO
    r = orc.ZigPrng(2026)
    counts = np.zeros(3)
    for _ in range(10000):
        counts[r.weighted_sample(f32(0.1, 0.3, 0.6))[1]] += 1
    assert abs(counts[0] - 1000) < 150 and abs(counts[2] - 6000) < 300


# ---- kmeans.fit: src/tac/kmeans.zig tests -----------------------------------

def test_fit_errors():  # kmeans.zig:373-389
    assert orc.kmeans_fit(f32(1, 0, 0, 1), 2, 0).status == ST_BUDGET
    assert orc.kmeans_fit(np.zeros(0, np.float32), 2, 1).status == ST_EMPTY_SET


def test_fit_degenerate():  # kmeans.zig:391-407
    r = orc.kmeans_fit(f32(1, 0, 0, 1), 2, 4)
    assert r.status == 0 and r.wcss == 0.0 and r.iters_run == 0
    assert list(r.assignments) == [0, 1]
    assert np.array_equal(r.centroids, f32(1, 0, 0, 1, 0, 1, 0, 1))
    r = orc.kmeans_fit(f32(1, 0, 0, 1, 1, 1), 2, 3)
    assert r.wcss == 0.0 and r.iters_run == 0


def _blobs(centers, offsets):
    return np.array([[c[0] + o[0], c[1] + o[1]] for c in centers for o in offsets], np.float32)


OFFS6 = [(-0.05, 0.02), (0.03, -0.04), (-0.01, -0.02), (0.02, 0.05), (-0.03, 0.01), (0.04, -0.03)]


def test_fit_recovers_blob_means():  # kmeans.zig:409-447
    centers = [(0, 0), (10, 0), (0, 10)]
    r = orc.kmeans_fit(_blobs(centers, OFFS6), 2, 3, max_iters=50, seed=42)
    cents = r.centroids.reshape(3, 2)
    for c in centers:
        assert min(math.hypot(*(cc - np.array(c))) for cc in cents) < 0.1


def test_fit_thread_count_byte_equal():  # kmeans.zig:449-485, :628-664
    v = np.random.default_rng(0xDE7E2).standard_normal(600 * 4).astype(np.float32)
    r1 = orc.kmeans_fit(v, 4, 32, seed=42, n_threads=1)
    for t in (3, 10, 64):
        rt = orc.kmeans_fit(v, 4, 32, seed=42, n_threads=t)
        assert rt.centroids.tobytes() == r1.centroids.tobytes()
        assert rt.assignments.tobytes() == r1.assignments.tobytes()
        assert rt.wcss == r1.wcss and rt.iters_run == r1.iters_run
    small = v[:20]
    assert orc.kmeans_fit(small, 4, 3, seed=7, n_threads=64).centroids.tobytes() == \
        orc.kmeans_fit(small, 4, 3, seed=7).centroids.tobytes()


def test_fit_wcss_non_increasing():  # kmeans.zig:503-521
    v = np.random.default_rng(1234).standard_normal(60).astype(np.float32)
    w = [orc.kmeans_fit(v, 3, 4, seed=111, max_iters=it, tol=0.0).wcss for it in (1, 5, 25)]
    assert w[1] <= w[0] and w[2] <= w[1]


def test_fit_wcss_trace_monotone_and_equals_sum():
    # Lloyd monotonicity per iteration (assign then update never increases
    # the objective) and wcss = serial fold of the per-vector distances.
    v = np.random.default_rng(3).standard_normal(4000 * 4).astype(np.float32)
    r = orc.kmeans_fit(v, 4, 16, max_iters=12, tol=NEVER, init=v[:64], trace=True)
    assert np.all(np.diff(r.wcss_trace.astype(np.float64)) <= 1e-6 * r.wcss_trace[0])
    cents = r.centroids.reshape(16, 4)
    pts = v.reshape(-1, 4)
    # after the last update, re-assigning can only lower the objective
    d = ((pts[:, None, :].astype(np.float64) - cents[None].astype(np.float64)) ** 2).sum(-1)
    assert d.min(1).sum() <= r.wcss * (1 + 1e-5)


def test_fit_assignments_valid():  # kmeans.zig:523-533
    v = np.random.default_rng(5).standard_normal(50).astype(np.float32)
    r = orc.kmeans_fit(v, 5, 3, seed=0)
    assert r.assignments.size == 10 and r.assignments.max() < 3


def test_fit_empty_cluster_path():  # kmeans.zig:535-543
    r = orc.kmeans_fit(f32(0.0, 0.0, 0.0001, 0.0, 100.0, 0.0), 2, 3, max_iters=10, seed=1)
    assert r.status == 0 and r.assignments.max() < 3


BLOBS5 = [(0, 0), (50, 0), (0, 50), (-50, 0), (0, -50)]
OFFS8 = [(-0.05, 0.02), (0.03, -0.04), (-0.01, -0.02), (0.02, 0.05), (-0.03, 0.01),
         (0.04, -0.03), (0.0, 0.0), (0.01, -0.01)]


def _lloyd_invariants(pts, r, k, d):
    # kmeans.zig:545-626: assignments are argmin under the returned centroids;
    # centroids equal the serial-order mean with a reciprocal multiply.
    n = pts.shape[0]
    cents = r.centroids.reshape(k, d)
    for i in range(n):
        mine = orc.l2sq(pts[i], cents[r.assignments[i]])
        assert all(mine <= orc.l2sq(pts[i], cents[c]) for c in range(k))
    sums = np.zeros((k, d), np.float32)
    counts = np.zeros(k, np.uint32)
    for i in range(n):
        a = r.assignments[i]
        sums[a] = (sums[a] + pts[i]).astype(np.float32)
        counts[a] += 1
    for c in range(k):
        if counts[c]:
            inv = np.float32(np.float32(1.0) / np.float32(counts[c]))
            assert np.array_equal((sums[c] * inv).astype(np.float32), cents[c])


def test_fit_lloyd_invariants():  # kmeans.zig:545-626
    pts = _blobs(BLOBS5, OFFS8)
    r = orc.kmeans_fit(pts, 2, 5, seed=7, max_iters=50)
    _lloyd_invariants(pts, r, 5, 2)


def test_fit_early_break_invariants():  # kmeans.zig:666-708
    pts = f32(0.00, 0.00, 0.01, -0.01, -0.02, 0.01, 0.01, 0.02, -0.01, -0.02, 0.00, 0.01,
              100.0, 100.0, 99.99, 100.01, 100.02, 99.98, 100.01, 99.99, 99.98, 100.02, 100.0,
              100.0).reshape(12, 2)
    r = orc.kmeans_fit(pts, 2, 2, seed=3, max_iters=25)
    assert r.iters_run <= 5
    _lloyd_invariants(pts, r, 2, 2)


def test_fit_brute_force_tiny():
    # Independent restatement on tiny inputs with forced ties: numpy float32
    # arithmetic in the reference's order, compared bit for bit.
    rng = np.random.default_rng(17)
    for trial in range(30):
        n, d, k = int(rng.integers(5, 40)), int(rng.integers(1, 6)), int(rng.integers(2, 6))
        if k >= n:
            continue
        pts = np.round(rng.standard_normal((n, d)) * 2).astype(np.float32)  # many ties
        init = pts[rng.permutation(n)[:k]].copy()
        iters = int(rng.integers(1, 6))
        r = orc.kmeans_fit(pts, d, k, max_iters=iters, tol=NEVER, init=init)
        c = init.copy()
        for _ in range(iters):
            dist = np.array([[_seq_l2sq(p, q) for q in c] for p in pts], np.float32)
            a = np.array([int(np.argmin(row)) for row in dist])  # numpy argmin: first min
            e = dist[np.arange(n), a].copy()
            sums = np.zeros((k, d), np.float32)
            cnt = np.zeros(k, np.uint32)
            for i in range(n):
                sums[a[i]] = (sums[a[i]] + pts[i]).astype(np.float32)
                cnt[a[i]] += 1
            for cc in range(k):
                if cnt[cc]:
                    c[cc] = (sums[cc] * np.float32(np.float32(1) / np.float32(cnt[cc]))).astype(
                        np.float32)
                else:
                    far = int(np.argmax(e))
                    c[cc] = pts[far]
                    e[far] = -np.inf
        assert r.centroids.tobytes() == c.reshape(-1).tobytes(), trial
        assert np.array_equal(r.assignments, a)


# ---- pq: src/index/pq.zig tests ---------------------------------------------

def test_pq_errors():  # pq.zig:357-370
    assert orc.pq_train(np.zeros(33, np.float32), 33, 32, 256).status == ST_DIM_NOT_DIV
    assert orc.pq_train(np.zeros(0, np.float32), 32, 32, 256).status == ST_EMPTY_CORPUS
    assert orc.pq_train(np.zeros(64, np.float32), 0, 32, 256).status == ST_DIM


def _normalize_rows(x):
    n = np.sqrt((x.astype(np.float32) ** 2).sum(1, dtype=np.float32)).astype(np.float32)
    return (x / np.where(n > 0, n, 1)[:, None]).astype(np.float32)


def test_pq_round_trip_idempotent():  # pq.zig:372-413
    x = _normalize_rows(np.random.default_rng(0x52017).standard_normal((300, 32)))
    init = np.stack([x[:256, m:m + 1] for m in range(32)])
    r = orc.pq_train(x, 32, 32, 256, init=init)
    assert r.status == 0
    codes = orc.pq_encode(x[:1], 32, 32, 256, r.codebooks)
    dec = orc.pq_decode(codes, 32, 32, 256, r.codebooks)
    assert np.array_equal(orc.pq_encode(dec, 32, 32, 256, r.codebooks), codes)


def test_pq_mse_bounded():  # pq.zig:415-444
    x = (np.random.default_rng(0xC0DE).standard_normal((1024, 32)) * 0.1).astype(np.float32)
    init = np.stack([x[:256, m:m + 1] for m in range(32)])
    r = orc.pq_train(x, 32, 32, 256, init=init)
    dec = orc.pq_decode(orc.pq_encode(x, 32, 32, 256, r.codebooks), 32, 32, 256, r.codebooks)
    assert float(((x.astype(np.float64) - dec) ** 2).mean()) < 1e-3


def test_pq_thread_counts_byte_equal():  # pq.zig:462-517
    x = _normalize_rows(np.random.default_rng(0xA701C).standard_normal((512, 32)))
    init = np.stack([x[100:356, m:m + 1] for m in range(32)])
    r1 = orc.pq_train(x, 32, 32, 256, init=init, n_threads=1)
    for t in (4, 10, 64):
        assert orc.pq_train(x, 32, 32, 256, init=init, n_threads=t).codebooks.tobytes() == \
            r1.codebooks.tobytes()


def test_pq_train_is_per_subspace_kmeans():
    # pq.zig:301-336: subspace m is kmeans.fit on the m-th column block with
    # seed +% m.
    x = np.random.default_rng(8).standard_normal((700, 16)).astype(np.float32)
    init = np.random.default_rng(9).standard_normal((4, 20, 4)).astype(np.float32)
    r = orc.pq_train(x, 16, 4, 20, init=init, max_iters=7, tol=NEVER)
    for m in range(4):
        f = orc.kmeans_fit(x[:, 4 * m:4 * m + 4], 4, 20, max_iters=7, tol=NEVER, init=init[m])
        assert f.centroids.tobytes() == r.codebooks.reshape(4, -1)[m].tobytes()


def test_encode_brute_force():
    # PQ.encode = first-index argmin of the reference distance per subspace.
    rng = np.random.default_rng(12)
    x = np.round(rng.standard_normal((64, 12)) * 3).astype(np.float32)
    cb = np.round(rng.standard_normal((3, 9, 4)) * 3).astype(np.float32)
    got = orc.pq_encode(x, 12, 3, 9, cb)
    for i in range(64):
        for m in range(3):
            d = [_seq_l2sq(x[i, 4 * m:4 * m + 4], cb[m, c]) for c in range(9)]
            assert got[i, m] == int(np.argmin(d))


def test_distance_table_layout_and_values():  # pq.zig:344-349, :519-585
    rng = np.random.default_rng(11)
    q = rng.standard_normal((4, 32)).astype(np.float32)
    cb = rng.standard_normal((32, 256, 1)).astype(np.float32)
    st, t = orc.pq_distance_table(q, 4, 32, 32, 256, cb)
    assert st == 0
    m, c, i = 5, 17, 2
    assert abs(t[((m * 256) + c) * 4 + i] - q[i, m] * cb[m, c, 0]) < 1e-6
    st, _ = orc.pq_distance_table(q, 4, 32, 32, 256, cb, table_len=4)
    assert st == 4  # OutBufferWrongSize


def _same_floats(a, b):
    a, b = np.asarray(a, np.float32).reshape(-1), np.asarray(b, np.float32).reshape(-1)
    na, nb = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32),
                                                          b[~nb].view(np.uint32)))


@pytest.mark.parametrize("dsub", [1, 2, 3, 4, 5, 6, 7, 8])
def test_vectorized_distances_equal_the_per_pair_form(dsub):
    """For d <= 8 the oracle forms all K distances of a vector at once from a
    transposed codebook and takes the first-index minimum in two passes; the
    per-pair form (orc_l2sq, then the strict-< scan) must give the same codes,
    codebooks, empties and wcss, on inputs with exact ties, duplicate
    codewords, signed zeros, NaN and infinities."""
    rng = np.random.default_rng(100 + dsub)
    m, ksub, n = 4, 37, 3000
    dim = m * dsub
    cb = rng.standard_normal((m, ksub, dsub)).astype(np.float32)
    cb[:, 3] = cb[:, 0]          # duplicates: the lower index wins
    cb[:, 20] = 0.0
    cb[:, 21] = -0.0             # equal to +0.0 under <
    x = rng.standard_normal((n, dim)).astype(np.float32)
    x[100:130] = cb[:, :30].transpose(1, 0, 2).reshape(30, dim)  # exact ties at distance 0
    x[::97] = 0.0
    x[5::101] = -0.0
    x[7, :dsub] = np.nan
    x[9, 0] = np.inf
    x[11, -1] = -np.inf
    x[13] = 3e19                 # squares overflow to +inf
    bad = cb.copy()
    bad[1, 5, 0] = np.nan
    bad[2, 6, 0] = np.inf
    for book in (cb, bad):
        fast = orc.pq_encode(x, dim, m, ksub, book, n_threads=4)
        with orc.scalar_distances():
            slow = orc.pq_encode(x, dim, m, ksub, book, n_threads=4)
        assert np.array_equal(fast, slow)
    # Lloyd iterations: vec.argmin from values[0] (finite data, forced ties)
    xt = x[14:].copy()
    xt[~np.isfinite(xt)] = 0.0
    xt[np.abs(xt) > 1e10] = 1.0
    init = cb.copy()
    a = orc.pq_train(xt, dim, m, ksub, init=init, max_iters=4, tol=float("-inf"), n_threads=3,
                     trace=True)
    with orc.scalar_distances():
        b = orc.pq_train(xt, dim, m, ksub, init=init, max_iters=4, tol=float("-inf"),
                         n_threads=3, trace=True)
    assert a.status == b.status == 0
    assert _same_floats(a.trace, b.trace)
    assert np.array_equal(a.empties, b.empties)
    assert _same_floats(a.wcss, b.wcss)
    # a NaN row: its subspace's codeword 0 turns NaN, and argmin from values[0]
    # then keeps 0 for every vector
    xn = xt.copy()
    xn[50, :dsub] = np.nan
    a = orc.pq_train(xn, dim, m, ksub, init=init, max_iters=3, tol=float("-inf"), trace=True)
    with orc.scalar_distances():
        b = orc.pq_train(xn, dim, m, ksub, init=init, max_iters=3, tol=float("-inf"),
                         trace=True)
    assert _same_floats(a.trace, b.trace)
    assert np.array_equal(a.empties, b.empties)
