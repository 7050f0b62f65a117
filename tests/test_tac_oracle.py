"""Pins of the TAC oracle (oracle/tac_oracle.c) on the CPU: every known
answer of the reference's own phase tests (src/tac/tac.zig:846-1130), the
clusterFlat invariants it tests (:1131-1306), and properties the mathematics
fixes (Welford against the two-pass variance, one centroid = the serial mean,
per-token fits through kmeans.fit, the thread grouping of wcss_total)."""
import numpy as np
import pytest

from oracle import binding as orc

OK, BUDGET_TOO_SMALL, BUDGET_TOO_LARGE, INVALID, EMPTY = 0, 21, 22, 23, 24


# ---- Phase 1 (tac.zig:846-880) ------------------------------------------------

def test_classify_boundaries_through_tail():
    # classifyToken(0/1/127/128/255/256/10000, 128, 256): E M M S S A A
    st, k, b = orc.tac_allocate_tail([0, 1, 127, 128, 255, 256, 10_000], 128, 256, 100)
    assert st == OK
    assert k.tolist() == [0, 1, 1, 2, 2, 0, 0]
    assert b == 100 - 6


def test_allocate_tail_small_thresholds():
    st, k, b = orc.tac_allocate_tail([0, 1, 2, 3, 4, 5, 6, 7], 3, 5, 50)
    assert (st, b) == (OK, 44)
    assert k.tolist() == [0, 1, 1, 2, 2, 0, 0, 0]


def test_allocate_tail_errors():
    assert orc.tac_allocate_tail([1, 1, 4], 3, 5, 3)[0] == BUDGET_TOO_SMALL
    for mu, tau in ((5, 5), (6, 5), (0, 5)):
        assert orc.tac_allocate_tail([1], mu, tau, 10)[0] == INVALID


# ---- Phase 2 (tac.zig:882-945) ------------------------------------------------

def test_damped_phase2_sqrt_n_split():
    st, k, frac = orc.tac_damped_phase2([9, 16], [2.0, 2.0], [0, 0], 70, 3, 5)
    assert st == OK and k.tolist() == [30, 40]
    assert np.allclose(frac, 0.0, atol=1e-3)


def test_damped_phase2_spread_dominates():
    st, k, _ = orc.tac_damped_phase2([25, 25], [1.0, 4.0], [0, 0], 100, 3, 5)
    assert st == OK and k.tolist() == [20, 80]


def test_damped_phase2_zero_spread_uniform():
    st, k, _ = orc.tac_damped_phase2([10, 10, 10], [0.0, 0.0, 0.0], [0, 0, 0], 11, 3, 5)
    assert st == OK and k.tolist() == [4, 4, 3]


def test_damped_phase2_fractional_remainder():
    st, k, frac = orc.tac_damped_phase2([9, 16], [1.0, 1.0], [0, 0], 10, 3, 5)
    assert st == OK and k.tolist() == [4, 5]
    assert abs(frac[0] - 0.2857) < 1e-3 and abs(frac[1] - 0.7143) < 1e-3
    # the exact values: f32 of 30/7 - 4 and 40/7 - 5 computed in f64
    assert frac[0] == np.float32(3.0 / 7.0 * 10.0 - 4.0)
    assert frac[1] == np.float32(4.0 / 7.0 * 10.0 - 5.0)


def test_damped_phase2_rejects_bad_weights():
    assert orc.tac_damped_phase2([300], [np.nan], [0], 10, 3, 5)[0] == INVALID
    assert orc.tac_damped_phase2([300], [-1.0], [0], 10, 3, 5)[0] == INVALID


# ---- Phase 3 (tac.zig:947-980) ------------------------------------------------

def test_bound_phase3_cases():
    assert orc.tac_bound_phase3([200], [1], 128, 156, 4, 39)[1].tolist() == [4]
    assert orc.tac_bound_phase3([156], [10], 128, 156, 4, 39)[1].tolist() == [4]
    st, k = orc.tac_bound_phase3([50, 200, 500], [1, 2, 1], 128, 256, 4, 39)
    assert st == OK and k.tolist() == [1, 2, 4]
    assert orc.tac_bound_phase3([100], [0], 50, 100, 4, 39)[0] == INVALID


# ---- Phase 4 (tac.zig:982-1039) -----------------------------------------------

def test_reconcile_surplus_largest_remainder():
    st, k = orc.tac_reconcile_phase4([10_000, 10_000], [4, 5], [0.3, 0.8], 12, 3, 5, 4, 39)
    assert st == OK and k.tolist() == [4, 8]


def test_reconcile_deficit_smallest_remainder():
    st, k = orc.tac_reconcile_phase4([10_000, 10_000], [10, 8], [0.1, 0.6], 14, 3, 5, 4, 39)
    assert st == OK and k.tolist() == [6, 8]


def test_reconcile_deficit_walks_to_next_token():
    st, k = orc.tac_reconcile_phase4([10_000, 10_000], [10, 5], [0.0, 0.9], 8, 3, 5, 4, 39)
    assert st == OK and k.tolist() == [4, 4]


def test_reconcile_surplus_without_room():
    assert orc.tac_reconcile_phase4([156], [4], [0.5], 10, 128, 156, 4, 39)[0] == BUDGET_TOO_LARGE


def test_reconcile_deficit_degrades_small_then_micro():
    st, k = orc.tac_reconcile_phase4([200, 10_000], [2, 4], [0.0, 0.0], 5, 128, 256, 4, 39)
    assert st == OK and k.tolist() == [1, 4]
    # one step further: the small token is at 1, the micro token drops to 0
    st, k = orc.tac_reconcile_phase4([50, 200, 10_000], [1, 1, 4], [0, 0, 0], 5, 128, 256, 4, 39)
    assert st == OK and k.tolist() == [0, 1, 4]
    assert orc.tac_reconcile_phase4([10_000], [4], [0.0], 3, 128, 256, 4, 39)[0] == BUDGET_TOO_SMALL


# ---- allocateBudgets (tac.zig:1041-1129) --------------------------------------

def test_allocate_budgets_small_vocab():
    p = orc.tac_params(18, 0, mu=3, tau=5, epsilon=4, theta=1)
    st, k, _ = orc.tac_allocate_budgets([0, 2, 4, 20, 20, 20], [0, 0, 0, 1.0, 2.0, 3.0], p)
    assert st == OK and k.tolist() == [0, 1, 2, 4, 4, 7]


def test_allocate_budgets_paper_defaults():
    p = orc.tac_params(100, 0)
    st, k, _ = orc.tac_allocate_budgets([50, 200, 5000, 5000], [0, 0, 1.0, 2.0], p)
    assert st == OK and k.sum() == 100
    assert k[0] == 1 and k[1] == 2
    assert 4 <= k[2] <= 128 and 4 <= k[3] <= 128 and k[3] >= k[2]


def test_allocate_budgets_deterministic():
    p = orc.tac_params(50, 999)
    a = orc.tac_allocate_budgets([0, 100, 250, 1000, 5000], [0, 0, 0, 0.7, 2.3], p)
    b = orc.tac_allocate_budgets([0, 100, 250, 1000, 5000], [0, 0, 0, 0.7, 2.3], p)
    assert a[0] == b[0] == OK and a[1].tolist() == b[1].tolist()


# ---- Welford spreads (tac.zig:604-638) ----------------------------------------

def _groups(ids):
    ids = np.asarray(ids, np.uint32)
    nd = int(ids.max()) + 1
    freqs = np.bincount(ids, minlength=nd).astype(np.uint32)
    offs = np.concatenate([[0], np.cumsum(freqs)]).astype(np.uint32)
    idx = np.argsort(ids, kind="stable").astype(np.uint32)
    return freqs, offs, idx


def test_spreads_closed_forms():
    # 1-D {0, 2}: mean 1, M2 = 2, spread 1.  2-D {(1,0),(3,0),(5,0)}: M2 = 8, spread 8/3.
    v = np.array([0.0, 2.0], np.float32)
    _, offs, idx = _groups([0, 0])
    assert orc.tac_spreads(v, 1, offs, idx)[0] == np.float32(1.0)
    v = np.array([1, 0, 3, 0, 5, 0], np.float32)
    _, offs, idx = _groups([0, 0, 0])
    assert orc.tac_spreads(v, 2, offs, idx)[0] == np.float32(8.0) / np.float32(3.0)


def test_spreads_match_two_pass_variance():
    rng = np.random.default_rng(3)
    ids = rng.integers(0, 40, 5000)
    ids[:40] = np.arange(40)
    v = (rng.standard_normal((5000, 16)) * rng.uniform(0.1, 3, (5000, 1))).astype(np.float32)
    freqs, offs, idx = _groups(ids)
    s = orc.tac_spreads(v, 16, offs, idx)
    for j in range(40):
        rows = v[ids == j].astype(np.float64)
        want = ((rows - rows.mean(0)) ** 2).sum() / len(rows)
        assert abs(s[j] - want) <= 1e-4 * max(want, 1e-6)


# ---- clusterFlat (tac.zig:1131-1306) ------------------------------------------

def _themes(counts, themes, sigma, seed):
    rng = np.random.default_rng(seed)
    ids, vec = [], []
    for tid, (c, t) in enumerate(zip(counts, themes)):
        for _ in range(c):
            ids.append(tid)
            vec.append(np.asarray(t, np.float32) + rng.standard_normal(len(t)).astype(np.float32) * sigma)
    return np.array(ids, np.uint32), np.array(vec, np.float32)


def test_cluster_flat_tiny_corpus_invariants():
    ids, v = _themes([10, 10, 6, 4], [(1, 0), (0, 1), (-1, 0), (0, -1)], 0.05, 7)
    p = orc.tac_params(14, 42, mu=3, tau=5, epsilon=1, theta=1)
    r = orc.tac_cluster_flat(ids, v, 2, p)
    assert r.status == OK
    assert r.kappa_per_token.sum() == 14 and r.kappa_per_token[3] == 2
    assert np.all(r.assignments < 14) and r.assignments.size == 30
    assert np.isfinite(r.wcss_total) and r.wcss_total >= 0


def test_cluster_flat_deterministic():
    rng = np.random.default_rng(1)
    ids = (np.arange(40) % 5).astype(np.uint32)
    v = rng.standard_normal((40, 3)).astype(np.float32)
    p = orc.tac_params(18, 12345, mu=3, tau=5, epsilon=1, theta=1)
    a, b = orc.tac_cluster_flat(ids, v, 3, p), orc.tac_cluster_flat(ids, v, 3, p)
    assert a.status == b.status == OK
    assert a.centroids.tobytes() == b.centroids.tobytes()
    assert np.array_equal(a.assignments, b.assignments)
    assert np.array_equal(a.kappa_per_token, b.kappa_per_token) and a.wcss_total == b.wcss_total


def test_cluster_flat_token_zero_absent():
    ids = np.array([1, 1, 1, 1, 2, 2, 2, 2, 3, 3, 3, 3], np.uint32)
    v = np.arange(1, 13, dtype=np.float32) / 10
    r = orc.tac_cluster_flat(ids, v, 1, orc.tac_params(6, 0, mu=3, tau=5, epsilon=1, theta=1))
    assert r.status == OK and r.kappa_per_token.tolist() == [0, 2, 2, 2]


def test_cluster_flat_errors():
    assert orc.tac_cluster_flat([], np.zeros(0, np.float32), 2, orc.tac_params(1, 0)).status \
        == EMPTY
    assert orc.tac_cluster_flat([0, 0], [1, 0, 0, 1], 2, orc.tac_params(0, 0)).status \
        == BUDGET_TOO_SMALL
    assert orc.tac_cluster_flat([0, 0, 0], [1, 0, 0, 1], 2, orc.tac_params(4, 0)).status == INVALID
    assert orc.tac_cluster_flat([0, 0], [1, 0, 0, 1], 0, orc.tac_params(4, 0)).status == INVALID


def test_cluster_flat_one_centroid_per_theme_is_the_serial_mean():
    themes = [(10, 0), (0, 10), (-10, 0)]
    ids, v = _themes([6, 6, 6], themes, 0.05, 99)
    r = orc.tac_cluster_flat(ids, v, 2, orc.tac_params(3, 0, mu=2, tau=5, epsilon=1, theta=1))
    assert r.status == OK and r.kappa_per_token.tolist() == [1, 1, 1]
    assert np.array_equal(r.assignments, ids)
    for j, t in enumerate(themes):
        rows = v[ids == j]
        s = np.zeros(2, np.float32)
        for row in rows:  # serial fp32 fold, then * fl(1 / fl(n))
            s = (s + row).astype(np.float32)
        mean = (s * (np.float32(1.0) / np.float32(len(rows)))).astype(np.float32)
        assert r.centroids[2 * j: 2 * j + 2].tobytes() == mean.tobytes()
        assert np.allclose(mean, t, atol=0.1)


def test_cluster_flat_per_token_fits_and_thread_grouping():
    # Each token's centroids and assignments are kmeans.fit on its gathered
    # rows with seed ^ token id (tac.zig:487-497); wcss_total groups the
    # per-token wcss by thread slice (tac.zig:688-820).
    rng = np.random.default_rng(11)
    ids = rng.integers(0, 7, 900).astype(np.uint32)
    v = rng.standard_normal((900, 4)).astype(np.float32)
    base = dict(mu=20, tau=60, epsilon=2, theta=10)
    r1 = orc.tac_cluster_flat(ids, v, 4, orc.tac_params(30, 77, **base))
    assert r1.status == OK
    goff = np.concatenate([[0], np.cumsum(r1.kappa_per_token)]).astype(np.int64)
    wj = []
    for j in range(7):
        rows = v[ids == j]
        f = orc.kmeans_fit(rows, 4, int(r1.kappa_per_token[j]), seed=77 ^ j)
        assert f.status == OK
        assert r1.centroids[goff[j] * 4: goff[j + 1] * 4].tobytes() == f.centroids.tobytes()
        assert np.array_equal(r1.assignments[ids == j], goff[j] + f.assignments)
        wj.append(np.float32(f.wcss))
    serial = np.float32(0)
    for w in wj:
        serial = np.float32(serial + w)
    assert np.float32(r1.wcss_total) == serial
    r3 = orc.tac_cluster_flat(ids, v, 4, orc.tac_params(30, 77, n_threads=3, **base))
    chunk = (7 + 2) // 3
    parts = [np.float32(0)] * 3
    for j, w in enumerate(wj):
        parts[j // chunk] = np.float32(parts[j // chunk] + w)
    total = np.float32(0)
    for x in parts:
        total = np.float32(total + x)
    assert np.float32(r3.wcss_total) == total
    assert r3.centroids.tobytes() == r1.centroids.tobytes()
