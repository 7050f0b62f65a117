"""GPU parity of the candidate-set Lloyd assignment and encode.

From the second iteration on, each vector is assigned by evaluating only the
codewords that can tie or beat its previous code under the reference
distance; the rest go to the pruned full search.  The first iteration (on
16,384 vectors or more) and encode anchor each vector at a grid cell's
codeword instead.  These tests train through
both paths on inputs built to stress the rule: exact duplicate points and
codewords (ties resolved by the first index), distances in the subnormal
range, large magnitudes, every sub-dimension 1-8 and K from 2 to 256, and
compare bit for bit with the oracle (src/tac/kmeans.zig:154-224 restated).
"""
import numpy as np
import pytest

from oracle import binding as orc
from tac_gpu import device, kmeans, pq, synth

NEVER = float("-inf")
pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _candidate_passes(monkeypatch):
    # By default the library keeps the candidate passes for dsub <= 4
    # (K <= 256); these tests exercise them at every dsub.  TAC_GPU_FULL_SEARCH=1 still wins where a test sets it.
    monkeypatch.setenv("TAC_GPU_CANDIDATES", "1")


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).reshape(-1).view(np.uint32)


def _train_both(x, dim, m, ksub, init, iters):
    got = pq.train(x, dim, 0, m=m, ksub=ksub, max_iters=iters, tol=NEVER, init_codebooks=init,
                   trace=True)
    ref = orc.pq_train(x, dim, m, ksub, init=init, max_iters=iters, tol=NEVER, n_threads=16,
                       trace=True)
    assert ref.status == 0
    for t in range(iters):
        diff = np.count_nonzero(_bits(got.stats.trace[t]) != _bits(ref.trace[t]))
        assert diff == 0, f"iteration {t}: {diff} codebook floats differ"
    assert np.array_equal(got.stats.empties, ref.empties)
    return got, ref


@pytest.mark.parametrize("dsub,ksub", [(1, 256), (2, 256), (3, 100), (4, 256), (5, 65),
                                       (6, 17), (7, 2), (8, 256), (4, 1024), (2, 512), (8, 1024),
                                       (1, 700), (3, 1000)])
def test_sub_dimensions_and_codebook_sizes(gpu, dsub, ksub):
    m = 4
    dim = m * dsub
    rng = np.random.default_rng(100 + dsub)
    x = (rng.standard_normal((9000, dim)) * 0.2).astype(np.float32)
    init = synth.shuffle_init(x, m, ksub, 5)
    _train_both(x, dim, m, ksub, init, 6)


@pytest.mark.parametrize("dsub,ksub", [(1, 256), (2, 200), (3, 100), (4, 256), (5, 65),
                                       (6, 17), (7, 2), (8, 256), (4, 1024), (2, 777), (8, 1024)])
def test_first_iteration_grid_anchors(gpu, dsub, ksub):
    # 20,000 vectors: iteration 0 takes the grid-anchored candidate pass.
    m = 2
    dim = m * dsub
    rng = np.random.default_rng(300 + dsub)
    x = (rng.standard_normal((20000, dim)) * 0.3).astype(np.float32)
    init = synth.shuffle_init(x, m, ksub, 9)
    _train_both(x, dim, m, ksub, init, 2)


def test_first_iteration_grid_ties_and_magnitudes(gpu):
    # Exact ties (vectors on duplicated codewords), subnormal and huge
    # distances, all through the grid-anchored first iteration.
    rng = np.random.default_rng(21)
    pts = (rng.standard_normal((300, 16)) * 0.3).astype(np.float32)
    x = pts[rng.integers(0, 300, 20000)]
    init = synth.shuffle_init(x, 4, 256, 3)
    init[:, 128:] = init[:, :128]
    _train_both(x, 16, 4, 256, init, 2)
    for scale in (1e-19, 1e15):
        xs = (rng.standard_normal((20000, 16)) * scale).astype(np.float32)
        _train_both(xs, 16, 4, 256, synth.shuffle_init(xs, 4, 256, 4), 2)


def test_duplicate_points_and_codewords(gpu):
    # 6,000 vectors drawn from 250 distinct points: every assignment has exact
    # ties, clusters empty out and get reseeded onto duplicates.
    rng = np.random.default_rng(7)
    pts = (rng.standard_normal((250, 16)) * 0.3).astype(np.float32)
    x = pts[rng.integers(0, 250, 6000)]
    init = synth.shuffle_init(x, 4, 256, 1)
    init[:, 128:] = init[:, :128]
    _, ref = _train_both(x, 16, 4, 256, init, 6)
    assert ref.empties.sum() > 0


@pytest.mark.parametrize("scale", [1e-19, 1e-12, 1e15])
def test_extreme_magnitudes(gpu, scale):
    # 1e-19: squared distances are subnormal, the candidate rows cannot
    # separate codewords and vectors go to the full search.  1e15: distances
    # near 1e30, inside the bound arithmetic's range.
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((5000, 16)) * scale).astype(np.float32)
    init = synth.shuffle_init(x, 4, 256, 2)
    _train_both(x, 16, 4, 256, init, 5)


def test_matches_full_search_on_the_chunk_workload(gpu, monkeypatch):
    # 117,645 x 64, m16 k256, 20 iterations: the default path (grid anchors
    # in iteration 0, previous codes from iteration 1) and
    # TAC_GPU_FULL_SEARCH=1 give the same bytes, and the candidate path
    # settles most vectors without the full search.
    w, x, init = synth.workload("chunk-117k")
    device.profile_enable(True)
    device.profile_read(reset=True)
    got = pq.train(x, w.dim, 0, m=w.m, ksub=w.ksub, max_iters=w.iters, tol=NEVER,
                   init_codebooks=init)
    prof = device.profile_read(reset=True)
    monkeypatch.setenv("TAC_GPU_FULL_SEARCH", "1")
    full = pq.train(x, w.dim, 0, m=w.m, ksub=w.ksub, max_iters=w.iters, tol=NEVER,
                    init_codebooks=init)
    prof_full = device.profile_read(reset=True)
    device.profile_enable(False)
    assert np.array_equal(_bits(got.codebooks), _bits(full.codebooks))
    assert prof.cand_vectors == w.iters * w.m * w.n
    assert 0 < prof.cand_deferred < 0.1 * prof.cand_vectors
    assert prof_full.cand_vectors == 0


def test_kmeans_fit_assignments(gpu):
    # M = 1 through kmeans.fit: assignments, wcss and iteration count.
    rng = np.random.default_rng(0x5EED)
    v = (rng.standard_normal((20000, 6)) * 0.5).astype(np.float32).reshape(-1)
    init = v[: 200 * 6].copy()
    got = kmeans.fit(v, 6, 200, max_iters=12, tol=1e-6, init_centroids=init)
    ref = orc.kmeans_fit(v, 6, 200, max_iters=12, tol=1e-6, init=init)
    assert got.iters_run == ref.iters_run
    assert np.array_equal(got.assignments, ref.assignments)
    assert np.array_equal(_bits(got.centroids), _bits(ref.centroids))
    assert np.float32(got.wcss).view(np.uint32) == np.float32(ref.wcss).view(np.uint32)


# ---- encode: anchors from a grid over the codebook's bounding box ----------

def _encode_both(x, cb, m, ksub):
    dim = x.shape[1]
    got = pq.PQ(dim, dim // m, np.ascontiguousarray(cb).reshape(-1), m, ksub).encode_many(x)
    ref = orc.pq_encode(x, dim, m, ksub, cb, n_threads=16)
    assert np.array_equal(got, ref), f"{np.count_nonzero(got != ref)} codes differ"
    return got


@pytest.mark.parametrize("dsub,ksub", [(1, 256), (2, 256), (3, 100), (4, 256), (5, 65),
                                       (6, 17), (7, 2), (8, 256), (4, 1024), (2, 512), (8, 1024),
                                       (3, 1000)])
def test_encode_sub_dimensions_and_codebook_sizes(gpu, dsub, ksub):
    m = 4
    rng = np.random.default_rng(200 + dsub)
    x = (rng.standard_normal((20000, m * dsub)) * 0.2).astype(np.float32)
    cb = (rng.standard_normal((m, ksub, dsub)) * 0.2).astype(np.float32)
    _encode_both(x, cb, m, ksub)


def test_encode_ties_outliers_and_non_finite(gpu):
    # Duplicate codewords (ties to the first index), vectors on codewords,
    # vectors far outside the codebook's box (clamped to edge cells) and
    # NaN / inf coordinates (PQ.encode keeps code 0 when every distance is
    # NaN).
    rng = np.random.default_rng(21)
    m, ksub, dsub = 8, 256, 4
    cb = (rng.standard_normal((m, ksub, dsub)) * 0.1).astype(np.float32)
    cb[:, 200:] = cb[:, 10:66]
    x = (rng.standard_normal((30000, m * dsub)) * 0.1).astype(np.float32)
    on = cb[np.arange(m)[None, :], rng.integers(0, ksub, (5000, m))].reshape(5000, m * dsub)
    x[:5000] = on
    x[5000:6000] *= 1e4
    x[6000, 3] = np.nan
    x[6001, :] = np.nan
    x[6002, 5] = np.inf
    x[6003, 7] = -np.inf
    _encode_both(x, cb, m, ksub)


@pytest.mark.parametrize("scale", [1e-19, 1e15])
def test_encode_extreme_magnitudes(gpu, scale):
    rng = np.random.default_rng(23)
    x = (rng.standard_normal((20000, 16)) * scale).astype(np.float32)
    cb = (rng.standard_normal((4, 256, 4)) * scale).astype(np.float32)
    _encode_both(x, cb, 4, 256)


def test_encode_non_finite_codeword(gpu):
    rng = np.random.default_rng(29)
    x = (rng.standard_normal((20000, 16)) * 0.3).astype(np.float32)
    cb = (rng.standard_normal((4, 256, 4)) * 0.3).astype(np.float32)
    cb[1, 17, 2] = np.nan
    cb[2, 99, 0] = np.inf
    _encode_both(x, cb, 4, 256)


def test_encode_matches_full_search_on_the_corpus(gpu, monkeypatch):
    w, x, init = synth.workload("corpus-1.52m", n=200000)
    p = pq.train(x, w.dim, 0, m=w.m, ksub=w.ksub, max_iters=3, tol=NEVER, init_codebooks=init)
    device.profile_enable(True)
    device.profile_read(reset=True)
    got = p.encode_many(x)
    prof = device.profile_read(reset=True)
    device.profile_enable(False)
    monkeypatch.setenv("TAC_GPU_FULL_SEARCH", "1")
    full = p.encode_many(x)
    assert np.array_equal(got, full)
    assert prof.cand_vectors == w.m * x.shape[0]
    assert 0 < prof.cand_deferred < 0.1 * prof.cand_vectors


def test_k1024_matches_full_search_on_the_corpus(gpu, monkeypatch):
    """m16 x k1024 on 200,000 corpus rows: 3 candidate iterations (the first
    from u16 grid anchors) and the candidate encode give the full search's
    codebooks and codes."""
    w = synth.WORKLOADS["corpus-1.52m-k1024"]
    x = synth.residuals(w, 200000)
    init = synth.shuffle_init(x, w.m, w.ksub, 0)
    device.profile_enable(True)
    device.profile_read(reset=True)
    p = pq.train(x, w.dim, 0, m=w.m, ksub=w.ksub, max_iters=3, tol=NEVER, init_codebooks=init)
    got = p.encode_many(x)
    prof = device.profile_read(reset=True)
    device.profile_enable(False)
    assert prof.cand_vectors > 0 and prof.cand_deferred < 0.2 * prof.cand_vectors
    monkeypatch.setenv("TAC_GPU_FULL_SEARCH", "1")
    q = pq.train(x, w.dim, 0, m=w.m, ksub=w.ksub, max_iters=3, tol=NEVER, init_codebooks=init)
    assert np.array_equal(_bits(p.codebooks), _bits(q.codebooks))
    assert got.dtype == np.uint16 and np.array_equal(got, q.encode_many(x))


@pytest.mark.parametrize("dsub,screen_off,train_cand,encode_cand",
                         [(4, False, True, True), (5, False, False, False),
                          (6, False, False, False), (8, False, False, False),
                          (5, True, True, False), (7, True, False, False)])
def test_default_pass_by_sub_dimension(gpu, monkeypatch, dsub, screen_off, train_cand,
                                       encode_cand):
    # Without the switch: the candidate passes where they are faster (up to
    # dsub 4, K <= 256), the full search through the matrix-core screen from
    # dsub 5 on; without the screen the Lloyd loop keeps the candidate passes
    # up to dsub 6 and the full search is the vector unit's.  The bytes are the
    # oracle's either way.
    monkeypatch.delenv("TAC_GPU_CANDIDATES")
    if screen_off:
        monkeypatch.setenv("TAC_GPU_SCREEN", "0")
    m, ksub, n = 2, 256, 20000
    dim = m * dsub
    rng = np.random.default_rng(600 + dsub)
    x = (rng.standard_normal((n, dim)) * 0.3).astype(np.float32)
    init = synth.shuffle_init(x, m, ksub, 3)
    device.profile_enable(True)
    device.profile_read(reset=True)
    got, _ = _train_both(x, dim, m, ksub, init, 3)
    prof_train = device.profile_read(reset=True)
    codes = got.encode_many(x)
    prof_enc = device.profile_read(reset=True)
    device.profile_enable(False)
    assert (prof_train.cand_vectors > 0) == train_cand
    assert (prof_enc.cand_vectors > 0) == encode_cand
    assert (prof_train.screen_vectors > 0) == (not train_cand and not screen_off)
    assert (prof_enc.screen_vectors > 0) == (not encode_cand and not screen_off)
    ref = orc.pq_encode(x, dim, m, ksub, got.codebooks, n_threads=16)
    assert np.array_equal(codes, ref)


@pytest.mark.parametrize("ksub", [256, 1024])
def test_deferred_search_lane_groups_match_one_lane(gpu, monkeypatch, ksub):
    """The deferred vectors' pruned full search with four lanes per vector
    (K >= 128) gives the one-lane search's codebooks and codes, on corpus rows
    whose candidate passes defer a few percent of the vector-subspaces."""
    w = synth.WORKLOADS["corpus-1.52m-k1024" if ksub == 1024 else "corpus-1.52m"]
    x = synth.residuals(w, 60000)
    init = synth.shuffle_init(x, w.m, w.ksub, 0)

    def run():
        device.profile_enable(True)
        device.profile_read(reset=True)
        p = pq.train(x, w.dim, 0, m=w.m, ksub=w.ksub, max_iters=3, tol=NEVER,
                     init_codebooks=init)
        codes = p.encode_many(x)
        prof = device.profile_read(reset=True)
        device.profile_enable(False)
        return p, codes, prof

    p4, c4, prof = run()
    assert prof.cand_deferred > 0
    monkeypatch.setenv("TAC_GPU_LIST_LANES", "1")
    p1, c1, _ = run()
    assert np.array_equal(_bits(p4.codebooks), _bits(p1.codebooks))
    assert np.array_equal(c4, c1)
