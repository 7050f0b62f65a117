"""GPU parity: the HIP path against the CPU oracle, bit for bit.

Every comparison is on bytes (codes) or float bit patterns (codebooks); the
oracle restates src/index/pq.zig and src/tac/kmeans.zig.
"""
import numpy as np
import pytest

from oracle import binding as orc
from tac_gpu import device, errors, kmeans, pq, synth

NEVER = float("-inf")
pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).reshape(-1).view(np.uint32)


def _workload_rows(n, seed=0, zipf=0.0, sigma=0.15):
    w = synth.Workload("t", n, 64, 4096, zipf, sigma, 16, 256, 1, seed)
    return synth.residuals(w, n)


@pytest.mark.parametrize("m,ksub", [(16, 256), (32, 256), (8, 256), (64, 256), (16, 1024),
                                    (16, 3), (21, 17)])
def test_encode_matches_oracle(gpu, m, ksub):
    dim = 64 if m != 21 else 63
    n = 5003
    x = _workload_rows(n, seed=3)[:, :dim].copy() if dim == 64 else \
        np.random.default_rng(1).standard_normal((n, dim)).astype(np.float32) * 0.2
    cb = synth.gauss_codebooks(7, m, ksub, dim // m, 0.05).reshape(-1)
    p = pq.PQ(dim=dim, sub_dim=dim // m, codebooks=cb, m=m, ksub=ksub)
    got = p.encode_many(x)
    ref = orc.pq_encode(x, dim, m, ksub, cb, n_threads=8)
    assert got.dtype == ref.dtype
    assert np.array_equal(got, ref), f"{np.count_nonzero(got != ref)} codes differ"


@pytest.mark.parametrize("tol,kpp", [(NEVER, False), (1e-3, False), (1e-4, True)])
def test_train_two_streams_match_one(gpu, monkeypatch, tol, kpp):
    """The k-means++ seeding and the Lloyd loop run the two halves of the
    subspaces on two streams when m is even; one stream
    (TAC_GPU_TRAIN_STREAMS=1) gives the same bits, also when subspaces of
    either half converge at different iterations."""
    w, x, init = synth.workload("chunk-117k", n=60000)
    if kpp:
        init = None

    def run():
        return pq.train(x, w.dim, 0xa1b2c3d4 if kpp else 0, m=w.m, ksub=w.ksub, max_iters=12,
                        tol=tol, init_codebooks=init, trace=True)

    two = run()
    monkeypatch.setenv("TAC_GPU_TRAIN_STREAMS", "1")
    one = run()
    assert np.array_equal(_bits(two.stats.trace), _bits(one.stats.trace))
    assert np.array_equal(_bits(two.codebooks), _bits(one.codebooks))
    assert np.array_equal(two.stats.iters_run, one.stats.iters_run)
    assert np.array_equal(two.stats.empties, one.stats.empties)
    assert np.array_equal(_bits(two.stats.wcss), _bits(one.stats.wcss))
    if tol != NEVER:
        ref = orc.pq_train(x, w.dim, w.m, w.ksub, init=init, max_iters=12, tol=tol,
                           n_threads=16, seed=0xa1b2c3d4 if kpp else 0)
        assert np.array_equal(two.stats.iters_run, ref.iters_run)
        assert np.array_equal(_bits(two.codebooks), _bits(ref.codebooks))


def test_encode_ties_pick_lowest_index(gpu):
    # Codewords 5, 9 and 200 of every subspace are identical and nearest to
    # every vector: the reference keeps the first (strict <), i.e. 5.
    m, ksub, dim, n = 16, 256, 64, 777
    rng = np.random.default_rng(5)
    cb = (rng.standard_normal((m, ksub, 4)) * 3.0 + 10.0).astype(np.float32)
    x = (rng.standard_normal((n, dim)) * 0.01).astype(np.float32)
    for j in (5, 9, 200):
        cb[:, j, :] = 0.0
    got = pq.PQ(dim, 4, cb.reshape(-1), m, ksub).encode_many(x)
    assert np.all(got == 5)
    assert np.array_equal(got, orc.pq_encode(x, dim, m, ksub, cb))


@pytest.mark.parametrize("n", [1, 63, 257, 4097, 16385])
def test_encode_ragged_sizes(gpu, n):
    x = _workload_rows(n, seed=11)
    cb = synth.gauss_codebooks(2, 16, 256, 4, 0.05)
    got = pq.PQ(64, 4, cb.reshape(-1), 16, 256).encode_many(x)
    assert np.array_equal(got, orc.pq_encode(x, 64, 16, 256, cb))


def test_train_chunk_matches_oracle_every_iteration(gpu):
    """Full small-chunk workload: 117,645 x 64, m16 k256, 20 Lloyd iterations,
    seeded-shuffle init; codebooks bit-exact after every iteration, codes
    bit-exact."""
    w, x, init = synth.workload("chunk-117k")
    got = pq.train(x, w.dim, 0, m=w.m, ksub=w.ksub, max_iters=w.iters, tol=NEVER,
                   init_codebooks=init, trace=True)
    ref = orc.pq_train(x, w.dim, w.m, w.ksub, init=init, max_iters=w.iters, tol=NEVER,
                       n_threads=16, trace=True)
    assert ref.status == 0
    for t in range(w.iters):
        diff = np.count_nonzero(_bits(got.stats.trace[t]) != _bits(ref.trace[t]))
        assert diff == 0, f"iteration {t}: {diff} codebook floats differ"
    assert np.array_equal(_bits(got.codebooks), _bits(ref.codebooks))
    assert np.array_equal(got.stats.iters_run, ref.iters_run)
    assert np.array_equal(got.stats.empties, ref.empties)
    codes = got.encode_many(x)
    assert np.array_equal(codes, orc.pq_encode(x, w.dim, w.m, w.ksub, ref.codebooks, n_threads=16))


@pytest.mark.parametrize("m,ksub,n", [(32, 256, 20000), (8, 256, 20000), (16, 1024, 30000),
                                      (64, 16, 3000), (16, 256, 257)])
def test_train_shapes_match_oracle(gpu, m, ksub, n):
    x = _workload_rows(n, seed=9, zipf=1.1)
    init = synth.shuffle_init(x, m, ksub, 4)
    got = pq.train(x, 64, 0, m=m, ksub=ksub, max_iters=6, tol=NEVER, init_codebooks=init)
    ref = orc.pq_train(x, 64, m, ksub, init=init, max_iters=6, tol=NEVER, n_threads=16)
    assert np.array_equal(_bits(got.codebooks), _bits(ref.codebooks))


def test_train_early_break_matches_oracle(gpu):
    # Default tol = 1e-4: subspaces stop at different iterations.
    x = _workload_rows(20000, seed=21)
    init = synth.shuffle_init(x, 16, 64, 8)
    got = pq.train(x, 64, 0, m=16, ksub=64, max_iters=25, tol=1e-4, init_codebooks=init)
    ref = orc.pq_train(x, 64, 16, 64, init=init, max_iters=25, tol=1e-4, n_threads=16)
    assert np.array_equal(got.stats.iters_run, ref.iters_run)
    assert np.array_equal(_bits(got.stats.wcss), _bits(ref.wcss))
    assert np.array_equal(_bits(got.codebooks), _bits(ref.codebooks))


def test_train_forced_empty_clusters(gpu):
    # Many init codewords sit on top of each other: most clusters empty in
    # iteration 0 and get reseeded from the farthest points.
    x = _workload_rows(5000, seed=4)
    init = np.repeat(x[:4].reshape(4, 16, 4).transpose(1, 0, 2), 64, axis=1).copy()  # [16][256][4]
    got = pq.train(x, 64, 0, m=16, ksub=256, max_iters=5, tol=NEVER, init_codebooks=init)
    ref = orc.pq_train(x, 64, 16, 256, init=init, max_iters=5, tol=NEVER, n_threads=16)
    assert ref.empties.sum() > 0
    assert np.array_equal(got.stats.empties, ref.empties)
    assert np.array_equal(_bits(got.codebooks), _bits(ref.codebooks))


def _same_floats(a, b):
    """Bit equality, with any NaN equal to any NaN (payloads are not compared)."""
    a = np.ascontiguousarray(a, dtype=np.float32).reshape(-1)
    b = np.ascontiguousarray(b, dtype=np.float32).reshape(-1)
    na, nb = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32),
                                                          b[~nb].view(np.uint32)))


@pytest.mark.parametrize("n", [5000, 40000])
def test_train_reseed_skips_nan_distances(gpu, n):
    # vec.argmax (src/util/vec.zig:285-299) starts from values[0] and moves on a
    # strict >, so a NaN distance past index 0 never wins the empty-cluster
    # reseed (src/tac/kmeans.zig:199-211).  Row 5 carries a NaN in subspace 3
    # (its distance there is NaN) and row 1029, far from everything, holds the
    # largest distance: it must seed the first empty cluster of every
    # subspace, subspace 3 included.  Later iterations then run with the NaN
    # codeword that row 5's cluster sum produces.
    x = _workload_rows(n, seed=4)
    x[5, 12:16] = np.nan
    x[1029] = 50.0
    init = np.repeat(x[:4].reshape(4, 16, 4).transpose(1, 0, 2), 64, axis=1).copy()
    for iters in (1, 3):
        got = pq.train(x, 64, 0, m=16, ksub=256, max_iters=iters, tol=NEVER,
                       init_codebooks=init)
        ref = orc.pq_train(x, 64, 16, 256, init=init, max_iters=iters, tol=NEVER, n_threads=16)
        assert ref.status == 0
        if iters == 1:
            # every subspace reseeds its first empty cluster (index 1) from row 1029
            assert np.all(ref.codebooks.reshape(16, 256, 4)[:, 1, :] == 50.0)
        assert np.array_equal(got.stats.empties, ref.empties)
        assert _same_floats(got.codebooks, ref.codebooks), f"{iters} iterations"


def test_train_degenerate_k_ge_n(gpu):
    x = _workload_rows(200, seed=2)
    got = pq.train(x, 64, 0, m=16, ksub=256, init_codebooks=None)
    ref = orc.pq_train(x, 64, 16, 256, init=None)
    assert np.array_equal(_bits(got.codebooks), _bits(ref.codebooks))
    assert np.all(got.stats.iters_run == 0)


def test_kmeans_fit_matches_oracle(gpu):
    rng = np.random.default_rng(0xDE7E2)
    v = rng.standard_normal(600 * 4).astype(np.float32)
    init = v[: 32 * 4].copy()
    got = kmeans.fit(v, 4, 32, max_iters=25, init_centroids=init)
    ref = orc.kmeans_fit(v, 4, 32, max_iters=25, init=init)
    assert got.iters_run == ref.iters_run
    assert np.array_equal(got.assignments, ref.assignments)
    assert np.array_equal(_bits(got.centroids), _bits(ref.centroids))
    assert np.float32(got.wcss).view(np.uint32) == np.float32(ref.wcss).view(np.uint32)


@pytest.mark.parametrize("dim,k,n,init", [(9, 12, 3000, False), (16, 40, 5000, True),
                                          (33, 17, 4000, False), (64, 50, 6000, False),
                                          (64, 30, 4000, True), (128, 9, 2500, False),
                                          (100, 3000, 2000, False), (512, 5, 700, True)])
def test_kmeans_fit_wide_rows(gpu, dim, k, n, init):
    """kmeans.fit past dim 8 (the token-clustering engine as one problem):
    vec.l2sq's 4-lane form at 64 and 128 and its generic form otherwise,
    k-means++ from `seed` or caller centroids, tol 1e-4 (the reference's
    default, so wcss decides the stop), and k >= n (the degenerate branch,
    kmeans.zig:88-104).  Centroids, assignments, wcss and iterations equal
    the oracle's bit for bit."""
    rng = np.random.default_rng(dim * 1000 + k)
    centres = rng.standard_normal((7, dim)).astype(np.float32)
    v = (centres[rng.integers(0, 7, n)] + 0.3 * rng.standard_normal((n, dim))).astype(np.float32)
    ini = v[rng.permutation(n)[:k]].copy() if init and k < n else None
    got = kmeans.fit(v, dim, k, seed=77, max_iters=25, tol=1e-4, init_centroids=ini)
    ref = orc.kmeans_fit(v, dim, k, max_iters=25, tol=1e-4, seed=77, init=ini)
    assert ref.status == 0
    assert got.iters_run == ref.iters_run
    assert np.array_equal(got.assignments, ref.assignments)
    assert np.array_equal(_bits(got.centroids), _bits(ref.centroids))
    assert np.float32(got.wcss).view(np.uint32) == np.float32(ref.wcss).view(np.uint32)


@pytest.mark.parametrize("case", ["tol", "one_stream", "k1024", "m8", "small_one_iter",
                                  "degenerate", "zero_iters"])
def test_train_encode_entry(gpu, monkeypatch, case):
    """tac_pq_train_encode_device: its codebooks equal tac_pq_train_device's
    and its codes tac_pq_encode_device's on those codebooks, and both equal
    the oracle: with tol 1e-3 (subspaces that stop early still encode), on
    one stream, with u16 codes, at dsub 8, and on the shapes that take the
    ordinary encode (one iteration of fewer than 16,384 vectors, n <= ksub,
    no iteration)."""
    m, ksub, n, iters, tol = 16, 256, 40_000, 8, NEVER
    if case == "tol":
        tol = 1e-3
    if case == "one_stream":
        monkeypatch.setenv("TAC_GPU_TRAIN_STREAMS", "1")
    if case == "k1024":
        ksub = 1024
    if case == "m8":
        m = 8
    if case == "small_one_iter":
        n, iters = 9000, 1
    if case == "degenerate":
        n = 200
    if case == "zero_iters":
        iters = 0
    x = _workload_rows(n, seed=5)
    init = synth.shuffle_init(x, m, ksub, 3) if ksub <= n else None
    dx = device.DeviceArray.from_host(x)
    dinit = device.DeviceArray.from_host(init) if init is not None else None
    dcb = device.DeviceArray((m, ksub, 64 // m), np.float32)
    dcodes = device.DeviceArray((n, m), pq.code_dtype(ksub))
    st = device.train_encode_device(dx, n, 64, m, ksub, dinit, dcb, dcodes, iters, tol, seed=11)
    cb, codes = dcb.to_host(), dcodes.to_host()
    # the separate entry points on the same input
    dcb2 = device.DeviceArray((m, ksub, 64 // m), np.float32)
    dcodes2 = device.DeviceArray((n, m), pq.code_dtype(ksub))
    st2 = device.train_device(dx, n, 64, m, ksub, dinit, dcb2, iters, tol, stats=True, seed=11)
    device.encode_device(dx, n, 64, m, ksub, dcb2, dcodes2)
    assert np.array_equal(_bits(cb), _bits(dcb2.to_host()))
    assert np.array_equal(codes, dcodes2.to_host())
    assert np.array_equal(st[0], st2[0]) and np.array_equal(_bits(st[1]), _bits(st2[1]))
    for a in (dx, dinit, dcb, dcodes, dcb2, dcodes2):
        if a is not None:
            a.free()
    ref = orc.pq_train(x, 64, m, ksub, init=init, seed=11, max_iters=iters, tol=tol, n_threads=8)
    assert ref.status == 0
    assert np.array_equal(_bits(cb), _bits(ref.codebooks))
    assert np.array_equal(codes, orc.pq_encode(x, 64, m, ksub, ref.codebooks, n_threads=8))


def test_device_resident_train_then_encode(gpu):
    w, x, init = synth.workload("chunk-117k", n=40000)
    dx = device.DeviceArray.from_host(x)
    dinit = device.DeviceArray.from_host(init)
    dcb = device.DeviceArray(init.shape, np.float32)
    dcodes = device.DeviceArray((x.shape[0], w.m), np.uint8)
    device.train_device(dx, x.shape[0], 64, w.m, w.ksub, dinit, dcb, 4, NEVER)
    device.encode_device(dx, x.shape[0], 64, w.m, w.ksub, dcb, dcodes)
    cb = dcb.to_host()
    ref = orc.pq_train(x, 64, w.m, w.ksub, init=init, max_iters=4, tol=NEVER, n_threads=16)
    assert np.array_equal(_bits(cb), _bits(ref.codebooks))
    assert np.array_equal(dcodes.to_host(), orc.pq_encode(x, 64, w.m, w.ksub, ref.codebooks, 16))


def test_argument_errors_on_device_path(gpu):
    with pytest.raises(errors.DimNotDivisibleByM):
        pq.train(np.zeros(33, np.float32), 33, 1)
    with pytest.raises(errors.EmptyCorpus):
        pq.train(np.zeros(0, np.float32), 32, 1)
    with pytest.raises(errors.AllZero):  # k-means++ on identical points (rng.zig:65)
        pq.train(np.zeros((300, 32), np.float32), 32, 1)


# ---- the pruned exact search against the exhaustive reference scan --------

def _encode_both(x, cb, m, ksub):
    dim = x.shape[1]
    got = pq.PQ(dim, dim // m, np.ascontiguousarray(cb, np.float32).reshape(-1), m,
                ksub).encode_many(x)
    return got, orc.pq_encode(x, dim, m, ksub, cb)


def test_pruned_search_near_ties_across_blocks(gpu):
    # Codewords 3 and 200 (different blocks of 8) sit symmetrically around
    # every vector's sub-vector, so their distances tie in exact arithmetic
    # and differ by at most rounding; codeword 77 is a few ulps farther.
    rng = np.random.default_rng(31)
    n, m, ksub = 4096, 16, 256
    x = (rng.standard_normal((n, 64)) * 0.2).astype(np.float32)
    cb = (rng.standard_normal((m, ksub, 4)) * 0.2 + 3.0).astype(np.float32)
    delta = np.float32(1e-3)
    for mm in range(m):
        centre = x[0, 4 * mm:4 * mm + 4]
        cb[mm, 3] = centre + delta
        cb[mm, 200] = centre - delta
        cb[mm, 77] = centre + delta * np.float32(1.0000005)
    x[:] = x[0]  # every vector equals the one the ties were built around
    x += (rng.integers(-2, 3, x.shape) * np.float32(1e-9)).astype(np.float32)
    got, ref = _encode_both(x, cb, m, ksub)
    assert np.array_equal(got, ref)


def test_pruned_search_duplicate_codewords_across_blocks(gpu):
    rng = np.random.default_rng(32)
    x = (rng.standard_normal((3000, 64)) * 0.2).astype(np.float32)
    cb = (rng.standard_normal((16, 256, 4)) * 0.2).astype(np.float32)
    cb[:, 8 * np.arange(32) + 5] = cb[:, 5:6]  # one codeword repeated in every block
    got, ref = _encode_both(x, cb, 16, 256)
    assert np.array_equal(got, ref)


def test_pruned_search_wide_bounds(gpu):
    # A few far-away codewords make cmax large, so the gap test is loose and
    # many searches fall back to the full scan; results must not change.
    rng = np.random.default_rng(33)
    x = (rng.standard_normal((5000, 64)) * 0.2).astype(np.float32)
    cb = (rng.standard_normal((16, 256, 4)) * 0.2).astype(np.float32)
    cb[:, 255] = 1e6
    got, ref = _encode_both(x, cb, 16, 256)
    assert np.array_equal(got, ref)


def test_pruned_search_non_finite_values(gpu):
    rng = np.random.default_rng(34)
    x = (rng.standard_normal((700, 64)) * 0.2).astype(np.float32)
    cb = (rng.standard_normal((16, 64, 4)) * 0.2).astype(np.float32)
    cb[0, 0, 0] = np.nan          # NaN codeword first: never wins under strict <
    cb[1, 10, 2] = np.inf
    cb[2, :, :] = np.float32(3e38)  # squared norms overflow
    x[5, 0:4] = np.nan
    x[6, 4:8] = np.inf
    x[7, :] = np.float32(2e38)
    got, ref = _encode_both(x, cb, 16, 64)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("ksub", [1, 2, 7, 8, 9, 100])
def test_pruned_search_small_and_ragged_ksub(gpu, ksub):
    x = _workload_rows(3001, seed=ksub)
    cb = synth.gauss_codebooks(ksub, 16, ksub, 4, 0.1)
    got, ref = _encode_both(x, cb, 16, ksub)
    assert np.array_equal(got, ref)


def test_train_with_duplicate_init_codewords_across_blocks(gpu):
    # Lloyd assignment with exact ties spanning codeword blocks in every
    # iteration's first pass.
    x = _workload_rows(20000, seed=35, zipf=1.1)
    init = synth.shuffle_init(x, 16, 256, 3)
    init[:, 8 * np.arange(32) + 1] = init[:, 1:2]
    got = pq.train(x, 64, 0, m=16, ksub=256, max_iters=4, tol=NEVER, init_codebooks=init)
    ref = orc.pq_train(x, 64, 16, 256, init=init, max_iters=4, tol=NEVER, n_threads=16)
    assert np.array_equal(got.stats.empties, ref.empties)
    assert np.array_equal(_bits(got.codebooks), _bits(ref.codebooks))


def test_cpp_mirror_round_trip_on_gpu(gpu):
    import subprocess
    from pathlib import Path
    exe = Path(__file__).resolve().parent.parent / "ir-multivector-retrieval_amd" / "lib" / \
        "host_mirror_check"
    r = subprocess.run([str(exe), "gpu"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr


# ---- k-means++ seeding (src/tac/kmeans.zig:106-136) ------------------------

@pytest.mark.parametrize("m,ksub,n,seed", [(16, 256, 20000, 0xa1b2c3d4), (32, 64, 3000, 7),
                                           (8, 256, 5000, 123)])
def test_kmeanspp_train_matches_oracle(gpu, m, ksub, n, seed):
    # The drop-in pq.train path: no initial codebooks, reference iteration
    # control (25 iterations, tol 1e-4).
    x = _workload_rows(n, seed=seed % 97, zipf=1.1)
    got = pq.train(x, 64, seed, m=m, ksub=ksub)
    ref = orc.pq_train(x, 64, m, ksub, seed=seed, n_threads=16)
    assert ref.status == 0
    assert np.array_equal(got.stats.iters_run, ref.iters_run)
    assert np.array_equal(_bits(got.codebooks), _bits(ref.codebooks))


@pytest.mark.parametrize("m,ksub,n,seed,dups", [(16, 256, 20000, 0xa1b2c3d4, False),
                                                (8, 64, 777, 5, False),
                                                (8, 128, 150_001, 9, False),
                                                (16, 64, 6000, 31, True)])
def test_kmeanspp_exact_evaluation_every_draw(gpu, monkeypatch, m, ksub, n, seed, dups):
    # TAC_GPU_KPP_EXACT=1 sends every draw through the exact chunked
    # evaluation of weightedSample (rng.zig:60-81) instead of only the
    # inconclusive ones; the picks must not change.  `dups` repeats rows so
    # that many weights are exactly zero.
    x = _workload_rows(n, seed=seed % 89)
    if dups:
        x = x[np.random.default_rng(seed).integers(0, 400, n)]
    monkeypatch.setenv("TAC_GPU_KPP_EXACT", "1")
    got = pq.train(x, 64, seed, m=m, ksub=ksub, max_iters=2, tol=NEVER)
    ref = orc.pq_train(x, 64, m, ksub, seed=seed, max_iters=2, tol=NEVER, n_threads=16)
    assert ref.status == 0
    assert np.array_equal(_bits(got.codebooks), _bits(ref.codebooks))


def test_kmeanspp_first_iteration_is_the_seed_plus_one_update(gpu):
    x = _workload_rows(8000, seed=5)
    got = pq.train(x, 64, 99, m=16, ksub=128, max_iters=1, tol=NEVER, trace=True)
    ref = orc.pq_train(x, 64, 16, 128, seed=99, max_iters=1, tol=NEVER, trace=True)
    assert np.array_equal(_bits(got.stats.trace[0]), _bits(ref.trace[0]))


def test_kmeanspp_all_zero_weights(gpu):
    # 300 identical points, k = 256: after the first pick every weight is 0
    # and weightedSample fails with AllZero (src/util/rng.zig:65).
    x = np.tile(np.linspace(-1, 1, 64, dtype=np.float32), (300, 1))
    assert orc.pq_train(x, 64, 16, 256, seed=1).status == 10
    with pytest.raises(errors.AllZero):
        pq.train(x, 64, 1, m=16, ksub=256)


def test_kmeanspp_non_finite_weights(gpu):
    # distances that overflow to +inf make weightedSample fail with NonFinite
    x = _workload_rows(600, seed=8)
    x[17] = 3e38
    assert orc.pq_train(x, 64, 16, 256, seed=3).status == 9
    with pytest.raises(errors.NonFinite):
        pq.train(x, 64, 3, m=16, ksub=256)


@pytest.mark.parametrize("k,seed", [(3, 42), (4, 7), (5, 0), (32, 42)])
def test_kmeans_fit_kmeanspp_matches_oracle(gpu, k, seed):
    # The reference's own seeded fit cases (src/tac/kmeans.zig:409-501) run
    # end to end on the GPU and agree with the oracle bit for bit.
    rng = np.random.default_rng(seed + k)
    v = rng.standard_normal(600 * 2).astype(np.float32)
    got = kmeans.fit(v, 2, k, seed=seed, max_iters=50)
    ref = orc.kmeans_fit(v, 2, k, seed=seed, max_iters=50)
    assert got.iters_run == ref.iters_run
    assert np.array_equal(got.assignments, ref.assignments)
    assert np.array_equal(_bits(got.centroids), _bits(ref.centroids))


@pytest.mark.timeout(300)
def test_cluster_past_2_pow_24_members(gpu):
    """One cluster of about 16.9M members (more than 2^24): its centroid is
    sum * fl(1.0 / fl(count)) with fl(count) rounded (src/tac/kmeans.zig:194),
    and its fp32 sum is a serial fold of 16.9M terms in ascending row order
    (kmeans.zig:177-184) whose running value passes 2^23, where a float's
    spacing exceeds the terms' scale and any other order rounds differently.
    dim 4, m 1, ksub 4, three blobs of 33,334 rows beside the big one,
    rows interleaved; 3 Lloyd iterations with every codebook and wcss
    compared with the oracle bit for bit."""
    rng = np.random.default_rng(24)
    big, small = 16_900_001, 33_334
    n = big + 3 * small
    centres = np.array([[0.5, 0.25, 0.75, 1.5], [-3, 0, 0, 0], [0, -3, 0, 0], [0, 0, -3, 0]],
                       np.float32)
    blob = np.concatenate([np.zeros(big, np.int64), np.repeat([1, 2, 3], small)])
    blob = blob[rng.permutation(n)]
    x = (centres[blob] + rng.standard_normal((n, 4), dtype=np.float32) * np.float32(0.01))
    x = x.astype(np.float32)
    init = np.stack([x[np.nonzero(blob == b)[0][0]] for b in range(4)])[None].astype(np.float32)
    got = pq.train(x, 4, 0, m=1, ksub=4, max_iters=3, tol=NEVER, init_codebooks=init,
                   trace=True)
    ref = orc.pq_train(x, 4, 1, 4, init=init, max_iters=3, tol=NEVER, n_threads=16, trace=True)
    assert ref.status == 0
    codes = orc.pq_encode(x, 4, 1, 4, ref.trace[1], n_threads=16)
    counts = np.bincount(codes[:, 0], minlength=4)
    assert counts.max() > 2 ** 24 and int(np.float32(counts.max())) != counts.max()
    for t in range(3):
        assert np.array_equal(_bits(got.stats.trace[t]), _bits(ref.trace[t])), t
    assert np.array_equal(_bits(got.stats.wcss), _bits(ref.wcss))
    assert np.array_equal(_bits(got.codebooks), _bits(ref.codebooks))
