"""The reference's host-dependent generic vec path (src/util/vec.zig:16,
:90-103, :159-175: lane_count = std.simd.suggestVectorLength(f32), 16 on
AVX-512, 8 on AVX2, 4 on NEON) on the GPU at each lane count, bit for bit
against the oracle set to the same count: PQ at sub-dimension 8 (train,
encode, the no-allocation encode, the distance table), kmeans.fit and token
clustering at generic dims."""
import numpy as np
import pytest

from oracle import binding as orc
from tac_gpu import device, errors, kmeans, lib, pq, synth, tac

NEVER = float("-inf")
pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).reshape(-1).view(np.uint32)


@pytest.fixture
def lanes(request):
    n = request.param
    with device.lanes(n), orc.lane_count(n):
        yield n


def test_default_and_rejected_values(gpu):
    assert device.lane_count() == 16
    for bad in (0, 2, 12, 32):
        with pytest.raises(errors.InvalidArgument):
            device.set_lane_count(bad)
    assert device.lane_count() == 16


@pytest.mark.parametrize("lanes", [4, 8, 16], indirect=True)
def test_pq_dsub8_train_and_encode(gpu, lanes):
    """m8 over dim 64 (dsub 8): every iteration's codebook, the codes of
    the grid-anchored encode, of the train-then-encode entry and of the
    no-allocation encode, all against the oracle at the same lane count."""
    w = synth.Workload("t", 40_000, 64, 4096, 1.1, 0.15, 8, 256, 1, 3)
    x = synth.residuals(w, w.n)
    init = synth.shuffle_init(x, 8, 256, 5)
    got = pq.train(x, 64, 0, m=8, ksub=256, max_iters=6, tol=NEVER, init_codebooks=init,
                   trace=True)
    ref = orc.pq_train(x, 64, 8, 256, init=init, max_iters=6, tol=NEVER, n_threads=8,
                       trace=True)
    assert ref.status == 0
    for t in range(6):
        assert np.array_equal(_bits(got.stats.trace[t]), _bits(ref.trace[t])), t
    # wcss folds every vector's distance to its centroid: it sees the last
    # bit of each, so it tells the lane counts' orders apart
    assert np.array_equal(_bits(got.stats.wcss), _bits(ref.wcss))
    if lanes != 8:
        with orc.lane_count(4 if lanes == 16 else 16):
            other = orc.pq_train(x, 64, 8, 256, init=init, max_iters=6, tol=NEVER, n_threads=8)
        assert not np.array_equal(_bits(other.wcss), _bits(ref.wcss))
    ref_codes = orc.pq_encode(x, 64, 8, 256, ref.codebooks, n_threads=8)
    assert np.array_equal(got.encode_many(x), ref_codes)
    dx = device.DeviceArray.from_host(x)
    dinit = device.DeviceArray.from_host(init)
    dcb = device.DeviceArray(init.shape, np.float32)
    dcodes = device.DeviceArray((w.n, 8), np.uint8)
    device.train_encode_device(dx, w.n, 64, 8, 256, dinit, dcb, dcodes, 6, NEVER)
    assert np.array_equal(_bits(dcb.to_host()), _bits(ref.codebooks))
    assert np.array_equal(dcodes.to_host(), ref_codes)
    errors.check(lib.tac_pq_encode_device_noalloc(dx.ptr, w.n, 64, 8, 256, dcb.ptr, dcodes.ptr,
                                                  None))
    device.synchronize()
    assert np.array_equal(dcodes.to_host(), ref_codes)
    for a in (dx, dinit, dcb, dcodes):
        a.free()


@pytest.mark.parametrize("lanes", [4, 16], indirect=True)
def test_distance_table_dsub8(gpu, lanes):
    rng = np.random.default_rng(8)
    q = rng.standard_normal((5, 64)).astype(np.float32)
    cb = rng.standard_normal(8 * 256 * 8).astype(np.float32)
    p = pq.PQ(dim=64, sub_dim=8, codebooks=cb, m=8, ksub=256)
    got = p.build_distance_table(q, 5)
    st, ref = orc.pq_distance_table(q, 5, 64, 8, 256, cb)
    assert st == 0
    assert np.array_equal(_bits(got), _bits(ref))
    with orc.lane_count(16 if lanes == 4 else 4):
        _, other = orc.pq_distance_table(q, 5, 64, 8, 256, cb)
    assert not np.array_equal(_bits(other), _bits(ref))  # the orders differ on these inputs


@pytest.mark.parametrize("lanes", [4, 8], indirect=True)
@pytest.mark.parametrize("dim", [8, 20, 100])
def test_kmeans_fit_generic_dims(gpu, lanes, dim):
    rng = np.random.default_rng(dim)
    v = rng.standard_normal((3000, dim)).astype(np.float32)
    got = kmeans.fit(v, dim, 24, seed=5, max_iters=15, tol=1e-4)
    ref = orc.kmeans_fit(v, dim, 24, max_iters=15, tol=1e-4, seed=5)
    assert ref.status == 0 and got.iters_run == ref.iters_run
    assert np.array_equal(got.assignments, ref.assignments)
    assert np.array_equal(_bits(got.centroids), _bits(ref.centroids))


@pytest.mark.parametrize("lanes", [4, 8], indirect=True)
@pytest.mark.parametrize("dim", [20, 100])
def test_token_clustering_generic_dims(gpu, lanes, dim):
    ids, v = synth.tac_vectors(20_000, dim, 600, 1.05, 0.15, dim)
    f = np.bincount(ids)
    kap = int(((f > 0) & (f < 20)).sum() + 2 * ((f >= 20) & (f < 40)).sum()
              + 0.6 * (f[f >= 40] // 8).sum())
    kw = dict(mu=20, tau=40, epsilon=4, theta=8)
    ref = orc.tac_cluster_flat(ids, v, dim, orc.tac_params(kap, 3, **kw))
    assert ref.status == 0
    got = tac.cluster_flat(ids, v, dim, tac.ClusteringParams(kappa_total=kap, seed=3, **kw))
    assert got.centroids.tobytes() == ref.centroids.tobytes()
    assert np.array_equal(got.assignments, ref.assignments)
