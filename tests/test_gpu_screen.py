"""GPU parity of the matrix-core first pass of the full search (sub-dimensions
5-8, K <= 256, screen_kernels.hpp), in the Lloyd assignment and in encode.

The full search at these sub-dimensions ranks codewords by a bf16
hi/lo screen on v_mfma_f32_32x32x16_bf16 and gives the reference distance to
the winning block of 8; a vector whose blocks the screen cannot separate goes
to the deferred list and its pruned exact search.  These cases train through
it (TAC_GPU_FULL_SEARCH=1: every iteration takes the full search) and compare every iteration's codebook
bit for bit with the oracle (src/tac/kmeans.zig:154-224 restated) and with
the vector-unit first pass (TAC_GPU_SCREEN=0): every sub-dimension 5-8, K
from 2 to 256 (codeword padding inside the 16-wide groups), exact ties from
duplicated points and codewords, magnitudes outside the screen's range
(every vector takes the reference scan), single non-finite components, and
row counts that end inside a 16-row group.
"""
import numpy as np
import pytest

from oracle import binding as orc
from tac_gpu import device, pq, synth

NEVER = float("-inf")
pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).reshape(-1).view(np.uint32)


def _train(x, dim, m, ksub, init, iters, monkeypatch, screen):
    # every iteration through the full search (not the candidate passes)
    monkeypatch.setenv("TAC_GPU_FULL_SEARCH", "1")
    monkeypatch.setenv("TAC_GPU_SCREEN", "1" if screen else "0")
    device.profile_enable(True)
    device.profile_read(reset=True)
    got = pq.train(x, dim, 0, m=m, ksub=ksub, max_iters=iters, tol=NEVER, init_codebooks=init,
                   trace=True)
    prof = device.profile_read(reset=True)
    device.profile_enable(False)
    return got, prof


def _check(x, dim, m, ksub, init, iters, monkeypatch):
    got, prof = _train(x, dim, m, ksub, init, iters, monkeypatch, True)
    ref = orc.pq_train(x, dim, m, ksub, init=init, max_iters=iters, tol=NEVER, n_threads=16,
                       trace=True)
    assert ref.status == 0
    for t in range(iters):
        diff = np.count_nonzero(_bits(got.stats.trace[t]) != _bits(ref.trace[t]))
        assert diff == 0, f"iteration {t}: {diff} codebook floats differ"
    assert np.array_equal(got.stats.empties, ref.empties)
    old, _ = _train(x, dim, m, ksub, init, iters, monkeypatch, False)
    assert np.array_equal(_bits(got.codebooks), _bits(old.codebooks))
    return prof


@pytest.mark.parametrize("dsub,ksub", [(5, 256), (6, 100), (7, 17), (8, 256), (8, 2), (5, 31),
                                       (6, 255), (7, 129)])
def test_sub_dimensions_and_codebook_sizes(gpu, monkeypatch, dsub, ksub):
    m = 4
    dim = m * dsub
    rng = np.random.default_rng(600 + 10 * dsub + ksub)
    x = (rng.standard_normal((9001, dim)) * 0.2).astype(np.float32)
    init = synth.shuffle_init(x, m, ksub, 5)
    prof = _check(x, dim, m, ksub, init, 6, monkeypatch)
    # every vector went through the screen, which settled most of them
    assert prof.screen_vectors == 6 * m * x.shape[0]
    assert prof.screen_deferred < 0.2 * prof.screen_vectors


def test_duplicate_points_and_codewords(gpu, monkeypatch):
    # 6,000 vectors from 250 distinct points, codewords duplicated: exact
    # ties in every assignment, clusters empty out and get reseeded.
    rng = np.random.default_rng(71)
    pts = (rng.standard_normal((250, 32)) * 0.3).astype(np.float32)
    x = pts[rng.integers(0, 250, 6000)]
    init = synth.shuffle_init(x, 4, 256, 1)
    init[:, 128:] = init[:, :128]
    _check(x, 32, 4, 256, init, 6, monkeypatch)


@pytest.mark.parametrize("scale", [1e-25, 1e-3, 1e15, 1e20])
def test_magnitudes(gpu, monkeypatch, scale):
    # 1e-25 and 1e20 lie outside the screen's range: every vector takes the
    # reference scan.  1e15 stays inside it.
    rng = np.random.default_rng(13)
    x = (rng.standard_normal((5000, 32)) * scale).astype(np.float32)
    init = synth.shuffle_init(x, 4, 256, 2)
    prof = _check(x, 32, 4, 256, init, 4, monkeypatch)
    if scale < 1e-18 or scale > 1e18:
        assert prof.screen_deferred == prof.screen_vectors


def test_non_finite_components(gpu, monkeypatch):
    rng = np.random.default_rng(17)
    x = (rng.standard_normal((7000, 32)) * 0.2).astype(np.float32)
    x[5, 3] = np.inf
    x[6, 9] = np.nan
    x[7, :8] = np.nan
    init = synth.shuffle_init(x, 4, 64, 3)
    got, _ = _train(x, 32, 4, 64, init, 3, monkeypatch, True)
    old, _ = _train(x, 32, 4, 64, init, 3, monkeypatch, False)
    for t in range(3):
        assert np.array_equal(_bits(got.stats.trace[t]), _bits(old.stats.trace[t]))


def _encode(x, dim, m, ksub, cb, monkeypatch, screen):
    monkeypatch.setenv("TAC_GPU_SCREEN", "1" if screen else "0")
    device.profile_enable(True)
    device.profile_read(reset=True)
    p = pq.PQ(dim=dim, sub_dim=dim // m, codebooks=cb, m=m, ksub=ksub)
    got = p.encode_many(x)
    prof = device.profile_read(reset=True)
    device.profile_enable(False)
    return got, prof


def _check_encode(x, dim, m, ksub, cb, monkeypatch):
    got, prof = _encode(x, dim, m, ksub, cb, monkeypatch, True)
    ref = orc.pq_encode(x, dim, m, ksub, cb, n_threads=16)
    assert got.dtype == ref.dtype
    assert np.array_equal(got, ref), f"{np.count_nonzero(got != ref)} codes differ"
    old, _ = _encode(x, dim, m, ksub, cb, monkeypatch, False)
    assert np.array_equal(got, old)
    return prof


@pytest.mark.parametrize("dsub,m,ksub", [(8, 8, 256), (8, 3, 100), (5, 4, 256), (6, 5, 31),
                                         (7, 3, 17), (7, 4, 256), (5, 2, 2), (6, 4, 129)])
def test_encode_sub_dimensions(gpu, monkeypatch, dsub, m, ksub):
    # PQ.encode through the screen: token-major rows, 16-byte loads at dsub 8
    # with dim % 4 == 0, element loads otherwise (dim 24, 20, 30, 21, 28, 10).
    dim = m * dsub
    rng = np.random.default_rng(900 + 10 * dsub + ksub)
    x = (rng.standard_normal((12_345, dim)) * 0.2).astype(np.float32)
    cb = synth.shuffle_init(x, m, ksub, 7).reshape(-1)
    prof = _check_encode(x, dim, m, ksub, cb, monkeypatch)
    assert prof.screen_vectors == m * x.shape[0]
    assert prof.screen_deferred < 0.2 * prof.screen_vectors


def test_encode_ties_and_non_finite(gpu, monkeypatch):
    # duplicated codewords (exact ties: lowest index), rows equal to
    # codewords, and rows with inf / NaN components (the deferred scan keeps
    # PQ.encode's best-from-+inf rule)
    rng = np.random.default_rng(23)
    dim, m, ksub = 64, 8, 256
    x = (rng.standard_normal((9000, dim)) * 0.2).astype(np.float32)
    cb = synth.shuffle_init(x, m, ksub, 4)
    cb[:, 200:] = cb[:, 100:156]
    x[:50] = cb[np.arange(8), np.arange(50)[:, None] % ksub].reshape(50, dim)
    x[60, 3] = np.inf
    x[61, 9] = np.nan
    x[62, :8] = np.nan
    _check_encode(x, dim, m, ksub, cb.reshape(-1), monkeypatch)


@pytest.mark.parametrize("scale", [1e-25, 1e15, 1e20])
def test_encode_magnitudes(gpu, monkeypatch, scale):
    rng = np.random.default_rng(29)
    x = (rng.standard_normal((6000, 64)) * scale).astype(np.float32)
    cb = synth.shuffle_init(x, 8, 256, 6).reshape(-1)
    prof = _check_encode(x, 64, 8, 256, cb, monkeypatch)
    if scale < 1e-18 or scale > 1e18:
        assert prof.screen_deferred == prof.screen_vectors
