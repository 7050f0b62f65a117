"""GPU parity of the cell-list encode (sub-dimensions 1-4, K <= 256).

A uniform grid over the codebook's box joined with mean +- 3 sigma of a
sample of the rows lists, per cell, every codeword that can be the
reference's first-index argmin somewhere in the cell; the encode evaluates a
vector's cell list with the reference distance.  These cases check the codes
bit for bit against the oracle's PQ.encode (src/index/pq.zig:59-76 restated)
and against the anchored candidate encode (TAC_GPU_ENCODE_CELLS=0): data
wider than the codebook (most vectors outside the codebook's box but inside
the grid), lattice codebooks with exact ties on the bisectors, vectors on
and beside cell edges (the grid's origin and scale recomputed here the way
the box kernel sets them when the codebook's box holds the sample's
mean +- 3 sigma), duplicate codewords whose lists pass the 32-item
(128-codeword) limit, lists that overflow the list space, and K below one
item of 4 codewords.
"""
import numpy as np
import pytest

from oracle import binding as orc
from tac_gpu import device, pq

pytestmark = pytest.mark.gpu

SIDES = {1: 65536, 2: 256, 3: 36, 4: 16}  # fine cells per dimension


def _encode(x, cb, m, ksub, monkeypatch=None, cells=True):
    dim = x.shape[1]
    if monkeypatch is not None:
        monkeypatch.setenv("TAC_GPU_ENCODE_CELLS", "1" if cells else "0")
    return pq.PQ(dim, dim // m, np.ascontiguousarray(cb).reshape(-1), m, ksub).encode_many(x)


def _check(x, cb, m, ksub, monkeypatch, max_deferred=None):
    device.profile_enable(True)
    device.profile_read(reset=True)
    got = _encode(x, cb, m, ksub, monkeypatch, cells=True)
    prof = device.profile_read(reset=True)
    device.profile_enable(False)
    ref = orc.pq_encode(x, x.shape[1], m, ksub, cb, n_threads=16)
    assert np.array_equal(got, ref), f"{np.count_nonzero(got != ref)} codes differ from the oracle"
    old = _encode(x, cb, m, ksub, monkeypatch, cells=False)
    assert np.array_equal(got, old)
    assert prof.cand_vectors == m * x.shape[0]
    finite = int(np.isfinite(cb.reshape(m, -1)).all(axis=1).sum())
    assert prof.cell_subspaces == finite  # forced: every tame subspace
    if max_deferred is not None:
        assert prof.cand_deferred <= max_deferred * prof.cand_vectors, (prof.cand_deferred,
                                                                         prof.cand_vectors)
    return prof


@pytest.mark.parametrize("dsub,ksub", [(1, 256), (2, 256), (3, 200), (4, 256), (4, 17), (2, 3),
                                       (4, 2), (3, 7)])
def test_data_wider_than_the_codebook(gpu, monkeypatch, dsub, ksub):
    rng = np.random.default_rng(500 + 10 * dsub + ksub)
    m = 4
    x = (rng.standard_normal((40000, m * dsub)) * 0.09).astype(np.float32)
    cb = (rng.standard_normal((m, ksub, dsub)) * 0.05).astype(np.float32)
    _check(x, cb, m, ksub, monkeypatch, max_deferred=0.1)


@pytest.mark.parametrize("dsub", [2, 4])
def test_lattice_ties(gpu, monkeypatch, dsub):
    # Codewords on a 4^dsub lattice of step 1/32 (duplicated past 4^dsub),
    # vectors on lattice midpoints and on the lattice: exact ties everywhere.
    rng = np.random.default_rng(77 + dsub)
    m, ksub = 4, 256
    cb = (rng.integers(0, 4, (m, ksub, dsub)) / 32.0).astype(np.float32)
    x = (rng.integers(0, 7, (30000, m * dsub)) / 64.0).astype(np.float32)
    _check(x, cb, m, ksub, monkeypatch, max_deferred=0.05)


def _grid_of(cb_sub, G):
    """The box kernel's origin and scale when the codebook's box holds the
    sample's mean +- 3 sigma (cell_grid_params over the codebook's box)."""
    lo = cb_sub.min(axis=0).astype(np.float64)
    hi = cb_sub.max(axis=0).astype(np.float64)
    w = hi - lo
    wmin = (np.abs(lo) + np.abs(hi)) * 2.0 ** -20 + 1e-30
    w = np.maximum(w, wmin)
    return lo.astype(np.float32), (G / w).astype(np.float32)


@pytest.mark.parametrize("dsub", [1, 2, 3, 4])
def test_vectors_on_cell_edges(gpu, monkeypatch, dsub):
    rng = np.random.default_rng(900 + dsub)
    m, ksub, n = 2, 256, 30000
    G = SIDES[dsub]
    cb = (rng.standard_normal((m, ksub, dsub)) * 0.3).astype(np.float32)
    # codewords at the box's corners widen it past the data's mean +- 3 sigma
    for q in range(2):
        cb[:, q] = np.float32(-1.5 if q == 0 else 1.5)
    x = np.empty((n, m * dsub), dtype=np.float32)
    for s in range(m):
        lo, sc = _grid_of(cb[s], G)
        # the central quarter of the grid keeps the rows' mean +- 3 sigma
        # inside the codebook's box
        k = rng.integers(G // 2 - G // 8, G // 2 + G // 8 + 1, (n, dsub))
        edge = (lo[None, :] + k.astype(np.float32) / sc[None, :]).astype(np.float32)
        steps = rng.integers(-2, 3, (n, dsub))
        for _ in range(2):
            edge = np.where(steps > 0, np.nextafter(edge, np.float32(np.inf)), edge)
            edge = np.where(steps < 0, np.nextafter(edge, np.float32(-np.inf)), edge)
            steps = steps - np.sign(steps)
        x[:, s * dsub:(s + 1) * dsub] = edge
    x[: n // 4] *= np.float32(0.1)  # some rows nearer the centre
    _check(x, cb, m, ksub, monkeypatch)


def test_duplicates_past_the_item_limit(gpu, monkeypatch):
    # 200 copies of one codeword: lists near it hold all 200 (ties), past the
    # 32-item (128-codeword) limit, so those cells defer; the first copy must
    # win.
    rng = np.random.default_rng(31)
    m, ksub, dsub = 4, 256, 4
    cb = (rng.standard_normal((m, ksub, dsub)) * 0.2).astype(np.float32)
    cb[:, 30:230] = cb[:, 30:31]
    x = (rng.standard_normal((30000, m * dsub)) * 0.2).astype(np.float32)
    _check(x, cb, m, ksub, monkeypatch)


def test_list_space_overflow(gpu, monkeypatch):
    # Two points, 128 copies each: every list holds one point's copies (ties,
    # 32 items) and some the other's too (past the item limit), far past the
    # space of 8 items per cell on average: later blocks defer their cells.  A second call reuses
    # the space from its start.
    rng = np.random.default_rng(37)
    m, ksub, dsub = 2, 256, 4
    a = rng.standard_normal((m, 1, dsub)).astype(np.float32) * 0.1
    b = rng.standard_normal((m, 1, dsub)).astype(np.float32) * 0.1
    cb = np.concatenate([np.repeat(a, 128, axis=1), np.repeat(b, 128, axis=1)], axis=1)
    cb = cb[:, rng.permutation(ksub)]
    x = (rng.standard_normal((30000, m * dsub)) * 0.1).astype(np.float32)
    _check(x, cb, m, ksub, monkeypatch)
    y = (rng.standard_normal((20000, m * dsub)) * 0.1).astype(np.float32)
    _check(y, cb, m, ksub, monkeypatch)


def test_outliers_nan_and_a_non_finite_codebook(gpu, monkeypatch):
    rng = np.random.default_rng(41)
    m, ksub, dsub = 4, 256, 4
    cb = (rng.standard_normal((m, ksub, dsub)) * 0.1).astype(np.float32)
    cb[3, 5, 1] = np.inf  # subspace 3 takes the full search
    x = (rng.standard_normal((25000, m * dsub)) * 0.1).astype(np.float32)
    x[:500] *= 1e3
    x[600, 2] = np.nan
    x[601, :] = np.nan
    x[602, 9] = -np.inf
    x[603:700] = 0.0
    _check(x, cb, m, ksub, monkeypatch)


def test_auto_choice_per_subspace(gpu, monkeypatch):
    # The choice (made by default from 4M rows; TAC_GPU_ENCODE_CELLS=auto
    # makes it here): a subspace whose sampled rows fall outside the
    # codebook's box takes the cell lists, the others the anchored pass.
    monkeypatch.setenv("TAC_GPU_ENCODE_CELLS", "auto")
    rng = np.random.default_rng(43)
    m, ksub, dsub, n = 4, 256, 4, 40000
    cb = (rng.standard_normal((m, ksub, dsub)) * 0.05).astype(np.float32)
    x = (rng.standard_normal((n, m * dsub)) * 0.09).astype(np.float32)  # wider than the codebook
    near = cb[np.arange(2)[None, :] + 2, rng.integers(0, ksub, (n, 2))].reshape(n, 2 * dsub)
    x[:, 2 * dsub:] = near + (rng.standard_normal((n, 2 * dsub)) * 1e-3).astype(np.float32)
    device.profile_enable(True)
    device.profile_read(reset=True)
    got = _encode(x, cb, m, ksub)
    prof = device.profile_read(reset=True)
    device.profile_enable(False)
    assert prof.cell_subspaces == 2  # subspaces 0 and 1
    ref = orc.pq_encode(x, x.shape[1], m, ksub, cb, n_threads=16)
    assert np.array_equal(got, ref)
    # below 4M rows the default keeps the anchored pass everywhere
    monkeypatch.delenv("TAC_GPU_ENCODE_CELLS")
    device.profile_enable(True)
    device.profile_read(reset=True)
    assert np.array_equal(_encode(x, cb, m, ksub), ref)
    assert device.profile_read(reset=True).cell_subspaces == 0
    device.profile_enable(False)
