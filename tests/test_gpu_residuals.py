"""GPU residual stage (tac_residuals / tac_residuals_device) against the
oracle, bit for bit: residuals and norms of src/index/storage.zig:255-278."""
import ctypes

import numpy as np
import pytest

from oracle import binding as orc
from tac_gpu import device, errors, lib, storage, synth

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def _case(n, dim, k, seed, spread=0.1):
    rng = np.random.default_rng(seed)
    c = rng.standard_normal((k, dim)).astype(np.float32)
    a = rng.integers(0, k, n).astype(np.uint32)
    v = (c[a] + spread * rng.standard_normal((n, dim))).astype(np.float32)
    return v, c, a


def _check(v, dim, c, a):
    st, r_ref, n_ref = orc.residuals(v, dim, c, a)
    assert st == 0
    r, n = storage.residuals_and_norms(v, dim, c, a)
    assert np.array_equal(_bits(n), _bits(n_ref))
    assert np.array_equal(_bits(r), _bits(r_ref))


@pytest.mark.parametrize("dim", [64, 128, 96, 4, 3, 1, 33, 1000])
@pytest.mark.parametrize("n", [1, 63, 64, 65, 5000])
def test_parity_shapes(gpu, n, dim):
    v, c, a = _case(n, dim, 37, seed=n * 7 + dim)
    _check(v, dim, c, a)


def test_special_values(gpu):
    v, c, a = _case(4096, 64, 16, seed=5)
    v[10] = c[a[10]]                      # zero residual
    v[11] = c[a[11]]
    v[11, 3] = -0.0
    c[a[11], 3] = 0.0                     # -0.0 component in a zero residual
    v[12, 7] = np.nan
    v[13, 0] = np.inf
    v[14, :2] = (3e19, -4e19)             # overflowing squares
    v[15] = c[a[15]] + np.float32(1e-30)  # tiny, subnormal squares
    _check(v, 64, c, a)


def test_full_corpus_scale(gpu):
    """1,521,797 tokens of dim 64 against 32,768 centroids (the corpus
    workload's tokens rebuilt as centre + residual)."""
    w = synth.WORKLOADS["corpus-1.52m"]
    r0, ids = synth.residuals(w, with_ids=True)
    cents = synth.centers(w.seed, w.n_centers, w.dim)
    v = (r0 + cents[ids]).astype(np.float32)
    _check(v, w.dim, cents, ids)


def test_device_entry_in_place_and_unaligned(gpu):
    v, c, a = _case(3000, 64, 20, seed=9)
    _, r_ref, n_ref = orc.residuals(v, 64, c, a)
    dv = device.DeviceArray.from_host(v)
    dc = device.DeviceArray.from_host(c)
    da = device.DeviceArray.from_host(a)
    dn = device.DeviceArray((3000,), np.float32)
    device.residuals_device(dv, 3000, 64, dc, 20, da, dv, dn)  # in place
    assert np.array_equal(_bits(dv.to_host()), _bits(r_ref))
    assert np.array_equal(_bits(dn.to_host()), _bits(n_ref))
    # 4-byte offset pointers take the scalar-load kernel
    raw = device.DeviceArray((3000 * 64 + 1,), np.float32)
    out = device.DeviceArray((3000 * 64 + 1,), np.float32)
    errors.check(lib.tac_gpu_memcpy_htod(ctypes.c_void_p(raw.ptr.value + 4),
                                         ctypes.c_void_p(v.ctypes.data), v.nbytes))
    errors.check(lib.tac_residuals_device(ctypes.c_void_p(raw.ptr.value + 4), 3000, 64, dc.ptr,
                                          20, da.ptr, ctypes.c_void_p(out.ptr.value + 4),
                                          dn.ptr, None))
    got = out.to_host()[1:].reshape(3000, 64)
    assert np.array_equal(_bits(got), _bits(r_ref))


def test_errors(gpu):
    v, c, a = _case(100, 64, 8, seed=1)
    a[57] = 8
    with pytest.raises(errors.InvalidArgument):
        storage.residuals_and_norms(v, 64, c, a)
    a[57] = 0
    with pytest.raises(errors.Unsupported):
        storage.residuals_and_norms(np.zeros((2, 5000), np.float32), 5000,
                                    np.zeros((1, 5000), np.float32), [0, 0])
    # the error leaves the library usable
    _check(v, 64, c, a)


def test_decode_rejects_out_of_range_codes(gpu):
    from tac_gpu import pq
    cb = np.random.default_rng(0).standard_normal((4, 100, 2)).astype(np.float32)
    q = pq.PQ(dim=8, sub_dim=2, codebooks=cb.reshape(-1), m=4, ksub=100)
    codes = np.array([[1, 2, 3, 99], [0, 0, 100, 0]], np.uint8)
    with pytest.raises(errors.InvalidArgument):
        q.decode_many(codes)
    ok = q.decode_many(codes[:1])
    assert np.array_equal(ok, orc.pq_decode(codes[:1], 8, 4, 100, cb))
