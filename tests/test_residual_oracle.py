"""Pins the oracle's residual stage (src/index/storage.zig:255-278).

The reference's own tests hold no known answers for this stage (they check
only that repeated builds give byte-equal norms,
tests/integration/build_determinism_test.zig:141-176), so the oracle is
pinned by closed forms worked out by hand, by special values whose result
IEEE arithmetic fixes, by the unit-norm and reconstruction properties, and
by planted mistakes (an FMA-contracted fold, a reversed fold order, a
normalisation by division) that must disagree with it.  No GPU needed.
"""
import numpy as np
import pytest

from oracle import binding as orc

ST_OK, ST_DIM, ST_INVALID = 0, 2, 14


def f32(*v):
    return np.array(v, dtype=np.float32)


def one(v, c):
    st, r, n = orc.residuals(f32(*v), len(v), f32(*c), [0])
    assert st == ST_OK
    return r[0], n[0]


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


def test_three_four_five():
    # diff (3, 4, 0, 0): sum 25 exactly, norm 5, fl(1/5) = 13421773 * 2^-26;
    # 3 * fl(1/5) = 0.60000000894 rounds to 0.6f, 4 * fl(1/5) = 0.8f exactly.
    r, n = one([4, 6, 1, -2], [1, 2, 1, -2])
    assert n == 5.0
    assert bits(r).tolist() == bits(f32(0.6, 0.8, 0, 0)).tolist()


def test_single_axis_is_a_signed_unit():
    # diff (0, -2, 0): norm 2, fl(1/2) = 0.5 exactly, r = (0, -1, 0)
    r, n = one([1, -1, 7], [1, 1, 7])
    assert n == 2.0 and r.tolist() == [0.0, -1.0, 0.0]


def test_zero_residual_is_left_unscaled():
    # norm 0 fails `norm > 0`, so no division happens (storage.zig:272)
    r, n = one([0.25, -3, 9], [0.25, -3, 9])
    assert n == 0.0 and bits(r).tolist() == [0, 0, 0]


def test_negative_zero_survives():
    # -0.0 - 0.0 = -0.0; norm 0 leaves the sign bit in place
    r, n = one([-0.0, 0.0], [0.0, 0.0])
    assert n == 0.0 and bits(r).tolist() == [0x80000000, 0]


def test_nan_propagates_without_scaling():
    r, n = one([np.nan, 3.0], [0.0, 1.0])
    assert np.isnan(n) and np.isnan(r[0]) and r[1] == 2.0  # NaN > 0 is false


def test_overflowing_norm_scales_by_zero():
    # squares overflow to +inf, norm = inf > 0, fl(1/inf) = 0, r = diff * 0
    r, n = one([3e19, -4e19], [0.0, 0.0])
    assert n == np.inf and bits(r).tolist() == [0, 0x80000000]


def test_infinite_component():
    r, n = one([np.inf, 1.0], [0.0, 0.0])
    assert n == np.inf and np.isnan(r[0]) and r[1] == 0.0  # inf * 0 = NaN


def test_errors():
    assert orc.residuals(f32(1, 2), 2, f32(0, 0), [1])[0] == ST_INVALID
    assert orc.residuals(f32(1, 2), 0, f32(0, 0), [0])[0] == ST_DIM


def _fold(diff, order=1, fused=False):
    s = np.float32(0.0)
    for x in diff[::order]:
        if fused:  # one rounding of x*x + s (exact in float64, then rounded)
            s = np.float32(np.float64(x) * np.float64(x) + np.float64(s))
        else:
            s = np.float32(s + np.float32(x * x))
    return s


def _random(n=2000, dim=64, k=50, seed=3):
    rng = np.random.default_rng(seed)
    c = rng.standard_normal((k, dim)).astype(np.float32)
    a = rng.integers(0, k, n).astype(np.uint32)
    v = (c[a] + 0.1 * rng.standard_normal((n, dim))).astype(np.float32)
    return v, c, a


def test_properties_on_random_tokens():
    v, c, a = _random()
    st, r, n = orc.residuals(v, 64, c, a)
    assert st == ST_OK
    diff = v - c[a]
    # unit norm after scaling, and r * norm reconstructs v - c to a few ulps
    assert np.allclose(np.linalg.norm(r.astype(np.float64), axis=1), 1.0, atol=2e-6)
    assert np.allclose(r * n[:, None], diff, rtol=3e-7, atol=1e-12)
    # the norm is the correctly rounded sqrt of the in-order unfused fold
    for i in range(0, 2000, 97):
        assert n[i] == np.sqrt(_fold(diff[i]))
        assert bits(r[i]).tolist() == bits(diff[i] * (np.float32(1.0) / n[i])).tolist()


def test_planted_mistakes_disagree():
    v, c, a = _random(seed=11)
    _, r, n = orc.residuals(v, 64, c, a)
    diff = v - c[a]
    fused = np.array([np.sqrt(_fold(d, fused=True)) for d in diff])
    rev = np.array([np.sqrt(_fold(d, order=-1)) for d in diff])
    divided = diff / n[:, None]  # x / norm instead of x * fl(1/norm)
    assert (fused != n).sum() > 0
    assert (rev != n).sum() > 0
    assert (bits(divided) != bits(r)).sum() > 0


@pytest.mark.parametrize("dim", [1, 3, 128, 300])
def test_any_dim(dim):
    v, c, a = _random(n=300, dim=dim, seed=dim)
    st, r, n = orc.residuals(v, dim, c, a)
    assert st == ST_OK
    diff = v - c[a]
    assert np.all(n[:50] == np.array([np.sqrt(_fold(d)) for d in diff[:50]]))
