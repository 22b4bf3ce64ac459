"""The seeded-noise oracle (oracle/es_noise.py), pinned without the GPU.

The generator has no reference counterpart (the reference draws its noise from
MLX or numpy, ``es.py:218-220``), so it is pinned by what the mathematics fixes:

* ``ln_fixed24`` against float64 log on all 2**24 inputs, ``sincos_turn24``
  against float64 sin/cos on all 2**24 inputs;
* the draws: moments, a Kolmogorov-Smirnov distance to N(0, 1), no correlation
  between the two components of a pair or between neighbouring members;
* ``perturb`` against the reference's ``theta + sigma * [eps; -eps]`` and
  ``update`` against a float64 evaluation of the reference's reduction
  (``es.py:224-226``).

Each planted-mistake test edits the oracle (on the CPU) the way a plausible bug
would and shows that one of the checks above fails.
"""

import math

import numpy as np
import pytest

from oracle import es_noise as E

F32 = np.float32


def ulps_off(got, ref):
    """|got - ref| in units of the float32 spacing at ref (ref float64)."""
    spacing = np.spacing(np.abs(ref).astype(F32)).astype(np.float64)
    spacing = np.maximum(spacing, np.spacing(F32(0)))
    return np.abs(got.astype(np.float64) - ref) / spacing


def ln_error(fn=E.ln_fixed24):
    n = np.arange(1, (1 << 24) + 1, dtype=np.int64)
    got = fn(n.astype(np.uint32))
    ref = np.log(n.astype(np.float64)) - 24 * math.log(2.0)
    return ulps_off(got, ref)


def sincos_error(fn=E.sincos_turn24):
    t = np.arange(0, 1 << 24, dtype=np.int64)
    s, c = fn(t.astype(np.uint32))
    a = t.astype(np.float64) * (2 * math.pi / 2.0**24)
    return max(np.abs(s - np.sin(a)).max(), np.abs(c - np.cos(a)).max())


def draws(noise=E.noise, n_members=200_000, d=8):
    return noise(12345, n_members, d).astype(np.float64)


def test_ln_fixed24_every_input():
    err = ln_error()
    assert err.max() <= 2.0, err.max()


def test_sincos_turn24_every_input():
    assert sincos_error() <= 1.2e-7


def test_sincos_special_angles():
    s, c = E.sincos_turn24(np.array([0, 1 << 22, 1 << 23, 3 << 22], dtype=np.uint32))
    np.testing.assert_array_equal(s, F32([0, 1, 0, -1]))
    np.testing.assert_array_equal(c, F32([1, 0, -1, 0]))


def test_ln_special_values():
    np.testing.assert_array_equal(E.ln_fixed24(np.array([1 << 24], dtype=np.uint32)), F32([0.0]))
    got = E.ln_fixed24(np.array([1, 1 << 23], dtype=np.uint32))
    np.testing.assert_allclose(got, [-24 * math.log(2), -math.log(2)], rtol=1e-7)


def test_draws_are_standard_normal():
    from scipy import stats

    z = draws().ravel()
    n = z.size
    assert abs(z.mean()) < 5 / math.sqrt(n)
    assert abs(z.var() - 1.0) < 0.01
    kurt = ((z - z.mean()) ** 4).mean() / z.var() ** 2
    assert abs(kurt - 3.0) < 0.05
    assert stats.kstest(z, "norm").statistic < 1.95 / math.sqrt(n)


def test_draws_are_uncorrelated():
    z = draws()
    # the two components of a Box-Muller pair, and neighbouring weights across pairs
    for a, b in ((0, 1), (1, 2), (0, 2)):
        assert abs(np.corrcoef(z[:, a], z[:, b])[0, 1]) < 0.01, (a, b)
    # neighbouring members, same weight
    assert abs(np.corrcoef(z[:-1, 0], z[1:, 0])[0, 1]) < 0.01


def test_seeds_and_members_differ():
    a = E.noise(1, 64, 10)
    b = E.noise(2, 64, 10)
    assert not np.any(a == b)
    assert len(np.unique(a[:, 0])) == 64


def test_noise_prefix_is_stable_in_d_and_p():
    """A weight's noise depends on (seed, member, weight) only, not on D or P."""
    big = E.noise(9, 40, 31)
    np.testing.assert_array_equal(E.noise(9, 17, 12), big[:17, :12])


def test_perturb_is_the_reference_expression():
    """theta[None, :] + sigma * [eps; -eps] in float32 (es.py:219-222)."""
    rng = np.random.default_rng(0)
    theta = rng.standard_normal(23).astype(F32)
    p, sigma = 10, 0.03
    eps = E.noise(77, p // 2, 23)
    full = np.concatenate([eps, -eps])
    ref = theta[None, :] + F32(sigma) * full
    np.testing.assert_array_equal(E.perturb(theta, p, 77, sigma), ref)
    with pytest.raises(ValueError):
        E.perturb(theta, 9, 77, sigma)


@pytest.mark.parametrize("p,d", [(2, 5), (64, 226), (40_000, 12)])
def test_update_matches_float64_reduction(p, d):
    rng = np.random.default_rng(p + d)
    theta = rng.standard_normal(d).astype(F32)
    ranks = (rng.permutation(p) / (p - 1) - 0.5).astype(F32)
    sigma, lr, seed = 0.1, 0.05, 31
    eps = E.noise(seed, p // 2, d).astype(np.float64)
    full = np.concatenate([eps, -eps])
    grad = (ranks.astype(np.float64)[:, None] * full).sum(axis=0) / (p * sigma)
    ref = theta.astype(np.float64) + lr * grad
    got = E.update(theta, ranks, seed, sigma, lr)
    scale = np.abs(theta).astype(np.float64) + lr * (np.abs(full).sum(axis=0) * 0.5) / (p * sigma)
    assert np.all(np.abs(got - ref) <= 4e-6 * scale + 1e-30), np.abs(got - ref).max()


def test_chunk_members():
    assert [E.chunk_members(h) for h in (1, 2048, 16384, 16385, 131072)] == [64, 64, 64, 128, 512]
    assert -(-131072 // E.chunk_members(131072)) == 256


# ---- planted mistakes: each must fail one of the checks above ------------------------------

def test_planted_missing_exponent_term_fails_ln_check():
    def ln_without_exponent(n):
        n = np.asarray(n, dtype=np.uint32)
        bits = n.astype(F32).view(np.uint32)
        m = ((bits & np.uint32(0x007FFFFF)) | np.uint32(0x3F800000)).view(F32)
        s = (m - F32(1)) / (m + F32(1))
        return (s + s)  # ln m only, k ln 2 dropped
    assert ln_error(ln_without_exponent).max() > 1e3


def test_planted_unreflected_odd_octant_fails_sincos_check():
    def sincos_no_reflection(t):
        t = np.asarray(t, dtype=np.uint32)
        octant, f = t >> np.uint32(21), t & np.uint32((1 << 21) - 1)
        phi = f.astype(F32) * E.PI_TURN24
        sp, cp = E._sin_poly(phi), E._cos_poly(phi)
        q = octant >> np.uint32(1)
        s = np.select([q == 0, q == 1, q == 2], [sp, cp, -sp], -cp)
        c = np.select([q == 0, q == 1, q == 2], [cp, -sp, -cp], sp)
        return s, c
    assert sincos_error(sincos_no_reflection) > 0.1


def test_planted_radius_without_factor_two_fails_variance(monkeypatch):
    def pair_half_radius(key, j):
        z0, z1 = orig(key, j)
        return z0 / F32(math.sqrt(2.0)), z1 / F32(math.sqrt(2.0))
    orig = E.gauss_pair
    monkeypatch.setattr(E, "gauss_pair", pair_half_radius)
    z = draws(n_members=20_000).ravel()
    assert abs(z.var() - 1.0) > 0.3


def test_planted_cos_twice_fails_correlation(monkeypatch):
    def pair_cos_twice(key, j):
        z0, _ = orig(key, j)
        return z0, z0
    orig = E.gauss_pair
    monkeypatch.setattr(E, "gauss_pair", pair_cos_twice)
    z = draws(n_members=20_000)
    assert abs(np.corrcoef(z[:, 0], z[:, 1])[0, 1]) > 0.9
