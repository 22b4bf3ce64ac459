"""The counter RNG of the oracle: known answers and distribution (CPU)."""

import numpy as np

from oracle import cartpole, rng

# pcg_hash known answers from the published algorithm (Jarzynski & Olano 2020),
# evaluated on Python integers with explicit 32-bit masking.
KAT = {
    0: 0x07BB2FE2,
    1: 0xA8BEEA3C,
    2: 0x7A7ECC88,
    3: 0x7F0EF6BC,
    0x9E3779B9: 0x9031965F,
    0xFFFFFFFF: 0xE62A4902,
    12345: 0xF45EAD0E,
    0x80000000: 0x21C72646,
}


def test_pcg_hash_known_answers():
    for v, expect in KAT.items():
        assert rng.pcg_hash_int(v) == expect
        assert int(rng.pcg_hash(np.array([v], dtype=np.uint32))[0]) == expect


def test_vectorised_hash_matches_integer_hash():
    v = np.random.default_rng(0).integers(0, 2**32, 20000, dtype=np.uint64).astype(np.uint32)
    got = rng.pcg_hash(v)
    assert all(int(g) == rng.pcg_hash_int(int(x)) for g, x in zip(got[:2000], v[:2000]))
    assert got.dtype == np.uint32


def test_uniform_is_top_24_bits():
    h = np.array([0, 0xFF, 0x100, 0x80000000, 0xFFFFFFFF], dtype=np.uint32)
    u = rng.uniform_pm(h, 1.0)
    np.testing.assert_array_equal(u, np.array([-1.0, -1.0, -1.0 + 2.0**-23, 0.0, 1.0 - 2.0**-23], dtype=np.float32))


def test_resets_are_uniform_in_bound_and_vary():
    """test_cartpole.py:160-172: in bound, different per call and per env, mean 0, std B/sqrt(3)."""
    n = 4096
    first, second = cartpole.reset(n, seed=1), cartpole.reset(n, seed=2)
    assert first.dtype == np.float32 and first.shape == (4, n)
    assert np.all(np.abs(first) <= cartpole.RESET_BOUND)
    assert not np.allclose(first, second)
    assert len(np.unique(first[0])) > n * 0.99
    assert abs(first.mean()) < 0.002
    assert abs(first.std() - cartpole.RESET_BOUND / np.sqrt(3)) < 0.002


def test_actions_are_fair_and_uniform():
    a = rng.action_bits(7, 1 << 16)
    assert set(np.unique(a)) == {0, 1} and abs(a.mean() - 0.5) < 0.01
    u = rng.uniform_actions(7, 1 << 16, 81)
    counts = np.bincount(u, minlength=81)
    assert u.min() == 0 and u.max() == 80 and counts.min() > 0.8 * (1 << 16) / 81
    t = rng.torque_uniform(3, 1 << 16)
    assert t.min() >= -1.0 and t.max() < 1.0 and abs(t.mean()) < 0.02
