"""The ABA pendulum oracle pinned by the reference's tests and by brute force (CPU)."""

import numpy as np
import pytest

import point_mass_chain
from oracle import pendulum as mm
from oracle import pendulum_aba as aba


def random_state(k, n, seed=0, vel=1.0):
    """test_pendulum.py:40-42."""
    r = np.random.default_rng(seed)
    return (np.concatenate([r.uniform(-np.pi, np.pi, (k, n)), r.uniform(-vel, vel, (k, n))]).astype(np.float32),
            r.integers(0, 3, n))


@pytest.mark.parametrize("trig", ["det", "numpy"])
def test_single_link_closed_form(trig):
    """test_pendulum_aba.py:13-18: theta'' = tau - g sin(theta)."""
    r = np.random.default_rng(0)
    state = r.uniform(-3, 3, (2, 50)).astype(np.float32)
    torque = r.uniform(-1, 1, 50).astype(np.float32)
    acc = aba.aba_accelerations(state[:1], state[1:], torque, 1, trig)[0]
    np.testing.assert_allclose(acc, torque - 9.8 * np.sin(state[0]), atol=1e-6)


@pytest.mark.parametrize("k,bound", [(2, 2e-6), (3, 5e-6), (4, 5e-6), (8, 1e-5), (16, 1e-5), (32, 1e-5), (64, 2e-5)])
def test_matches_point_mass_chain(k, bound):
    """test_pendulum_aba.py's textbook double pendulum (test_pendulum.py:14-37, rtol 1e-3),
    at every K: the float32 recursion against the chain's accelerations by the Jacobian
    method in float64 (tests/point_mass_chain.py), relative to |a| + 1. Measured: 5.6e-7 at
    K = 2, 1.7e-6 at 3, 2.2e-6 at 8, 3.2e-6 at 32, 6.0e-6 at 64."""
    r = np.random.default_rng(k)
    theta = r.uniform(-np.pi, np.pi, (k, 60)).astype(np.float32)
    omega = r.uniform(-1, 1, (k, 60)).astype(np.float32)
    torque = r.uniform(-1, 1, 60).astype(np.float32)
    out = aba.aba_accelerations(theta, omega, torque, k)
    ref = point_mass_chain.batch_accelerations(theta.astype(np.float64), omega.astype(np.float64),
                                               torque.astype(np.float64))
    assert (np.abs(out - ref) / (np.abs(ref) + 1.0)).max() < bound


@pytest.mark.parametrize("k", [1, 2, 4, 16, 64])
def test_float64_mass_matrix_is_the_point_mass_chain(k):
    """The oracle's float64 mass-matrix solve, which the tests below use past K = 16, is the
    same mechanics as the chain derived from the masses' positions (measured 2.0e-12 at
    K = 64)."""
    r = np.random.default_rng(100 + k)
    theta = r.uniform(-np.pi, np.pi, (k, 40)).astype(np.float32)
    omega = r.uniform(-1, 1, (k, 40)).astype(np.float32)
    torque = r.uniform(-1, 1, 40).astype(np.float32)
    got = mm.mass_matrix_accelerations_f64(theta, omega, torque, k)
    ref = point_mass_chain.batch_accelerations(theta.astype(np.float64), omega.astype(np.float64),
                                               torque.astype(np.float64))
    assert (np.abs(got - ref) / (np.abs(ref) + 1.0)).max() < 1e-10


@pytest.mark.parametrize("k", [2, 3, 4, 8, 16])
def test_matches_mass_matrix(k):
    """test_pendulum_aba.py:21-28: the O(K) recursion and the O(K^3) solve agree."""
    state, action = random_state(k, 300, seed=k)
    torque = ((action - 1) * 1.0).astype(np.float32)
    ref = mm.mass_matrix_dsdt(state, torque, k)[k:]
    out = aba.aba_accelerations(state[:k], state[k:], torque, k)
    np.testing.assert_allclose(out, ref, atol=1e-3, err_msg=f"K={k}")


@pytest.mark.parametrize("k", [4, 16, 32, 64])
def test_matches_float64_solve_at_every_k(k):
    """Past the reference's K = 16 oracle: the same equations in float64 by numpy.linalg.solve."""
    r = np.random.default_rng(k)
    state = np.concatenate([r.uniform(-np.pi, np.pi, (k, 60)), r.uniform(-1, 1, (k, 60))]).astype(np.float32)
    torque = r.uniform(-1, 1, 60).astype(np.float32)
    out = aba.aba_accelerations(state[:k], state[k:], torque, k)
    ref = mm.mass_matrix_accelerations_f64(state[:k], state[k:], torque, k)
    assert (np.abs(out - ref) / (np.abs(ref) + 1.0)).max() < 5e-5


@pytest.mark.parametrize("k,tol", [(16, 0.01), (32, 0.03), (64, 0.1)])
def test_rk4_energy_is_conserved_at_large_k(k, tol):
    """test_pendulum_aba.py:31-41."""
    p = aba.Pendulum(k)
    r = np.random.default_rng(k)
    state = np.concatenate([r.uniform(-0.5, 0.5, (k, 32)), r.uniform(-0.3, 0.3, (k, 32))]).astype(np.float32)
    e0 = mm.energy(state, k)
    for _ in range(200):
        state = p.physics(state, np.ones(32, dtype=np.int64))
    drift = np.abs(mm.energy(state, k) - e0) / (np.abs(e0) + 1e-6)
    assert drift.max() < tol, (k, drift.max())


@pytest.mark.parametrize("k", [4, 16])
def test_euler_energy_drift_is_first_order(k):
    """Semi-implicit Euler is symplectic: without torque the energy error stays bounded and
    shrinks with the step; pinned against RK4 of the same accelerations."""
    p = aba.Pendulum(k)
    r = np.random.default_rng(k)
    state = np.concatenate([r.uniform(-0.3, 0.3, (k, 32)), np.zeros((k, 32))]).astype(np.float32)
    e0 = mm.energy(state, k)
    s = state
    worst = 0.0
    for _ in range(400):
        s = p.physics_euler(s, np.zeros(32, np.float32))
        worst = max(worst, (np.abs(mm.energy(s, k) - e0) / (np.abs(e0) + 1e-6)).max())
    assert worst < 0.05, worst
    # one Euler step equals the composition of the pinned accelerations with the integrator
    acc = aba.aba_accelerations(state[:k], state[k:], np.zeros(32, np.float32), k)
    om1 = state[k:] + np.float32(0.01) * acc
    th1 = state[:k] + np.float32(0.01) * om1
    np.testing.assert_array_equal(p.physics_euler(state, np.zeros(32, np.float32))[k:], om1)
    np.testing.assert_array_equal(p.physics_euler(state, np.zeros(32, np.float32))[:k], mm.wrap(th1))


def test_terminated_envs_reset_in_place():
    """test_pendulum.py:67-75 for the ABA body."""
    p = aba.Pendulum(4)
    state = np.zeros((8, 2), dtype=np.float32)
    state[:4, 0] = np.pi
    assert mm.terminated(state, 4).tolist() == [True, False]
    next_state, reward, done = p.step(state, np.ones(2, dtype=np.int64), seed=1)
    assert done.tolist() == [True, False] and reward.tolist() == [0.0, -1.0]
    assert np.all(np.abs(next_state[:, 0]) <= aba.RESET_BOUND)
    ns, _, d = p.step_euler(state, np.zeros(2, np.float32), seed=1)
    assert d.tolist() == [True, False] and np.all(ns[4:, 0] == 0) and np.all(np.abs(ns[:4, 0]) <= 0.1)
