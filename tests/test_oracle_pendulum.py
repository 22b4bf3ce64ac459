"""The mass-matrix K-link pendulum oracle (oracle/pendulum.py, the oracle of the HIP
pendulum_metal step) pinned by the reference's test_pendulum.py (CPU): a chain of point
masses by the Jacobian method (the textbook double pendulum at K = 2), energy
conservation, resets in place; and numpy's reduction order, which the kernel
reproduces, made explicit."""

import numpy as np
import pytest

import point_mass_chain
from oracle import detmath
from oracle import pendulum as op

F32 = np.float32


def random_state(k, n, seed=0, vel=1.0):
    r = np.random.default_rng(seed)
    s = np.concatenate([r.uniform(-np.pi, np.pi, (k, n)), r.uniform(-vel, vel, (k, n))]).astype(F32)
    return s, r.integers(0, 3, n)


@pytest.mark.parametrize("trig", ["numpy", "det"])
@pytest.mark.parametrize("k,bound", [(2, 3e-6), (3, 6e-6), (4, 1e-5), (8, 3e-5), (16, 1e-4)])
def test_matches_point_mass_chain(trig, k, bound):
    """test_pendulum.py:32-38's textbook double pendulum (rtol 1e-3) at every K: the float32
    mass-matrix step's accelerations against the chain's by the Jacobian method in float64
    (tests/point_mass_chain.py), relative to |a| + 1. Measured: 1.4e-6 at K = 2, 4.3e-6 at
    4, 1.5e-5 at 8, 4.3e-5 at 16."""
    state, action = random_state(k, 100, seed=k)
    torque = ((action - 1) * op.TORQUE).astype(F32)
    acc = op.mass_matrix_dsdt(state, torque, k, trig=trig)[k:]
    expect = point_mass_chain.batch_accelerations(state[:k].astype(np.float64), state[k:].astype(np.float64),
                                                  torque.astype(np.float64))
    assert (np.abs(acc - expect) / (np.abs(expect) + 1.0)).max() < bound


def test_energy_is_conserved_without_torque():
    """test_pendulum.py:41-51: drift under 1 % over 200 RK4 steps for every K."""
    for k in (2, 4, 8, 16):
        p = op.Pendulum(k, trig="det")
        r = np.random.default_rng(k)
        state = np.concatenate([r.uniform(-0.5, 0.5, (k, 64)), r.uniform(-0.3, 0.3, (k, 64))]).astype(F32)
        e0 = op.energy(state, k)
        for _ in range(200):
            state = p.physics(state, np.ones(64, dtype=np.int64))
        drift = np.abs(op.energy(state, k) - e0) / (np.abs(e0) + 1e-6)
        assert drift.max() < 0.01, (k, drift.max())


def test_terminated_envs_reset_in_place():
    """test_pendulum.py:54-62."""
    p = op.Pendulum(4)
    state = np.zeros((8, 2), dtype=F32)
    state[:4, 0] = np.pi
    next_state, reward, done = p.step(state, np.ones(2, dtype=np.int64), seed=3)
    assert done.tolist() == [True, False] and reward.tolist() == [0.0, -1.0]
    assert np.all(np.abs(next_state[:, 0]) <= op.RESET_BOUND)


@pytest.mark.parametrize("k", [1, 2, 3, 4, 8, 16])
def test_numpy_reduction_order_is_sequential(k):
    """The right-hand side's sum over j (numpy's reduction of axis 1 of a (K, K, N) array)
    equals the sequential float32 sum in j order that the kernel computes, bit for bit."""
    state, action = random_state(k, 257, seed=k)
    torque = ((action - 1) * op.TORQUE).astype(F32)
    got = op.mass_matrix_dsdt(state, torque, k, trig="det")[k:]
    sin_f, cos_f, _ = detmath.trig_functions("det")
    th, om = state[:k], state[k:]
    c, s = cos_f(th), sin_f(th)
    mu = op.hanging_mass(k)
    rhs = []
    for i in range(k):
        r = None
        for j in range(k):
            t = (mu[i, j] * (s[i] * c[j] - c[i] * s[j])) * (om[j] * om[j])
            r = t if r is None else r + t
        rhs.append((-r) - (F32(op.GRAVITY) * mu[i, i]) * s[i])
    rhs[0] = rhs[0] + torque
    m = [[mu[i, j] * (c[i] * c[j] + s[i] * s[j]) for j in range(k)] for i in range(k)]
    np.testing.assert_array_equal(got, op.cholesky_solve(m, np.stack(rhs), k))


@pytest.mark.parametrize("k", [2, 8, 16])
def test_accelerations_match_float64_solve(k):
    state, action = random_state(k, 64, seed=10 + k)
    torque = ((action - 1) * op.TORQUE).astype(F32)
    got = op.mass_matrix_dsdt(state, torque, k, trig="det")[k:]
    ref = op.mass_matrix_accelerations_f64(state[:k], state[k:], torque, k)
    scale = np.abs(ref).max(axis=0) + 1.0
    assert np.all(np.abs(got - ref) <= 1e-3 * scale)
