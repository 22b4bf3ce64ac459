"""The CartPole oracle against the reference's own CPU tests (test_cartpole.py)."""

import math

import numpy as np
import pytest

from oracle import cartpole as env
from oracle import rng


def _cartpole_equations_step(x, x_dot, theta, theta_dot, action):
    """One explicit-Euler step of the cart-pole as Barto, Sutton & Anderson (1983) and Gym
    define it, written from its equations of motion rather than from any program: cart
    mass 1, pole mass 0.1, pole half-length l = 0.5 (a uniform rod, so its inertia about
    the pivot is 4/3 m l^2), g = 9.8, force +-10, tau = 0.02. The cart's and the pole's
    equations form a 2x2 system for the accelerations, solved in float64:

        [M             m l cos(theta)] [x'']       [F + m l theta'^2 sin(theta)]
        [cos(theta)    4/3 l         ] [theta''] = [g sin(theta)                ]

    with M the total mass; then x += tau x', x' += tau x'', theta += tau theta',
    theta' += tau theta''."""
    m_cart, m_pole, half, g, tau = 1.0, 0.1, 0.5, 9.8, 0.02
    force = 10.0 if action == 1 else -10.0
    c, s_ = math.cos(theta), math.sin(theta)
    total = m_cart + m_pole
    system = np.array([[total, m_pole * half * c], [c, 4.0 / 3.0 * half]])
    rhs = np.array([force + m_pole * half * theta_dot * theta_dot * s_, g * s_])
    x_acc, theta_acc = np.linalg.solve(system, rhs)
    return (x + tau * x_dot, x_dot + tau * x_acc, theta + tau * theta_dot, theta_dot + tau * theta_acc)


def _random_batch(n, seed=0):
    r = np.random.default_rng(seed)
    return r.uniform(-1, 1, size=(4, n)).astype(np.float32), r.integers(0, 2, size=n)


@pytest.mark.parametrize("trig", ["det", "numpy"])
def test_matches_gym_scalar_reference(trig):
    """test_cartpole.py:40-44, against the equations of motion solved in float64. The
    reference allows 1e-5; the float32 step is within float32 rounding of them (measured
    max 1.1e-7 on these 100 states), so the bound here is 5e-7."""
    state, action = _random_batch(100)
    stepped = env.physics(state, action, trig)
    expected = np.array([_cartpole_equations_step(*s, a) for s, a in zip(state.T.tolist(), action)]).T
    np.testing.assert_allclose(stepped, expected, rtol=0, atol=5e-7)


def test_det_trig_within_1e5_relative_of_numpy_trig():
    """The bit-exact (det) oracle vs the reference's literal np.sin/np.cos path."""
    state, action = _random_batch(100_000, seed=3)
    a, b = env.physics(state, action, "det"), env.physics(state, action, "numpy")
    np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-7)


def test_stays_float32():
    """test_cartpole.py:47-55."""
    state = env.reset(8, seed=1)
    next_state, reward, done = env.step(state, np.zeros(8, dtype=np.int64), seed=2)
    assert state.shape == (4, 8) and state.dtype == np.float32
    assert next_state.dtype == np.float32 and reward.dtype == np.float32 and done.dtype == np.bool_


def two_terminal_one_live():
    """test_cartpole.py:58-63: env 0 past the x limit, env 1 past the theta limit, env 2 fine."""
    state = np.zeros((4, 3), dtype=np.float32)
    state[0, 0] = 2.5
    state[2, 1] = 0.3
    return state


def test_terminated_envs_reset_in_place_others_untouched():
    """test_cartpole.py:66-73."""
    state = two_terminal_one_live()
    next_state, reward, done = env.step(state, np.ones(3, dtype=np.int64), seed=1)
    assert done.tolist() == [True, True, False]
    assert np.all(np.abs(next_state[:, :2]) <= env.RESET_BOUND)
    np.testing.assert_array_equal(next_state[:, :2], env.reset(3, seed=1)[:, :2])
    assert np.array_equal(next_state[:, 2], env.physics(state, np.ones(3))[:, 2])
    assert reward.tolist() == [1.0, 1.0, 1.0]


def test_random_policy_episodes_end():
    """test_cartpole.py:76-87: the Gym random policy averages ~22 steps."""
    n, steps = 1024, 500
    state = env.reset(n, seed=0)
    terminations = np.zeros(n, dtype=np.int64)
    for t in range(1, steps + 1):
        state, _, done = env.step(state, rng.action_bits(t, n), seed=t)
        terminations += done
    assert terminations.min() >= 1
    assert 10 < steps / terminations.mean() < 40


def test_chain_never_leaves_a_terminal_state():
    """test_cartpole.py:111-124: after any step no column is in a terminal region."""
    n = 4096
    state = env.reset(n, seed=0)
    for t in range(1, 101):
        state, _, _ = env.step(state, rng.action_bits(t, n), seed=t)
        assert not env.terminated(state).any()
    assert np.isfinite(state).all()


def test_step_k_equals_chained_steps():
    n, k = 257, 12
    state = env.reset(n, seed=9)
    fin, rewards, dones = env.step_k(state, 100, k)
    s = state
    for t in range(k):
        s, r, d = env.step(s, rng.action_bits(100 + t, n), seed=100 + t)
        np.testing.assert_array_equal(rewards[t], r)
        np.testing.assert_array_equal(dones[t], d)
    np.testing.assert_array_equal(fin, s)
