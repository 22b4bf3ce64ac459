"""The Acrobot oracle against the reference's own CPU tests (test_acrobot.py)."""

import math

import numpy as np
import pytest

from oracle import acrobot as env
from oracle import rng


def _acrobot_lagrangian_step(theta1, theta2, dtheta1, dtheta2, action):
    """One step of the Acrobot as Sutton & Barto's book (and Gym's AcrobotEnv, "book"
    dynamics) define it, written from the equations of motion rather than from any
    program: unit link masses, lengths and inertias, centres of mass at half length,
    g = 9.8, dt = 0.2, torque -1/0/+1, one classical RK4 step with the torque held, angles
    wrapped into [-pi, pi] and velocities clipped to 4 pi and 9 pi.

    The accelerations come from the 2x2 system of the Lagrangian, solved in float64 with a
    linear solve (not the closed-form elimination):

        [d11 d12] [q1'']   [-h1 - phi1      ]
        [d12 d22] [q2''] = [tau - h2 - phi2 ]

    d11 = m1 lc1^2 + m2 (l1^2 + lc2^2 + 2 l1 lc2 cos q2) + I1 + I2,
    d12 = m2 (lc2^2 + l1 lc2 cos q2) + I2, d22 = m2 lc2^2 + I2,
    h1 = -m2 l1 lc2 sin q2 (q2'^2 + 2 q1' q2'), h2 = m2 l1 lc2 sin q2 q1'^2,
    phi2 = m2 lc2 g cos(q1 + q2 - pi/2), phi1 = (m1 lc1 + m2 l1) g cos(q1 - pi/2) + phi2.
    """
    m1 = m2 = l1 = i1 = i2 = 1.0
    lc1 = lc2 = 0.5
    g, dt = 9.8, 0.2
    tau = float(action) - 1.0

    def accelerations(q1, q2, w1, w2):
        c2, s2 = math.cos(q2), math.sin(q2)
        d11 = m1 * lc1 * lc1 + m2 * (l1 * l1 + lc2 * lc2 + 2.0 * l1 * lc2 * c2) + i1 + i2
        d12 = m2 * (lc2 * lc2 + l1 * lc2 * c2) + i2
        d22 = m2 * lc2 * lc2 + i2
        h1 = -m2 * l1 * lc2 * s2 * (w2 * w2 + 2.0 * w1 * w2)
        h2 = m2 * l1 * lc2 * s2 * w1 * w1
        phi2 = m2 * lc2 * g * math.cos(q1 + q2 - math.pi / 2.0)
        phi1 = (m1 * lc1 + m2 * l1) * g * math.cos(q1 - math.pi / 2.0) + phi2
        mass = np.array([[d11, d12], [d12, d22]])
        rhs = np.array([-h1 - phi1, tau - h2 - phi2])
        return np.linalg.solve(mass, rhs)

    def derivative(y):
        a1, a2 = accelerations(*y)
        return np.array([y[2], y[3], a1, a2])

    y = np.array([theta1, theta2, dtheta1, dtheta2], dtype=np.float64)
    k1 = derivative(y)
    k2 = derivative(y + 0.5 * dt * k1)
    k3 = derivative(y + 0.5 * dt * k2)
    k4 = derivative(y + dt * k3)
    y = y + dt / 6.0 * (k1 + 2.0 * k2 + 2.0 * k3 + k4)

    def wrap(x):  # whole turns off an angle outside [-pi, pi]
        return x if -math.pi <= x <= math.pi else x - 2.0 * math.pi * math.floor((x + math.pi) / (2.0 * math.pi))

    return (wrap(y[0]), wrap(y[1]), min(max(y[2], -4.0 * math.pi), 4.0 * math.pi),
            min(max(y[3], -9.0 * math.pi), 9.0 * math.pi))


def random_batch(n, seed=0):
    """test_acrobot.py:52-56."""
    r = np.random.default_rng(seed)
    state = np.stack([r.uniform(-np.pi, np.pi, n), r.uniform(-np.pi, np.pi, n),
                      r.uniform(-2, 2, n), r.uniform(-2, 2, n)]).astype(np.float32)
    return state, r.integers(0, 3, size=n)


@pytest.mark.parametrize("trig", ["det", "numpy"])
def test_matches_gym_scalar_reference(trig):
    """test_acrobot.py:59-63, against the equations of motion solved in float64. The
    reference allows 1e-3; the float32 step is within float32 rounding of it (measured max
    4.2e-7 on these 200 states), so the bound here is 2e-6."""
    state, action = random_batch(200)
    stepped = env.physics(state, action, trig)
    expected = np.array([_acrobot_lagrangian_step(*s, a) for s, a in zip(state.T.tolist(), action)]).T
    # a wrapped angle may land on the other side of +-pi between float32 and float64
    diff = np.abs(stepped - expected)
    diff[:2] = np.minimum(diff[:2], np.abs(diff[:2] - 2 * np.pi))
    assert diff.max() < 2e-6, diff.max()


def test_det_trig_close_to_numpy_trig():
    """One RK4 step with the kernels' sin/cos against numpy's on 50,000 states: measured max
    4.77e-7 absolute (a few float32 ulps of the velocities), 99.9th percentile 2.4e-7."""
    state, action = random_batch(50_000, seed=4)
    a, b = env.physics(state, action, "det"), env.physics(state, action, "numpy")
    d = np.abs(a - b)
    d[:2] = np.minimum(d[:2], np.abs(d[:2] - 2 * np.pi))
    assert np.percentile(d, 99.9) <= 3e-7 and d.max() <= 6e-7, (np.percentile(d, 99.9), d.max())


def test_terminated_envs_reset_in_place_others_untouched():
    """test_acrobot.py:66-83: link 1 straight up is terminal and stays so after a step."""
    state = np.zeros((4, 2), dtype=np.float32)
    state[0, 0] = np.pi
    assert env.terminated(state).tolist() == [True, False]
    next_state, reward, done = env.step(state, np.ones(2, dtype=np.int64), seed=1)
    assert done.tolist() == [True, False]
    assert np.all(np.abs(next_state[:, 0]) <= env.RESET_BOUND)
    assert reward.tolist() == [0.0, -1.0]


def test_random_policy_stays_in_bounds():
    """test_acrobot.py:86-95."""
    n, steps = 1024, 300
    state = env.reset(n, seed=0)
    for t in range(1, steps + 1):
        state, _, _ = env.step(state, rng.uniform_actions(t, n, 3), seed=t)
    assert np.isfinite(state).all()
    assert np.all(np.abs(state[:2]) <= np.pi)
    assert np.all(np.abs(state[2]) <= env.MAX_VEL_1) and np.all(np.abs(state[3]) <= env.MAX_VEL_2)
