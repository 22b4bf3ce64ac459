"""The Acrobot oracle against the reference's own CPU tests (test_acrobot.py)."""

import math

import numpy as np
import pytest

from oracle import acrobot as env
from oracle import rng


def _gym_acrobot_step_scalar(theta1, theta2, dtheta1, dtheta2, action):
    """Gym's AcrobotEnv.step (book dynamics) in float64 with its rk4 on the torque-augmented
    state and its while-loop wrap, as test_acrobot.py:13-49 transcribes it."""
    m1 = m2 = l1 = I1 = I2 = 1.0
    lc1 = lc2 = 0.5
    g, dt = 9.8, 0.2
    torque = [-1.0, 0.0, 1.0][action]

    def dsdt(s):
        th1, th2, dth1, dth2, a = s
        d1 = m1 * lc1**2 + m2 * (l1**2 + lc2**2 + 2 * l1 * lc2 * math.cos(th2)) + I1 + I2
        d2 = m2 * (lc2**2 + l1 * lc2 * math.cos(th2)) + I2
        phi2 = m2 * lc2 * g * math.cos(th1 + th2 - math.pi / 2.0)
        phi1 = (-m2 * l1 * lc2 * dth2**2 * math.sin(th2) - 2 * m2 * l1 * lc2 * dth2 * dth1 * math.sin(th2)
                + (m1 * lc1 + m2 * l1) * g * math.cos(th1 - math.pi / 2) + phi2)
        ddth2 = (a + d2 / d1 * phi1 - m2 * l1 * lc2 * dth1**2 * math.sin(th2) - phi2) / (m2 * lc2**2 + I2 - d2**2 / d1)
        ddth1 = -(d2 * ddth2 + phi1) / d1
        return [dth1, dth2, ddth1, ddth2, 0.0]

    def rk4(y0):
        k1 = dsdt(y0)
        k2 = dsdt([y + dt / 2 * k for y, k in zip(y0, k1)])
        k3 = dsdt([y + dt / 2 * k for y, k in zip(y0, k2)])
        k4 = dsdt([y + dt * k for y, k in zip(y0, k3)])
        return [y + dt / 6.0 * (a + 2 * b + 2 * c + d) for y, a, b, c, d in zip(y0, k1, k2, k3, k4)]

    def wrap(x, m, M):
        diff = M - m
        while x > M:
            x -= diff
        while x < m:
            x += diff
        return x

    ns = rk4([theta1, theta2, dtheta1, dtheta2, torque])
    return (wrap(ns[0], -math.pi, math.pi), wrap(ns[1], -math.pi, math.pi),
            max(-4 * math.pi, min(4 * math.pi, ns[2])), max(-9 * math.pi, min(9 * math.pi, ns[3])))


def random_batch(n, seed=0):
    """test_acrobot.py:52-56."""
    r = np.random.default_rng(seed)
    state = np.stack([r.uniform(-np.pi, np.pi, n), r.uniform(-np.pi, np.pi, n),
                      r.uniform(-2, 2, n), r.uniform(-2, 2, n)]).astype(np.float32)
    return state, r.integers(0, 3, size=n)


@pytest.mark.parametrize("trig", ["det", "numpy"])
def test_matches_gym_scalar_reference(trig):
    """test_acrobot.py:59-63 (atol 1e-3)."""
    state, action = random_batch(200)
    stepped = env.physics(state, action, trig)
    expected = np.array([_gym_acrobot_step_scalar(*s, a) for s, a in zip(state.T.tolist(), action)]).T
    # a wrapped angle may land on the other side of +-pi between float32 and float64
    diff = np.abs(stepped - expected)
    diff[:2] = np.minimum(diff[:2], np.abs(diff[:2] - 2 * np.pi))
    assert diff.max() < 1e-3


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
