"""Acrobot restated in numpy: the CPU oracle for the HIP Acrobot step and rollout kernels.

TEST INFRASTRUCTURE: part of the CPU oracle (see ``oracle/__init__.py``).

Follows ``acrobot_np.py`` line by line with its Python-scalar groupings kept
(they decide which constants numpy folds in float64 before rounding to
float32, NEP 50):

* constants ``acrobot_np.py:18-28``;
* ``physics`` = ``_physics`` ``acrobot_np.py:47-61`` (RK4 at dt 0.2 on
  (theta1, theta2, dtheta1, dtheta2), wrap, clip);
* ``dsdt`` = ``_dsdt`` ``acrobot_np.py:64-84`` (Gym's book dynamics);
* ``wrap`` = ``_wrap`` ``acrobot_np.py:87-89``;
* ``terminated`` = ``_terminated`` ``acrobot_np.py:92-93``;
* ``step`` = ``step`` ``acrobot_np.py:35-44`` (reward -1, 0 on done).

As for CartPole, resets come from the kernels' counter RNG
(``acrobot_metal.py:79-83``) and the transcendentals default to ``detmath``.
``rollout_steps`` restates the fused ES kernel ``acrobot_rollout_metal.py:21-58``.
"""

import numpy as np

from . import detmath, rng

F32 = np.float32

LINK_LENGTH_1 = 1.0
LINK_MASS_1 = 1.0
LINK_MASS_2 = 1.0
LINK_COM_POS_1 = 0.5
LINK_COM_POS_2 = 0.5
LINK_MOI = 1.0
GRAVITY = 9.8
DT = 0.2
MAX_VEL_1 = 4 * np.pi
MAX_VEL_2 = 9 * np.pi
RESET_BOUND = 0.1


def reset(n, seed=0):
    return rng.reset_rows4(seed, n, RESET_BOUND)


def dsdt(s, torque, trig="det"):
    """Time derivative of the state; ``acrobot_np.py:64-84``."""
    sin_f, cos_f, _ = detmath.trig_functions(trig)
    theta1, theta2, dtheta1, dtheta2 = s
    m1, m2, l1 = LINK_MASS_1, LINK_MASS_2, LINK_LENGTH_1
    lc1, lc2, I1, I2, g = LINK_COM_POS_1, LINK_COM_POS_2, LINK_MOI, LINK_MOI, GRAVITY
    c2, s2 = cos_f(theta2), sin_f(theta2)
    d1 = m1 * lc1**2 + m2 * (l1**2 + lc2**2 + 2 * l1 * lc2 * c2) + I1 + I2
    d2 = m2 * (lc2**2 + l1 * lc2 * c2) + I2
    phi2 = m2 * lc2 * g * cos_f(theta1 + theta2 - np.pi / 2)
    phi1 = (
        -m2 * l1 * lc2 * dtheta2**2 * s2
        - 2 * m2 * l1 * lc2 * dtheta2 * dtheta1 * s2
        + (m1 * lc1 + m2 * l1) * g * cos_f(theta1 - np.pi / 2)
        + phi2
    )
    ddtheta2 = (torque + d2 / d1 * phi1 - m2 * l1 * lc2 * dtheta1**2 * s2 - phi2) / (
        m2 * lc2**2 + I2 - d2**2 / d1
    )
    ddtheta1 = -(d2 * ddtheta2 + phi1) / d1
    return np.stack([dtheta1, dtheta2, ddtheta1, ddtheta2])


def wrap(x):
    """Angle to [-pi, pi), branch-free; ``acrobot_np.py:87-89``."""
    return x - 2 * np.pi * np.floor((x + np.pi) / (2 * np.pi))


def physics_torque(state, torque, trig="det"):
    """RK4 + wrap + clip with a float32 torque per column; ``acrobot_np.py:47-61``."""
    k1 = dsdt(state, torque, trig)
    k2 = dsdt(state + DT / 2 * k1, torque, trig)
    k3 = dsdt(state + DT / 2 * k2, torque, trig)
    k4 = dsdt(state + DT * k3, torque, trig)
    ns = state + DT / 6 * (k1 + 2 * k2 + 2 * k3 + k4)
    return np.stack(
        [
            wrap(ns[0]),
            wrap(ns[1]),
            np.clip(ns[2], -MAX_VEL_1, MAX_VEL_1),
            np.clip(ns[3], -MAX_VEL_2, MAX_VEL_2),
        ]
    ).astype(F32)


def physics(state, action, trig="det"):
    torque = (np.asarray(action) - 1).astype(F32)
    return physics_torque(np.asarray(state, dtype=F32), torque, trig)


def terminated(state, trig="det"):
    """Tip above height 1; ``acrobot_np.py:92-93``."""
    _, cos_f, _ = detmath.trig_functions(trig)
    return -cos_f(state[0]) - cos_f(state[1] + state[0]) > 1.0


def step(state, action, seed, trig="det"):
    """(next_state, reward, done) for step counter `seed`; ``acrobot_np.py:35-44``."""
    state = np.asarray(state, dtype=F32)
    n = state.shape[1]
    stepped = physics(state, action, trig)
    done = terminated(stepped, trig)
    fresh = reset(n, seed)
    next_state = np.where(done[None, :], fresh, stepped).astype(F32)
    reward = np.where(done, 0.0, -1.0).astype(F32)
    return next_state, reward, done


def policy_logits(state, w1, b1, w2, b2, trig="det"):
    """6-H-3 policy on Gym's observation (cos th1, sin th1, cos th2, sin th2, dth1, dth2) in the
    fused kernel's order (``acrobot_rollout_metal.py:31-39``); returns (3, P)."""
    sin_f, cos_f, tanh_f = detmath.trig_functions(trig)
    th1, th2, dth1, dth2 = state
    obs = (cos_f(th1), sin_f(th1), cos_f(th2), sin_f(th2), dth1, dth2)
    logits = [b2[:, k].copy() for k in range(3)]
    for j in range(w1.shape[2]):
        pre = obs[0] * w1[:, 0, j]
        for i in range(1, 6):
            pre = pre + obs[i] * w1[:, i, j]
        h = tanh_f(pre + b1[:, j])
        for k in range(3):
            logits[k] = logits[k] + h * w2[:, j, k]
    return np.stack(logits)


def rollout_steps(state, theta_pop, hidden, horizon, trig="det"):
    """Steps before the first termination per member (P,) float32 from state (4, P) and
    theta_pop (P, 10H+3); ``acrobot_rollout_metal.py:21-58``."""
    from .es import first_argmax, unflatten

    state = np.asarray(state, dtype=F32).copy()
    w1, b1, w2, b2 = unflatten(np.asarray(theta_pop, dtype=F32), hidden, 6, 3)
    p = state.shape[1]
    alive = np.ones(p, dtype=bool)
    steps = np.zeros(p, dtype=F32)
    for _ in range(horizon):
        torque = (first_argmax(policy_logits(state, w1, b1, w2, b2, trig)) - 1).astype(F32)
        stepped = physics_torque(state, torque, trig)
        done = terminated(stepped, trig)
        alive = alive & ~done
        steps = steps + alive.astype(F32)
        state = np.where(alive[None, :], stepped, state)
        if not alive.any():
            break
    return steps
