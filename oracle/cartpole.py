"""CartPole restated in numpy: the CPU oracle for the HIP step and rollout kernels.

TEST INFRASTRUCTURE: part of the CPU oracle (see ``oracle/__init__.py``).

Follows ``cartpole_np.py`` line by line, in the same float32 operation order
(numpy's NEP 50 rules turn every Python-float constant into float32 before the
operation, which is what the HIP kernel's ``f`` literals do):

* constants ``cartpole_np.py:20-31``;
* ``physics`` = ``_physics`` ``cartpole_np.py:58-76``;
* ``terminated`` = ``_terminated`` ``cartpole_np.py:79-83``;
* ``step`` = ``step`` ``cartpole_np.py:39-55``: physics, done, a fresh state for
  every env, select by ``done``, reward 1.

Two deliberate differences from the reference, both needed for identical
results on two devices:

* the fresh state comes from the counter RNG of ``oracle.rng`` keyed by the
  step counter ``seed`` (the reference's Metal kernel's generator,
  ``cartpole_metal.py:39-51,89-93``), not from ``np.random``;
* sin and cos are ``oracle.detmath`` by default (``trig="numpy"`` selects the
  reference's own ``np.sin``/``np.cos``, used by the CPU timing baseline and by
  the tests that bound the difference).

``rollout_survived`` restates the fused ES kernel ``cartpole_rollout_metal.py:46-77``
(policy 4-H-2, first-index argmax, early exit) for a population.
"""

import numpy as np

from . import detmath, rng

F32 = np.float32

GRAVITY = 9.8
CART_MASS = 1.0
POLE_MASS = 0.1
TOTAL_MASS = CART_MASS + POLE_MASS
HALF_POLE_LENGTH = 0.5
POLE_MASS_LENGTH = POLE_MASS * HALF_POLE_LENGTH
FORCE_MAG = 10.0
TAU = 0.02
X_LIMIT = 2.4
THETA_LIMIT = 12 * 2 * np.pi / 360
RESET_BOUND = 0.05


def reset(n, seed=0):
    """(4, n) float32 fresh states: what the step kernel writes into a reset column at counter `seed`."""
    return rng.reset_rows4(seed, n, RESET_BOUND)


def physics(state, action, trig="det"):
    """One explicit-Euler step of Gym's CartPole for every column; ``cartpole_np.py:58-76``."""
    sin_f, cos_f, _ = detmath.trig_functions(trig)
    x, x_dot, theta, theta_dot = state
    force = np.where(np.asarray(action) == 1, FORCE_MAG, -FORCE_MAG).astype(F32)
    cos, sin = cos_f(theta), sin_f(theta)
    temp = (force + POLE_MASS_LENGTH * theta_dot**2 * sin) / TOTAL_MASS
    theta_acc = (GRAVITY * sin - cos * temp) / (
        HALF_POLE_LENGTH * (4.0 / 3.0 - POLE_MASS * cos**2 / TOTAL_MASS)
    )
    x_acc = temp - POLE_MASS_LENGTH * theta_acc * cos / TOTAL_MASS
    return np.stack(
        [
            x + TAU * x_dot,
            x_dot + TAU * x_acc,
            theta + TAU * theta_dot,
            theta_dot + TAU * theta_acc,
        ]
    ).astype(F32)


def terminated(state):
    """``cartpole_np.py:79-83``: |x| > 2.4 or |theta| > 12 degrees, compared in float32."""
    x, theta = state[0], state[2]
    return (np.abs(x) > X_LIMIT) | (np.abs(theta) > THETA_LIMIT)


def step(state, action, seed, trig="det"):
    """(next_state, reward, done) for step counter `seed`; ``cartpole_np.py:39-55``."""
    state = np.asarray(state, dtype=F32)
    n = state.shape[1]
    stepped = physics(state, action, trig)
    done = terminated(stepped)
    fresh = reset(n, seed)
    next_state = np.where(done[None, :], fresh, stepped).astype(F32)
    reward = np.ones(n, dtype=F32)
    return next_state, reward, done


def step_k(state, seed0, k, actions=None, trig="det"):
    """k chained steps with counters seed0, seed0+1, ...; actions (k, n) or, when None,
    the counter-RNG Bernoulli actions ``rng.action_bits(seed0 + t, n)``.
    Returns (final_state, rewards (k, n), dones (k, n))."""
    n = state.shape[1]
    rewards, dones = [], []
    for t in range(k):
        seed = (seed0 + t) & 0xFFFFFFFF
        a = rng.action_bits(seed, n) if actions is None else actions[t]
        state, r, d = step(state, a, seed, trig)
        rewards.append(r)
        dones.append(d)
    return state, np.stack(rewards), np.stack(dones)


def policy_logits(obs, w1, b1, w2, b2, trig="det"):
    """4-H-2 policy logits for a population in the fused kernel's summation order
    (``cartpole_rollout_metal.py:56-62``): hidden pre-activation
    ((o0 w0 + o1 w1) + o2 w2) + o3 w3 + b, then logits b2 + sum_j h_j w2[j] in j order.
    obs (4, P); w1 (P, 4, H); b1 (P, H); w2 (P, H, 2); b2 (P, 2). Returns (2, P)."""
    _, _, tanh_f = detmath.trig_functions(trig)
    hidden = w1.shape[2]
    l0 = b2[:, 0].copy()
    l1 = b2[:, 1].copy()
    for j in range(hidden):
        pre = obs[0] * w1[:, 0, j] + obs[1] * w1[:, 1, j] + obs[2] * w1[:, 2, j] + obs[3] * w1[:, 3, j] + b1[:, j]
        h = tanh_f(pre)
        l0 = l0 + h * w2[:, j, 0]
        l1 = l1 + h * w2[:, j, 1]
    return np.stack([l0, l1])


def rollout_survived(state, theta_pop, hidden, horizon, trig="det"):
    """Steps survived per member (P,) float32 from state (4, P) and theta_pop (P, 7H+2):
    ``cartpole_rollout_metal.py:46-77``. Members stop at their first termination; the
    terminating step is not counted."""
    from .es import unflatten

    state = np.asarray(state, dtype=F32).copy()
    w1, b1, w2, b2 = unflatten(np.asarray(theta_pop, dtype=F32), hidden, 4, 2)
    p = state.shape[1]
    alive = np.ones(p, dtype=bool)
    survived = np.zeros(p, dtype=F32)
    for _ in range(horizon):
        l0, l1 = policy_logits(state, w1, b1, w2, b2, trig)
        action = (l1 > l0).astype(np.int32)
        stepped = physics(state, action, trig)
        done = terminated(stepped)
        alive = alive & ~done
        survived = survived + alive.astype(F32)
        state = np.where(alive[None, :], stepped, state)
        if not alive.any():
            break
    return survived
