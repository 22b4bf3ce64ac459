"""The fused greedy evaluation against the reference's evaluation loop, in the oracle (CPU).

``es.py:308-322`` steps every env each iteration through the env step (auto-reset),
clears ``alive`` at the first termination and sums ``(reward - 1 + eval_bonus) * alive``.
The fused evaluation kernels stop each env at its first termination instead. Here the
early-exit restatements that the kernels follow equal the reference-shaped loop over the
oracle's env steps, per env and bit for bit, for all three bodies.
"""

import numpy as np
import pytest

from oracle import acrobot as oa
from oracle import cartpole as oc
from oracle import es as oes
from oracle import legged as olg

F32 = np.float32


def shared_theta(d, seed, scale=0.5):
    return (np.random.default_rng(seed).standard_normal(d) * scale).astype(F32)


def broadcast(theta, n):
    return np.broadcast_to(theta, (n, theta.shape[0])).copy()


def test_cartpole_evaluate_is_steps_survived():
    hidden, n, steps = 8, 128, 150
    theta = shared_theta(7 * hidden + 2, 1)
    w = oes.unflatten(broadcast(theta, n), hidden, 4, 2)
    state = oc.reset(n, seed=11)

    def action_of(s):
        l0, l1 = oc.policy_logits(s, *w)
        return (l1 > l0).astype(np.int32)

    loop = oes.evaluate_loop(oc.step, action_of, state, steps, seed0=100, eval_bonus=1.0)
    fused = oc.rollout_survived(state, broadcast(theta, n), hidden, steps)
    np.testing.assert_array_equal(loop, fused)
    assert 0 < fused.mean() < steps


def test_acrobot_evaluate_is_minus_steps():
    hidden, n, steps = 8, 96, 120
    theta = shared_theta(10 * hidden + 3, 2)
    w = oes.unflatten(broadcast(theta, n), hidden, 6, 3)
    state = oa.reset(n, seed=12)

    def action_of(s):
        return oes.first_argmax(oa.policy_logits(s, *w)).astype(np.int32)

    loop = oes.evaluate_loop(oa.step, action_of, state, steps, seed0=200, eval_bonus=1.0)
    fused = -oa.rollout_steps(state, broadcast(theta, n), hidden, steps)
    np.testing.assert_array_equal(loop, fused + F32(0.0))
    assert fused.min() < 0


@pytest.mark.parametrize("c", [1, 2, 3, 4])
def test_legged_evaluate_is_forward_distance(c):
    hidden, n, steps = 8, 48, 60
    theta = shared_theta(olg_n_params(hidden, c), 3 + c, scale=0.3)
    w = oes.unflatten(broadcast(theta, n), hidden, 5 + 2 * c, 3 * c)
    body = olg.Legged(c)
    state = body.reset(n, seed=13)

    def action_of(s):
        q, v = s[:3 + c], s[3 + c:]
        return oes.legged_action(olg.policy_logits(q, v, *w, c).T, c)

    loop = oes.evaluate_loop(body.step, action_of, state, steps, seed0=300, eval_bonus=0.0)
    fused = olg.evaluate_fused(state, theta, hidden, steps, c)
    np.testing.assert_array_equal(loop, fused)
    assert np.any(fused != 0)


def olg_n_params(hidden, c):
    return oes.n_params(hidden, 5 + 2 * c, 3 * c)
