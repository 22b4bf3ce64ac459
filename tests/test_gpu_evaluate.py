"""Fused greedy evaluation through the C ABI (GPU): per-env scores against the oracle bit
for bit, and the learner's score against the reference-shaped torch loop.
"""

import numpy as np
import pytest
import torch

from oracle import acrobot as oa
from oracle import cartpole as oc
from oracle import es as oes
from oracle import legged as olg

pytestmark = pytest.mark.gpu


def to_np(t):
    return t.detach().cpu().numpy()


def shared_theta(d, seed, scale=0.5):
    return (np.random.default_rng(seed).standard_normal(d) * scale).astype(np.float32)


@pytest.mark.parametrize("n", [2048, 20_000])
@pytest.mark.parametrize("hidden", [8, 32])
def test_cartpole_and_acrobot_evaluate_match_oracle(dev, n, hidden):
    """n = 2,048 (the learner's evaluation, lane groups) and 20,000 (one env per lane)."""
    from hipenvs import acrobot_rollout, cartpole_rollout

    theta = shared_theta(7 * hidden + 2, hidden)
    state = oc.reset(n, seed=21)
    got = cartpole_rollout.evaluate(torch.from_numpy(state).to(dev), torch.from_numpy(theta).to(dev), hidden, 300)
    expect = oc.rollout_survived(state, np.broadcast_to(theta, (n, theta.size)), hidden, 300)
    np.testing.assert_array_equal(to_np(got), expect)

    theta = shared_theta(10 * hidden + 3, hidden + 1)
    state = oa.reset(n, seed=22)
    got = acrobot_rollout.evaluate(torch.from_numpy(state).to(dev), torch.from_numpy(theta).to(dev), hidden, 100)
    expect = -oa.rollout_steps(state, np.broadcast_to(theta, (n, theta.size)), hidden, 100) + np.float32(0.0)
    np.testing.assert_array_equal(to_np(got), expect)
    assert not np.any(np.signbit(to_np(got)) & (to_np(got) == 0))  # no -0 scores


@pytest.mark.parametrize("c,hidden", [(1, 8), (2, 16), (3, 32), (4, 64)])
def test_legged_evaluate_matches_oracle(dev, c, hidden):
    from hipenvs import legged, legged_rollout

    n, steps = 256, 80
    theta = shared_theta(legged_rollout.n_params(hidden, c), c * hidden, scale=0.3)
    state = legged.Legged(c).reset(n, seed=23, device=dev)
    got = legged_rollout.evaluate(state, torch.from_numpy(theta).to(dev), hidden, steps, c)
    expect = olg.evaluate_fused(to_np(state), theta, hidden, steps, c)
    np.testing.assert_array_equal(to_np(got), expect)
    assert np.any(expect != 0)


def standing_theta(hidden, c, scale=0.02, seed=5):
    """Small random weights and head biases that favour each leg's middle (zero-torque) action:
    a policy under which the bodies stand for the whole evaluation, as a trained one does."""
    from hipenvs import legged_rollout

    obs, out = 5 + 2 * c, 3 * c
    theta = shared_theta(legged_rollout.n_params(hidden, c), seed, scale=scale)
    b2 = obs * hidden + hidden + hidden * out
    for leg in range(c):
        theta[b2 + 3 * leg + 1] = 1.0
    return theta


@pytest.mark.parametrize("c,hidden", [(2, 64), (3, 16), (4, 64)])
def test_legged_evaluate_standing_policy(dev, c, hidden):
    """Long episodes in the group form (batches of at most one wave per SIMD): most envs stand
    for every step, and the per-env sums equal the oracle's bit for bit."""
    from hipenvs import legged, legged_rollout

    n, steps = 300, 150
    theta = standing_theta(hidden, c)
    state = legged.Legged(c).reset(n, seed=31, device=dev)
    got = legged_rollout.evaluate(state, torch.from_numpy(theta).to(dev), hidden, steps, c, eval_bonus=10.0)
    expect = olg.evaluate_fused(to_np(state), theta, hidden, steps, c, eval_bonus=10.0)
    np.testing.assert_array_equal(to_np(got), expect)
    assert np.mean(expect > 10.0 * (steps - 1)) > 0.5  # most envs stood to the end (10 per step)


def test_legged_evaluate_one_lane_form(dev):
    """A batch past the group form's bound (16 envs per CU at C = 4) runs one env per lane:
    the same sums as the oracle."""
    from hipenvs import legged, legged_rollout

    c, hidden, steps = 4, 16, 24
    n = 16 * torch.cuda.get_device_properties(dev).multi_processor_count + 37
    theta = standing_theta(hidden, c, scale=0.2, seed=6)
    state = legged.Legged(c).reset(n, seed=32, device=dev)
    got = legged_rollout.evaluate(state, torch.from_numpy(theta).to(dev), hidden, steps, c)
    expect = olg.evaluate_fused(to_np(state), theta, hidden, steps, c)
    np.testing.assert_array_equal(to_np(got), expect)


@pytest.mark.parametrize("task_name", ["cartpole", "acrobot", "legged2"])
def test_learner_score_matches_torch_loop(dev, task_name):
    """es.evaluate_theta (one fused launch) against es.evaluate with the torch mean policy and
    the env step per iteration (the reference's loop): the same episodes up to the policy's
    summation order (a matmul in the loop), so per-env scores agree for nearly every env."""
    from hipenvs import es

    task = es.TASKS[task_name]
    hidden = 16
    d = es.n_params(hidden, task)
    theta = torch.from_numpy(shared_theta(d, 7, scale=0.3)).to(dev)
    fused = es.evaluate_theta(task, theta, hidden, n=2048, steps=200, device=dev)
    loop = es.evaluate(task, es.mean_policy(theta, hidden, task), n=2048, steps=200, device=dev)
    assert abs(fused - loop) <= 0.02 * max(1.0, abs(loop)), (fused, loop)
