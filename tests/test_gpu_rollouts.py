"""Fused ES rollout kernels vs the oracle, through the C ABI (GPU).

Bar: bit-exact fitness for every member. The oracle's fused-rollout restatement
is itself checked against its es.loop_fitness restatement (test_oracle_es.py),
which is the reference's test_es.py:46-69 gate made exact.
"""

import numpy as np
import pytest
import torch

from oracle import acrobot as oa
from oracle import cartpole as oc
from oracle import es as oes

pytestmark = pytest.mark.gpu


def to_np(t):
    return t.detach().cpu().numpy()


def population(p, d, seed, scale=None, sigma=0.1):
    """theta_pop: scale * N(0,1) rows, or (scale None) the antithetic ES population
    theta0 + sigma * [half; -half] around theta0 = 0.1 * N(0, 1)."""
    r = np.random.default_rng(seed)
    if scale is not None:
        return (r.standard_normal((p, d)) * scale).astype(np.float32)
    theta0 = (r.standard_normal(d) * 0.1).astype(np.float32)
    half = r.standard_normal((p // 2, d)).astype(np.float32)
    eps = np.concatenate([half, -half])
    return (theta0[None, :] + np.float32(sigma) * eps).astype(np.float32)


@pytest.mark.parametrize("hidden", [4, 8, 16, 32, 64])
def test_cartpole_rollout_matches_oracle(dev, hidden):
    from hipenvs import cartpole_rollout

    p, horizon = 512, 200
    theta = population(p, 7 * hidden + 2, hidden, scale=0.5)
    state = oc.reset(p, seed=3)
    got = cartpole_rollout.rollout_steps(torch.from_numpy(state).to(dev), torch.from_numpy(theta).to(dev), hidden, horizon)
    np.testing.assert_array_equal(to_np(got), oc.rollout_survived(state, theta, hidden, horizon))


@pytest.mark.parametrize("hidden", [4, 8, 16, 32, 64])
def test_acrobot_rollout_matches_oracle(dev, hidden):
    from hipenvs import acrobot_rollout

    p, horizon = 512, 120
    theta = population(p, 10 * hidden + 3, hidden, scale=0.5)
    state = oa.reset(p, seed=4)
    got = acrobot_rollout.rollout_steps(torch.from_numpy(state).to(dev), torch.from_numpy(theta).to(dev), hidden, horizon)
    np.testing.assert_array_equal(to_np(got), oa.rollout_steps(state, theta, hidden, horizon))


@pytest.mark.parametrize("hidden", [8, 32])
def test_large_populations_one_member_per_lane(dev, hidden):
    """Populations above the lane-group limit (16 members per CU) run one member per lane;
    both bodies, bit for bit against the oracle."""
    from hipenvs import acrobot_rollout, cartpole_rollout

    p = 20_000
    theta = population(p, 7 * hidden + 2, 100 + hidden, scale=0.5)
    state = oc.reset(p, seed=5)
    got = cartpole_rollout.rollout_steps(torch.from_numpy(state).to(dev), torch.from_numpy(theta).to(dev), hidden, 150)
    np.testing.assert_array_equal(to_np(got), oc.rollout_survived(state, theta, hidden, 150))
    theta = population(p, 10 * hidden + 3, 200 + hidden, scale=0.5)
    state = oa.reset(p, seed=6)
    got = acrobot_rollout.rollout_steps(torch.from_numpy(state).to(dev), torch.from_numpy(theta).to(dev), hidden, 60)
    np.testing.assert_array_equal(to_np(got), oa.rollout_steps(state, theta, hidden, 60))


def test_config2_cartpole_population(dev):
    """P = 4,096 antithetic members (sigma 0.1) around theta0 = 0.1 N(0,1), H = 32, horizon 500."""
    from hipenvs import cartpole_rollout

    p, hidden, horizon = 4096, 32, 500
    theta = population(p, 7 * hidden + 2, 0)
    state = oc.reset(p, seed=0)
    got = to_np(cartpole_rollout.rollout_steps(torch.from_numpy(state).to(dev), torch.from_numpy(theta).to(dev),
                                               hidden, horizon))
    np.testing.assert_array_equal(got, oc.rollout_survived(state, theta, hidden, horizon))


def test_config2_acrobot_population(dev):
    from hipenvs import acrobot_rollout

    p, hidden, horizon = 4096, 32, 500
    theta = population(p, 10 * hidden + 3, 1)
    state = oa.reset(p, seed=0)
    got = to_np(acrobot_rollout.rollout_steps(torch.from_numpy(state).to(dev), torch.from_numpy(theta).to(dev),
                                              hidden, horizon))
    np.testing.assert_array_equal(got, oa.rollout_steps(state, theta, hidden, horizon))


def test_rollout_edge_cases(dev):
    """Horizon 0, a single member, a population that is not a multiple of the wave size."""
    from hipenvs import cartpole_rollout

    for p, horizon in ((1, 50), (65, 0), (130, 7)):
        theta = population(p, 7 * 8 + 2, p, scale=1.0)
        state = oc.reset(p, seed=p)
        got = cartpole_rollout.rollout_steps(torch.from_numpy(state).to(dev), torch.from_numpy(theta).to(dev), 8, horizon)
        np.testing.assert_array_equal(to_np(got), oc.rollout_survived(state, theta, 8, horizon))


def test_unsupported_hidden_raises(dev):
    from hipenvs import cartpole_rollout

    with pytest.raises(ValueError):
        cartpole_rollout.rollout_steps(torch.zeros((4, 8), device=dev), torch.zeros((8, 7 * 5 + 2), device=dev), 5, 10)
