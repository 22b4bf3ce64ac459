"""The hopper and the mass-matrix K-link pendulum (the reference's hopper_metal and
pendulum_metal) through the C ABI (GPU), against their oracles bit for bit: single
steps from mixed-regime states and 100-step trajectories with identical flags.
"""

import numpy as np
import pytest
import torch

from oracle import hopper as oh
from oracle import pendulum as op

pytestmark = pytest.mark.gpu


def to_np(t):
    return t.detach().cpu().numpy()


def hopper_states(n, seed=0):
    """test_hopper.py:116-121: feet below and above the floor, tilted legs, moving."""
    r = np.random.default_rng(seed)
    q = np.stack([r.uniform(-1, 1, n), r.uniform(0.7, 1.3, n), r.uniform(-0.6, 0.6, n), r.uniform(-0.8, 0.8, n)])
    v = r.uniform(-2, 2, (4, n))
    return np.concatenate([q, v]).astype(np.float32), r.integers(0, 3, n).astype(np.int32)


def pendulum_states(k, n, seed=0, vel=1.0):
    """test_pendulum.py:27-29: angles U[-pi, pi], velocities U[-vel, vel]."""
    r = np.random.default_rng(seed)
    s = np.concatenate([r.uniform(-np.pi, np.pi, (k, n)), r.uniform(-vel, vel, (k, n))]).astype(np.float32)
    return s, r.integers(0, 3, n).astype(np.int32)


def test_hopper_step_matches_oracle(dev):
    from hipenvs import hopper

    state, action = hopper_states(4000)
    state[1, :200] = 0.5   # torsos already below the fall height: these terminate and reset
    state[2, 200:400] = 1.2  # and tilted past the fall angle
    env = hopper.Hopper()
    env.reseed(77)
    nxt, rew, done = env.step(torch.from_numpy(state).to(dev), torch.from_numpy(action).to(dev))
    e_next, e_rew, e_done = oh.Hopper().step(state, action, 78)
    np.testing.assert_array_equal(to_np(done), e_done)
    np.testing.assert_array_equal(to_np(rew), e_rew)
    np.testing.assert_array_equal(to_np(nxt), e_next)
    assert 0 < e_done.sum() < len(e_done)


def test_hopper_step_at_the_benchmark_size(dev):
    """N = 65,536, the bench's hopper step shape."""
    from hipenvs import hopper

    state, action = hopper_states(1 << 16, seed=16)
    env = hopper.Hopper()
    env.reseed(8)
    nxt, rew, done = env.step(torch.from_numpy(state).to(dev), torch.from_numpy(action).to(dev))
    e_next, e_rew, e_done = oh.Hopper().step(state, action, 9)
    np.testing.assert_array_equal(to_np(done), e_done)
    np.testing.assert_array_equal(to_np(nxt), e_next)
    np.testing.assert_array_equal(to_np(rew), e_rew)


def test_hopper_trajectory_and_reset(dev):
    """100 steps from fresh resets with random actions: identical states and flags."""
    from hipenvs import hopper

    n = 512
    env = hopper.Hopper()
    env.reseed(0)
    state = env.reset(n, seed=5, device=dev)
    expect = oh.Hopper().reset(n, 5)
    np.testing.assert_array_equal(to_np(state), expect)
    r = np.random.default_rng(1)
    dones = 0
    for t in range(100):
        a = r.integers(0, 3, n).astype(np.int32)
        state, rew, done = env.step(state, torch.from_numpy(a).to(dev))
        expect, e_rew, e_done = oh.Hopper().step(expect, a, t + 1)
        np.testing.assert_array_equal(to_np(done), e_done, err_msg=f"step {t}")
        np.testing.assert_array_equal(to_np(state), expect, err_msg=f"step {t}")
        dones += int(e_done.sum())
    assert dones > 0


@pytest.mark.parametrize("k", [1, 2, 3, 4, 8, 16])
def test_pendulum_step_matches_oracle(dev, k):
    from hipenvs import pendulum

    state, action = pendulum_states(k, 1000, seed=k)
    env = pendulum.Pendulum(k)
    env.reseed(10)
    nxt, rew, done = env.step(torch.from_numpy(state).to(dev), torch.from_numpy(action).to(dev))
    e_next, e_rew, e_done = op.Pendulum(k).step(state, action, 11)
    np.testing.assert_array_equal(to_np(done), e_done)
    np.testing.assert_array_equal(to_np(rew), e_rew)
    np.testing.assert_array_equal(to_np(nxt), e_next)


def test_pendulum_step_at_the_benchmark_size(dev):
    """K = 16 at N = 65,536, the bench's largest mass-matrix pendulum shape."""
    from hipenvs import pendulum

    state, action = pendulum_states(16, 1 << 16, seed=16)
    env = pendulum.Pendulum(16)
    env.reseed(20)
    nxt, rew, done = env.step(torch.from_numpy(state).to(dev), torch.from_numpy(action).to(dev))
    e_next, e_rew, e_done = op.Pendulum(16).step(state, action, 21)
    np.testing.assert_array_equal(to_np(done), e_done)
    np.testing.assert_array_equal(to_np(nxt), e_next)
    np.testing.assert_array_equal(to_np(rew), e_rew)
    assert 0 < e_done.sum() < len(e_done)


@pytest.mark.parametrize("k", [2, 4, 16])
def test_pendulum_trajectory(dev, k):
    from hipenvs import pendulum

    n = 256
    env = pendulum.Pendulum(k)
    env.reseed(0)
    state = env.reset(n, seed=3, device=dev)
    expect = op.Pendulum(k).reset(n, 3)
    np.testing.assert_array_equal(to_np(state), expect)
    r = np.random.default_rng(k)
    for t in range(100):
        a = r.integers(0, 3, n).astype(np.int32)
        state, rew, done = env.step(state, torch.from_numpy(a).to(dev))
        expect, _, e_done = op.Pendulum(k).step(expect, a, t + 1)
        np.testing.assert_array_equal(to_np(done), e_done, err_msg=f"step {t}")
        np.testing.assert_array_equal(to_np(state), expect, err_msg=f"step {t}")


@pytest.mark.parametrize("k", [2, 8, 16])
def test_pendulum_accelerations_match_oracle_and_aba(dev, k):
    """The mass-matrix solve bit for bit against its oracle, and within float32 rounding of
    the articulated-body algorithm's accelerations for the same states."""
    from hipenvs import pendulum, pendulum_aba

    state, _ = pendulum_states(k, 512, seed=100 + k)
    torque = np.random.default_rng(k).uniform(-1, 1, 512).astype(np.float32)
    s, t = torch.from_numpy(state).to(dev), torch.from_numpy(torque).to(dev)
    got = to_np(pendulum.Pendulum(k).accelerations(s, t))
    np.testing.assert_array_equal(got, op.mass_matrix_dsdt(state, torque, k, trig="det")[k:])
    aba = to_np(pendulum_aba.Pendulum(k).accelerations(s, t))
    ref = op.mass_matrix_accelerations_f64(state[:k], state[k:], torque, k)
    scale = np.abs(ref).max(axis=0) + 1.0
    assert np.all(np.abs(got - ref) <= 1e-3 * scale)
    assert np.all(np.abs(aba - ref) <= 1e-3 * scale)
