"""ABA pendulum HIP kernels vs the oracle, through the C ABI (GPU). Bar: bit-exact."""

import numpy as np
import pytest
import torch

from oracle import pendulum as mm
from oracle import pendulum_aba as oaba
from oracle import rng
from test_oracle_pendulum_aba import random_state

pytestmark = pytest.mark.gpu
KS = [1, 2, 3, 4, 8, 16, 32, 64]


def to_np(t):
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("k", KS)
def test_accelerations_match_oracle(dev, k):
    from hipenvs import pendulum_aba

    state, _ = random_state(k, 300, seed=k)
    torque = np.random.default_rng(k).uniform(-1, 1, 300).astype(np.float32)
    got = pendulum_aba.Pendulum(k).accelerations(torch.from_numpy(state).to(dev), torch.from_numpy(torque).to(dev))
    np.testing.assert_array_equal(to_np(got), oaba.aba_accelerations(state[:k], state[k:], torque, k))


@pytest.mark.parametrize("k", KS)
def test_rk4_step_matches_oracle(dev, k):
    """test_pendulum_aba.py:44-54's states, every column compared."""
    from hipenvs import pendulum_aba

    state, action = random_state(k, 200, seed=k)
    p = pendulum_aba.Pendulum(k)
    p.reseed(6)
    ns, rew, done = p.step(torch.from_numpy(state).to(dev), torch.from_numpy(action.astype(np.int32)).to(dev))
    ens, erew, edone = oaba.Pendulum(k).step(state, action, seed=7)
    np.testing.assert_array_equal(to_np(ns), ens)
    np.testing.assert_array_equal(to_np(rew), erew)
    np.testing.assert_array_equal(to_np(done), edone)


@pytest.mark.parametrize("k", KS)
def test_euler_step_matches_oracle(dev, k):
    from hipenvs import pendulum_aba

    state, _ = random_state(k, 257, seed=100 + k)
    torque = rng.torque_uniform(9, 257)
    p = pendulum_aba.Pendulum(k)
    p.reseed(8)
    ns, rew, done = p.step_euler(torch.from_numpy(state).to(dev), torch.from_numpy(torque).to(dev))
    ens, erew, edone = oaba.Pendulum(k).step_euler(state, torque, seed=9)
    np.testing.assert_array_equal(to_np(ns), ens)
    np.testing.assert_array_equal(to_np(done), edone)
    p.reseed(8)
    ns2, _, _ = p.step_euler(torch.from_numpy(state).to(dev))     # in-kernel counter-RNG torques
    np.testing.assert_array_equal(to_np(ns2), ens)


@pytest.mark.parametrize("k", [4, 16, 64])
def test_config3_euler_chain(dev, k):
    """The K-link configuration: angles U[-0.1, 0.1], velocities 0, torques U[-1, 1] per step,
    semi-implicit Euler dt 0.01; 50 free-running steps with identical states and flags."""
    from hipenvs import pendulum_aba

    n = 2048
    p = pendulum_aba.Pendulum(k)
    ref = oaba.Pendulum(k)
    s_dev = p.reset(n, seed=0, device=dev, zero_velocity=True)
    s_ref = ref.reset_euler(n, seed=0)
    np.testing.assert_array_equal(to_np(s_dev), s_ref)
    p.reseed(0)
    for t in range(1, 51):
        s_dev, _, d_dev = p.step_euler(s_dev)
        s_ref, _, d_ref = ref.step_euler(s_ref, None, seed=t)
        np.testing.assert_array_equal(to_np(d_dev), d_ref, err_msg=f"step {t}")
    np.testing.assert_array_equal(to_np(s_dev), s_ref)


def test_resets_and_lazy_chain(dev):
    """test_pendulum_aba.py:57-69 on the device."""
    from hipenvs import pendulum_aba

    p = pendulum_aba.Pendulum(8)
    n = 4096
    up = torch.zeros((16, n), device=dev)
    up[:8] = np.pi
    ones = torch.ones(n, dtype=torch.int32, device=dev)
    first = to_np(p.step(up, ones)[0])
    second = to_np(p.step(up, ones)[0])
    assert np.all(np.abs(first) <= oaba.RESET_BOUND) and not np.allclose(first, second)
    state = p.reset(n, device=dev)
    for _ in range(100):
        state, _, _ = p.step(state, torch.randint(0, 3, (n,), device=dev, dtype=torch.int32))
    out = to_np(state)
    assert np.isfinite(out).all() and np.all(np.abs(out[:8]) <= np.pi)


def test_k64_euler_full_size_with_terminations(dev):
    """The staged K = 64 Euler kernel at the benchmark's N = 65,536: one step bit for bit
    against the oracle, with chains pointing up (terminated, reset to angles U[+-0.1] and
    zero velocities) in some columns and random chains elsewhere."""
    from hipenvs import pendulum_aba

    k, n = 64, 65_536
    state, _ = random_state(k, n, seed=64)
    state[:k, ::97] = np.float32(np.pi)  # tip at height 64 > 32: these terminate
    torque = rng.torque_uniform(11, n)
    p = pendulum_aba.Pendulum(k)
    p.reseed(10)
    ns, rew, done = p.step_euler(torch.from_numpy(state).to(dev), torch.from_numpy(torque).to(dev))
    ens, erew, edone = oaba.Pendulum(k).step_euler(state, torque, seed=11)
    assert edone.sum() >= n // 97
    np.testing.assert_array_equal(to_np(done), edone)
    np.testing.assert_array_equal(to_np(rew), erew)
    np.testing.assert_array_equal(to_np(ns), ens)
