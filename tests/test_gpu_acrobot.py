"""Acrobot HIP step kernel vs the oracle, through the C ABI (GPU). Bar: bit-exact."""

import numpy as np
import pytest
import torch

from oracle import acrobot as oa
from oracle import rng
from test_oracle_acrobot import random_batch

pytestmark = pytest.mark.gpu


def to_np(t):
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("n", [1, 200, 4096, 5000])
def test_step_matches_oracle_on_random_states(dev, n):
    """test_acrobot.py:98-122's random states, every column compared (terminal ones too)."""
    from hipenvs import acrobot

    state, action = random_batch(n, seed=n)
    acrobot.reseed(10)
    ns, rew, done = acrobot.step(torch.from_numpy(state).to(dev), torch.from_numpy(action).to(dev))
    ens, erew, edone = oa.step(state, action, seed=11)
    np.testing.assert_array_equal(to_np(ns), ens)
    np.testing.assert_array_equal(to_np(rew), erew)
    np.testing.assert_array_equal(to_np(done), edone)


def test_step_bit_exact_at_the_benchmark_size(dev):
    """N = 262,144, the reference's Acrobot step benchmark shape, with mixed terminations."""
    from hipenvs import acrobot

    state, action = random_batch(1 << 18, seed=18)
    acrobot.reseed(30)
    ns, rew, done = acrobot.step(torch.from_numpy(state).to(dev), torch.from_numpy(action).to(dev))
    ens, erew, edone = oa.step(state, action, seed=31)
    np.testing.assert_array_equal(to_np(done), edone)
    np.testing.assert_array_equal(to_np(ns), ens)
    np.testing.assert_array_equal(to_np(rew), erew)
    assert 0 < edone.sum() < len(edone)


def test_reset_matches_counter_rng(dev):
    from hipenvs import acrobot

    np.testing.assert_array_equal(to_np(acrobot.reset(3000, seed=4, device=dev)), oa.reset(3000, seed=4))


def test_teacher_forced_and_free_running_chains(dev):
    """300 teacher-forced steps (each step from the oracle's state) then 100 free-running
    steps with identical done flags at every step."""
    from hipenvs import acrobot

    n = 4096
    state = oa.reset(n, seed=0)
    acrobot.reseed(0)
    for t in range(1, 301):
        a = rng.uniform_actions(t, n, 3)
        ns, _, done = acrobot.step(torch.from_numpy(state).to(dev), torch.from_numpy(a).to(dev))
        ens, _, edone = oa.step(state, a, seed=t)
        assert np.array_equal(to_np(ns), ens) and np.array_equal(to_np(done), edone), f"step {t}"
        state = ens
    s_dev = torch.from_numpy(state).to(dev)
    for t in range(301, 401):
        a = rng.uniform_actions(t, n, 3)
        s_dev, _, d_dev = acrobot.step(s_dev, torch.from_numpy(a).to(dev))
        state, _, d_ref = oa.step(state, a, seed=t)
        np.testing.assert_array_equal(to_np(d_dev), d_ref, err_msg=f"step {t}")
    np.testing.assert_array_equal(to_np(s_dev), state)


def test_resets_and_lazy_chain(dev):
    """test_acrobot.py:125-146 on the device."""
    from hipenvs import acrobot

    n = 4096
    terminal = torch.zeros((4, n), device=dev)
    terminal[0] = np.pi
    ones = torch.ones(n, dtype=torch.int32, device=dev)
    first = to_np(acrobot.step(terminal, ones)[0])
    second = to_np(acrobot.step(terminal, ones)[0])
    assert np.all(np.abs(first) <= oa.RESET_BOUND) and not np.allclose(first, second)
    assert abs(first.std() - oa.RESET_BOUND / np.sqrt(3)) < 0.002
    state = acrobot.reset(n, device=dev)
    for t in range(100):
        state, _, _ = acrobot.step(state, torch.randint(0, 3, (n,), device=dev, dtype=torch.int32))
    out = to_np(state)
    assert np.isfinite(out).all() and np.all(np.abs(out[:2]) <= np.pi)
