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


@pytest.mark.parametrize("k", [32, 64])
def test_rk4_full_size_with_terminations(dev, k):
    """The staged RK4 kernel (K = 32, 64) at the benchmark's N = 65,536: one step bit for bit
    against the oracle, with chains pointing up (terminated, every row reset U[+-0.1]) in
    some columns, random wide chains in most and near-rest chains in the first 4,096 (64
    waves that take the sin/cos polynomial)."""
    from hipenvs import pendulum_aba

    n = 65_536
    state, action = random_state(k, n, seed=640 + k)
    state[:, :4096] = oaba.Pendulum(k).reset(4096, seed=12)
    state[:k, 4096::89] = np.float32(np.pi)
    p = pendulum_aba.Pendulum(k)
    p.reseed(12)
    ns, rew, done = p.step(torch.from_numpy(state).to(dev), torch.from_numpy(action.astype(np.int32)).to(dev))
    ens, erew, edone = oaba.Pendulum(k).step(state, action, seed=13)
    assert edone.sum() >= (n - 4096) // 89
    np.testing.assert_array_equal(to_np(done), edone)
    np.testing.assert_array_equal(to_np(rew), erew)
    np.testing.assert_array_equal(to_np(ns), ens)


@pytest.mark.parametrize("k", [4, 16, 32, 64])
def test_rk4_reference_benchmark_chain(dev, k):
    """The reference's own benchmark shape for the RK4 drop-in (bench_aba.py:26-37): every
    row from the reset distribution, uniform actions in {0, 1, 2}, free-running; 16 steps at
    2,048 envs with identical states and flags."""
    from hipenvs import pendulum_aba

    n = 2048
    p = pendulum_aba.Pendulum(k)
    ref = oaba.Pendulum(k)
    s_dev = p.reset(n, seed=0, device=dev)
    s_ref = ref.reset(n, seed=0)
    np.testing.assert_array_equal(to_np(s_dev), s_ref)
    p.reseed(0)
    for t in range(1, 17):
        act = rng.uniform_actions(500 + t, n, 3)
        s_dev, _, d_dev = p.step(s_dev, torch.from_numpy(act).to(dev))
        s_ref, _, d_ref = ref.step(s_ref, act, seed=t)
        np.testing.assert_array_equal(to_np(d_dev), d_ref, err_msg=f"step {t}")
    np.testing.assert_array_equal(to_np(s_dev), s_ref)


def test_k64_past_32bit_offsets(dev):
    """The staged K = 64 kernels address the (128, n) arrays with 32-bit byte offsets, so from
    n = 4,194,304 (2 GiB per array) the RK4 and the Euler step take the generic kernels. One
    step of each at n = 4,194,304 + 200 (random wide chains drawn on the device), checked
    against the oracle on the first 256 columns, 64 in the middle and the last 456 (the
    envs are independent, so the oracle steps only those columns)."""
    from hipenvs import pendulum_aba

    k, n = 64, (1 << 22) + 200
    print(f"K = 64 past 32-bit offsets: n = {n}", flush=True)
    g = torch.Generator(device=dev).manual_seed(64)
    state = torch.empty((2 * k, n), device=dev)
    state[:k].uniform_(-np.pi, np.pi, generator=g)
    state[k:].uniform_(-1.0, 1.0, generator=g)
    cols = np.concatenate([np.arange(256), np.arange(n // 2, n // 2 + 64), np.arange(n - 456, n)])
    cols_dev = torch.from_numpy(cols).to(dev)
    sub = to_np(state[:, cols_dev])
    action = np.random.default_rng(5).integers(0, 3, n).astype(np.int32)
    torque = np.random.default_rng(6).uniform(-1, 1, n).astype(np.float32)
    p = pendulum_aba.Pendulum(k)
    p.reseed(20)
    ns, rew, done = p.step(state, torch.from_numpy(action).to(dev))
    ens, erew, edone = oaba.Pendulum(k).step(sub, action[cols], seed=21)
    assert not edone.any()  # the oracle's resets are keyed by column, so none may occur here
    np.testing.assert_array_equal(to_np(ns[:, cols_dev]), ens)
    np.testing.assert_array_equal(to_np(done[cols_dev]), edone)
    del ns
    p.reseed(30)
    ns, rew, done = p.step_euler(state, torch.from_numpy(torque).to(dev))
    ens, erew, edone = oaba.Pendulum(k).step_euler(sub, torque[cols], seed=31)
    assert not edone.any()
    np.testing.assert_array_equal(to_np(ns[:, cols_dev]), ens)
    np.testing.assert_array_equal(to_np(done[cols_dev]), edone)


def near_rest_states(k, seed):
    """Angles U[-0.38, 0.38] (every joint angle and every angle within 0.78 of zero), zero
    velocities, in six waves of 64 envs: waves 0 and 1 stay within the bound (wave 1 with one
    angle at 0.78 exactly), wave 2 has one root angle a float above 0.78, wave 3 one link at
    3.0, wave 4 one negative zero, wave 5 one link at -0.8."""
    r = np.random.default_rng(seed)
    n = 6 * 64
    s = np.zeros((2 * k, n), np.float32)
    s[:k] = r.uniform(-0.38, 0.38, (k, n)).astype(np.float32)
    s[0, 64 + 17] = np.float32(0.78)
    s[0, 128 + 5] = np.nextafter(np.float32(0.78), np.float32(1.0))
    s[k - 1, 192 + 40] = np.float32(3.0)
    s[0, 256 + 9] = np.float32(-0.0)
    s[k // 2, 320 + 63] = np.float32(-0.8)
    return s


@pytest.mark.parametrize("k", [4, 16, 32, 64])
def test_near_rest_waves_match_oracle(dev, k):
    """A wave whose angles all lie within 0.78 of zero takes the sin/cos polynomial without
    the range reduction; a wave with one angle outside takes the full reduction. Both give
    the oracle's bits: accelerations, the Euler step (with its termination cosines) and the
    RK4 step of the articulated-body model, and the mass-matrix model's step."""
    from hipenvs import pendulum, pendulum_aba

    state = near_rest_states(k, seed=300 + k)
    n = state.shape[1]
    s_dev = torch.from_numpy(state).to(dev)
    torque = rng.torque_uniform(5, n)
    t_dev = torch.from_numpy(torque).to(dev)
    p = pendulum_aba.Pendulum(k)
    np.testing.assert_array_equal(to_np(p.accelerations(s_dev, t_dev)),
                                  oaba.aba_accelerations(state[:k], state[k:], torque, k))
    p.reseed(2)
    ns, rew, done = p.step_euler(s_dev, t_dev)
    ens, erew, edone = oaba.Pendulum(k).step_euler(state, torque, seed=3)
    np.testing.assert_array_equal(to_np(ns), ens)
    np.testing.assert_array_equal(to_np(done), edone)
    action = np.random.default_rng(k).integers(0, 3, n)
    p.reseed(4)
    ns, rew, done = p.step(s_dev, torch.from_numpy(action.astype(np.int32)).to(dev))
    ens, erew, edone = oaba.Pendulum(k).step(state, action, seed=5)
    np.testing.assert_array_equal(to_np(ns), ens)
    np.testing.assert_array_equal(to_np(done), edone)
    if k <= 16:
        env = pendulum.Pendulum(k)
        env.reseed(6)
        nxt, rew, done = env.step(s_dev, torch.from_numpy(action.astype(np.int32)).to(dev))
        e_next, e_rew, e_done = mm.Pendulum(k).step(state, action.astype(np.int32), 7)
        np.testing.assert_array_equal(to_np(nxt), e_next)
        np.testing.assert_array_equal(to_np(done), e_done)
