"""CartPole HIP kernels vs the oracle, through the C ABI (GPU).

Bar: bit-exact. The kernels and the oracle evaluate the same float32 program
(reference op order, no FMA, deterministic transcendentals, counter RNG), so
next_state, reward and done must be identical, and termination/reset flags
identical over the whole horizon. The reference's own gate was atol 1e-4 on
live columns (test_cartpole.py:147-157); this is strictly stronger.
"""

import numpy as np
import pytest
import torch

from oracle import cartpole as oc
from oracle import detmath, rng

pytestmark = pytest.mark.gpu


def to_np(t):
    return t.detach().cpu().numpy()


def assert_same_floats(got, expect):
    """Bit-exact equality of values (+0 == -0, NaN == NaN)."""
    np.testing.assert_array_equal(np.asarray(got), np.asarray(expect))


def test_device_detmath_bit_exact(dev):
    from hipenvs import _lib

    r = np.random.default_rng(0)
    x = np.concatenate([
        r.uniform(-1, 1, 300_000), r.uniform(-40, 40, 300_000), r.uniform(-1e5, 1e5, 200_000),
        r.standard_normal(200_000) * 3,
        (np.arange(1, 50_000) * np.pi / 2),
        [0.0, -0.0, 1e-30, -1e-38, np.inf, -np.inf, np.nan, 256.0, -256.0, 256.00003, 3e9, 10.0, 20.0, -45.0],
    ]).astype(np.float32)
    xt = torch.from_numpy(x).to(dev)
    s, c, t = torch.empty_like(xt), torch.empty_like(xt), torch.empty_like(xt)
    _lib.call("hipenvs_detmath", _lib.ptr(xt), _lib.ptr(s), _lib.ptr(c), _lib.ptr(t), x.size, _lib.stream_of(dev))
    es, ec = detmath.sincos(x)
    assert_same_floats(to_np(s), es)
    assert_same_floats(to_np(c), ec)
    assert_same_floats(to_np(t), detmath.tanh(x))


def test_sample_actions_and_reset_match_the_counter_rng(dev):
    from hipenvs import cartpole

    for n in (1, 5, 4096, 100_003):
        a = cartpole.sample_actions(n, seed=77, device=dev)
        np.testing.assert_array_equal(to_np(a), rng.action_bits(77, n))
        u = cartpole.sample_actions(n, seed=78, m=81, device=dev)
        np.testing.assert_array_equal(to_np(u), rng.uniform_actions(78, n, 81))
        s = cartpole.reset(n, seed=12, device=dev)
        assert_same_floats(to_np(s), oc.reset(n, seed=12))


@pytest.mark.parametrize("offset", [0, 1, 2, 3])
def test_sample_actions_into_rows_at_any_alignment(dev, offset):
    """The sampler writes several consecutive envs per thread, as 16-byte vectors where the
    row is 16-byte aligned: rows at every 4-byte offset (out = a slice of a larger buffer),
    with lengths on and off multiples of 16, each equal to the counter RNG's draws and with
    the elements around the row untouched."""
    from hipenvs import cartpole

    for n in (1, 7, 16, 33, 262_144 + 5):
        buf = torch.full((n + 8,), -7, dtype=torch.int32, device=dev)
        out = buf[offset:offset + n]
        cartpole.sample_actions(n, seed=91, device=dev, out=out)
        got = to_np(buf)
        np.testing.assert_array_equal(got[offset:offset + n], rng.action_bits(91, n))
        assert (got[:offset] == -7).all() and (got[offset + n:] == -7).all()
        cartpole.sample_actions(n, seed=92, m=3, device=dev, out=out)
        np.testing.assert_array_equal(to_np(out), rng.uniform_actions(92, n, 3))


@pytest.mark.parametrize("n", [1, 3, 100, 4096, 4099])
def test_step_matches_oracle_on_random_states(dev, n):
    """Random states in [-1, 1] (test_cartpole.py:33-37), sizes on and off multiples of the
    wave and block sizes; every column compared, terminal ones included."""
    from hipenvs import cartpole

    r = np.random.default_rng(n)
    state = r.uniform(-1, 1, size=(4, n)).astype(np.float32)
    action = r.integers(0, 2, size=n).astype(np.int32)
    cartpole.reseed(41)
    ns, rew, done = cartpole.step(torch.from_numpy(state).to(dev), torch.from_numpy(action).to(dev))
    ens, erew, edone = oc.step(state, action, seed=42)
    assert_same_floats(to_np(ns), ens)
    assert_same_floats(to_np(rew), erew)
    np.testing.assert_array_equal(to_np(done), edone)
    assert ns.dtype == torch.float32 and rew.dtype == torch.float32 and done.dtype == torch.bool


def assert_same_bits(got, expect):
    """Bit-pattern equality, the sign of zero included; any NaN equals any NaN."""
    got, expect = np.asarray(got, dtype=np.float32), np.asarray(expect, dtype=np.float32)
    both_nan = np.isnan(got) & np.isnan(expect)
    np.testing.assert_array_equal(np.where(both_nan, 0, got.view(np.uint32)),
                                  np.where(both_nan, 0, expect.view(np.uint32)))


def test_step_bit_exact_on_extreme_states(dev):
    """Signed zeros, subnormals, huge angles (the float64 reduction), infinities and NaN in
    every state row: the constant divisions, the sin/cos reduction and the termination test
    agree with numpy's float32 arithmetic bit for bit, sign of zero included."""
    from hipenvs import cartpole

    specials = np.array([0.0, -0.0, 1e-40, -1e-40, 1e-45, 3e-39, 1e-20, -7e-12, 0.3, -2.0, 300.0, -1e5, 3.4e38,
                         -3.4e38, np.inf, -np.inf, np.nan], dtype=np.float32)
    r = np.random.default_rng(5)
    n = 4096
    state = r.choice(specials, size=(4, n)).astype(np.float32)
    state[:, :64] = 0.0
    state[2, :32] = -0.0
    action = r.integers(0, 2, size=n).astype(np.int32)
    cartpole.reseed(90)
    ns, rew, done = cartpole.step(torch.from_numpy(state).to(dev), torch.from_numpy(action).to(dev))
    with np.errstate(all="ignore"):
        ens, erew, edone = oc.step(state, action, seed=91)
    assert_same_bits(to_np(ns), ens)
    assert_same_bits(to_np(rew), erew)
    np.testing.assert_array_equal(to_np(done), edone)


def test_terminal_fixture(dev):
    """test_cartpole.py:147-157 with the fixture of test_cartpole.py:58-63."""
    from hipenvs import cartpole

    state = np.zeros((4, 3), dtype=np.float32)
    state[0, 0] = 2.5
    state[2, 1] = 0.3
    cartpole.reseed(0)
    ns, rew, done = cartpole.step(torch.from_numpy(state).to(dev), torch.ones(3, dtype=torch.int32, device=dev))
    assert to_np(done).tolist() == [True, True, False]
    assert np.all(np.abs(to_np(ns)[:, :2]) <= oc.RESET_BOUND)
    assert to_np(rew).tolist() == [1.0, 1.0, 1.0]
    assert_same_floats(to_np(ns)[:, 2], oc.physics(state, np.ones(3))[:, 2])


def test_config0_teacher_forced_1000_steps(dev):
    """N = 4,096, uniform[-0.05, 0.05] states from the seed, Bernoulli(0.5) actions,
    1,000 steps. Each step's input is the oracle's state (teacher forcing), so every
    step is compared from identical inputs; bit-exact, hence within the 1e-5 bar."""
    from hipenvs import cartpole

    n, steps = 4096, 1000
    state = oc.reset(n, seed=0)
    cartpole.reseed(0)
    total_done = 0
    for t in range(1, steps + 1):
        action = rng.action_bits(t, n)
        ns, rew, done = cartpole.step(torch.from_numpy(state).to(dev), torch.from_numpy(action).to(dev))
        ens, erew, edone = oc.step(state, action, seed=t)
        got_ns, got_done = to_np(ns), to_np(done)
        if not (np.array_equal(got_ns, ens) and np.array_equal(got_done, edone)):
            bad = np.flatnonzero((got_ns != ens).any(axis=0) | (got_done != edone))
            raise AssertionError(f"step {t}: {bad.size} columns differ, first {bad[:5]}")
        assert (to_np(rew) == 1.0).all()
        total_done += int(edone.sum())
        state = ens
    assert total_done > n * steps / 60, "a random policy terminates every ~22 steps"


def test_free_running_flags_identical_over_100_steps(dev):
    """Kernel-only chain of 100 steps against the oracle's chain: identical done flags at
    every step and identical final states (the flag-identity bar over 100 steps)."""
    from hipenvs import cartpole

    n = 4096
    cartpole.reseed(500)
    s_dev = cartpole.reset(n, seed=3, device=dev)
    s_ref = oc.reset(n, seed=3)
    for t in range(501, 601):
        a = cartpole.sample_actions(n, seed=t, device=dev)
        s_dev, _, d_dev = cartpole.step(s_dev, a)
        s_ref, _, d_ref = oc.step(s_ref, rng.action_bits(t, n), seed=t)
        np.testing.assert_array_equal(to_np(d_dev), d_ref, err_msg=f"step {t}")
    assert_same_floats(to_np(s_dev), s_ref)
    assert not oc.terminated(to_np(s_dev)).any()


@pytest.mark.parametrize("n", [4096, 4098])
@pytest.mark.parametrize("array_actions", [True, False])
def test_step_k_equals_k_single_steps(dev, n, array_actions):
    from hipenvs import cartpole

    k = 32
    s0 = cartpole.reset(n, seed=5, device=dev)
    acts = torch.stack([cartpole.sample_actions(n, seed=1000 + t, device=dev) for t in range(k)])
    cartpole.reseed(999)
    fin, rewards, dones = cartpole.step_k(s0, k, acts if array_actions else None)
    cartpole.reseed(999)
    s = s0
    for t in range(k):
        s, r, d = cartpole.step(s, acts[t])
        assert_same_floats(to_np(rewards[t]), to_np(r))
        np.testing.assert_array_equal(to_np(dones[t]), to_np(d))
    assert_same_floats(to_np(fin), to_np(s))
    efin, erew, edone = oc.step_k(to_np(s0), 1000, k, actions=None if not array_actions else to_np(acts))
    assert_same_floats(to_np(fin), efin)
    np.testing.assert_array_equal(to_np(dones), edone)


def test_full_size_properties(dev):
    """At N = 2^20 (the sweep's largest size): the fused kernel equals the single-step chain,
    no post-step state is terminal, and every column stays finite."""
    from hipenvs import cartpole

    n, k = 1 << 20, 32
    s0 = cartpole.reset(n, seed=11, device=dev)
    cartpole.reseed(2000)
    fin, _, dones = cartpole.step_k(s0, k)
    cartpole.reseed(2000)
    s = s0
    for t in range(k):
        a = cartpole.sample_actions(n, seed=2001 + t, device=dev)
        s, _, d = cartpole.step(s, a)
        assert torch.equal(d, dones[t])
    assert torch.equal(fin, s)
    out = to_np(s)
    assert np.isfinite(out).all() and not oc.terminated(out).any()
    frac = dones.float().mean().item()
    assert 1 / 60 < frac < 1 / 10, frac


def test_step_bit_exact_at_the_largest_sweep_size(dev):
    """N = 2^24, the sweep's largest size (and the 32-bit seed mixing of env indices past
    2^23): one step from states in the reset range and beyond it (so a share of the envs
    terminate and reset), every column bit for bit against the oracle."""
    from hipenvs import cartpole

    n = 1 << 24
    r = np.random.default_rng(24)
    state = r.uniform(-0.3, 0.3, size=(4, n)).astype(np.float32)
    action = r.integers(0, 2, size=n).astype(np.int32)
    cartpole.reseed(90)
    ns, rew, done = cartpole.step(torch.from_numpy(state).to(dev), torch.from_numpy(action).to(dev))
    ens, erew, edone = oc.step(state, action, seed=91)
    np.testing.assert_array_equal(to_np(done), edone)
    assert_same_bits(to_np(ns), ens)
    assert_same_bits(to_np(rew), erew)
    assert 0.05 < edone.mean() < 0.95


def test_resets_vary_and_are_uniform(dev):
    """test_cartpole.py:160-172 on the device."""
    from hipenvs import cartpole

    n = 4096
    all_done = torch.full((4, n), 3.0, device=dev)
    cartpole.reseed(0)
    first = to_np(cartpole.step(all_done, torch.zeros(n, dtype=torch.int32, device=dev))[0])
    second = to_np(cartpole.step(all_done, torch.zeros(n, dtype=torch.int32, device=dev))[0])
    assert np.all(np.abs(first) <= oc.RESET_BOUND)
    assert not np.allclose(first, second)
    assert len(np.unique(first[0])) > n * 0.99
    assert abs(first.mean()) < 0.002
    assert abs(first.std() - oc.RESET_BOUND / np.sqrt(3)) < 0.002


def test_int64_actions_accepted(dev):
    from hipenvs import cartpole

    n = 64
    s = cartpole.reset(n, seed=1, device=dev)
    a = torch.ones(n, dtype=torch.int64, device=dev)
    cartpole.reseed(7)
    out64 = cartpole.step(s, a)[0]
    cartpole.reseed(7)
    out32 = cartpole.step(s, a.to(torch.int32))[0]
    assert torch.equal(out64, out32)
