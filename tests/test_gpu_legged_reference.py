"""The reference-precision legged step (hipenvs_legged_step_reference, GPU).

It runs legged_np's own arithmetic: float64 from the contact solve on, a float64 state
out, as numpy promotes it. Bars:

* bit for bit (float64 state bits, float32 rewards, flags) against the oracle's literal
  restatement in its reference mode with deterministic trig (``trig="det64"``), from
  float32 and from float64 states, over every C, sweep count and the assisted case;
* against the fixtures written by the reference's own numpy: one step from each of its
  float64 states within 1e-5 relative per component, measured at
  about 1e-12; from its float32 initial state within the deterministic-float32-trig bound.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import legged as olg
from oracle import rng
from test_oracle_legged import legged_states

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
LEGGED = [(c, s, 0) for c in (1, 2, 4) for s in (4, 8, 16)] + [(4, 8, 20)] + [(3, s, 0) for s in (4, 8, 16)]


def to_np(t):
    return t.detach().cpu().numpy()


def gpu_step(dev, body, state, action, seed, assist):
    body.reseed(seed - 1)            # step() pre-increments the counter, as the reference does
    return body.step(torch.from_numpy(np.ascontiguousarray(state)).to(dev),
                     torch.from_numpy(np.asarray(action, dtype=np.int32)).to(dev), assist)


def assert_same(got, want):
    ns, rew, done = got
    ens, erew, edone = want
    assert ns.dtype == torch.float64 and ens.dtype == np.float64
    np.testing.assert_array_equal(to_np(done), edone)
    np.testing.assert_array_equal(to_np(ns).view(np.uint64), ens.view(np.uint64))
    np.testing.assert_array_equal(to_np(rew), erew)


@pytest.mark.parametrize("c,s,assist", LEGGED)
def test_fixture_steps_bit_exact_and_within_the_bar(dev, c, s, assist):
    from hipenvs import legged

    g = np.load(GOLDEN / "legged_physics.npz", allow_pickle=False)
    tag = f"c{c}_s{s}_a{assist}"
    traj, acts = g[f"{tag}_traj"], g[f"{tag}_actions"]
    body = legged.Legged(c, s, precision="reference")
    oracle = olg.Legged(c, s, mode="reference", trig="det64")
    print(f"legged reference step {tag}", flush=True)
    for t in range(traj.shape[0]):
        inp = g[f"{tag}_state0"] if t == 0 else traj[t - 1]
        got = gpu_step(dev, body, inp, acts[t], 100 + t, float(assist))
        assert_same(got, oracle.step(inp, acts[t], 100 + t, float(assist)))
        live = ~to_np(got[2])
        ns = to_np(got[0])[:, live]
        want = traj[t][:, live]
        big = np.abs(want) > 1e-3
        rel = (np.abs(ns - want)[big] / np.abs(want[big])).max()
        if t == 0:
            assert rel <= 4e-5, (tag, rel)      # float32 first substep: float32 trig differences
        else:
            assert rel <= 1e-5, (tag, t, rel)   # the bar
            assert rel <= 1e-11, (tag, t, rel)  # measured: <= 2.4e-12


@pytest.mark.parametrize("c", [1, 2, 3, 4])
@pytest.mark.parametrize("iters", [1, 4, 8, 16])
def test_random_states_three_chained_steps(dev, c, iters):
    """float32 states in (with planted falls), then the float64 states out fed back in."""
    from hipenvs import legged

    state, action = legged_states(c, 2048, seed=40 + c)
    state[1, :100] = 0.4
    state[2, 100:200] = 1.3
    body = legged.Legged(c, iters, precision="reference")
    oracle = olg.Legged(c, iters, mode="reference", trig="det64")
    print(f"legged reference chain c={c} iters={iters}", flush=True)
    x_gpu, x_cpu = state, state
    for t in range(3):
        act = rng.uniform_actions(500 + t, state.shape[1], 3 ** c)
        got = gpu_step(dev, body, x_gpu, act, 7 + t, 0.0)
        want = oracle.step(x_cpu, act, 7 + t)
        assert_same(got, want)
        x_gpu, x_cpu = to_np(got[0]), want[0]
    assert want[2].sum() > 0


def test_hundred_step_horizon_flags_identical(dev):
    """100 free-running steps at C = 4, 8 sweeps, N = 512: identical flags and state bits
    at every step (the north-star 100-step horizon), resets included."""
    from hipenvs import legged

    n = 512
    body = legged.Legged(4, 8, precision="reference")
    oracle = olg.Legged(4, 8, mode="reference", trig="det64")
    x = oracle.reset(n, seed=1)
    xg = torch.from_numpy(x).to(dev)
    resets = 0
    for t in range(1, 101):
        act = rng.uniform_actions(t, n, 81)
        body.reseed(t - 1)
        ns, rew, done = body.step(xg, torch.from_numpy(act).to(dev))
        x, erew, edone = oracle.step(x, act, t)
        np.testing.assert_array_equal(to_np(done), edone, err_msg=f"step {t}")
        np.testing.assert_array_equal(to_np(ns).view(np.uint64), x.view(np.uint64), err_msg=f"step {t}")
        np.testing.assert_array_equal(to_np(rew), erew, err_msg=f"step {t}")
        resets += int(edone.sum())
        xg = ns
    assert resets > 0


def test_argument_checks(dev):
    from hipenvs import _lib, legged

    with pytest.raises(ValueError):
        legged.Legged(4, 0, precision="reference")
    with pytest.raises(ValueError):
        legged.Legged(4, 8, precision="float64")
    body = legged.Legged(2, 8, precision="reference")
    with pytest.raises(TypeError):
        body.step(torch.zeros((10, 4), dtype=torch.float16, device=dev), torch.zeros(4, dtype=torch.int32, device=dev))
    ns, rew, done = body.step(torch.zeros((10, 0), device=dev), torch.zeros(0, dtype=torch.int32, device=dev))
    assert ns.shape == (10, 0) and ns.dtype == torch.float64
    null = _lib.ptr(None)
    assert _lib.lib().hipenvs_legged_step_reference(4, 0, 0.0, null, 0, null, 0, null, null, null, null, 0,
                                                    null) == _lib.E_ARG
