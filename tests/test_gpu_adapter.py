"""The learner-facing DeviceEnv (ppo.MLXEnv's shape) over the step bodies (GPU): trajectories
of counter-RNG actions checked bit for bit against the oracle's env steps, resets included."""

import numpy as np
import pytest
import torch

from oracle import acrobot as oac
from oracle import cartpole as ocp
from oracle import hopper as ohp
from oracle import legged as olg
from oracle import pendulum as opd
from oracle import pendulum_aba as oab
from oracle import rng

pytestmark = pytest.mark.gpu

# name -> (hipenvs body factory, oracle step(state, action, seed), number of actions)
BODIES = {
    "cartpole": (lambda m: m.cartpole, lambda s, a, sd: ocp.step(s, a, sd), 2),
    "acrobot": (lambda m: m.acrobot, lambda s, a, sd: oac.step(s, a, sd), 3),
    "hopper": (lambda m: m.hopper.Hopper(), lambda s, a, sd: ohp.Hopper().step(s, a, sd), 3),
    "legged2": (lambda m: m.legged.Legged(2), lambda s, a, sd: olg.Legged(2).step(s, a, sd), 9),
    "pendulum4": (lambda m: m.pendulum.Pendulum(4), lambda s, a, sd: opd.Pendulum(4).step(s, a, sd), 3),
    "pendulum_aba8": (lambda m: m.pendulum_aba.Pendulum(8), lambda s, a, sd: oab.Pendulum(8).step(s, a, sd), 3),
}
# Bodies whose random-action episodes rarely end within 40 steps from their reset: every
# fourth env starts pointing up (tip above the termination height), so the first step
# terminates and resets it.
RAISED = {"acrobot": 1, "pendulum4": 4, "pendulum_aba8": 8}  # leading rows set to pi: theta1 (Acrobot), every absolute angle (chains)


@pytest.mark.parametrize("name", sorted(BODIES))
def test_device_env_matches_the_oracle(dev, name):
    """40 steps of uniform counter-RNG actions from the env's own reset: the adapter's state,
    rewards and done flags equal the oracle's env step at every step (the step counter the
    body pre-increments is the oracle's seed)."""
    import hipenvs
    from hipenvs import acrobot, adapter, cartpole, hopper, legged, pendulum, pendulum_aba  # noqa: F401

    make, oracle_step, n_actions = BODIES[name]
    n = 300
    body = make(hipenvs)
    env = adapter.DeviceEnv(body, n, seed=9, device=dev)
    if name in RAISED:
        env.state[:RAISED[name], ::4] = float(np.pi)
    state = env.state.cpu().numpy()
    assert env.obs().shape == (n, state.shape[0])
    body.reseed(100)
    resets = 0
    for t in range(101, 141):
        a = rng.uniform_actions(t, n, n_actions)
        reward, done = env.step(torch.from_numpy(a).to(dev))
        state, er, ed = oracle_step(state, a, t)
        np.testing.assert_array_equal(env.state.cpu().numpy(), state, err_msg=f"{name} step {t}")
        np.testing.assert_array_equal(reward.cpu().numpy(), er, err_msg=f"{name} step {t}")
        np.testing.assert_array_equal(done.cpu().numpy(), ed, err_msg=f"{name} step {t}")
        resets += int(ed.sum())
    # random actions end CartPole, hopper and biped episodes within 40 steps; the swinging
    # chains terminate from their raised starts
    assert resets >= (n // 4 if name in RAISED else 1), (name, resets)
