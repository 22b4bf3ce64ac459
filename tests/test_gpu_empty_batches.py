"""Empty batches through every step, reset and rollout module (GPU): N = 0 returns empty
outputs of the right shapes and launches nothing (the C ABI returns before any launch, so
no zero-size grid reaches the runtime), and the stream stays usable afterwards.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _empty_actions(dev):
    return torch.zeros(0, dtype=torch.int32, device=dev)


def test_step_and_reset_modules_accept_empty_batches(dev):
    from hipenvs import acrobot, cartpole, hopper, legged, pendulum, pendulum_aba

    for mod, rows in ((cartpole, 4), (acrobot, 4)):
        s = mod.reset(0, seed=1, device=dev)
        assert s.shape == (rows, 0)
        nxt, rew, done = mod.step(s, _empty_actions(dev))
        assert nxt.shape == (rows, 0) and rew.shape == (0,) and done.shape == (0,)
    nxt, rew, done = cartpole.step_k(cartpole.reset(0, seed=1, device=dev), 32)
    assert nxt.shape == (4, 0) and rew.shape == (32, 0) and done.shape == (32, 0)
    assert cartpole.sample_actions(0, seed=3, device=dev).shape == (0,)

    bodies = [(pendulum_aba.Pendulum(4), 8), (pendulum.Pendulum(4), 8), (hopper.Hopper(), 8),
              (legged.Legged(4), 14)]
    for body, rows in bodies:
        s = body.reset(0, seed=2, device=dev)
        assert s.shape == (rows, 0)
        nxt, rew, done = body.step(s, _empty_actions(dev))
        assert nxt.shape == (rows, 0) and rew.shape == (0,) and done.shape == (0,)
    nxt, rew, done = pendulum_aba.Pendulum(64).step_euler(torch.zeros((128, 0), device=dev))
    assert nxt.shape == (128, 0) and rew.shape == (0,) and done.shape == (0,)

    # the stream is still good: a real step right after
    nxt, _, _ = cartpole.step(cartpole.reset(8, seed=4, device=dev), torch.ones(8, dtype=torch.int32, device=dev))
    torch.cuda.synchronize()
    assert nxt.shape == (4, 8) and torch.isfinite(nxt).all()


def test_rollouts_accept_empty_populations(dev):
    from hipenvs import acrobot_rollout, cartpole_rollout

    for mod, d_of in ((cartpole_rollout, lambda h: 7 * h + 2), (acrobot_rollout, lambda h: 10 * h + 3)):
        got = mod.rollout_steps(torch.zeros((4, 0), device=dev), torch.zeros((0, d_of(8)), device=dev), 8, 100)
        assert got.shape == (0,)
    torch.cuda.synchronize()
