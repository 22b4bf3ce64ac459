"""The learner-facing DeviceEnv (ppo.MLXEnv's shape) over the step bodies (GPU): the same
trajectory as calling the body directly."""

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["cartpole", "acrobot", "hopper", "legged2", "pendulum4"])
def test_device_env_follows_the_body(dev, name):
    from hipenvs import acrobot, adapter, cartpole, hopper, legged, pendulum

    make = {"cartpole": lambda: cartpole, "acrobot": lambda: acrobot, "hopper": hopper.Hopper,
            "legged2": lambda: legged.Legged(2), "pendulum4": lambda: pendulum.Pendulum(4)}[name]
    n_actions = {"cartpole": 2, "acrobot": 3, "hopper": 3, "legged2": 9, "pendulum4": 3}[name]
    body_a, body_b = make(), make()  # the same module object for module bodies: reseed before each step
    env = adapter.DeviceEnv(body_a, 300, seed=9, device=dev)
    state = body_b.reset(300, seed=9, device=dev)
    assert env.obs().shape == (300, state.shape[0])
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    for t in range(20):
        a = torch.randint(0, n_actions, (300,), generator=g, device=dev, dtype=torch.int32)
        body_a.reseed(100 + t)
        reward, done = env.step(a)
        body_b.reseed(100 + t)
        state, r2, d2 = body_b.step(state, a)
        assert torch.equal(env.state, state) and torch.equal(reward, r2) and torch.equal(done, d2)
