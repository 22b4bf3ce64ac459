"""A device-resident environment object for learners: the shape of the reference's
``ppo.MLXEnv`` (``ppo.py:84-95``) over any hipenvs step body.

``DeviceEnv(body, n)`` holds the (D, N) state on the GPU. ``obs()`` is its (N, D)
transpose for a policy, ``step(action)`` advances all N envs with one kernel launch and
returns (reward, done); terminated envs reset inside the step, as in the reference.
Nothing here synchronises: a learner's rollout of T steps is T launches on the current
stream. ``body`` is a step module (``hipenvs.cartpole``, ``hipenvs.acrobot``) or a body
object (``hipenvs.legged.Legged(c)``, ``hipenvs.hopper.Hopper()``,
``hipenvs.pendulum.Pendulum(k)``, ``hipenvs.pendulum_aba.Pendulum(k)``).
"""

import torch

from . import _lib


class DeviceEnv:
    def __init__(self, body, n, seed=None, device=None):
        self.body = body
        self.device = torch.device(device) if device is not None else _lib.default_device()
        self.state = body.reset(int(n), seed=seed, device=self.device)

    @property
    def n(self):
        return self.state.shape[1]

    def obs(self):
        """(N, D) view of the state for the policy; the env keeps (D, N)."""
        return self.state.T

    def step(self, action):
        """One step of every env; returns (reward (N,) float32, done (N,) bool)."""
        self.state, reward, done = self.body.step(self.state, action)
        return reward, done
