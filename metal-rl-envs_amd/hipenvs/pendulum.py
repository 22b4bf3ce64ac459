"""The K-link pendulum in its mass-matrix form on MI355X: drop-in for the reference's
``pendulum_metal`` module.

``Pendulum(k)`` keeps the surface of ``pendulum_metal.Pendulum``
(``pendulum_metal.py:104-131``): ``reseed(seed)`` and ``step(state, action)`` over a
(2K, N) float32 state of absolute angles then velocities, action in {0, 1, 2} meaning
root torque -1, 0, +1, RK4 at dt 0.02 with each stage's K x K mass matrix
M_ij = mu_ij cos(th_i - th_j) built from K cosines and K sines and solved by Cholesky,
wrap, clip, reward -1 / 0 on termination, terminated columns reset in place from the
counter RNG. K in {1, 2, 3, 4, 8, 16} (the reference's own limit is K = 16 too).
``reset(n, seed=None)`` replaces ``pendulum_mlx.Pendulum.reset``;
``accelerations(state, torque)`` returns the solved accelerations alone. The reference's
``pairwise_trig`` variant (2K^2 transcendentals per stage) is a slower way to the same
equations and is not provided.
"""

import torch

from . import _lib
from .pendulum_aba import DT, GRAVITY, MAX_VEL, RESET_BOUND, TORQUE  # noqa: F401  (same task constants)

SUPPORTED_K = (1, 2, 3, 4, 8, 16)
RESET_SEED_BASE = 0xA0000000


class Pendulum:
    def __init__(self, k):
        if int(k) not in SUPPORTED_K:
            raise ValueError(f"k must be one of {SUPPORTED_K}, got {k}")
        self.k = int(k)
        self.calls = 0
        self.reset_calls = 0

    def reseed(self, seed=0):
        self.calls = int(seed)

    def reset(self, n, seed=None, device=None):
        device = torch.device(device) if device is not None else _lib.default_device()
        if seed is None:
            seed = RESET_SEED_BASE + self.reset_calls
            self.reset_calls += 1
        state = torch.empty((2 * self.k, n), dtype=torch.float32, device=device)
        with _lib.on(device):
            _lib.call("hipenvs_pendulum_aba_reset", self.k, 0, _lib.ptr(state), n, _lib.u32(seed),
                      _lib.stream_of(device))
        return state

    def step(self, state, action):
        """RK4 step of all N envs in one launch (``pendulum_metal.py:121-131``)."""
        n = _lib.check_state(state, 2 * self.k)
        device = state.device
        action = _lib.as_actions(action, n, device)
        self.calls += 1
        next_state = torch.empty_like(state)
        reward = torch.empty(n, dtype=torch.float32, device=device)
        done = torch.empty(n, dtype=torch.bool, device=device)
        with _lib.on(device):
            _lib.call("hipenvs_pendulum_step", self.k, _lib.ptr(state), _lib.ptr(action), _lib.u32(self.calls),
                      _lib.ptr(next_state), _lib.ptr(reward), _lib.ptr(done), n, _lib.stream_of(device))
        return next_state, reward, done

    def accelerations(self, state, torque):
        """Absolute angular accelerations (K, N) of the mass-matrix solve for a root torque (N,)."""
        n = _lib.check_state(state, 2 * self.k)
        torque = _lib.as_f32_vector(torque, n, state.device, "torque")
        acc = torch.empty((self.k, n), dtype=torch.float32, device=state.device)
        with _lib.on(state.device):
            _lib.call("hipenvs_pendulum_accelerations", self.k, _lib.ptr(state), _lib.ptr(torque), _lib.ptr(acc), n,
                      _lib.stream_of(state.device))
        return acc
