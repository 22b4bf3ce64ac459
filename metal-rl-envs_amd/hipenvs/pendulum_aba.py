"""The K-link pendulum by the articulated-body algorithm on MI355X: drop-in for the
reference's ``pendulum_aba_metal`` module.

``Pendulum(k)`` keeps the surface of ``pendulum_aba_metal.Pendulum``
(``pendulum_aba_metal.py:119-144``): ``reseed(seed)`` and ``step(state, action)``
over a (2K, N) float32 state of absolute angles then velocities, action in
{0, 1, 2} meaning root torque -1, 0, +1, RK4 at dt 0.02, reward -1 / 0 on
termination (tip above half the chain's length), terminated columns reset in
place from the counter RNG. K in {1, 2, 3, 4, 8, 16, 32, 64}.

Additions with no reference counterpart:

* ``step_euler(state, torque=None)``: one semi-implicit Euler step at dt 0.01
  with a continuous root torque per env (a (N,) float32 tensor, or the counter
  RNG's U[-1, 1) when None); resets to angles U[+-0.1] with zero velocities.
* ``accelerations(state, torque)``: the ABA's absolute accelerations alone
  (``pendulum_aba_np.aba_accelerations``, ``pendulum_aba_np.py:30-99``).
* ``reset(n, seed=None, zero_velocity=False)`` from the counter RNG.
"""

import torch

from . import _lib

GRAVITY = 9.8
DT = 0.02
DT_EULER = 0.01
TORQUE = 1.0
MAX_VEL = 10 * 3.141592653589793
RESET_BOUND = 0.1
SUPPORTED_K = (1, 2, 3, 4, 8, 16, 32, 64)
RESET_SEED_BASE = 0x80000000


class Pendulum:
    def __init__(self, k):
        if int(k) not in SUPPORTED_K:
            raise ValueError(f"k must be one of {SUPPORTED_K}, got {k}")
        self.k = int(k)
        self.calls = 0
        self.reset_calls = 0

    def reseed(self, seed=0):
        self.calls = int(seed)

    def reset(self, n, seed=None, device=None, zero_velocity=False):
        device = torch.device(device) if device is not None else _lib.default_device()
        if seed is None:
            seed = RESET_SEED_BASE + self.reset_calls
            self.reset_calls += 1
        state = torch.empty((2 * self.k, n), dtype=torch.float32, device=device)
        with _lib.on(device):
            _lib.call("hipenvs_pendulum_aba_reset", self.k, int(bool(zero_velocity)), _lib.ptr(state), n,
                      _lib.u32(seed), _lib.stream_of(device))
        return state

    def step(self, state, action):
        """RK4 step of all N envs in one launch (``pendulum_aba_metal.py:134-144``)."""
        n = _lib.check_state(state, 2 * self.k)
        device = state.device
        action = _lib.as_actions(action, n, device)
        self.calls += 1
        return self._launch("hipenvs_pendulum_aba_step", state, action, n, device)

    def step_euler(self, state, torque=None):
        """Semi-implicit Euler step with a continuous root torque (N,) f32, or counter-RNG torques."""
        n = _lib.check_state(state, 2 * self.k)
        device = state.device
        if torque is not None:
            torque = _lib.as_f32_vector(torque, n, device, "torque")
        self.calls += 1
        return self._launch("hipenvs_pendulum_aba_step_euler", state, torque, n, device)

    def _launch(self, entry, state, extra, n, device):
        next_state = torch.empty_like(state)
        reward = torch.empty(n, dtype=torch.float32, device=device)
        done = torch.empty(n, dtype=torch.bool, device=device)
        with _lib.on(device):
            _lib.call(entry, self.k, _lib.ptr(state), _lib.ptr(extra), _lib.u32(self.calls), _lib.ptr(next_state),
                      _lib.ptr(reward), _lib.ptr(done), n, _lib.stream_of(device))
        return next_state, reward, done

    def accelerations(self, state, torque):
        """Absolute angular accelerations (K, N) of state (2K, N) under root torque (N,)."""
        n = _lib.check_state(state, 2 * self.k)
        torque = _lib.as_f32_vector(torque, n, state.device, "torque")
        acc = torch.empty((self.k, n), dtype=torch.float32, device=state.device)
        with _lib.on(state.device):
            _lib.call("hipenvs_pendulum_aba_accelerations", self.k, _lib.ptr(state), _lib.ptr(torque), _lib.ptr(acc),
                      n, _lib.stream_of(state.device))
        return acc
