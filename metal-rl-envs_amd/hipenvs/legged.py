"""The C-legged body with hard contacts on MI355X: drop-in for the reference's
``legged_metal`` module.

``Legged(c, iters=8)`` keeps the surface of ``legged_metal.Legged``
(``legged_metal.py:158-185``): ``reseed(seed)`` and ``step(state, action,
assist=None)`` over a (2(3+C), N) float32 state (q = x, y, phi, psi_1..C, then
their velocities), action in [0, 3**C) giving leg k the torque
((a // 3**k) % 3 - 1) * TORQUE, four semi-implicit Euler substeps of 0.01 s
with ``iters`` sweeps of block projected Gauss-Seidel over the C contacts,
reward forward velocity + 1 (0 on a fall), terminated columns reset to the
standing pose plus U[+-0.05] noise from the counter RNG. C in {1, 2, 3, 4}.
``reset(n, seed=None)`` replaces ``legged_mlx.Legged.reset``.

``precision="reference"`` runs ``legged_np``'s own arithmetic instead of the Metal
kernel's float32: numpy promotes the tangential impulse to float64 in its contact
solve (``hopper_np.py:100``), and with it the velocities and the state, so
``legged_np.Legged.step`` returns a float64 state and every later step runs in
float64. In this mode ``step`` takes a float32 or float64 state and returns a
float64 one, with the same dtype flow (iters >= 1).
"""

import numpy as np
import torch

from . import _lib

M_T, I_T, M_F, L = 1.0, 0.1, 0.2, 1.0
GRAVITY = 9.8
TORQUE = 2.0
MU = 0.7
H, SUBSTEPS = 0.01, 4
BAUMGARTE = 0.2
FALL_HEIGHT, FALL_ANGLE = 0.6, 1.0
RESET_BOUND = 0.05
ITERS = 8
SUPPORTED_C = (1, 2, 3, 4)
RESET_SEED_BASE = 0x80000000


def leg_angles(c):
    """Resting leg angles, a symmetric spread (``legged_np.py:30-32``)."""
    return np.linspace(-0.25 * (c - 1), 0.25 * (c - 1), c) if c > 1 else np.zeros(1)


def stand_pose(c):
    """The reset pose (``legged_np.py:45-48``): hip at the height of the innermost foot on the floor."""
    angles = leg_angles(c)
    q = np.concatenate([[0.0, L * np.cos(np.abs(angles).min()), 0.0], angles])
    return np.concatenate([q, np.zeros_like(q)]).astype(np.float32)


PRECISIONS = ("f32", "reference")


class Legged:
    def __init__(self, c, iters=ITERS, precision="f32"):
        if int(c) not in SUPPORTED_C:
            raise ValueError(f"c must be one of {SUPPORTED_C}, got {c}")
        if not 0 <= int(iters) <= 4096:
            raise ValueError("iters must be in [0, 4096]")
        if precision not in PRECISIONS:
            raise ValueError(f"precision must be one of {PRECISIONS}, got {precision!r}")
        if precision == "reference" and int(iters) < 1:
            raise ValueError("precision='reference' needs iters >= 1 (with no sweep the reference never leaves "
                             "float32: use precision='f32')")
        self.precision = precision
        self.c, self.iters = int(c), int(iters)
        self.n_actions = 3 ** self.c
        self.rows = 2 * (3 + self.c)
        self.stand = stand_pose(self.c)
        self._stand_dev = {}
        self.calls = 0
        self.reset_calls = 0

    def stand_on(self, device):
        key = str(device)
        if key not in self._stand_dev:
            self._stand_dev[key] = torch.from_numpy(self.stand).to(device)
        return self._stand_dev[key]

    def reseed(self, seed=0):
        self.calls = int(seed)

    def reset(self, n, seed=None, device=None):
        device = torch.device(device) if device is not None else _lib.default_device()
        if seed is None:
            seed = RESET_SEED_BASE + self.reset_calls
            self.reset_calls += 1
        state = torch.empty((self.rows, n), dtype=torch.float32, device=device)
        with _lib.on(device):
            _lib.call("hipenvs_legged_reset", self.c, _lib.ptr(self.stand_on(device)), _lib.ptr(state), n,
                      _lib.u32(seed), _lib.stream_of(device))
        return state

    def step(self, state, action, assist=None):
        """All N envs by one control step (four substeps) in one launch, asynchronously.
        ``assist`` (a float) is the torso spring-damper stiffness of the curriculum."""
        if self.precision == "reference":
            return self._step_reference(state, action, assist)
        n = _lib.check_state(state, self.rows)
        device = state.device
        action = _lib.as_actions(action, n, device)
        self.calls += 1
        next_state = torch.empty_like(state)
        reward = torch.empty(n, dtype=torch.float32, device=device)
        done = torch.empty(n, dtype=torch.bool, device=device)
        with _lib.on(device):
            _lib.call("hipenvs_legged_step", self.c, self.iters, float(assist or 0.0), _lib.ptr(state),
                      _lib.ptr(action), _lib.u32(self.calls), _lib.ptr(self.stand_on(device)), _lib.ptr(next_state),
                      _lib.ptr(reward), _lib.ptr(done), n, _lib.stream_of(device))
        return next_state, reward, done

    def _step_reference(self, state, action, assist):
        is_f64 = int(isinstance(state, torch.Tensor) and state.dtype == torch.float64)
        n = _lib.check_state(state, self.rows, dtypes=(torch.float32, torch.float64))
        device = state.device
        action = _lib.as_actions(action, n, device)
        self.calls += 1
        next_state = torch.empty((self.rows, n), dtype=torch.float64, device=device)
        reward = torch.empty(n, dtype=torch.float32, device=device)
        done = torch.empty(n, dtype=torch.bool, device=device)
        with _lib.on(device):
            _lib.call("hipenvs_legged_step_reference", self.c, self.iters, float(assist or 0.0), _lib.ptr(state),
                      is_f64, _lib.ptr(action), _lib.u32(self.calls), _lib.ptr(self.stand_on(device)),
                      _lib.ptr(next_state), _lib.ptr(reward), _lib.ptr(done), n, _lib.stream_of(device))
        return next_state, reward, done
