"""The one-contact hopper on MI355X: drop-in for the reference's ``hopper_metal`` module.

``Hopper()`` keeps the surface of ``hopper_metal.Hopper`` (``hopper_metal.py:113-138``):
``reseed(seed)`` and ``step(state, action)`` over an (8, N) float32 state (q = x, y,
phi, psi, then their velocities), hip torque (action - 1) * TORQUE, four
semi-implicit Euler substeps of 0.01 s with the exact single-contact solve, reward
forward velocity + 1 (0 on a fall), terminated columns reset to the standing pose plus
U[+-0.05] noise from the counter RNG. ``reset(n, seed=None)`` replaces
``hopper_mlx.Hopper.reset``.

The kernel is the legged body's at one contact with one sweep, adding the two impulse
terms in the hopper's order (``hopper_np.py:76``), so its results are the hopper's bit
for bit in float32.
"""

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
STAND = (0.0, L, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0)
RESET_SEED_BASE = 0x90000000


class Hopper:
    rows = 8
    n_actions = 3

    def __init__(self):
        self.calls = 0
        self.reset_calls = 0

    def reseed(self, seed=0):
        self.calls = int(seed)

    def reset(self, n, seed=None, device=None):
        device = torch.device(device) if device is not None else _lib.default_device()
        if seed is None:
            seed = RESET_SEED_BASE + self.reset_calls
            self.reset_calls += 1
        return _lib.launch_reset("hipenvs_hopper_reset", self.rows, n, seed, device)

    def step(self, state, action):
        """All N envs by one control step in one launch, asynchronously."""
        self.calls += 1
        return _lib.launch_step("hipenvs_hopper_step", self.rows, state, action, self.calls)
