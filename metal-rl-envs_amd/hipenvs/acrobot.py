"""Batched Acrobot on MI355X: drop-in for the reference's ``acrobot_metal`` module.

Same surface as ``acrobot_metal.py:93-111``: ``reseed(seed)`` and
``step(state, action) -> (next_state, reward, done)`` over a (4, N) float32
state of rows theta1, theta2, dtheta1, dtheta2; action in {0, 1, 2} is a torque
of -1, 0, +1; reward -1 per step, 0 on the terminating step. Gym's book
dynamics, RK4 at dt 0.2, wrap and clip (``acrobot_np.py:18-93``), with the
terminated columns reset in place from the kernel's counter RNG. ``reset(n,
seed=None)`` replaces ``acrobot_mlx.reset``.
"""

from . import _lib

LINK_LENGTH_1 = 1.0
LINK_MASS_1 = 1.0
LINK_MASS_2 = 1.0
LINK_COM_POS_1 = 0.5
LINK_COM_POS_2 = 0.5
LINK_MOI = 1.0
GRAVITY = 9.8
DT = 0.2
MAX_VEL_1 = 4 * 3.141592653589793
MAX_VEL_2 = 9 * 3.141592653589793
RESET_BOUND = 0.1

ROWS = 4
_calls = 0
_reset_calls = 0
RESET_SEED_BASE = 0x80000000


def reseed(seed=0):
    global _calls
    _calls = int(seed)


def reset(n, seed=None, device=None):
    """(4, n) fresh states uniform in +-RESET_BOUND from the counter RNG (see cartpole.reset)."""
    import torch

    global _reset_calls
    device = torch.device(device) if device is not None else _lib.default_device()
    if seed is None:
        seed = RESET_SEED_BASE + _reset_calls
        _reset_calls += 1
    return _lib.launch_reset("hipenvs_acrobot_reset", ROWS, n, seed, device)


def step(state, action):
    """One RK4 step for all N envs in one launch, asynchronously."""
    global _calls
    _calls += 1
    return _lib.launch_step("hipenvs_acrobot_step", ROWS, state, action, _calls)
