"""Batched CartPole on MI355X: drop-in for the reference's ``cartpole_metal`` module.

Same surface as ``cartpole_metal.py:106-125``: ``reseed(seed)``, and
``step(state, action) -> (next_state, reward, done)`` over a (4, N) float32
state of rows x, x_dot, theta, theta_dot, one column per environment. Calls are
asynchronous on torch's current stream (the reference's lazy evaluation); new
output tensors every call; inputs are never written. ``step`` pre-increments a
module-level counter and hands it to the kernel as the reset RNG's seed, as
``cartpole_metal.step`` does (``cartpole_metal.py:106-117``).

Additions with no reference counterpart:

* ``reset(n, seed=None)`` draws fresh states from the kernels' counter RNG
  instead of MLX's global key (``cartpole_mlx.py:30-31``).
* ``step_k(state, k, actions=None)`` runs k steps in one launch; identical to k
  ``step`` calls, with in-kernel Bernoulli(0.5) actions when ``actions`` is None.
* ``sample_actions(n, seed)``: the device action sampler of the benchmark loop.

Physical constants are those of Gym CartPole-v1 (``cartpole_np.py:20-31``).
"""

import torch

from . import _lib

GRAVITY = 9.8
CART_MASS = 1.0
POLE_MASS = 0.1
TOTAL_MASS = CART_MASS + POLE_MASS
HALF_POLE_LENGTH = 0.5
POLE_MASS_LENGTH = POLE_MASS * HALF_POLE_LENGTH
FORCE_MAG = 10.0
TAU = 0.02
X_LIMIT = 2.4
THETA_LIMIT = 12 * 2 * 3.141592653589793 / 360
RESET_BOUND = 0.05

ROWS = 4
_calls = 0
_reset_calls = 0
RESET_SEED_BASE = 0x80000000


def reseed(seed=0):
    """Set the step counter; the next ``step`` uses counter seed + 1 (``cartpole_metal.py:109-111``)."""
    global _calls
    _calls = int(seed)


def reset(n, seed=None, device=None):
    """(4, n) float32 fresh states, uniform in +-RESET_BOUND, from the counter RNG.
    With ``seed`` given, the values a reset column receives at step counter ``seed``;
    without, successive calls draw counters 2**31, 2**31 + 1, ..."""
    global _reset_calls
    device = torch.device(device) if device is not None else _lib.default_device()
    if seed is None:
        seed = RESET_SEED_BASE + _reset_calls
        _reset_calls += 1
    state = torch.empty((ROWS, n), dtype=torch.float32, device=device)
    with _lib.on(device):
        _lib.call("hipenvs_cartpole_reset", _lib.ptr(state), n, _lib.u32(seed), _lib.stream_of(device))
    return state


def step(state, action):
    """Advance all N envs by one step in one kernel launch, asynchronously.
    Returns (next_state (4, N) f32, reward (N,) f32 = 1, done (N,) bool)."""
    global _calls
    n = _lib.check_state(state, ROWS)
    device = state.device
    action = _lib.as_actions(action, n, device)
    _calls += 1
    next_state = torch.empty_like(state)
    reward = torch.empty(n, dtype=torch.float32, device=device)
    done = torch.empty(n, dtype=torch.bool, device=device)
    with _lib.on(device):
        _lib.call("hipenvs_cartpole_step", _lib.ptr(state), _lib.ptr(action), _lib.u32(_calls),
                  _lib.ptr(next_state), _lib.ptr(reward), _lib.ptr(done), n, _lib.stream_of(device))
    return next_state, reward, done


def step_k(state, k, actions=None):
    """k steps in one launch: (final state (4, N), rewards (k, N), dones (k, N)).
    Step t uses counter seed+1+t and ``actions[t]`` or, if ``actions`` is None, the
    in-kernel Bernoulli(0.5) action. The module counter advances by k."""
    global _calls
    n = _lib.check_state(state, ROWS)
    device = state.device
    k = int(k)
    if k < 0:
        raise ValueError("k must be >= 0")
    if actions is not None:
        if not isinstance(actions, torch.Tensor) or actions.shape != (k, n):
            raise ValueError(f"actions must be a ({k}, {n}) tensor")
        if actions.device != device:
            raise ValueError(f"actions is on {actions.device}, state is on {device}")
        actions = actions.to(torch.int32).contiguous()
    seed = _calls + 1
    _calls += k
    next_state = torch.empty_like(state)
    rewards = torch.empty((k, n), dtype=torch.float32, device=device)
    dones = torch.empty((k, n), dtype=torch.bool, device=device)
    if k == 0:
        next_state.copy_(state)
        return next_state, rewards, dones
    with _lib.on(device):
        _lib.call("hipenvs_cartpole_step_k", _lib.ptr(state), _lib.ptr(actions), _lib.u32(seed), k,
                  _lib.ptr(next_state), _lib.ptr(rewards), _lib.ptr(dones), n, _lib.stream_of(device))
    return next_state, rewards, dones


def sample_actions(n, seed, m=2, device=None, out=None):
    """(n,) int32 counter-RNG actions: Bernoulli(0.5) for m == 2, else uniform in [0, m)."""
    device = torch.device(device) if device is not None else (out.device if out is not None else _lib.default_device())
    if out is None:
        out = torch.empty(n, dtype=torch.int32, device=device)
    elif out.dtype != torch.int32 or out.shape != (n,) or not out.is_contiguous():
        raise ValueError("out must be a contiguous (n,) int32 tensor")
    with _lib.on(device):
        _lib.call("hipenvs_sample_actions", _lib.ptr(out), n, int(m), _lib.u32(seed), _lib.stream_of(device))
    return out
