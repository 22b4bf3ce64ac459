"""The whole legged ES rollout as one kernel launch: drop-in for the reference's
``legged_rollout_metal`` module (``legged_rollout_metal.py:70-83``).

Each of P members runs its (5+2C)-H-3C tanh policy (one three-way head per
leg, observation everything but x) and the contact physics for the horizon,
accumulating the shaped reward (forward velocity while the torso is above
``height_gate``, plus ``alive_bonus`` per step) until its first fall, when it
pays ``fall_penalty`` once. Returns (fitness, steps taken).

Additions: ``iters`` (the reference fixes ITERS = 8 at build time) and
``layout``: "rows" reads ``theta_pop`` (P, D) in ``es.unflatten``'s layout, as
the reference does; "columns" reads ``theta_cols`` (D, P), the transpose, in
which the 64 members of a wave load 256 contiguous bytes per weight.
"""

import torch

from . import _lib

LAYOUTS = {"rows": 0, "columns": 1}
SUPPORTED_C = (1, 2, 4)


def n_params(hidden, c):
    obs, out = 5 + 2 * c, 3 * c
    return obs * hidden + hidden + hidden * out + out


def rollout(state, theta_pop, hidden, horizon, c, alive_bonus=1.0, fall_penalty=0.0, height_gate=0.0, assist=0.0,
            iters=8, layout="rows"):
    """(fitness (P,), steps (P,)) float32 from state (2(3+C), P); asynchronous."""
    if int(c) not in SUPPORTED_C:
        raise ValueError(f"c must be one of {SUPPORTED_C}, got {c}")
    if layout not in LAYOUTS:
        raise ValueError(f"layout must be one of {tuple(LAYOUTS)}")
    if not 0 <= int(iters) <= 4096:
        raise ValueError("iters must be in [0, 4096]")
    c = int(c)
    p = _lib.check_state(state, 2 * (3 + c))
    hidden = _lib.check_hidden(hidden)
    horizon = _lib.check_horizon(horizon)
    d = n_params(hidden, c)
    shape = (p, d) if layout == "rows" else (d, p)
    theta_pop = _lib.check_theta(theta_pop, *shape, state.device)
    fitness = torch.empty(p, dtype=torch.float32, device=state.device)
    steps = torch.empty(p, dtype=torch.float32, device=state.device)
    with torch.cuda.device(state.device):
        _lib.call("hipenvs_legged_es_rollout", c, hidden, int(iters), LAYOUTS[layout], _lib.ptr(state),
                  _lib.ptr(theta_pop), p, horizon, float(alive_bonus), float(fall_penalty), float(height_gate),
                  float(assist), _lib.ptr(fitness), _lib.ptr(steps), _lib.stream_of(state.device))
    return fitness, steps
