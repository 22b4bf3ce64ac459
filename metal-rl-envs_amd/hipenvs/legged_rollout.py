"""The whole legged ES rollout as one kernel launch: drop-in for the reference's
``legged_rollout_metal`` module (``legged_rollout_metal.py:70-83``).

Each of P members runs its (5+2C)-H-3C tanh policy (one three-way head per
leg, observation everything but x) and the contact physics for the horizon,
accumulating the shaped reward (forward velocity while the torso is above
``height_gate``, plus ``alive_bonus`` per step) until its first fall, when it
pays ``fall_penalty`` once. Returns (fitness, steps taken).

Additions: ``iters`` (the reference fixes ITERS = 8 at build time) and
``schedule``:

* "chunked" (default): the rollout runs in chunks of ``chunk_steps`` steps (for
  ``c <= 2`` a first chunk of 16 when ``chunk_steps`` is longer) and
  the survivors of each chunk (state, accumulators, weights) are packed into a
  dense column buffer before the next. Episode lengths are heavy-tailed (mean
  ~43 steps at the benchmark's shape while a few members last the whole
  horizon), so this keeps waves full. The first chunk reads ``theta_pop``'s
  (P, D) rows directly (each lane its member's row, front to back), or the
  (D, P) columns when they are given as ``theta_cols``.
* "rows": one member per lane for the whole rollout, ``theta_pop`` (P, D).
* "columns": one member per lane, ``theta_cols`` (D, P), the transpose, in which
  the 64 members of a wave load 256 contiguous bytes per weight.

All three give identical results.
"""

import torch

from . import _lib

LAYOUTS = {"rows": 0, "columns": 1}
SCHEDULES = ("chunked", "rows", "columns")
CHUNK_STEPS = 32
SUPPORTED_C = (1, 2, 3, 4)


def n_params(hidden, c):
    obs, out = 5 + 2 * c, 3 * c
    return obs * hidden + hidden + hidden * out + out


def rollout(state, theta_pop, hidden, horizon, c, alive_bonus=1.0, fall_penalty=0.0, height_gate=0.0, assist=0.0,
            iters=8, schedule="chunked", layout=None, theta_cols=None, chunk_steps=CHUNK_STEPS):
    """(fitness (P,), steps (P,)) float32 from state (2(3+C), P); asynchronous.
    ``theta_pop`` is (P, D) rows, or (D, P) for schedule "columns"; with schedule
    "chunked" the columns may be given directly as ``theta_cols`` (then
    ``theta_pop`` may be None). ``layout`` is the older name of ``schedule``."""
    if layout is not None:
        schedule = layout
    if int(c) not in SUPPORTED_C:
        raise ValueError(f"c must be one of {SUPPORTED_C}, got {c}")
    if schedule not in SCHEDULES:
        raise ValueError(f"schedule must be one of {SCHEDULES}")
    if not 0 <= int(iters) <= 4096:
        raise ValueError("iters must be in [0, 4096]")
    c = int(c)
    p = _lib.check_state(state, 2 * (3 + c))
    hidden = _lib.check_hidden(hidden)
    horizon = _lib.check_horizon(horizon)
    d = n_params(hidden, c)
    rows = schedule == "chunked" and theta_cols is None
    if rows:
        theta_pop = _lib.check_theta(theta_pop, p, d, state.device)
        if p * d * 4 >= 1 << 31:  # past the rows form's 32-bit offsets: the columns form on the transpose
            rows, theta_cols = False, theta_pop.T.contiguous()
    if schedule == "chunked" and not rows:
        theta_pop = _lib.check_theta(theta_cols, d, p, state.device, "theta_cols")
    elif not rows:
        shape = (d, p) if schedule == "columns" else (p, d)
        theta_pop = _lib.check_theta(theta_pop, *shape, state.device)
    fitness = torch.empty(p, dtype=torch.float32, device=state.device)
    steps = torch.empty(p, dtype=torch.float32, device=state.device)
    args = (float(alive_bonus), float(fall_penalty), float(height_gate), float(assist), _lib.ptr(fitness),
            _lib.ptr(steps))
    with _lib.on(state.device):
        if schedule == "chunked":
            nbytes = _lib.lib().hipenvs_legged_es_rollout_workspace_bytes(c, hidden, p)
            workspace = torch.empty(nbytes, dtype=torch.uint8, device=state.device)
            entry = "hipenvs_legged_es_rollout_chunked_rows" if rows else "hipenvs_legged_es_rollout_chunked"
            _lib.call(entry, c, hidden, int(iters), int(chunk_steps), _lib.ptr(state), _lib.ptr(theta_pop), p,
                      horizon, *args, _lib.ptr(workspace), nbytes, _lib.stream_of(state.device))
        else:
            _lib.call("hipenvs_legged_es_rollout", c, hidden, int(iters), LAYOUTS[schedule], _lib.ptr(state),
                      _lib.ptr(theta_pop), p, horizon, *args, _lib.stream_of(state.device))
    return fitness, steps


def rollout_seeded(state, theta, seed, sigma, hidden, horizon, c, alive_bonus=1.0, fall_penalty=0.0,
                   height_gate=0.0, assist=0.0, iters=8, chunk_steps=CHUNK_STEPS):
    """The chunked rollout on the antithetic population theta + sigma * [eps; -eps] of
    ``es_noise`` (P = state.shape[1], even). The weights are generated on the device straight
    into the packed member tiles of the workspace, so no (P, D) tensor is made. Equals
    ``rollout(state, es_noise.perturb(theta, P, seed, sigma), hidden, horizon, c, ...)`` bit
    for bit. Returns (fitness (P,), steps (P,)); asynchronous."""
    if int(c) not in SUPPORTED_C:
        raise ValueError(f"c must be one of {SUPPORTED_C}, got {c}")
    if not 0 <= int(iters) <= 4096:
        raise ValueError("iters must be in [0, 4096]")
    if int(chunk_steps) < 1:
        raise ValueError("chunk_steps must be >= 1")
    c = int(c)
    p = _lib.check_population(_lib.check_state(state, 2 * (3 + c)))
    hidden = _lib.check_hidden(hidden)
    horizon = _lib.check_horizon(horizon)
    theta = _lib.check_theta_vector(theta, n_params(hidden, c), state.device)
    fitness = torch.empty(p, dtype=torch.float32, device=state.device)
    steps = torch.empty(p, dtype=torch.float32, device=state.device)
    nbytes = _lib.lib().hipenvs_legged_es_rollout_workspace_bytes(c, hidden, p)
    workspace = torch.empty(nbytes, dtype=torch.uint8, device=state.device)
    with _lib.on(state.device):
        _lib.call("hipenvs_legged_es_rollout_seeded", c, hidden, int(iters), int(chunk_steps), _lib.ptr(state),
                  _lib.ptr(theta), p, _lib.u32(seed), float(sigma), horizon, float(alive_bonus),
                  float(fall_penalty), float(height_gate), float(assist), _lib.ptr(fitness), _lib.ptr(steps),
                  _lib.ptr(workspace), nbytes, _lib.stream_of(state.device))
    return fitness, steps


def evaluate(state, theta, hidden, steps, c, iters=8, eval_bonus=0.0):
    """Per-env score of the greedy policy ``theta`` (D,) shared by every env of `state`
    (2(3+C), n), without assist, over up to ``steps`` steps: the reference's evaluation sum
    (``es.py:308-322``) of (reward - 1) + eval_bonus with reward v_x + 1 while the body stands
    (forward distance for eval_bonus 0), ending at the first fall. One launch; asynchronous."""
    if int(c) not in SUPPORTED_C:
        raise ValueError(f"c must be one of {SUPPORTED_C}, got {c}")
    if not 0 <= int(iters) <= 4096:
        raise ValueError("iters must be in [0, 4096]")
    c = int(c)
    n = _lib.check_state(state, 2 * (3 + c))
    hidden = _lib.check_hidden(hidden)
    steps = _lib.check_horizon(steps)
    theta = _lib.check_theta_vector(theta, n_params(hidden, c), state.device)
    out = torch.empty(n, dtype=torch.float32, device=state.device)
    with _lib.on(state.device):
        _lib.call("hipenvs_legged_evaluate", c, hidden, int(iters), _lib.ptr(state), _lib.ptr(theta), n, steps,
                  float(eval_bonus), _lib.ptr(out), _lib.stream_of(state.device))
    return out
