"""The whole Acrobot ES rollout as one kernel launch: drop-in for the reference's
``acrobot_rollout_metal`` module (``acrobot_rollout_metal.py:69-81``).

Each of P members runs its own 6-H-3 tanh MLP policy on Gym's observation
(cos and sin of both angles, both velocities) against the RK4 physics and
returns the steps taken before the tip first clears height 1 (the horizon if it
never does).
"""

import torch

from . import _lib


def n_params(hidden):
    return 10 * hidden + 3


def rollout_steps(state, theta_pop, hidden, horizon):
    """Steps before the first termination for each of P members from `state` (4, P),
    each with its own policy row of `theta_pop` (P, 10*hidden+3). Returns (P,) float32."""
    p = _lib.check_state(state, 4)
    hidden = _lib.check_hidden(hidden)
    horizon = _lib.check_horizon(horizon)
    theta_pop = _lib.check_theta(theta_pop, p, n_params(hidden), state.device)
    steps = torch.empty(p, dtype=torch.float32, device=state.device)
    with _lib.on(state.device):
        _lib.call("hipenvs_acrobot_es_rollout", _lib.ptr(state), _lib.ptr(theta_pop), p, hidden, horizon,
                  _lib.ptr(steps), _lib.stream_of(state.device))
    return steps


def rollout_steps_seeded(state, theta, seed, sigma, hidden, horizon):
    """``rollout_steps`` on the antithetic population theta + sigma * [eps; -eps] of
    ``es_noise`` (P = state.shape[1], even), generated on the device into a (P, D)
    workspace; asynchronous. Equals ``rollout_steps(state, es_noise.perturb(theta, P, seed,
    sigma), hidden, horizon)`` bit for bit."""
    p = _lib.check_population(_lib.check_state(state, 4))
    hidden = _lib.check_hidden(hidden)
    horizon = _lib.check_horizon(horizon)
    d = n_params(hidden)
    theta = _lib.check_theta_vector(theta, d, state.device)
    workspace = torch.empty((p, d), dtype=torch.float32, device=state.device)
    out = torch.empty(p, dtype=torch.float32, device=state.device)
    with _lib.on(state.device):
        _lib.call("hipenvs_acrobot_es_rollout_seeded", _lib.ptr(state), _lib.ptr(theta), p, _lib.u32(seed),
                  float(sigma), hidden, horizon, _lib.ptr(out), _lib.ptr(workspace), workspace.numel() * 4,
                  _lib.stream_of(state.device))
    return out


def evaluate(state, theta, hidden, steps):
    """Per-env score of the greedy policy ``theta`` (D,) shared by every env of `state` (4, n)
    over up to ``steps`` steps: the reference's evaluation sum (``es.py:308-322``) of
    reward - 1 + 1 to the first termination, i.e. minus the steps taken before the tip first clears height 1. One launch; asynchronous.
    Returns (n,) float32; ``.mean()`` is the canonical score."""
    n = _lib.check_state(state, 4)
    hidden = _lib.check_hidden(hidden)
    steps = _lib.check_horizon(steps)
    theta = _lib.check_theta_vector(theta, n_params(hidden), state.device)
    out = torch.empty(n, dtype=torch.float32, device=state.device)
    with _lib.on(state.device):
        _lib.call("hipenvs_acrobot_evaluate", _lib.ptr(state), _lib.ptr(theta), n, hidden, steps, _lib.ptr(out),
                  _lib.stream_of(state.device))
    return out
