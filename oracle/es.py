"""Evolution-strategies pieces restated in numpy for the oracle.

TEST INFRASTRUCTURE: part of the CPU oracle (see ``oracle/__init__.py``).

* ``n_params`` / ``unflatten``: ``es.py:152-164``. A member's row is w1 (I, H)
  row-major, b1 (H), w2 (H, O) row-major, b2 (O).
* ``centered_ranks``: ``es.py:214-215`` with ties broken by index (a stable
  sort on both sides), which the reference's quicksort-based argsort leaves
  unspecified.
* ``legged_action``: ``es.py:86-93``: per-leg first-index argmax of each
  three-way head, composed as sum_k a_k 3**k.
* ``loop_fitness``: ``es.py:174-193``: step the whole population once per
  iteration with auto-reset, count ``steps += alive``, then
  ``fit += (forward + alive_bonus) * alive - fall_penalty * fell``.
* ``evaluate_loop``: ``es.py:308-322``: every env steps each iteration with
  auto-reset, ``alive &= ~done``, ``fit += (reward - 1 + eval_bonus) * alive``
  in float32 (MLX's default dtype for ``mx.zeros``).
"""

import numpy as np

F32 = np.float32


def n_params(hidden, obs_dim, n_out):
    return obs_dim * hidden + hidden + hidden * n_out + n_out


def unflatten(theta_pop, hidden, obs_dim, n_out):
    """(P, D) rows to (w1 (P, I, H), b1 (P, H), w2 (P, H, O), b2 (P, O)); ``es.py:156-164``."""
    p, h, i, o = theta_pop.shape[0], hidden, obs_dim, n_out
    k = 0
    w1 = theta_pop[:, k:k + i * h].reshape(p, i, h); k += i * h
    b1 = theta_pop[:, k:k + h]; k += h
    w2 = theta_pop[:, k:k + h * o].reshape(p, h, o); k += h * o
    b2 = theta_pop[:, k:k + o]
    return w1, b1, w2, b2


def centered_ranks(values):
    """Ranks in [-0.5, 0.5], ties broken by index; ``es.py:214-215``."""
    values = np.asarray(values)
    order = np.argsort(values, kind="stable")
    ranks = np.empty(values.shape[0], dtype=np.int64)
    ranks[order] = np.arange(values.shape[0])
    return ranks.astype(values.dtype) / (values.shape[0] - 1) - 0.5


def first_argmax(logits):
    """First-index argmax over axis 0 of a (m, P) stack, as the fused kernels' strict '>' chain."""
    best = logits[0]
    idx = np.zeros(best.shape, dtype=np.int32)
    for j in range(1, logits.shape[0]):
        better = logits[j] > best
        idx = np.where(better, j, idx)
        best = np.where(better, logits[j], best)
    return idx


def legged_action(logits, c):
    """logits (P, 3C) -> action index sum_k argmax(logits[:, 3k:3k+3]) * 3**k; ``es.py:86-93``."""
    out = np.zeros(logits.shape[0], dtype=np.int32)
    for k in range(c):
        out = out + np.argmax(logits[:, 3 * k:3 * k + 3], axis=-1).astype(np.int32) * 3**k
    return out


def steps_fitness(steps_survived, horizon, sign):
    """(fitness, steps taken) from a fused kernel's steps survived; ``es.py:96-103``:
    fitness = sign * steps, steps taken = min(steps + 1, horizon)."""
    steps_survived = np.asarray(steps_survived, dtype=F32)
    return F32(sign) * steps_survived, np.minimum(steps_survived + 1, horizon)


def loop_fitness(step, logits, action_of, state, params, horizon, seed0, alive_bonus=1.0, fall_penalty=0.0,
                 height_gate=0.0):
    """Reward sum to the first termination and steps taken, stepping the whole population
    once per iteration with auto-reset; ``es.py:174-193``.

    ``step(state, action, seed)`` is an oracle env step, ``logits(state, *params)`` the
    population policy, ``action_of(logits)`` the action rule; step t uses counter seed0 + t.
    Accumulators are float64, as numpy's ``xp.zeros((P,))`` makes them in the reference."""
    p = state.shape[1]
    alive = np.ones(p, dtype=bool)
    fit = np.zeros(p)
    steps = np.zeros(p)
    for t in range(horizon):
        action = action_of(logits(state, *params))
        state, reward, done = step(state, action, (seed0 + t) & 0xFFFFFFFF)
        steps = steps + alive.astype(steps.dtype)
        fell = alive & done
        alive = alive & ~done
        if height_gate:
            forward = (reward - 1.0) * (state[1] >= height_gate).astype(fit.dtype)
        else:
            forward = reward - 1.0
        fit = fit + (forward + alive_bonus) * alive.astype(fit.dtype) - fall_penalty * fell.astype(fit.dtype)
    return fit, steps


def generation_update(theta, eps, fitness, sigma, lr):
    """theta + lr * sum(rank * eps) / (P * sigma) with stable centered ranks; ``es.py:218-227``
    given the noise ``eps`` (P, D) and the population fitness."""
    p = eps.shape[0]
    ranks = centered_ranks(np.asarray(fitness, dtype=F32))
    grad = (ranks[:, None] * eps).sum(axis=0) / (p * sigma)
    return theta + lr * grad


def evaluate_loop(step, action_of, state, steps, seed0, eval_bonus=1.0):
    """Per-env sums of the greedy evaluation (``es.py:308-322``) before the final mean.

    ``step(state, action, seed)`` is an oracle env step with auto-reset, ``action_of(state)``
    the greedy action of the shared policy; step t uses counter seed0 + t."""
    n = state.shape[1]
    alive = np.ones(n, dtype=bool)
    fit = np.zeros(n, dtype=F32)
    for t in range(steps):
        state, reward, done = step(state, action_of(state), (seed0 + t) & 0xFFFFFFFF)
        alive = alive & ~done
        fit = fit + ((reward - F32(1.0)) + F32(eval_bonus)) * alive.astype(F32)
    return fit
