"""The C-legged body with hard contacts, restated in numpy: the CPU oracle for the HIP
legged step and legged ES rollout kernels.

TEST INFRASTRUCTURE: part of the CPU oracle (see ``oracle/__init__.py``).

Follows ``legged_np.py`` line by line: ``leg_angles``/``static_pose``/
``stand_pose`` (30-48), ``torques`` (51-54), ``substep`` (57-97: foot
Jacobians, mass matrix M = M_T diag(1,1,0..) + I_T e_phi e_phi^T + M_F sum_c
J_c^T J_c, bias, gravity, leg torques and the assist spring-damper, a dense
Cholesky of M reused for the free velocity and the 2C columns M^-1 J^T,
Delassus blocks, ITERS sweeps of block projected Gauss-Seidel with the exact
single-contact solve, semi-implicit Euler), ``Legged`` (105-132).

``mode="reference"`` is the literal numpy program, including the float64
promotion the reference picks up in ``contact_impulse`` (see ``oracle.hopper``):
after the first contact solve its impulses, and from the second substep on the
whole state, are float64. ``mode="f32"`` is the same program held in float32
(the reference Metal kernel's arithmetic, ``legged_metal.py:13-155``) and is
what the HIP kernels reproduce bit for bit; tests bound the distance between
the two modes per step.

``rollout_fused`` restates the fused ES kernel ``legged_rollout_metal.py:19-59``
(policy with bias-first sums, one three-way head per leg, early exit at the
first fall, shaped reward) in the f32 mode.
"""

import numpy as np

from . import detmath, rng
from .hopper import (BAUMGARTE, FALL_ANGLE, FALL_HEIGHT, GRAVITY, H, I_T, L, M_F, M_T, MU, RESET_BOUND,  # noqa: F401
                     SUBSTEPS, TORQUE, contact_impulse)
from .pendulum import cholesky_solve

F32 = np.float32
ITERS = 8


def leg_angles(c):
    """``legged_np.py:30-32``."""
    return np.linspace(-0.25 * (c - 1), 0.25 * (c - 1), c) if c > 1 else np.zeros(1)


def static_pose(c):
    """``legged_np.py:35-42``."""
    angles = np.array([-0.25, 0.25] * (c // 2)) if c > 1 else np.zeros(1)
    q = np.concatenate([[0.0, L * np.cos(np.abs(angles).min()), 0.0], np.sort(angles)])
    return np.concatenate([q, np.zeros_like(q)]).astype(np.float32)


def stand_pose(c):
    """``legged_np.py:45-48``."""
    angles = leg_angles(c)
    q = np.concatenate([[0.0, L * np.cos(np.abs(angles).min()), 0.0], angles])
    return np.concatenate([q, np.zeros_like(q)]).astype(np.float32)


def torques(action, c):
    """Action index a in [0, 3**C) -> per-leg torque ((a // 3**k) % 3 - 1) * TORQUE; ``legged_np.py:51-54``."""
    action = np.asarray(action)
    return [((action // 3**k) % 3 - 1).astype(np.float32) * TORQUE for k in range(c)]


def substep(q, v, torque, c, iters=ITERS, mu=MU, assist=0.0, mode="f32", trig=None, hopper_sum=False):
    """One semi-implicit Euler substep with block-PGS contacts; ``legged_np.py:57-97``.
    ``hopper_sum`` (C = 1) adds the impulse terms in the hopper's order,
    ``(v_free + MiJt lt) + MiJn ln`` (``hopper_np.py:76``), as the HIP hopper step does."""
    trig = trig or ("det" if mode == "f32" else "numpy")
    sin_f, cos_f, _ = detmath.trig_functions(trig)
    n = 3 + c
    zero = np.zeros_like(q[0])
    one = zero + 1.0
    Jt, Jn, drift, depth = [], [], [], []
    for k in range(c):
        a = q[2] + q[3 + k]
        ca, sa = cos_f(a), sin_f(a)
        ad = v[2] + v[3 + k]
        row_t = [one, zero, L * ca] + [L * ca if j == k else zero for j in range(c)]
        row_n = [zero, one, L * sa] + [L * sa if j == k else zero for j in range(c)]
        Jt.append(row_t)
        Jn.append(row_n)
        drift.append((-L * sa * ad * ad, L * ca * ad * ad))
        depth.append(-(q[1] - L * ca))
    base = [[0.0] * n for _ in range(n)]
    base[0][0], base[1][1], base[2][2] = M_T, M_T, I_T
    M = [[base[i][j] + M_F * sum(Jt[k][i] * Jt[k][j] + Jn[k][i] * Jn[k][j] for k in range(c)) for j in range(n)]
         for i in range(n)]
    force = [-M_F * sum(Jt[k][i] * drift[k][0] + Jn[k][i] * drift[k][1] for k in range(c))
             - GRAVITY * (M_F * sum(Jn[k][i] for k in range(c)) + (M_T if i == 1 else 0.0)) for i in range(n)]
    for k in range(c):
        force[3 + k] = force[3 + k] + torque[k]
    force[2] = force[2] - assist * q[2] - 0.1 * assist * v[2]
    Mmat = np.stack([np.stack(row) for row in M])
    v_free = [v[i] + H * acc for i, acc in enumerate(cholesky_solve(Mmat, np.stack(force), n))]
    MiJt = [cholesky_solve(Mmat, np.stack(Jt[k]), n) for k in range(c)]
    MiJn = [cholesky_solve(Mmat, np.stack(Jn[k]), n) for k in range(c)]

    def dot(r, s):
        return sum(r[i] * s[i] for i in range(n))

    A = [[(dot(Jt[k], MiJt[l]), dot(Jt[k], MiJn[l]), dot(Jn[k], MiJt[l]), dot(Jn[k], MiJn[l])) for l in range(c)]
         for k in range(c)]
    w0 = [(dot(Jt[k], v_free), dot(Jn[k], v_free)) for k in range(c)]
    lt = [zero] * c
    ln = [zero] * c
    for _ in range(iters):
        for k in range(c):
            wt = w0[k][0] + sum(A[k][l][0] * lt[l] + A[k][l][1] * ln[l] for l in range(c) if l != k)
            wn = w0[k][1] + sum(A[k][l][2] * lt[l] + A[k][l][3] * ln[l] for l in range(c) if l != k)
            lt[k], ln[k] = contact_impulse(A[k][k][0], A[k][k][1], A[k][k][3], wt, wn, depth[k], mu, mode)
    if hopper_sum:
        v_new = np.stack([v_free[i] + MiJt[0][i] * lt[0] + MiJn[0][i] * ln[0] for i in range(n)])
    else:
        v_new = np.stack([v_free[i] + sum(MiJt[k][i] * lt[k] + MiJn[k][i] * ln[k] for k in range(c))
                          for i in range(n)])
    return q + H * v_new, v_new


class Legged:
    """``legged_np.Legged`` (``legged_np.py:105-132``) with counter-RNG resets."""

    def __init__(self, c, iters=ITERS, mode="f32", trig=None):
        self.c, self.iters, self.mode, self.trig = c, iters, mode, trig
        self.n_actions = 3**c
        self.stand = stand_pose(c)

    def reset(self, n, seed=0):
        """stand + U[+-0.05] on every row, row j hashed at j * 0x85EBCA6B (legged_metal.py:148-151)."""
        return (self.stand[:, None] + rng.reset_rows(seed, n, 2 * (3 + self.c), RESET_BOUND)).astype(F32)

    def physics(self, state, action, assist=0.0):
        d = 3 + self.c
        q, v = state[:d], state[d:]
        tq = torques(action, self.c)
        for _ in range(SUBSTEPS):
            q, v = substep(q, v, tq, self.c, self.iters, assist=assist, mode=self.mode, trig=self.trig)
        return np.concatenate([q, v])

    def physics_torques(self, state, tq, assist=0.0):
        d = 3 + self.c
        q, v = state[:d], state[d:]
        for _ in range(SUBSTEPS):
            q, v = substep(q, v, tq, self.c, self.iters, assist=assist, mode=self.mode, trig=self.trig)
        return q, v

    @staticmethod
    def terminated(state):
        return (state[1] < FALL_HEIGHT) | (np.abs(state[2]) > FALL_ANGLE)

    def step(self, state, action, seed, assist=0.0):
        """``legged_np.py:114-121``: reward forward velocity + 1, 0 on done. In the f32 mode the
        state is float32 throughout; in the reference mode a float32 state is promoted as the
        reference promotes it and the next state is float64, like legged_np's."""
        n = state.shape[1]
        state = np.asarray(state)
        stepped = self.physics(state.astype(F32) if self.mode == "f32" else state, action, assist)
        done = self.terminated(stepped)
        fresh = self.reset(n, seed)
        next_state = np.where(done[None, :], fresh, stepped)
        reward = np.where(done, 0.0, stepped[3 + self.c] + 1.0).astype(np.float32)
        if self.mode == "f32":
            next_state = next_state.astype(F32)
        return next_state, reward, done


def policy_logits(q, v, w1, b1, w2, b2, c, trig="det"):
    """(5+2C)-H-3C policy in the fused kernel's order (``legged_rollout_metal.py:218-231``):
    hidden = tanh(b1 + sum over obs (y, phi, psi_1..C, then all velocities)), each head
    b2 + sum_j h_j w2[j]. Returns logits (3C, P)."""
    _, _, tanh_f = detmath.trig_functions(trig)
    n = 3 + c
    obs = [q[k] for k in range(1, n)] + [v[k] for k in range(n)]
    hidden = w1.shape[2]
    hs = []
    for j in range(hidden):
        s = b1[:, j].copy()
        for i, o in enumerate(obs):
            s = s + o * w1[:, i, j]
        hs.append(tanh_f(s))
    out = []
    for o in range(3 * c):
        s = b2[:, o].copy()
        for j in range(hidden):
            s = s + hs[j] * w2[:, j, o]
        out.append(s)
    return np.stack(out)


def head_torques(logits, c):
    """Per leg, first-index argmax of its three logits -> torque in {-1, 0, 1} * TORQUE."""
    from .es import first_argmax

    return [((first_argmax(logits[3 * k:3 * k + 3]) - 1).astype(F32) * F32(TORQUE)) for k in range(c)]


def rollout_fused(state, theta_pop, hidden, horizon, c, iters=ITERS, alive_bonus=1.0, fall_penalty=0.0,
                  height_gate=0.0, assist=0.0, trig="det"):
    """(fitness, steps taken) per member; ``legged_rollout_metal.py:19-59`` in float32:
    step, then on a fall count the step and subtract the penalty and stop, else add
    (v_x if y >= gate else 0) + alive and count the step."""
    from .es import unflatten

    n = 3 + c
    state = np.asarray(state, dtype=F32)
    w1, b1, w2, b2 = unflatten(np.asarray(theta_pop, dtype=F32), hidden, 5 + 2 * c, 3 * c)
    q, v = state[:n].copy(), state[n:].copy()
    p = state.shape[1]
    alive = np.ones(p, dtype=bool)
    total = np.zeros(p, dtype=F32)
    taken = np.zeros(p, dtype=F32)
    body = Legged(c, iters, mode="f32")
    alive_f, fall_f, gate_f = F32(alive_bonus), F32(fall_penalty), F32(height_gate)
    for _ in range(horizon):
        tq = head_torques(policy_logits(q, v, w1, b1, w2, b2, c, trig), c)
        nq, nv = body.physics_torques(np.concatenate([q, v]), tq, assist)
        fell = alive & ((nq[1] < FALL_HEIGHT) | (np.abs(nq[2]) > FALL_ANGLE))
        live = alive & ~fell
        taken = np.where(alive, taken + F32(1.0), taken)
        total = np.where(fell, total - fall_f, total)
        gain = np.where(nq[1] >= gate_f, nv[0], F32(0.0)) + alive_f
        total = np.where(live, total + gain, total)
        alive = live
        q = np.where(alive[None, :], nq, q)
        v = np.where(alive[None, :], nv, v)
        if not alive.any():
            break
    return total.astype(F32), taken.astype(F32)


def evaluate_fused(state, theta, hidden, steps, c, iters=ITERS, eval_bonus=0.0, trig="det"):
    """Per-env greedy-evaluation sums of one policy ``theta`` (D,) shared by every env, as the
    fused evaluation kernel runs them: no assist; each env stops at its first fall (which adds
    nothing), and each standing step adds ((v_x + 1) - 1) + eval_bonus, the reference's
    ``reward - 1.0 + task.eval_bonus`` with ``reward = v_x + 1`` (``es.py:314-319``,
    ``legged_np.py:118-121``)."""
    from .es import unflatten

    n = 3 + c
    state = np.asarray(state, dtype=F32)
    p = state.shape[1]
    theta_pop = np.broadcast_to(np.asarray(theta, dtype=F32), (p, theta.shape[0]))
    w1, b1, w2, b2 = unflatten(theta_pop, hidden, 5 + 2 * c, 3 * c)
    q, v = state[:n].copy(), state[n:].copy()
    alive = np.ones(p, dtype=bool)
    total = np.zeros(p, dtype=F32)
    body = Legged(c, iters, mode="f32")
    bonus = F32(eval_bonus)
    for _ in range(steps):
        tq = head_torques(policy_logits(q, v, w1, b1, w2, b2, c, trig), c)
        nq, nv = body.physics_torques(np.concatenate([q, v]), tq, 0.0)
        live = alive & ~((nq[1] < FALL_HEIGHT) | (np.abs(nq[2]) > FALL_ANGLE))
        total = np.where(live, total + (((nv[0] + F32(1.0)) - F32(1.0)) + bonus), total)
        alive = live
        q = np.where(alive[None, :], nq, q)
        v = np.where(alive[None, :], nv, v)
        if not alive.any():
            break
    return total.astype(F32)
