"""The one-contact hopper and the exact single-contact impulse, restated in numpy.

TEST INFRASTRUCTURE: part of the CPU oracle (see ``oracle/__init__.py``).

It is the oracle of the HIP hopper step (the reference's ``hopper_metal``),
and the legged body reuses its constants and its contact law
(``legged_np.py:25``); the reference pins the legged body by "C = 1 with one
sweep is the hopper" (test_legged.py:20-26). Follows ``hopper_np.py``:
constants (26-34), ``foot`` (37-40), ``substep`` (43-77), ``contact_impulse``
(80-109), ``Hopper`` (117-138), with the counter-RNG reset of
``hopper_metal.py:118-121``.

``mode`` selects the arithmetic of ``contact_impulse``: ``"reference"`` is
literal, including numpy's promotion of ``np.where(slip_p <= 0, 1.0, -1.0)``
to float64 (two Python-float branches), which makes the tangential impulse
and everything downstream float64; ``"f32"`` keeps that sign in float32 so
the whole computation stays float32, the arithmetic of the reference's Metal
kernel (``legged_metal.py:53-71``) and of the HIP kernels.
"""

import numpy as np

from . import detmath, rng
from .pendulum import cholesky_solve

M_T, I_T, M_F, L = 1.0, 0.1, 0.2, 1.0
GRAVITY = 9.8
TORQUE = 2.0
MU = 0.7
H, SUBSTEPS = 0.01, 4
BAUMGARTE = 0.2
FALL_HEIGHT, FALL_ANGLE = 0.6, 1.0
RESET_BOUND = 0.05
STAND = np.array([0.0, L, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0], dtype=np.float32)


def foot(q, trig="numpy"):
    """Foot position (2, N) for q (4, N); ``hopper_np.py:37-40``."""
    sin_f, cos_f, _ = detmath.trig_functions(trig)
    a = q[2] + q[3]
    return np.stack([q[0] + L * sin_f(a), q[1] - L * cos_f(a)])


def contact_impulse(Att, Atn, Ann, wt, wn, depth, mu=MU, mode="reference"):
    """Exact impulse (lt, ln) of one contact; ``hopper_np.py:80-109``."""
    touching = depth >= 0.0
    target = BAUMGARTE / H * np.maximum(depth, 0.0)
    det = Att * Ann - Atn * Atn
    ln_stick = (Att * (target - wn) + Atn * wt) / det
    lt_stick = (-Ann * wt - Atn * (target - wn)) / det
    sticks = np.abs(lt_stick) <= mu * ln_stick
    den_p, den_m = Ann + mu * Atn, Ann - mu * Atn
    ln_p = np.where(den_p > 0.0, np.maximum((target - wn) / np.where(den_p > 0.0, den_p, 1.0), 0.0), 0.0)
    ln_m = np.where(den_m > 0.0, np.maximum((target - wn) / np.where(den_m > 0.0, den_m, 1.0), 0.0), 0.0)
    slip_p = wt + (Att * mu + Atn) * ln_p
    if mode == "reference":
        s = np.where(slip_p <= 0.0, 1.0, -1.0)
    elif mode == "f32":
        s = np.where(slip_p <= 0.0, np.float32(1.0), np.float32(-1.0))
    else:
        raise ValueError(f"unknown mode {mode!r}")
    ln_slide = np.where(slip_p <= 0.0, ln_p, ln_m)
    lt_slide = mu * s * ln_slide
    ln = np.where(sticks, ln_stick, ln_slide)
    lt = np.where(sticks, lt_stick, lt_slide)
    active = touching & (ln > 0.0) & (wn < target)
    return np.where(active, lt, 0.0), np.where(active, ln, 0.0)


def substep(q, v, torque, mu=MU, mode="reference", trig="numpy"):
    """One semi-implicit Euler substep with the exact single-contact solve; ``hopper_np.py:43-77``."""
    sin_f, cos_f, _ = detmath.trig_functions(trig)
    a = q[2] + q[3]
    ca, sa = cos_f(a), sin_f(a)
    ad = v[2] + v[3]
    zero = np.zeros_like(q[0])
    Jt = (zero + 1.0, zero, L * ca, L * ca)
    Jn = (zero, zero + 1.0, L * sa, L * sa)
    M = [[None] * 4 for _ in range(4)]
    base = ((M_T, 0.0, 0.0, 0.0), (0.0, M_T, 0.0, 0.0), (0.0, 0.0, I_T, 0.0), (0.0, 0.0, 0.0, 0.0))
    for i in range(4):
        for j in range(4):
            M[i][j] = base[i][j] + M_F * (Jt[i] * Jt[j] + Jn[i] * Jn[j])
    drift_x, drift_y = -L * sa * ad * ad, L * ca * ad * ad
    force = [
        -M_F * (Jt[i] * drift_x + Jn[i] * drift_y) - GRAVITY * (M_F * Jn[i] + (M_T if i == 1 else 0.0))
        for i in range(4)
    ]
    force[3] = force[3] + torque
    Mmat = np.stack([np.stack(row) for row in M])
    v_free = [v[i] + H * acc for i, acc in enumerate(cholesky_solve(Mmat, np.stack(force), 4))]
    MiJt = cholesky_solve(Mmat, np.stack(Jt), 4)
    MiJn = cholesky_solve(Mmat, np.stack(Jn), 4)
    Att = sum(Jt[i] * MiJt[i] for i in range(4))
    Atn = sum(Jt[i] * MiJn[i] for i in range(4))
    Ann = sum(Jn[i] * MiJn[i] for i in range(4))
    wt = sum(Jt[i] * v_free[i] for i in range(4))
    wn = sum(Jn[i] * v_free[i] for i in range(4))
    depth = -(q[1] - L * ca)
    lt, ln = contact_impulse(Att, Atn, Ann, wt, wn, depth, mu, mode)
    v_new = np.stack([v_free[i] + MiJt[i] * lt + MiJn[i] * ln for i in range(4)])
    return q + H * v_new, v_new


class Hopper:
    """``hopper_np.Hopper`` (``hopper_np.py:117-138``); resets from the counter RNG."""

    def reset(self, n, seed=0):
        """STAND + U[+-0.05] on every row, row j hashed at j * 0x85EBCA6B (hopper_metal.py:118-120)."""
        return (STAND[:, None] + rng.reset_rows(seed, n, 8, RESET_BOUND)).astype(np.float32)

    def step(self, state, action, seed, mode="f32", trig="det"):
        """``hopper_np.py:121-127``: reward forward velocity + 1, 0 on done; fresh state on done."""
        n = state.shape[1]
        stepped = self.physics(np.asarray(state, dtype=np.float32), action, mode=mode, trig=trig)
        done = self.terminated(stepped)
        next_state = np.where(done[None, :], self.reset(n, seed), stepped).astype(np.float32)
        reward = np.where(done, 0.0, stepped[4] + 1.0).astype(np.float32)
        return next_state, reward, done

    def physics(self, state, action, mode="reference", trig="numpy"):
        torque = ((np.asarray(action) - 1) * TORQUE).astype(np.float32)
        q, v = state[:4], state[4:]
        for _ in range(SUBSTEPS):
            q, v = substep(q, v, torque, mode=mode, trig=trig)
        return np.concatenate([q, v])

    def terminated(self, state):
        return (state[1] < FALL_HEIGHT) | (np.abs(state[2]) > FALL_ANGLE)
