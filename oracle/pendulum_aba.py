"""The K-link pendulum by the articulated-body algorithm, restated in numpy: the CPU
oracle for the HIP ABA kernels.

TEST INFRASTRUCTURE: part of the CPU oracle (see ``oracle/__init__.py``).

* ``aba_accelerations`` follows ``pendulum_aba_np.py:30-99`` term by term
  (Featherstone's planar ABA: outward link velocities and velocity-product
  biases, inward articulated inertias and biases into the parent, outward
  accelerations with the base accelerating at -g, then the running sum that
  turns joint accelerations into absolute ones).
* ``Pendulum.physics`` / ``step`` follow ``pendulum_aba_np.py:102-132``: RK4
  at dt 0.02 with discrete actions {0, 1, 2} -> torque -1, 0, +1 at the root,
  wrap, clip at 10 pi, termination ``-sum cos > K/2``, reward -1 / 0, reset
  U[+-0.1] on all 2K rows from the counter RNG (``pendulum_aba_metal.py:109-113``).
* ``Pendulum.physics_euler`` / ``step_euler`` are the semi-implicit Euler
  variant with a continuous root torque (no reference counterpart): one ABA
  evaluation per step, omega' = omega + dt * acc, theta' = theta + dt * omega'
  at dt 0.01, the same wrap/clip/termination, reset to angles U[+-0.1] with
  zero velocities. It is pinned by composing the pinned accelerations with the
  integrator and by its energy behaviour.
"""

import numpy as np

from . import detmath, rng
from .pendulum import DT, GRAVITY, MAX_VEL, RESET_BOUND, TORQUE, terminated, wrap

F32 = np.float32
DT_EULER = 0.01


def aba_accelerations(th, om, torque, k, trig="det"):
    """Absolute angular accelerations (K, N) from absolute angles and velocities (K, N)."""
    sin_f, cos_f, _ = detmath.trig_functions(trig)
    zero = np.zeros_like(th[0])
    q = [th[0]] + [th[i] - th[i - 1] for i in range(1, k)]
    qd = [om[0]] + [om[i] - om[i - 1] for i in range(1, k)]
    X, v, c, IA, p = [], [], [], [], []
    v_prev = (zero, zero, zero)
    for i in range(k):
        cs, sn = cos_f(q[i]), sin_f(q[i])
        r = 1.0 if i > 0 else 0.0
        X.append((cs, sn, r))
        w, x, y = v_prev
        xy = y + w * r
        vi = (w + qd[i], cs * x + sn * xy, -sn * x + cs * xy)
        v.append(vi)
        c.append((zero, qd[i] * vi[2], -qd[i] * vi[1]))
        n, fx, fy = vi[0] + vi[2], vi[1], vi[0] + vi[2]
        p.append((vi[1] * fy - vi[2] * fx, -vi[0] * fy, vi[0] * fx))
        one = zero + 1.0
        IA.append([one, zero, one, one, zero, one])
        v_prev = vi
    U, D, u = [None] * k, [None] * k, [None] * k
    for i in reversed(range(k)):
        a00, a01, a02, a11, a12, a22 = IA[i]
        U[i] = (a00, a01, a02)
        D[i] = a00
        u[i] = (torque if i == 0 else zero) - p[i][0]
        if i == 0:
            break
        Ui, Di = U[i], D[i]
        Ia = (a00 - Ui[0] * Ui[0] / Di, a01 - Ui[0] * Ui[1] / Di, a02 - Ui[0] * Ui[2] / Di,
              a11 - Ui[1] * Ui[1] / Di, a12 - Ui[1] * Ui[2] / Di, a22 - Ui[2] * Ui[2] / Di)
        ci = c[i]
        Iac = (Ia[0] * ci[0] + Ia[1] * ci[1] + Ia[2] * ci[2],
               Ia[1] * ci[0] + Ia[3] * ci[1] + Ia[4] * ci[2],
               Ia[2] * ci[0] + Ia[4] * ci[1] + Ia[5] * ci[2])
        g = u[i] / Di
        pa = (p[i][0] + Iac[0] + Ui[0] * g, p[i][1] + Iac[1] + Ui[1] * g, p[i][2] + Iac[2] + Ui[2] * g)
        cs, sn, r = X[i]
        x1, x2 = sn * r, cs * r
        rows = ((Ia[0], Ia[1], Ia[2]), (Ia[1], Ia[3], Ia[4]), (Ia[2], Ia[4], Ia[5]))
        B = [(m0 + m1 * x1 + m2 * x2, m1 * cs - m2 * sn, m1 * sn + m2 * cs) for m0, m1, m2 in rows]
        cols_X = ((one, x1, x2), (zero, cs, -sn), (zero, sn, cs))

        def xtb(a, b):
            return cols_X[a][0] * B[0][b] + cols_X[a][1] * B[1][b] + cols_X[a][2] * B[2][b]

        parent = IA[i - 1]
        IA[i - 1] = [parent[0] + xtb(0, 0), parent[1] + xtb(0, 1), parent[2] + xtb(0, 2),
                     parent[3] + xtb(1, 1), parent[4] + xtb(1, 2), parent[5] + xtb(2, 2)]
        pp = p[i - 1]
        p[i - 1] = (pp[0] + pa[0] + x1 * pa[1] + x2 * pa[2], pp[1] + cs * pa[1] - sn * pa[2],
                    pp[2] + sn * pa[1] + cs * pa[2])
    a_prev = (zero, zero - GRAVITY, zero)
    qdd = []
    for i in range(k):
        cs, sn, r = X[i]
        w, x, y = a_prev
        xy = y + w * r
        ap = (w + c[i][0], cs * x + sn * xy + c[i][1], -sn * x + cs * xy + c[i][2])
        qddi = (u[i] - (U[i][0] * ap[0] + U[i][1] * ap[1] + U[i][2] * ap[2])) / D[i]
        qdd.append(qddi)
        a_prev = (ap[0] + qddi, ap[1], ap[2])
    acc, run = [], zero
    for i in range(k):
        run = run + qdd[i]
        acc.append(run)
    return np.stack(acc)


class Pendulum:
    """``pendulum_aba_np.Pendulum`` (``pendulum_aba_np.py:102-132``) with counter-RNG resets."""

    def __init__(self, k, trig="det"):
        self.k = k
        self.trig = trig

    def reset(self, n, seed=0):
        """(2K, n): every row U[+-0.1] (the RK4 task's reset)."""
        return rng.reset_rows(seed, n, 2 * self.k, RESET_BOUND)

    def reset_euler(self, n, seed=0):
        """(2K, n): angles U[+-0.1], velocities 0 (the semi-implicit Euler task's reset)."""
        s = self.reset(n, seed)
        s[self.k:] = 0.0
        return s

    def dsdt(self, s, torque):
        k = self.k
        return np.concatenate([s[k:], aba_accelerations(s[:k], s[k:], torque, k, self.trig)])

    def physics(self, state, action):
        """RK4 at dt 0.02 with torque (action - 1) * TORQUE; ``pendulum_aba_np.py:117-123``."""
        state = np.asarray(state, dtype=F32)
        torque = ((np.asarray(action) - 1) * TORQUE).astype(F32)
        k1 = self.dsdt(state, torque)
        k2 = self.dsdt(state + DT / 2 * k1, torque)
        k3 = self.dsdt(state + DT / 2 * k2, torque)
        k4 = self.dsdt(state + DT * k3, torque)
        ns = state + DT / 6 * (k1 + 2 * k2 + 2 * k3 + k4)
        return np.concatenate([wrap(ns[: self.k]), np.clip(ns[self.k:], -MAX_VEL, MAX_VEL)]).astype(F32)

    def physics_euler(self, state, torque):
        """One semi-implicit Euler step of DT_EULER with a float32 root torque per env."""
        k = self.k
        state = np.asarray(state, dtype=F32)
        th, om = state[:k], state[k:]
        acc = aba_accelerations(th, om, np.asarray(torque, dtype=F32), k, self.trig)
        om_new = om + DT_EULER * acc
        th_new = th + DT_EULER * om_new
        return np.concatenate([wrap(th_new), np.clip(om_new, -MAX_VEL, MAX_VEL)]).astype(F32)

    def _finish(self, stepped, fresh):
        done = terminated(stepped, self.k, self.trig)
        next_state = np.where(done[None, :], fresh, stepped).astype(F32)
        reward = np.where(done, 0.0, -1.0).astype(F32)
        return next_state, reward, done

    def step(self, state, action, seed):
        stepped = self.physics(state, action)
        return self._finish(stepped, self.reset(stepped.shape[1], seed))

    def step_euler(self, state, torque, seed):
        """Semi-implicit Euler step; ``torque`` (n,) float32 or None for the counter-RNG
        torque U[-1, 1) of step counter ``seed``."""
        n = np.asarray(state).shape[1]
        if torque is None:
            torque = rng.torque_uniform(seed, n)
        stepped = self.physics_euler(state, torque)
        return self._finish(stepped, self.reset_euler(n, seed))
