"""The K-link pendulum's mass-matrix form, restated in numpy (test oracle for the ABA).

TEST INFRASTRUCTURE: part of the CPU oracle (see ``oracle/__init__.py``).

Follows ``pendulum_np.py``: constants (29-34), ``hanging_mass`` (37-39), the
Lagrangian derivative ``Pendulum._dsdt`` (68-79) with K x K mass matrix
M_ij = mu_ij cos(th_i - th_j) solved by ``cholesky_solve`` (85-107), the
termination rule (81-82), ``_wrap`` (110-111) and ``energy`` (114-120). It is
an independent derivation of the accelerations the articulated-body algorithm
computes, which is how the reference's test_pendulum_aba.py:21-28 uses it.
"""

import numpy as np

from . import detmath, rng

F32 = np.float32

GRAVITY = 9.8
DT = 0.02
TORQUE = 1.0
MAX_VEL = 10 * np.pi
RESET_BOUND = 0.1
PI = np.pi


def hanging_mass(k):
    """mu_ij = unit masses at or beyond the outer of joints i and j; ``pendulum_np.py:37-39``."""
    return np.array([[k - max(i, j) for j in range(k)] for i in range(k)], dtype=np.float32)


def mass_matrix_dsdt(s, torque, k, trig="numpy"):
    """[omega; acc] from the mass-matrix form; ``pendulum_np.py:68-79``."""
    sin_f, cos_f, _ = detmath.trig_functions(trig)
    mu = hanging_mass(k)
    th, om = s[:k], s[k:]
    c, sn = cos_f(th), sin_f(th)
    cos_d = c[:, None, :] * c[None, :, :] + sn[:, None, :] * sn[None, :, :]
    sin_d = sn[:, None, :] * c[None, :, :] - c[:, None, :] * sn[None, :, :]
    m = mu[:, :, None] * cos_d
    rhs = -(mu[:, :, None] * sin_d * (om**2)[None, :, :]).sum(axis=1)
    rhs = rhs - GRAVITY * np.diag(mu)[:, None] * sn
    rhs[0] = rhs[0] + torque
    acc = cholesky_solve(m, rhs, k)
    return np.concatenate([om, acc])


def cholesky_solve(m, b, k):
    """Solve M x = b for K x K SPD M batched over the last axis; ``pendulum_np.py:85-107``:
    loops over K of vector ops over N, the factor's rows built left to right."""
    lo = [[None] * k for _ in range(k)]
    for i in range(k):
        for j in range(i + 1):
            s = m[i, j] if not isinstance(m, list) else m[i][j]
            for p in range(j):
                s = s - lo[i][p] * lo[j][p]
            lo[i][j] = np.sqrt(s) if i == j else s / lo[j][j]
    y = [None] * k
    for i in range(k):
        s = b[i]
        for p in range(i):
            s = s - lo[i][p] * y[p]
        y[i] = s / lo[i][i]
    x = [None] * k
    for i in reversed(range(k)):
        s = y[i]
        for p in range(i + 1, k):
            s = s - lo[p][i] * x[p]
        x[i] = s / lo[i][i]
    return np.stack(x)


def wrap(x):
    """``pendulum_np.py:110-111``."""
    return x - 2 * PI * np.floor((x + PI) / (2 * PI))


def terminated(state, k, trig="det"):
    """Tip above half the chain's length: -sum cos(th) > k/2; ``pendulum_np.py:81-82``.
    numpy reduces axis 0 of a C-ordered (K, N) array row by row, in order."""
    _, cos_f, _ = detmath.trig_functions(trig)
    return -cos_f(state[:k]).sum(axis=0) > k / 2


def energy(state, k):
    """Total mechanical energy per env (unit masses and rods); ``pendulum_np.py:114-120``."""
    th, om = state[:k], state[k:]
    vx = np.cumsum(om * np.cos(th), axis=0)
    vy = np.cumsum(om * np.sin(th), axis=0)
    y = np.cumsum(-np.cos(th), axis=0)
    return 0.5 * (vx**2 + vy**2).sum(axis=0) + GRAVITY * y.sum(axis=0)


def mass_matrix_accelerations_f64(th, om, torque, k):
    """The same equations assembled and solved in float64 with numpy.linalg.solve, for
    any K: the brute-force check of the ABA past the reference's K = 16 oracle."""
    th = th.astype(np.float64)
    om = om.astype(np.float64)
    mu = hanging_mass(k).astype(np.float64)
    n = th.shape[1]
    out = np.empty((k, n))
    for e in range(n):
        d = th[:, e][:, None] - th[:, e][None, :]
        m = mu * np.cos(d)
        rhs = -(mu * np.sin(d) * (om[:, e] ** 2)[None, :]).sum(axis=1) - GRAVITY * np.diag(mu) * np.sin(th[:, e])
        rhs[0] += float(torque[e])
        out[:, e] = np.linalg.solve(m, rhs)
    return out


class Pendulum:
    """``pendulum_np.Pendulum`` (``pendulum_np.py:42-82``), the mass-matrix body of the
    reference's ``pendulum_metal``, with counter-RNG resets (``pendulum_metal.py:94-98``):
    RK4 at dt 0.02 of ``mass_matrix_dsdt``, wrap, clip, termination, reward -1 / 0."""

    def __init__(self, k, trig="det"):
        self.k = k
        self.trig = trig

    def reset(self, n, seed=0):
        """(2K, n): every row U[+-0.1], row j hashed at j * 0x85EBCA6B."""
        return rng.reset_rows(seed, n, 2 * self.k, RESET_BOUND)

    def physics(self, state, action):
        """``pendulum_np.py:59-66``."""
        state = np.asarray(state, dtype=F32)
        torque = ((np.asarray(action) - 1) * TORQUE).astype(F32)
        k1 = mass_matrix_dsdt(state, torque, self.k, self.trig)
        k2 = mass_matrix_dsdt(state + DT / 2 * k1, torque, self.k, self.trig)
        k3 = mass_matrix_dsdt(state + DT / 2 * k2, torque, self.k, self.trig)
        k4 = mass_matrix_dsdt(state + DT * k3, torque, self.k, self.trig)
        ns = state + DT / 6 * (k1 + 2 * k2 + 2 * k3 + k4)
        return np.concatenate([wrap(ns[: self.k]), np.clip(ns[self.k:], -MAX_VEL, MAX_VEL)]).astype(F32)

    def step(self, state, action, seed):
        """``pendulum_np.py:50-57``."""
        stepped = self.physics(state, action)
        done = terminated(stepped, self.k, self.trig)
        next_state = np.where(done[None, :], self.reset(stepped.shape[1], seed), stepped).astype(F32)
        reward = np.where(done, 0.0, -1.0).astype(F32)
        return next_state, reward, done
