"""A planar chain of K unit point masses on unit massless rods, link angles absolute (from
the downward vertical), torque on the first joint, g = 9.8: its accelerations by the
Jacobian method of multibody dynamics, in float64. Test-side physics, derived here from
the positions of the masses and independent of the oracle's and the reference's formulas.

Mass i sits at p_i = sum_{j <= i} (sin t_j, -cos t_j), so its velocity is J_i w with
column j of J_i equal to (cos t_j, sin t_j) for j <= i (zero after), and its acceleration
is J_i w' + a_i with a_i = sum_{j <= i} (-sin t_j, cos t_j) w_j^2. Projecting Newton's law
for every mass onto the generalised coordinates gives

    (sum_i J_i^T J_i) w' = sum_i J_i^T ((0, -g) - a_i) + (torque, 0, ..., 0).
"""

import numpy as np

GRAVITY = 9.8


def accelerations(theta, omega, torque, g=GRAVITY):
    """(K,) absolute angular accelerations of one chain."""
    theta = np.asarray(theta, dtype=np.float64)
    omega = np.asarray(omega, dtype=np.float64)
    k = theta.shape[0]
    c, s = np.cos(theta), np.sin(theta)
    mass = np.zeros((k, k))
    rhs = np.zeros(k)
    rhs[0] = float(torque)
    for i in range(k):
        jx = np.where(np.arange(k) <= i, c, 0.0)
        jy = np.where(np.arange(k) <= i, s, 0.0)
        ax = -np.sum(s[: i + 1] * omega[: i + 1] ** 2)
        ay = np.sum(c[: i + 1] * omega[: i + 1] ** 2)
        mass += np.outer(jx, jx) + np.outer(jy, jy)
        rhs += jx * (0.0 - ax) + jy * (-g - ay)
    return np.linalg.solve(mass, rhs)


def batch_accelerations(theta, omega, torque, g=GRAVITY):
    """(K, N) accelerations of N chains given (K, N) angles and velocities and (N,) torques."""
    return np.stack([accelerations(theta[:, n], omega[:, n], torque[n], g) for n in range(theta.shape[1])], axis=1)
