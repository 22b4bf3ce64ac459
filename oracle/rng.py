"""The counter-based RNG shared by the oracle and the HIP kernels, restated in numpy.

TEST INFRASTRUCTURE: part of the CPU oracle (see ``oracle/__init__.py``).

The hash is the PCG hash of Jarzynski & Olano, "Hash Functions for GPU
Rendering" (JCGT 2020), as the reference's Metal kernels use it
(``cartpole_metal.py:39-51``): one LCG step, a random xorshift, a multiply and
a final xorshift, all on uint32. A uniform in ``[-bound, bound)`` takes the top
24 bits (``cartpole_metal.py:47-50``). Per-env streams are seeded with
``seed ^ (env * 0x9E3779B9)`` and per-row offsets (``cartpole_metal.py:89-93``
for the 4-row bodies, ``row * 0x85EBCA6B`` for the generic ones at
``pendulum_aba_metal.py:109-112`` and ``legged_metal.py:148-151``). ``seed`` is
the per-call counter the reference's ``step`` pre-increments
(``cartpole_metal.py:106-117``).

Additions that have no counterpart in the reference (the reference draws these
from MLX's or numpy's RNG, which no other device can reproduce):

* ``action_bits``: Bernoulli(0.5) actions, bit 31 of ``pcg(h + ACTION_OFFSET)``.
* ``uniform_actions``: a uniform integer action in ``[0, m)`` as
  ``(pcg(h + ACTION_OFFSET) >> 8) * m >> 24``.
* ``torque_uniform``: a continuous torque U[-1, 1) from ``pcg(h + TORQUE_OFFSET)``.

All arithmetic is exact uint32 (wrapping) plus one float32 multiply, so the
numpy and HIP versions agree bit for bit; ``tests/test_rng.py`` pins the hash
against known-answer values computed from the published algorithm with
Python integers.
"""

import numpy as np

U32 = np.uint32
GOLDEN = U32(0x9E3779B9)
ROW_OFFSETS_4 = (U32(0), U32(0x85EBCA6B), U32(0xC2B2AE35), U32(0x27D4EB2F))
ROW_STRIDE = U32(0x85EBCA6B)
ACTION_OFFSET = U32(0x165667B1)
TORQUE_OFFSET = U32(0xD3A2646C)
TWO_POW_M24 = np.float32(1.0 / 16777216.0)


def pcg_hash(v):
    """uint32 PCG hash, vectorised; input and output are uint32 arrays."""
    v = np.asarray(v, dtype=U32)
    with np.errstate(over="ignore"):
        s = v * U32(747796405) + U32(2891336453)
        w = ((s >> ((s >> U32(28)) + U32(4))) ^ s) * U32(277803737)
    return (w >> U32(22)) ^ w


def pcg_hash_int(v):
    """The same hash on one Python int, written from the published algorithm with
    explicit masking; the known-answer reference for ``pcg_hash``."""
    m = 0xFFFFFFFF
    s = (v * 747796405 + 2891336453) & m
    w = (((s >> ((s >> 28) + 4)) ^ s) * 277803737) & m
    return ((w >> 22) ^ w) & m


def uniform_pm(h, bound):
    """float32 in [-bound, bound) from the top 24 bits of uint32 hashes."""
    f = (np.asarray(h, dtype=U32) >> U32(8)).astype(np.float32)
    return (f * TWO_POW_M24 * np.float32(2.0) - np.float32(1.0)) * np.float32(bound)


def env_hash(seed, n):
    """Per-env stream base ``seed ^ (env * 0x9E3779B9)`` for envs 0..n-1."""
    i = np.arange(n, dtype=U32)
    with np.errstate(over="ignore"):
        return U32(seed & 0xFFFFFFFF) ^ (i * GOLDEN)


def reset_rows4(seed, n, bound):
    """(4, n) float32: the fresh state the 4-row kernels (CartPole, Acrobot) write on reset."""
    h = env_hash(seed, n)
    with np.errstate(over="ignore"):
        return np.stack([uniform_pm(pcg_hash(h + off), bound) for off in ROW_OFFSETS_4])


def reset_rows(seed, n, rows, bound):
    """(rows, n) float32: the fresh noise of the generic kernels, row j hashed at h + j * 0x85EBCA6B."""
    h = env_hash(seed, n)
    with np.errstate(over="ignore"):
        return np.stack([uniform_pm(pcg_hash(h + U32(j) * ROW_STRIDE), bound) for j in range(rows)])


def action_bits(seed, n):
    """int32 (n,) Bernoulli(0.5) actions for step counter `seed`."""
    h = env_hash(seed, n)
    with np.errstate(over="ignore"):
        return (pcg_hash(h + ACTION_OFFSET) >> U32(31)).astype(np.int32)


def uniform_actions(seed, n, m):
    """int32 (n,) uniform actions in [0, m) for step counter `seed` (m <= 2**8)."""
    h = env_hash(seed, n)
    with np.errstate(over="ignore"):
        top = (pcg_hash(h + ACTION_OFFSET) >> U32(8)).astype(np.uint64)
    return ((top * np.uint64(m)) >> np.uint64(24)).astype(np.int32)


def torque_uniform(seed, n):
    """float32 (n,) continuous torques U[-1, 1) for step counter `seed`."""
    h = env_hash(seed, n)
    with np.errstate(over="ignore"):
        return uniform_pm(pcg_hash(h + TORQUE_OFFSET), 1.0)
