"""Counter-RNG antithetic Gaussian perturbations and the seeded ES update, restated in numpy.

TEST INFRASTRUCTURE: part of the CPU oracle (see ``oracle/__init__.py``).

The reference's ``generation`` (``es.py:218-227``) draws ``half`` = (P/2, D)
standard normals from MLX's or numpy's generator, materialises
``eps = [half; -half]``, rolls out ``theta + sigma * eps`` and reduces
``sum(centered_ranks(fit)[:, None] * eps, axis=0) / (P * sigma)``. The seeded
form keeps that algorithm but draws ``eps`` from a counter RNG keyed by
(seed, member pair, weight pair), so the (P, D) noise never exists: the
rollouts regenerate the population and the update regenerates the noise.
The generator has no counterpart in the reference (no device reproduces MLX's
or numpy's streams); what is restated here is this package's own definition:

* member key ``k = pcg(seed ^ pcg(m + MEMBER_SALT))`` for member pair m < P/2;
* weight pair j (weights 2j and 2j + 1): ``h1 = pcg(k + 2j * GOLDEN)``,
  ``h2 = pcg(k + (2j + 1) * GOLDEN)``;
* Box-Muller on 24-bit fixed point: ``u1 = ((h1 >> 8) + 1) * 2**-24`` in (0, 1],
  ``t = h2 >> 8``; ``r = sqrt(-2 ln u1)``, angle ``2 pi t / 2**24``;
  ``eps[2j] = r cos``, ``eps[2j + 1] = r sin``; member ``m + P/2`` gets ``-eps``.

``ln`` and ``sin``/``cos`` are written out in float32 elementary operations
(exact bit tricks, one division, Horner polynomials with the Taylor
coefficients, no fused multiply-add), so the HIP kernels reproduce every bit.

What pins them (``tests/test_es_noise.py``):

* ``ln_fixed24`` against float64 ``math.log`` on every one of its 2**24
  inputs, ``sincos_turn24`` against float64 sin/cos on every one of its 2**24
  inputs (error bounds stated in the test);
* the draws' moments, independence of the pair's two components, a
  Kolmogorov-Smirnov distance to the standard normal CDF, and the antithetic
  sign;
* ``perturb`` equal to ``theta + sigma * [eps; -eps]`` computed the
  reference's way from the materialised noise, and ``update`` within float32
  rounding of the float64 evaluation of the reference's reduction.
"""

import numpy as np

from .rng import GOLDEN, U32, pcg_hash

F32 = np.float32
MEMBER_SALT = U32(0x6A09E667)


def _h(x):
    return F32(float.fromhex(x))


# ln(m) = 2 atanh(s), s = (m - 1) / (m + 1): 2s + s * z * (2/3 + 2/5 z + 2/7 z^2 + 2/9 z^3 + 2/11 z^4), z = s^2
LN_C = tuple(_h(x) for x in ("0x1.555556p-1", "0x1.99999ap-2", "0x1.24924ap-2", "0x1.c71c72p-3", "0x1.745d18p-3"))
LN2_HI = _h("0x1.62e4p-1")        # 17 significant bits: k * LN2_HI is exact for |k| <= 127
LN2_LO = _h("0x1.7f7d1cp-20")
SQRT2 = _h("0x1.6a09e6p+0")
# sin(x) = x + x * z * (-1/6 + z/120 - z^2/5040 + z^3/362880); cos(x) = 1 + z * (-1/2 + z/24 - ... - z^4/3628800)
SIN_C = tuple(_h(x) for x in ("-0x1.555556p-3", "0x1.111112p-7", "-0x1.a01a02p-13", "0x1.71de3ap-19"))
COS_C = tuple(_h(x) for x in ("-0x1p-1", "0x1.555556p-5", "-0x1.6c16c2p-10", "0x1.a01a02p-16", "-0x1.27e4fcp-22"))
PI_TURN24 = _h("0x1.921fb6p-22")  # float32(pi) * 2**-23: one 2**24-th of a turn is 2 pi / 2**24
OCTANT = U32(1 << 21)


def member_key(seed, m):
    return pcg_hash(U32(seed) ^ pcg_hash(np.asarray(m, dtype=U32) + MEMBER_SALT))


def ln_fixed24(n):
    """float32 ln(n * 2**-24) for uint32 n in [1, 2**24]."""
    n = np.asarray(n, dtype=U32)
    bits = n.astype(F32).view(U32)                       # exact: n < 2**25
    e = (bits >> U32(23)).astype(np.int32) - 127
    m = ((bits & U32(0x007FFFFF)) | U32(0x3F800000)).view(F32)   # n / 2**e in [1, 2)
    big = m > SQRT2
    m = np.where(big, m * F32(0.5), m)
    k = (e + big.astype(np.int32) - 24).astype(F32)
    s = (m - F32(1.0)) / (m + F32(1.0))
    z = s * s
    c1, c2, c3, c4, c5 = LN_C
    poly = c1 + z * (c2 + z * (c3 + z * (c4 + z * c5)))
    ln_m = (s + s) + s * (z * poly)
    return k * LN2_HI + (k * LN2_LO + ln_m)


def _sin_poly(x):
    z = x * x
    s1, s2, s3, s4 = SIN_C
    return x + x * (z * (s1 + z * (s2 + z * (s3 + z * s4))))


def _cos_poly(x):
    z = x * x
    k1, k2, k3, k4, k5 = COS_C
    return F32(1.0) + z * (k1 + z * (k2 + z * (k3 + z * (k4 + z * k5))))


def sincos_turn24(t):
    """float32 (sin, cos) of 2 pi t / 2**24 for uint32 t in [0, 2**24)."""
    t = np.asarray(t, dtype=U32)
    octant = t >> U32(21)
    f = t & (OCTANT - U32(1))
    odd = (octant & U32(1)) == 1
    phi = np.where(odd, OCTANT - f, f).astype(F32) * PI_TURN24   # in [0, pi/4]
    sp, cp = _sin_poly(phi), _cos_poly(phi)
    s_psi = np.where(odd, cp, sp)                               # angle within the quadrant
    c_psi = np.where(odd, sp, cp)
    q = octant >> U32(1)
    s = np.select([q == 0, q == 1, q == 2], [s_psi, c_psi, -s_psi], -c_psi)
    c = np.select([q == 0, q == 1, q == 2], [c_psi, -s_psi, -c_psi], s_psi)
    return s.astype(F32), c.astype(F32)


def gauss_pair(key, j):
    """The standard-normal pair (eps[2j], eps[2j + 1]) of member key ``key`` (broadcasting)."""
    key = np.asarray(key, dtype=U32)
    j2 = np.asarray(j, dtype=U32) * U32(2)
    with np.errstate(over="ignore"):
        h1 = pcg_hash(key + j2 * GOLDEN)
        h2 = pcg_hash(key + (j2 + U32(1)) * GOLDEN)
    r = np.sqrt(F32(-2.0) * ln_fixed24((h1 >> U32(8)) + U32(1)))
    s, c = sincos_turn24(h2 >> U32(8))
    return r * c, r * s


def noise(seed, half, d):
    """(half, d) float32: eps of member pairs 0 .. half-1 (member m + half carries -eps[m])."""
    keys = member_key(seed, np.arange(half, dtype=np.int64).astype(U32))[:, None]
    pairs = np.arange((d + 1) // 2, dtype=np.int64).astype(U32)[None, :]
    z0, z1 = gauss_pair(keys, pairs)
    out = np.empty((half, 2 * pairs.shape[1]), dtype=F32)
    out[:, 0::2], out[:, 1::2] = z0, z1
    return out[:, :d]


def perturb(theta, p, seed, sigma):
    """(p, d) rows theta + sigma * [eps; -eps], float32 as the reference evaluates it (``es.py:218-222``)."""
    if p % 2:
        raise ValueError("p must be even (antithetic pairs)")
    theta = np.asarray(theta, dtype=F32)
    eps = noise(seed, p // 2, theta.shape[0])
    sig = F32(sigma)
    return np.concatenate([theta[None, :] + sig * eps, theta[None, :] + sig * -eps])


def chunk_members(half):
    """Member pairs per partial sum in ``update``: a multiple of 64, at most 256 partials."""
    return 64 * max(1, -(-half // (64 * 256)))


def update(theta, ranks, seed, sigma, lr):
    """theta + lr * (sum_m ranks[m] eps[m]) / (P sigma) over antithetic pairs, in the HIP kernels'
    order: weights w[m] = ranks[m] - ranks[m + P/2]; per chunk of ``chunk_members`` pairs a
    sequential float32 sum of w[m] * eps[m]; then a sequential sum of the chunks; then
    ``theta + f32(lr) * (S / f32(P * sigma))`` (``es.py:224-226`` under numpy's float32 rules)."""
    theta = np.asarray(theta, dtype=F32)
    ranks = np.asarray(ranks, dtype=F32)
    p, d = ranks.shape[0], theta.shape[0]
    if p % 2:
        raise ValueError("p must be even (antithetic pairs)")
    half = p // 2
    w = ranks[:half] - ranks[half:]
    eps = noise(seed, half, d)
    mc = chunk_members(half)
    total = np.zeros(d, dtype=F32)
    for c0 in range(0, half, mc):
        acc = np.zeros(d, dtype=F32)
        for m in range(c0, min(half, c0 + mc)):
            acc = acc + w[m] * eps[m]
        total = total + acc
    scale = F32(float(p) * float(sigma))
    return theta + F32(lr) * (total / scale)
