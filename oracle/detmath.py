"""Deterministic float32 sin, cos and tanh, restated in numpy for the oracle.

TEST INFRASTRUCTURE: everything under ``oracle/`` is the CPU oracle the HIP
library's results are checked against. Only ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg may import it, and only to check results.
The product path never calls into it.

Why these exist. The reference evaluates ``np.sin``/``np.cos``/``np.tanh`` on
float32 arrays (``cartpole_np.py:63``, ``acrobot_np.py:70-77``,
``pendulum_aba_np.py:39``, ``legged_np.py:204``, ``es.py:170``) and its Metal
kernels call ``metal::sin``/``metal::tanh``. Neither library is bit-reproducible
on the other device, so a 1-ULP difference in one transcendental is enough to
flip a termination flag at a threshold or an argmax between nearly tied logits.
The HIP kernels and this oracle therefore both evaluate the SAME float32
program, built only from IEEE-754 operations that numpy and the GPU round
identically (``+ - * /``, ``rint``, ``floor``, comparisons, exponent bit
manipulation), with no fused multiply-add on either side:

* sin/cos: Cody-Waite reduction by pi/2 split into four float32 pieces
  (12 + 12 + 12 + 24 significant bits, so ``k * P1``, ``k * P2`` and ``k * P3``
  are exact for ``|k| < 2**12``), then the Taylor series of sin (to r**9) and
  cos (to r**10) on ``|r| <= pi/4``; truncation error < 2.5e-9 relative.
  Arguments with ``|x| > 256`` take a float64 reduction (pi/2 split into a
  33-bit head and a tail, exact products for ``|k| < 2**20``), which is still
  plain IEEE arithmetic on both devices.
* tanh: ``tanh|x| = E / (E + 2)`` with ``E = expm1(2|x|)``; expm1 by
  Cody-Waite reduction by ln 2 (16-bit head) and the Taylor series of
  ``e**r - 1`` to r**8 on ``|r| <= ln2/2``, recombined as
  ``2**k * p + (2**k - 1)``. ``|x|`` is clamped at 10, where tanh rounds to 1.

The coefficients are the Taylor coefficients 1/n! rounded to float32; the
reduction constants are derived from pi/2 and ln 2 in ``_constants`` below.
Accuracy against float64 ``math`` is checked in ``tests/test_detmath.py``
(<= 2 ULP for sin/cos, <= 3 ULP for tanh over dense sweeps); the same tests
bound the distance to numpy's own float32 functions, which is what ties this
oracle to the reference's arithmetic.

The HIP twin of every function here is in
``metal-rl-envs_amd/csrc/hipenvs_device.h``; a GPU test checks the two
bit-for-bit over a million arguments.
"""

import math

import numpy as np

F32 = np.float32
SMALL_ARG = F32(256.0)
TANH_CLAMP = F32(10.0)


def _f32_truncated(x, keep_bits):
    """float32(x) with only the leading `keep_bits` significant bits kept."""
    b = int(np.array(x, dtype=np.float32).view(np.uint32))
    drop = 24 - keep_bits
    return F32(np.array(b & ~((1 << drop) - 1), dtype=np.uint32).view(np.float32))


# pi to 60 significant digits; the reduction pieces are cut from the exact rational
PI_DIGITS = "3.14159265358979323846264338327950288419716939937510582097494"


def _constants():
    from fractions import Fraction
    pio2 = Fraction(PI_DIGITS) / 2
    p1 = _f32_truncated(float(pio2), 12)
    p2 = _f32_truncated(float(pio2 - Fraction(float(p1))), 12)
    p3 = _f32_truncated(float(pio2 - Fraction(float(p1)) - Fraction(float(p2))), 12)
    p4 = F32(float(pio2 - Fraction(float(p1)) - Fraction(float(p2)) - Fraction(float(p3))))
    ln2 = math.log(2.0)
    ln2_hi = _f32_truncated(ln2, 16)
    ln2_lo = F32(ln2 - float(ln2_hi))
    # float64 head of pi/2 with 33 significant bits: kd * head is exact for |kd| < 2**20
    b = np.array(float(pio2), dtype=np.float64).view(np.uint64)
    head = (b & ~np.uint64((1 << 20) - 1)).view(np.float64)
    tail = np.float64(float(pio2 - Fraction(float(head))))
    return p1, p2, p3, p4, ln2_hi, ln2_lo, np.float64(head), tail


PIO2_1, PIO2_2, PIO2_3, PIO2_4, LN2_HI, LN2_LO, PIO2_1D, PIO2_2D = _constants()
TWO_OVER_PI = F32(2.0 / math.pi)
TWO_OVER_PI_D = np.float64(2.0 / math.pi)
LOG2E = F32(1.0 / math.log(2.0))

S3, S5, S7, S9 = (F32(v) for v in (-1 / 6, 1 / 120, -1 / 5040, 1 / 362880))
C2, C4, C6, C8, C10 = (F32(v) for v in (-1 / 2, 1 / 24, -1 / 720, 1 / 40320, -1 / 3628800))
E2, E3, E4, E5, E6, E7, E8 = (F32(1.0 / math.factorial(n)) for n in range(2, 9))

# Expected values of the derived constants; tests/test_detmath.py checks them
# against the literals compiled into the HIP header.
CONSTANT_HEX = {
    "PIO2_1": float(PIO2_1).hex(), "PIO2_2": float(PIO2_2).hex(), "PIO2_3": float(PIO2_3).hex(), "PIO2_4": float(PIO2_4).hex(),
    "LN2_HI": float(LN2_HI).hex(), "LN2_LO": float(LN2_LO).hex(),
    "TWO_OVER_PI": float(TWO_OVER_PI).hex(), "LOG2E": float(LOG2E).hex(),
    "PIO2_1D": float(PIO2_1D).hex(), "PIO2_2D": float(PIO2_2D).hex(),
}


def _reduce(x):
    """(r, q): x = r + (k mod 4) * pi/2 + 2*pi*m with |r| <= ~pi/4, r float32, q int32 in 0..3."""
    x = np.asarray(x, dtype=F32)
    with np.errstate(invalid="ignore", over="ignore"):
        k = np.rint(x * TWO_OVER_PI)
        r = (((x - k * PIO2_1) - k * PIO2_2) - k * PIO2_3) - k * PIO2_4
        q = np.zeros(x.shape, dtype=np.int32)
        small = np.abs(x) <= SMALL_ARG
        q[small] = k[small].astype(np.int32) & 3
        big = ~small
        if big.any():
            xd = x[big].astype(np.float64)
            kd = np.rint(xd * TWO_OVER_PI_D)
            r[big] = ((xd - kd * PIO2_1D) - kd * PIO2_2D).astype(F32)
            qd = kd - 4.0 * np.floor(kd * 0.25)
            # the GPU converts a NaN quadrant to 0; numpy would give INT_MIN. The
            # result is NaN either way, so pin the integer to 0 like the GPU does.
            qd = np.where(np.isfinite(qd), qd, 0.0)
            q[big] = qd.astype(np.int32) & 3
    return r, q


def _poly(r):
    z = r * r
    sp = S7 + z * S9
    sp = S5 + z * sp
    sp = S3 + z * sp
    s = r + (r * z) * sp
    cp = C8 + z * C10
    cp = C6 + z * cp
    cp = C4 + z * cp
    cp = C2 + z * cp
    c = F32(1.0) + z * cp
    return s, c


def sincos(x):
    """(sin x, cos x) as float32 arrays, bit-identical to det_sincos in hipenvs_device.h."""
    r, q = _reduce(x)
    with np.errstate(invalid="ignore", over="ignore"):
        s, c = _poly(r)
    sin = np.where(q == 0, s, np.where(q == 1, c, np.where(q == 2, -s, -c)))
    cos = np.where(q == 0, c, np.where(q == 1, -s, np.where(q == 2, -c, s)))
    return sin.astype(F32), cos.astype(F32)


def sin(x):
    return sincos(x)[0]


def cos(x):
    return sincos(x)[1]


def expm1_nonneg(y):
    """e**y - 1 for float32 y in [0, 20] (the range tanh uses)."""
    y = np.asarray(y, dtype=F32)
    with np.errstate(invalid="ignore", over="ignore"):
        k = np.rint(y * LOG2E)
        r = (y - k * LN2_HI) - k * LN2_LO
        p = E7 + r * E8
        p = E6 + r * p
        p = E5 + r * p
        p = E4 + r * p
        p = E3 + r * p
        p = E2 + r * p
        p = r + (r * r) * p
        ki = np.where(np.isfinite(k), k, 0.0).astype(np.int32)
        two_k = ((ki + 127) << 23).astype(np.int32).view(F32)
        return two_k * p + (two_k - F32(1.0))


def tanh(x):
    """float32 tanh, bit-identical to det_tanh in hipenvs_device.h."""
    x = np.asarray(x, dtype=F32)
    a = np.abs(x)
    with np.errstate(invalid="ignore"):
        a = np.where(a > TANH_CLAMP, TANH_CLAMP, a)   # NaN compares false and stays NaN
        e = expm1_nonneg(a + a)
        t = e / (e + F32(2.0))
    return np.copysign(t, x).astype(F32)


# ---------------------------------------------------------------------------
# Deterministic float64 sin/cos, for the float64 arithmetic the reference's legged
# body falls into (its numpy promotes the state to float64; legged_np.py:66 then
# evaluates np.cos/np.sin on float64 arrays). Same construction as the float32 pair:
# Cody-Waite reduction by pi/2 in three float64 pieces (33 + 33 + 53 significant
# bits: k * D1 and k * D2 exact for |k| < 2**20), then the Taylor series of sin to
# r**19 and of cos to r**20 on |r| <= pi/4 (truncation below 2**-70 relative), with
# plain float64 operations and no fused multiply-add, so the GPU reproduces every bit.
# ---------------------------------------------------------------------------

def _constants64():
    from fractions import Fraction
    pio2 = Fraction(PI_DIGITS) / 2

    def head33(v):
        b = np.array(float(v), dtype=np.float64).view(np.uint64)
        return float((b & ~np.uint64((1 << 20) - 1)).view(np.float64))

    d1 = head33(pio2)
    d2 = head33(pio2 - Fraction(d1))
    d3 = float(pio2 - Fraction(d1) - Fraction(d2))
    sin_c = tuple(float(Fraction((-1) ** i, math.factorial(2 * i + 1))) for i in range(1, 10))   # r**3 .. r**19
    cos_c = tuple(float(Fraction((-1) ** i, math.factorial(2 * i))) for i in range(1, 11))       # r**2 .. r**20
    return np.float64(d1), np.float64(d2), np.float64(d3), sin_c, cos_c


PIO2_D1, PIO2_D2, PIO2_D3, SIN64_C, COS64_C = _constants64()
TWO_OVER_PI_64 = np.float64(2.0 / math.pi)
CONSTANT_HEX.update({"PIO2_D1": float(PIO2_D1).hex(), "PIO2_D2": float(PIO2_D2).hex(),
                     "PIO2_D3": float(PIO2_D3).hex(), "TWO_OVER_PI_64": float(TWO_OVER_PI_64).hex()})


def sincos64(x):
    """(sin x, cos x) as float64 arrays, bit-identical to det_sincos64 in hipenvs_device.h.
    Any float64 x: the same operations run for every argument (accurate for |x| < 2**20 * pi/2;
    NaN and infinities give NaN)."""
    x = np.asarray(x, dtype=np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        k = np.rint(x * TWO_OVER_PI_64)
        r = ((x - k * PIO2_D1) - k * PIO2_D2) - k * PIO2_D3
        z = r * r
        sp = np.float64(SIN64_C[-1])
        for c in SIN64_C[-2::-1]:
            sp = c + z * sp
        s = r + (r * z) * sp
        cp = np.float64(COS64_C[-1])
        for c in COS64_C[-2::-1]:
            cp = c + z * cp
        co = 1.0 + z * cp
        q = k - 4.0 * np.floor(k * 0.25)
    sin_v = np.where(q == 0.0, s, np.where(q == 1.0, co, np.where(q == 2.0, -s, -co)))
    cos_v = np.where(q == 0.0, co, np.where(q == 1.0, -s, np.where(q == 2.0, -co, s)))
    return sin_v, cos_v


def _by_dtype(f32_fn, f64_fn):
    def fn(x):
        x = np.asarray(x)
        return f64_fn(x) if x.dtype == np.float64 else f32_fn(x)
    return fn


sin_by_dtype = _by_dtype(sin, lambda x: sincos64(x)[0])
cos_by_dtype = _by_dtype(cos, lambda x: sincos64(x)[1])


def trig_functions(kind):
    """(sin, cos, tanh) callables for the oracle: 'det' (bit-identical to the HIP
    kernels, the default), 'det64' (det on float32 arrays, sincos64 on float64 ones:
    the HIP reference-precision legged step) or 'numpy' (the reference's own
    np.sin/np.cos/np.tanh)."""
    if kind == "det":
        return sin, cos, tanh
    if kind == "det64":
        return sin_by_dtype, cos_by_dtype, tanh
    if kind == "numpy":
        return np.sin, np.cos, np.tanh
    raise ValueError(f"unknown trig kind {kind!r}")
