"""The oracle's deterministic transcendentals: accuracy and header agreement (CPU).

The HIP kernels evaluate the same float32 programs (hipenvs_device.h); the GPU
test test_gpu_cartpole.py::test_device_detmath_bit_exact checks the two bit for
bit. Here the oracle's functions are pinned against float64 ``math`` (the
mathematics) and against numpy's float32 functions (what the reference calls).
"""

import re
from pathlib import Path

import numpy as np
import pytest

from oracle import detmath as dm

HEADER = Path(__file__).resolve().parents[1] / "metal-rl-envs_amd" / "csrc" / "hipenvs_device.h"


def ulp_error(got, ref64):
    ulp = np.spacing(np.abs(ref64).astype(np.float32)).astype(np.float64)
    return np.abs(got.astype(np.float64) - ref64) / ulp


@pytest.mark.parametrize("lo,hi", [(-0.8, 0.8), (-10.0, 10.0), (-256.0, 256.0), (-1e5, 1e5)])
def test_sincos_within_1_5_ulp_of_float64(lo, hi):
    x = np.random.default_rng(0).uniform(lo, hi, 400_000).astype(np.float32)
    s, c = dm.sincos(x)
    xd = x.astype(np.float64)
    assert ulp_error(s, np.sin(xd)).max() <= 1.5
    assert ulp_error(c, np.cos(xd)).max() <= 1.5


def test_sincos_near_multiples_of_half_pi():
    """Where the reduction cancels: the nearest float32s to k*pi/2 for k up to 2e5."""
    t = np.arange(1, 200_000) * np.pi / 2
    x0 = t.astype(np.float32)
    x = np.concatenate([x0, np.nextafter(x0, np.float32(np.inf)), np.nextafter(x0, np.float32(0))])
    s, c = dm.sincos(x)
    xd = x.astype(np.float64)
    assert ulp_error(s, np.sin(xd)).max() <= 1.5
    assert ulp_error(c, np.cos(xd)).max() <= 1.5


@pytest.mark.parametrize("lo,hi", [(-0.3, 0.3), (-3.0, 3.0), (-12.0, 12.0)])
def test_tanh_within_2_5_ulp_of_float64(lo, hi):
    x = np.random.default_rng(1).uniform(lo, hi, 400_000).astype(np.float32)
    assert ulp_error(dm.tanh(x), np.tanh(x.astype(np.float64))).max() <= 2.5


def test_close_to_numpy_float32():
    """The reference's own np.sin/np.cos/np.tanh differ from these by at most a few ULP."""
    x = np.random.default_rng(2).uniform(-10, 10, 400_000).astype(np.float32)
    s, c = dm.sincos(x)
    for got, ref in ((s, np.sin(x)), (c, np.cos(x)), (dm.tanh(x), np.tanh(x))):
        ulp = np.spacing(np.abs(ref)).astype(np.float64)
        assert (np.abs(got.astype(np.float64) - ref) / ulp).max() <= 3.0


def test_special_values():
    x = np.array([0.0, -0.0, 1e-30, -1e-38, np.inf, -np.inf, np.nan, 300.0, -7000.5, 3e9], dtype=np.float32)
    s, c = dm.sincos(x)
    assert s[0] == 0 and s[1] == 0 and c[0] == 1 and c[1] == 1   # sin(-0) is +0 here: sign of zero not kept
    assert s[2] == np.float32(1e-30) and c[2] == 1
    assert np.isnan(s[4:7]).all() and np.isnan(c[4:7]).all()
    xd = x[7:9].astype(np.float64)
    assert ulp_error(s[7:9], np.sin(xd)).max() <= 1.5 and ulp_error(c[7:9], np.cos(xd)).max() <= 1.5
    # past |x| = 2**20 * pi/2 the float64 head product is no longer exact: still a
    # deterministic value in [-1, 1], no longer accurate to the last bits
    assert abs(s[9]) <= 1 and abs(c[9]) <= 1 and abs(s[9] ** 2 + c[9] ** 2 - 1) < 1e-5
    t = dm.tanh(np.array([0.0, -0.0, 1e-30, 20.0, -20.0, np.inf, -np.inf, np.nan], dtype=np.float32))
    assert t[0] == 0 and np.signbit(t[1]) and t[2] == np.float32(1e-30)
    assert t[3] == 1 and t[4] == -1 and t[5] == 1 and t[6] == -1 and np.isnan(t[7])


def test_header_constants_match_the_oracle():
    """Every reduction constant compiled into the HIP header equals the oracle's derivation."""
    text = HEADER.read_text()
    for name, hexval in dm.CONSTANT_HEX.items():
        m = re.search(rf"constexpr (?:float|double) {name} = (-?0x[0-9a-fA-F.]+p[+-]?\d+)f?;", text)
        assert m, name
        assert float.fromhex(m.group(1)) == float.fromhex(hexval), name
    coeffs = dict(S3=dm.S3, S5=dm.S5, S7=dm.S7, S9=dm.S9, C2=dm.C2, C4=dm.C4, C6=dm.C6, C8=dm.C8, C10=dm.C10,
                  E2=dm.E2, E3=dm.E3, E4=dm.E4, E5=dm.E5, E6=dm.E6, E7=dm.E7, E8=dm.E8)
    for name, value in coeffs.items():
        m = re.search(rf"\b{name} = (-?0x[0-9a-fA-F.]+p[+-]?\d+)f", text)
        assert m, name
        assert float.fromhex(m.group(1)) == float(value), name
    for name, values in (("SIN64_C", dm.SIN64_C), ("COS64_C", dm.COS64_C)):
        m = re.search(rf"constexpr double {name}\[\d+\] = \{{([^}}]*)\}};", text)
        assert m, name
        got = [float.fromhex(v.strip()) for v in m.group(1).split(",")]
        assert got == [float(v) for v in values], name


def _ulp64(got, exact):
    import mpmath

    out = []
    for g, t in zip(got, exact):
        out.append(0.0 if t == 0 and g == 0 else float(abs(mpmath.mpf(float(g)) - t) / np.spacing(abs(float(t)))))
    return np.array(out)


def test_sincos64_against_exact_values():
    """The float64 pair (reference-precision legged step) within 2 ulp of the exact sin/cos
    (mpmath at 200 bits) on the legged body's angle range and far beyond it."""
    import mpmath

    mpmath.mp.prec = 200
    rng = np.random.default_rng(64)
    x = np.concatenate([rng.uniform(-4, 4, 3000), rng.uniform(-1e4, 1e4, 1000), rng.uniform(-1e-6, 1e-6, 200),
                        [0.0, np.pi / 4, np.pi / 2, 3.0, 1e-300]])
    s, c = dm.sincos64(x)
    assert s.dtype == np.float64 and c.dtype == np.float64
    es = _ulp64(s, [mpmath.sin(mpmath.mpf(float(v))) for v in x])
    ec = _ulp64(c, [mpmath.cos(mpmath.mpf(float(v))) for v in x])
    assert es.max() <= 2.0 and ec.max() <= 2.0, (es.max(), ec.max())
    assert es.mean() < 0.5 and ec.mean() < 0.5


def test_sincos64_close_to_numpy_and_special_values():
    x = np.random.default_rng(65).uniform(-8, 8, 1_000_000)
    s, c = dm.sincos64(x)
    assert np.max(np.abs(s - np.sin(x)) / np.spacing(np.abs(np.sin(x)))) <= 2.0
    assert np.max(np.abs(c - np.cos(x)) / np.spacing(np.abs(np.cos(x)))) <= 2.0
    s, c = dm.sincos64(np.array([np.nan, np.inf, -np.inf]))
    assert np.isnan(s).all() and np.isnan(c).all()


def test_trig_by_dtype_dispatch():
    """'det64' evaluates float32 arrays with the float32 functions and float64 arrays with
    sincos64, as numpy's np.sin keeps each array's dtype."""
    sin_f, cos_f, _ = dm.trig_functions("det64")
    x32 = np.linspace(-3, 3, 101, dtype=np.float32)
    assert np.array_equal(sin_f(x32), dm.sin(x32)) and sin_f(x32).dtype == np.float32
    x64 = x32.astype(np.float64)
    assert np.array_equal(cos_f(x64), dm.sincos64(x64)[1]) and cos_f(x64).dtype == np.float64


def test_reduction_is_the_identity_within_078():
    """The kernels' near-rest vote (one wave vote, then the polynomial alone) relies on the
    reduction returning the argument itself (bit for bit but for -0, which reduces to +0;
    both give the same sin and cos) with quadrant 0, for |x| <= 0.78. Checked for every
    float32 in [0.5, 0.78] of both signs (below 0.5, x * 2/pi < 0.32 and rint gives 0), for
    random smaller magnitudes, and for the zeros and subnormals; and the first
    float32 above 0.78 still has quadrant 0 (the bound is conservative)."""
    lo, hi = np.float32(0.5).view(np.uint32), np.float32(0.78).view(np.uint32)
    pos = np.arange(lo, hi + 1, dtype=np.uint32).view(np.float32)
    small = np.random.default_rng(78).uniform(0, 0.5, 1_000_000).astype(np.float32)
    special = np.array([0.0, 1e-45, 1e-40, 1.17549435e-38, 1e-30], dtype=np.float32)
    x = np.concatenate([pos, -pos, small, -small, special, -special])
    for part in np.array_split(x, 8):
        r, q = dm._reduce(part)
        same = r.view(np.uint32) == part.view(np.uint32)
        assert np.all(same | ((part == 0) & (r == 0)))
        assert not q.any()
        s, c = dm.sincos(part)
        ps, pc = dm._poly(part)
        assert np.array_equal(s.view(np.uint32), ps.view(np.uint32))
        assert np.array_equal(c.view(np.uint32), pc.view(np.uint32))
    above = np.nextafter(np.float32(0.78), np.float32(1.0))
    assert dm._reduce(np.array([above]))[1][0] == 0
