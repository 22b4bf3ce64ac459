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
