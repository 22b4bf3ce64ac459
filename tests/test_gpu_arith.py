"""The kernels' shared arithmetic on the device, bit for bit against numpy's IEEE float32.

``hipenvs_div_recip`` divides as the legged kernels divide by a shared divisor (float64
reciprocal, IEEE redo for a subnormal quotient). Operands: random bit patterns (NaN, infinities,
zeros and subnormals included), quotients near 1, quotients near float32 rounding midpoints,
and exact subnormal midpoints, where the plain product rounds the wrong way and the redo
must fix it.
"""

import numpy as np
import pytest
import torch

from hipenvs import _lib


def _operands(rng):
    n = 1 << 20
    a = rng.integers(0, 1 << 32, size=n, dtype=np.uint64).astype(np.uint32).view(np.float32)
    d = rng.integers(0, 1 << 32, size=n, dtype=np.uint64).astype(np.uint32).view(np.float32)
    m1 = (rng.uniform(1, 2, n) * 2.0 ** rng.integers(-20, 20, n)).astype(np.float32)
    m2 = (rng.uniform(1, 2, n) * 2.0 ** rng.integers(-20, 20, n)).astype(np.float32)
    # near midpoints: a = RN32(m * d) for float32 midpoints m across the whole range
    mid = (2 * rng.integers(0, 1 << 23, n) + 1).astype(np.float64) * 2.0 ** rng.integers(-175, 110, n)
    dd = (1 + rng.integers(0, 4096, n) / 4096.0) * 2.0 ** rng.integers(-30, 30, n)
    d3 = dd.astype(np.float32)
    with np.errstate(over="ignore"):  # some products overflow float32 to inf, a wanted case
        a3 = (mid * d3.astype(np.float64)).astype(np.float32)
    # exact subnormal midpoints: a = (2j + 1) 2^-150 * d exactly, d an odd integer times 2^e
    j = rng.integers(0, 64, n)
    odd = (2 * rng.integers(1, 2048, n) + 1).astype(np.float64)
    d4 = (odd * 2.0 ** rng.integers(1, 8, n)).astype(np.float32)
    a4_64 = (2 * j + 1) * 2.0 ** -150 * d4.astype(np.float64)
    a4 = a4_64.astype(np.float32)
    exact = a4.astype(np.float64) == a4_64
    a4, d4 = a4[exact], d4[exact]
    specials = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 1.1754942e-38, 3.4028235e38, 1.0],
                        dtype=np.float32)
    sa, sd = np.meshgrid(specials, specials)
    return (np.concatenate([a, m1, a3, a4, sa.ravel()]).astype(np.float32),
            np.concatenate([d, m2, d3, d4, sd.ravel()]).astype(np.float32), len(a4))


@pytest.mark.gpu
def test_div_recip_is_ieee_division(dev):
    rng = np.random.default_rng(7)
    a, d, n_mid = _operands(rng)
    assert n_mid > 1000
    ta, td = torch.from_numpy(a).to(dev), torch.from_numpy(d).to(dev)
    q = torch.empty_like(ta)
    marked = torch.empty(a.shape, dtype=torch.uint8, device=dev)
    _lib.call("hipenvs_div_recip", _lib.ptr(ta), _lib.ptr(td), _lib.ptr(q), _lib.ptr(marked), a.size,
              _lib.stream_of(dev))
    q, marked = q.cpu().numpy(), marked.cpu().numpy().astype(bool)
    with np.errstate(all="ignore"):
        want = a / d
        fast = (a.astype(np.float64) * (1.0 / d.astype(np.float64))).astype(np.float32)
    both_nan = np.isnan(q) & np.isnan(want)
    np.testing.assert_array_equal(np.where(both_nan, 0, q.view(np.uint32)), np.where(both_nan, 0, want.view(np.uint32)))
    fb = fast.view(np.uint32) & 0x7FFFFFFF
    np.testing.assert_array_equal(marked, (fb != 0) & (fb <= 0x7FFFFF))
    # the redo path ran and mattered: exact subnormal midpoints where the product alone is wrong
    wrong = (fast.view(np.uint32) != want.view(np.uint32)) & ~(np.isnan(fast) & np.isnan(want))
    assert wrong.sum() > 100 and marked[wrong].all()


@pytest.mark.gpu
def test_sqrt_and_recip_match_ieee_for_every_float32(dev):
    """The kernels' square root (float64 reciprocal square root estimate, one Newton step,
    rounded to float32) and float64 reciprocal (hardware estimate, two Newton steps) against
    IEEE sqrtf and 1.0 / (double)x, over all 2^32 float32 bit patterns, in 16 launches of
    2^28. The Cholesky pivots and the shared-reciprocal divisions rest on both."""
    counts = torch.zeros(2, dtype=torch.int64, device=dev)
    step = 1 << 28
    for first in range(0, 1 << 32, step):
        _lib.call("hipenvs_sqrt_recip_check", first, step, _lib.ptr(counts), _lib.stream_of(dev))
    sqrt_bad, recip_bad = counts.cpu().tolist()
    assert (sqrt_bad, recip_bad) == (0, 0)


@pytest.mark.gpu
def test_sqrt_recip_check_argument_bounds(dev):
    """The check's own arguments: a range past 2^32 is refused, an empty one does nothing."""
    counts = torch.zeros(2, dtype=torch.int64, device=dev)
    with pytest.raises(RuntimeError):
        _lib.call("hipenvs_sqrt_recip_check", (1 << 32) - 4, 8, _lib.ptr(counts), _lib.stream_of(dev))
    _lib.call("hipenvs_sqrt_recip_check", 0, 0, _lib.ptr(counts), _lib.stream_of(dev))
    assert counts.cpu().tolist() == [0, 0]

