"""The oracle against golden fixtures written by the reference's own numpy modules
(``tests/golden/make_golden.py``): bit for bit where the oracle restates the reference's
arithmetic literally (numpy trig, the reference's float64 promotions), and within stated
bounds for the float32 variants the HIP kernels compute (deterministic trig, float32
held throughout).
"""

from pathlib import Path

import numpy as np
import pytest

from oracle import acrobot as oa
from oracle import hopper as oh
from oracle import legged as ol
from oracle import pendulum_aba as op

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    return np.load(GOLDEN / name, allow_pickle=False)


def assert_bits(got, want):
    got, want = np.asarray(got), np.asarray(want)
    assert got.dtype == want.dtype, (got.dtype, want.dtype)
    assert got.shape == want.shape
    both_nan = np.isnan(got) & np.isnan(want)
    assert np.array_equal(np.where(both_nan, 0, got), np.where(both_nan, 0, want))
    # sign of zero too
    assert np.array_equal(np.signbit(got) | both_nan, np.signbit(want) | both_nan)


def test_acrobot_physics_bit_exact():
    g = load("acrobot_physics.npz")
    assert_bits(oa.physics(g["state"], g["action"], trig="numpy"), g["next_state"])


def test_acrobot_physics_det_trig_close():
    """Kernel arithmetic (deterministic sin/cos, <= 1.5 ULP) vs the reference's np.sin/np.cos."""
    g = load("acrobot_physics.npz")
    got = oa.physics(g["state"], g["action"], trig="det")
    np.testing.assert_allclose(got, g["next_state"], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("k", [1, 2, 3, 4, 8, 16, 32, 64])
def test_aba_accelerations_bit_exact(k):
    g = load("pendulum_aba.npz")
    got = op.aba_accelerations(g[f"k{k}_theta"], g[f"k{k}_omega"], g[f"k{k}_torque"], k, trig="numpy")
    assert_bits(got, g[f"k{k}_acc"])


@pytest.mark.parametrize("k", [2, 4, 16])
def test_aba_rk4_physics_bit_exact(k):
    g = load("pendulum_aba.npz")
    got = op.Pendulum(k, trig="numpy").physics(g[f"rk4_k{k}_state"], g[f"rk4_k{k}_action"])
    assert_bits(got, g[f"rk4_k{k}_next"])


@pytest.mark.parametrize("k", [2, 4, 16])
def test_aba_rk4_physics_det_trig_close(k):
    g = load("pendulum_aba.npz")
    got = op.Pendulum(k, trig="det").physics(g[f"rk4_k{k}_state"], g[f"rk4_k{k}_action"])
    np.testing.assert_allclose(got, g[f"rk4_k{k}_next"], rtol=1e-5, atol=5e-7)


def test_contact_impulse_bit_exact():
    g = load("contact_impulse.npz")
    lt, ln = oh.contact_impulse(g["Att"], g["Atn"], g["Ann"], g["wt"], g["wn"], g["depth"], mode="reference")
    assert_bits(lt, g["lt"])
    assert_bits(ln, g["ln"])


def test_contact_impulse_f32_close():
    g = load("contact_impulse.npz")
    lt, ln = oh.contact_impulse(g["Att"], g["Atn"], g["Ann"], g["wt"], g["wn"], g["depth"], mode="f32")
    assert np.asarray(lt).dtype == np.float32
    np.testing.assert_allclose(lt, g["lt"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(ln, g["ln"], rtol=1e-5, atol=1e-6)


LEGGED = [(c, s, 0) for c in (1, 2, 4) for s in (4, 8, 16)] + [(4, 8, 20)]


@pytest.mark.parametrize("c,s,assist", LEGGED)
def test_legged_physics_bit_exact_over_eight_steps(c, s, assist):
    """legged_np.Legged._physics chained eight times, float64 promotion and all."""
    g = load("legged_physics.npz")
    tag = f"c{c}_s{s}_a{assist}"
    body = ol.Legged(c, s, mode="reference")
    state = g[f"{tag}_state0"]
    for t in range(g[f"{tag}_traj"].shape[0]):
        state = body.physics(state, g[f"{tag}_actions"][t], float(assist))
        assert str(state.dtype) == g[f"{tag}_dtypes"][t]
        assert_bits(state.astype(np.float64), g[f"{tag}_traj"][t])


@pytest.mark.parametrize("c,s,assist", LEGGED)
def test_legged_physics_f32_one_step_close(c, s, assist):
    """The kernels' float32 arithmetic vs the reference's promoted one, one step from the
    same float32 state (observed: max abs 7.8e-6 over all cases). The reference itself
    runs this step in float64 after its first contact solve, so its result is not a float32
    trajectory and no float32 program can meet it bit for bit."""
    g = load("legged_physics.npz")
    tag = f"c{c}_s{s}_a{assist}"
    state0 = g[f"{tag}_state0"]
    got = ol.Legged(c, s, mode="f32").physics(state0, g[f"{tag}_actions"][0], float(assist))
    assert got.dtype == np.float32
    want = g[f"{tag}_traj"][0]
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=2e-5)
