"""The kernels' arithmetic against the reference's own, on the CPU (oracle only).

The HIP kernels reproduce the oracle's default arithmetic bit for bit (deterministic
float32 sin/cos, the float32 legged step; the GPU tests check every kernel that way). The
oracle with ``trig="numpy"`` (and, for the legged body, ``mode="reference"``) is the
reference's numpy program bit for bit: ``test_golden.py`` checks it against fixtures written
by the reference's own modules. Here the two arithmetics are compared, so the reference's
parity targets -- each step's float32 state within 1e-5 relative, and identical termination
and reset flags over 100 steps -- are checked against the reference's arithmetic rather
than against the oracle the kernels match:

* per-step gaps, measured per body and chain length K, on the golden inputs and on the
  benchmark's own states (each bound is the measured maximum, rounded up);
* conditioning: every gap is at most what the reference's own step does when its input
  moves by one ulp (seven perturbation patterns). Where a gap exceeds 1e-5 relative on a
  component, the reference's step itself is that sensitive there, so no float32 program
  whose sin/cos round differently from numpy's can do better;
* flags identical over 100 steps: free-running from the benchmarks' start distributions,
  and teacher-forced (both arithmetics stepping from the reference's state at every step)
  from states near or across the termination boundary, where flags actually flip.

Relative errors are taken over components with |x| > 1e-3, absolute ones over all.
"""

from pathlib import Path

import numpy as np
import pytest

from oracle import acrobot as oa
from oracle import cartpole as oc
from oracle import legged as ol
from oracle import pendulum_aba as op
from oracle import rng

GOLDEN = Path(__file__).resolve().parent / "golden"
INF = np.float32(np.inf)


def gaps(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    err = np.abs(got - want)
    big = np.abs(want) > 1e-3
    return float(err.max()), float((err[big] / np.abs(want[big])).max()) if big.any() else 0.0


def one_ulp_inputs(x, row_blocks):
    """x with one block of rows moved one ulp up or down, and with every component moved one
    ulp in a random direction (three draws)."""
    out = []
    for rows in row_blocks:
        for d in (INF, -INF):
            y = x.copy()
            y[rows] = np.nextafter(y[rows], d)
            out.append(y)
    r = np.random.default_rng(0)
    for _ in range(3):
        up = r.integers(0, 2, size=x.shape).astype(bool)
        out.append(np.where(up, np.nextafter(x, INF), np.nextafter(x, -INF)).astype(np.float32))
    return out


def reference_move(step, x, row_blocks, want):
    """The largest (abs, rel) change of the reference's own step over the one-ulp inputs."""
    worst_abs = worst_rel = 0.0
    for y in one_ulp_inputs(x, row_blocks):
        a, r = gaps(step(y), want)
        worst_abs, worst_rel = max(worst_abs, a), max(worst_rel, r)
    return worst_abs, worst_rel


def check(gap, bound, move=None):
    """gap within its measured bound and, when given, within the reference's one-ulp move."""
    (ga, gr), (ba, br) = gap, bound
    assert ga <= ba and gr <= br, f"gap abs {ga:.3e} rel {gr:.3e} above the measured bound {ba:.1e} / {br:.1e}"
    if move is not None:
        ma, mr = move
        assert ga <= ma and gr <= mr, f"gap {ga:.3e} / {gr:.3e} above the reference's one-ulp move {ma:.3e} / {mr:.3e}"


# ---------------------------------------------------------------------------
# K-link pendulum (articulated-body algorithm)
# ---------------------------------------------------------------------------

# (abs, rel) bounds: measured maxima rounded up. Golden inputs: angles U[-pi, pi], rates
# U[-3, 3] (tests/golden/make_golden.py), wide enough that accelerations reach ~1e2 and
# cancel; the deterministic trig's ~1 ulp differences from np.sin/np.cos then reach
# 5.9e-4 relative on a component at K = 64, against 1.9e-3 for the reference's own
# one-ulp move.
ABA_ACC_GOLDEN = {1: (5e-7, 7e-8), 2: (1e-6, 5e-7), 3: (1e-6, 2.4e-6), 4: (4.3e-6, 2.2e-4), 8: (1.1e-5, 2.1e-3),
                  16: (1.4e-5, 6.0e-5), 32: (2.0e-5, 2.3e-4), 64: (4.1e-5, 6.0e-4)}
ABA_RK4_GOLDEN = {2: (6e-8, 1.9e-6), 4: (6e-8, 6.5e-7), 16: (1.2e-7, 1.9e-6)}
# One step from the benchmark's own states: config-3 chains (angles U[+-0.1], rates 0,
# torques U[-1, 1], semi-implicit Euler dt 0.01) after 300 steps, 256 envs; the Euler step
# and the reference's RK4 step (discrete torque) from those states.
ABA_EULER_C3 = {4: (1e-8, 7e-8), 16: (1.2e-7, 8e-7), 32: (1.2e-7, 1.1e-6), 64: (2.4e-7, 2.1e-5)}
ABA_RK4_C3 = {4: (2e-8, 1.5e-7), 16: (1.2e-7, 1.9e-6), 32: (2.4e-7, 3.8e-6), 64: (2.4e-7, 4.1e-5)}


def load(name):
    return np.load(GOLDEN / name, allow_pickle=False)


@pytest.mark.parametrize("k", [1, 2, 3, 4, 8, 16, 32, 64])
def test_aba_accelerations_gap_on_golden(k):
    g = load("pendulum_aba.npz")
    th, om, tq, want = g[f"k{k}_theta"], g[f"k{k}_omega"], g[f"k{k}_torque"], g[f"k{k}_acc"]
    gap = gaps(op.aba_accelerations(th, om, tq, k, trig="det"), want)
    move = reference_move(lambda y: op.aba_accelerations(y[:k], y[k:], tq, k, trig="numpy"),
                          np.concatenate([th, om]), (slice(0, k), slice(k, 2 * k)), want)
    check(gap, ABA_ACC_GOLDEN[k], move)


@pytest.mark.parametrize("k", [2, 4, 16])
def test_aba_rk4_step_gap_on_golden(k):
    g = load("pendulum_aba.npz")
    state, action, want = g[f"rk4_k{k}_state"], g[f"rk4_k{k}_action"], g[f"rk4_k{k}_next"]
    gap = gaps(op.Pendulum(k, trig="det").physics(state, action), want)
    move = reference_move(lambda y: op.Pendulum(k, trig="numpy").physics(y, action), state,
                          (slice(0, k), slice(k, 2 * k)), want)
    check(gap, ABA_RK4_GOLDEN[k], move)


_C3_STATES = {}


def config3_states(k, n=256, steps=300):
    """Config-3 chains after `steps` Euler steps in the kernels' arithmetic (cached per K)."""
    if k not in _C3_STATES:
        p = op.Pendulum(k, trig="det")
        s = p.reset_euler(n, seed=0)
        for t in range(1, steps + 1):
            s, _, _ = p.step_euler(s, None, t)
        _C3_STATES[k] = s
    return _C3_STATES[k]


@pytest.mark.parametrize("k", [4, 16, 32, 64])
def test_aba_euler_step_gap_on_config3_states(k):
    s = config3_states(k)
    tq = rng.torque_uniform(301, s.shape[1])
    want = op.Pendulum(k, trig="numpy").physics_euler(s, tq)
    gap = gaps(op.Pendulum(k, trig="det").physics_euler(s, tq), want)
    move = reference_move(lambda y: op.Pendulum(k, trig="numpy").physics_euler(y, tq), s,
                          (slice(0, k), slice(k, 2 * k)), want)
    check(gap, ABA_EULER_C3[k], move)
    if k <= 32:  # the 1e-5 relative bar itself holds up to K = 32
        assert gap[1] <= 1e-5


@pytest.mark.parametrize("k", [4, 16, 32, 64])
def test_aba_rk4_step_gap_on_config3_states(k):
    s = config3_states(k)
    act = rng.uniform_actions(302, s.shape[1], 3)
    want = op.Pendulum(k, trig="numpy").physics(s, act)
    gap = gaps(op.Pendulum(k, trig="det").physics(s, act), want)
    move = reference_move(lambda y: op.Pendulum(k, trig="numpy").physics(y, act), s,
                          (slice(0, k), slice(k, 2 * k)), want)
    check(gap, ABA_RK4_C3[k], move)
    if k <= 32:
        assert gap[1] <= 1e-5


# ---------------------------------------------------------------------------
# CartPole and Acrobot
# ---------------------------------------------------------------------------

def test_cartpole_step_gap():
    """Random states across the live region, one step: the deterministic sin/cos of theta
    differ from numpy's by at most an ulp, and the step's state moves by less than 1e-5
    relative."""
    r = np.random.default_rng(7)
    n = 65536
    s = np.stack([r.uniform(-2.4, 2.4, n), r.uniform(-3, 3, n), r.uniform(-0.21, 0.21, n),
                  r.uniform(-3, 3, n)]).astype(np.float32)
    a = r.integers(0, 2, n)
    want = oc.physics(s, a, trig="numpy")
    gap = gaps(oc.physics(s, a, trig="det"), want)
    move = reference_move(lambda y: oc.physics(y, a, trig="numpy"), s, (slice(2, 3),), want)
    check(gap, (2.4e-7, 2e-6), move)
    assert gap[1] <= 1e-5


def test_acrobot_step_gap_on_golden():
    g = load("acrobot_physics.npz")
    want = g["next_state"]
    gap = gaps(oa.physics(g["state"], g["action"], trig="det"), want)
    move = reference_move(lambda y: oa.physics(y, g["action"], trig="numpy"), g["state"],
                          (slice(0, 2), slice(2, 4)), want)
    check(gap, ACROBOT_GOLDEN, move)


ACROBOT_GOLDEN = (2.7e-5, 6.5e-6)


# ---------------------------------------------------------------------------
# Flags over 100 steps
# ---------------------------------------------------------------------------

def free_running(step_a, step_b, s, steps):
    """Two chains from the same start, each on its own state; (mismatched flags, terminations)."""
    sa = sb = s
    mismatches = terminations = 0
    for t in range(1, steps + 1):
        sa, _, da = step_a(sa, t)
        sb, _, db = step_b(sb, t)
        mismatches += int((da != db).sum())
        terminations += int(db.sum())
    return mismatches, terminations


def teacher_forced(step_a, step_b, s, steps):
    """Both arithmetics step from the reference chain's state at every step."""
    mismatches = terminations = 0
    for t in range(1, steps + 1):
        _, _, da = step_a(s, t)
        s, _, db = step_b(s, t)
        mismatches += int((da != db).sum())
        terminations += int(db.sum())
    return mismatches, terminations


def test_cartpole_flags_free_running_100_steps():
    """Config 0's shape: 4,096 envs from the reset distribution, Bernoulli actions."""
    n = 4096
    acts = [rng.action_bits(1000 + t, n) for t in range(101)]
    mism, term = free_running(lambda s, t: oc.step(s, acts[t], t, trig="det"),
                              lambda s, t: oc.step(s, acts[t], t, trig="numpy"), oc.reset(n, seed=0), 100)
    assert mism == 0 and term > 10000, (mism, term)


def test_acrobot_flags_teacher_forced_100_steps():
    """Half the envs from the reset distribution, half from wide states (both angles
    U[-pi, pi], rates U[-4, 4] and U[-8, 8]) that swing up and terminate."""
    r = np.random.default_rng(5)
    n = 4096
    s = oa.reset(n, seed=0)
    h = n // 2
    s[:, :h] = np.stack([r.uniform(-np.pi, np.pi, h), r.uniform(-np.pi, np.pi, h), r.uniform(-4, 4, h),
                         r.uniform(-8, 8, h)]).astype(np.float32)
    acts = [rng.uniform_actions(1000 + t, n, 3) for t in range(101)]
    mism, term = teacher_forced(lambda s, t: oa.step(s, acts[t], t, trig="det"),
                                lambda s, t: oa.step(s, acts[t], t, trig="numpy"), s, 100)
    assert mism == 0 and term > 1000, (mism, term)


def boundary_chains(k, n, reset):
    """Half the chains from `reset`, half raised around the termination boundary: joint
    angles such that -sum cos th sits near K/2 (absolute angles 2 pi / 3 + U[-0.25, 0.25]),
    rates U[-1, 1]."""
    r = np.random.default_rng(k)
    s = reset.copy()
    h = n // 2
    s[:k, :h] = (2 * np.pi / 3 + r.uniform(-0.25, 0.25, (k, h))).astype(np.float32)
    s[k:, :h] = r.uniform(-1, 1, (k, h)).astype(np.float32)
    return s


@pytest.mark.parametrize("k", [4, 16, 64])
def test_aba_euler_flags_teacher_forced_100_steps(k):
    n = 512
    pa, pb = op.Pendulum(k, trig="det"), op.Pendulum(k, trig="numpy")
    s = boundary_chains(k, n, pa.reset_euler(n, seed=0))
    mism, term = teacher_forced(lambda s, t: pa.step_euler(s, None, t), lambda s, t: pb.step_euler(s, None, t), s, 100)
    assert mism == 0 and term > 50, (mism, term)


@pytest.mark.parametrize("k", [4, 16, 64])
def test_aba_rk4_flags_teacher_forced_100_steps(k):
    n = 256
    pa, pb = op.Pendulum(k, trig="det"), op.Pendulum(k, trig="numpy")
    s = boundary_chains(k, n, pa.reset(n, seed=0))
    acts = [rng.uniform_actions(1000 + t, n, 3) for t in range(101)]
    mism, term = teacher_forced(lambda s, t: pa.step(s, acts[t], t), lambda s, t: pb.step(s, acts[t], t), s, 100)
    assert mism == 0 and term > 25, (mism, term)


@pytest.mark.parametrize("k", [4, 16, 64])
def test_aba_euler_flags_free_running_config3(k):
    """Config 3's own chains (reset U[+-0.1], rates 0, torques U[-1, 1]) never reach the
    boundary in 100 steps in either arithmetic; the flags agree (all clear)."""
    n = 256
    pa, pb = op.Pendulum(k, trig="det"), op.Pendulum(k, trig="numpy")
    mism, term = free_running(lambda s, t: pa.step_euler(s, None, t), lambda s, t: pb.step_euler(s, None, t),
                              pa.reset_euler(n, seed=0), 100)
    assert mism == 0, (mism, term)


@pytest.mark.parametrize("c", [2, 4])
def test_legged_flags_free_running_100_steps(c):
    """The legged body, 8 sweeps, 256 envs from the stand reset with uniform actions: the
    float32 step (the kernels' arithmetic) and the reference-precision step (deterministic
    float32/float64 trig) each against the reference's numpy program."""
    n = 256
    ref = ol.Legged(c, 8, mode="reference", trig="numpy")
    f32 = ol.Legged(c, 8, mode="f32", trig="det")
    det64 = ol.Legged(c, 8, mode="reference", trig="det64")
    s = f32.reset(n, seed=0)
    acts = [rng.uniform_actions(1000 + t, n, 3**c) for t in range(101)]
    ref_step = lambda s, t: ref.step(s, acts[t], t)  # noqa: E731
    mism, term = free_running(lambda s, t: f32.step(s, acts[t], t), ref_step, s, 100)
    assert mism == 0 and term > 500, ("float32", mism, term)
    mism, term = free_running(lambda s, t: det64.step(s, acts[t], t), ref_step, s, 100)
    assert mism == 0 and term > 500, ("reference precision", mism, term)
