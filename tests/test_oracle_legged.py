"""The hopper and legged oracles pinned by the reference's physics tests (CPU):
test_hopper.py (analytic flight, standing, landing, friction, contact laws) and
test_legged.py (C = 1 is the hopper, sweep convergence, landing, finiteness), in
both the literal ("reference") and the float32 ("f32") arithmetic."""

import numpy as np
import pytest

from oracle import hopper as hp
from oracle import legged as lg

MODES = ["reference", "f32"]


def _run(q, v, torque, substeps, mu=hp.MU, mode="reference"):
    for _ in range(substeps):
        q, v = hp.substep(q, v, torque, mu=mu, mode=mode)
    return q, v


def _col(*vals):
    return np.array(vals, dtype=np.float32)[:, None]


@pytest.mark.parametrize("mode", MODES)
def test_free_flight_is_a_parabola(mode):
    """test_hopper.py:21-28."""
    q, v = _col(0.0, 10.0, 0.0, 0.0), _col(0.3, 0.0, 0.0, 0.0)
    q, v = _run(q, v, np.zeros(1, dtype=np.float32), 100, mode=mode)
    t = 100 * hp.H
    assert abs(q[1, 0] - (10.0 - 0.5 * hp.GRAVITY * t * t)) < 0.06
    assert abs(q[0, 0] - 0.3 * t) < 1e-4 and abs(q[2, 0]) < 1e-6 and abs(q[3, 0]) < 1e-6


@pytest.mark.parametrize("mode", MODES)
def test_energy_conserved_in_flight_with_rotation(mode):
    """test_hopper.py:31-40."""
    q, v = _col(0.0, 10.0, 0.3, -0.5), _col(0.0, 0.0, 2.0, 3.0)

    def energy(q, v):
        f = hp.foot(q)
        a = q[2] + q[3]
        ad = v[2] + v[3]
        vf = (v[0] + hp.L * np.cos(a) * ad, v[1] + hp.L * np.sin(a) * ad)
        return (0.5 * hp.M_T * (v[0] ** 2 + v[1] ** 2) + 0.5 * hp.I_T * v[2] ** 2 + 0.5 * hp.M_F * (vf[0] ** 2 + vf[1] ** 2)
                + hp.GRAVITY * (hp.M_T * q[1] + hp.M_F * f[1]))[0]

    e0 = energy(q, v)
    q, v = _run(q, v, np.zeros(1, dtype=np.float32), 100, mode=mode)
    assert abs(energy(q, v) - e0) / abs(e0) < 0.01


@pytest.mark.parametrize("mode", MODES)
def test_standing_body_does_not_drift(mode):
    """test_hopper.py:43-48."""
    q, v = _col(0.0, hp.L, 0.0, 0.0), _col(0.0, 0.0, 0.0, 0.0)
    q, v = _run(q, v, np.zeros(1, dtype=np.float32), 400, mode=mode)
    assert np.abs(q[:, 0] - [0.0, hp.L, 0.0, 0.0]).max() < 1e-3
    assert np.abs(v[:, 0]).max() < 1e-3


@pytest.mark.parametrize("mode", MODES)
def test_inelastic_drop_lands_and_stays(mode):
    """test_hopper.py:51-58."""
    q, v = _col(0.0, hp.L + 0.5, 0.0, 0.0), _col(0.0, 0.0, 0.0, 0.0)
    min_foot = 0.0
    for _ in range(300):
        q, v = _run(q, v, np.zeros(1, dtype=np.float32), 1, mode=mode)
        min_foot = min(min_foot, hp.foot(q)[1, 0])
    assert min_foot > -0.02
    assert abs(q[1, 0] - hp.L) < 0.01 and abs(v[1, 0]) < 1e-2


@pytest.mark.parametrize("mode", MODES)
def test_friction_slows_a_sliding_foot_and_zero_friction_does_not(mode):
    """test_hopper.py:61-69."""
    q0, v0 = _col(0.0, hp.L, 0.0, 0.0), _col(1.0, 0.0, 0.0, 0.0)

    def foot_speed(q, v):
        a = q[2] + q[3]
        return (v[0] + hp.L * np.cos(a) * (v[2] + v[3]))[0]

    q, v = _run(q0, v0, np.zeros(1, dtype=np.float32), 5, mode=mode)
    assert 0.0 <= foot_speed(q, v) < 1.0
    q, v = _run(q0, v0, np.zeros(1, dtype=np.float32), 5, mu=0.0, mode=mode)
    assert abs(foot_speed(q, v) - 1.0) < 0.05


@pytest.mark.parametrize("mode", MODES)
def test_contact_impulse_satisfies_complementarity(mode):
    """test_hopper.py:84-113 on 2,000 random SPD Delassus matrices."""
    r = np.random.default_rng(0)
    n = 2000
    b = r.uniform(-1, 1, (n, 2, 2))
    A = np.einsum("nij,nkj->nik", b, b) + 0.05 * np.eye(2)
    Att, Atn, Ann = A[:, 0, 0].astype(np.float32), A[:, 0, 1].astype(np.float32), A[:, 1, 1].astype(np.float32)
    wt, wn = r.uniform(-2, 2, n).astype(np.float32), r.uniform(-2, 2, n).astype(np.float32)
    depth = r.uniform(-0.1, 0.1, n).astype(np.float32)
    lt, ln = hp.contact_impulse(Att, Atn, Ann, wt, wn, depth, hp.MU, mode)
    target = hp.BAUMGARTE / hp.H * np.maximum(depth, 0.0)
    wt2, wn2 = wt + Att * lt + Atn * ln, wn + Atn * lt + Ann * ln
    assert (ln >= 0).all() and (ln[depth < 0] == 0).all()
    well_posed = Ann > hp.MU * np.abs(Atn)
    assert 0.5 < well_posed.mean() < 0.95
    assert (ln[~well_posed & (wn >= target)] == 0).all()
    sel = well_posed
    lt, ln, target, wt2, wn2 = (x[sel] for x in (lt, ln, target, wt2, wn2))
    pushing = ln > 0
    np.testing.assert_allclose(wn2[pushing], target[pushing], atol=1e-3)
    assert (np.abs(lt) <= hp.MU * ln + 1e-5).all()
    inside = pushing & (np.abs(lt) < hp.MU * ln - 1e-4)
    np.testing.assert_allclose(wt2[inside], 0.0, atol=1e-3)
    edge = pushing & ~inside
    assert (np.sign(wt2[edge]) * np.sign(lt[edge]) <= 0).all()


def hopper_states(n, seed=0):
    """test_hopper.py:116-121: mixed regimes."""
    r = np.random.default_rng(seed)
    q = np.stack([r.uniform(-1, 1, n), r.uniform(0.7, 1.3, n), r.uniform(-0.6, 0.6, n), r.uniform(-0.8, 0.8, n)])
    v = r.uniform(-2, 2, (4, n))
    return np.concatenate([q, v]).astype(np.float32), r.integers(0, 3, n)


def legged_states(c, n, seed=0):
    """test_legged.py:11-16."""
    r = np.random.default_rng(seed)
    d = 3 + c
    q = np.concatenate([np.stack([r.uniform(-1, 1, n), r.uniform(0.7, 1.3, n), r.uniform(-0.6, 0.6, n)]),
                        r.uniform(-0.8, 0.8, (c, n))])
    v = r.uniform(-2, 2, (d, n))
    return np.concatenate([q, v]).astype(np.float32), r.integers(0, 3**c, n)


@pytest.mark.parametrize("mode", MODES)
def test_one_leg_is_the_hopper(mode):
    """test_legged.py:20-26: C = 1 with one sweep reproduces the hopper step."""
    state, action = hopper_states(300)
    ref = hp.Hopper().physics(state, action, mode=mode, trig="numpy" if mode == "reference" else "det")
    out = lg.Legged(1, iters=1, mode=mode).physics(state, action)
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-5)


def test_hopper_is_one_leg_with_the_hoppers_impulse_order():
    """In float32 the hopper step is the C = 1, one-sweep legged substep exactly once the two
    impulse terms are added in the hopper's order; the HIP hopper kernel is built that way."""
    state, action = hopper_states(3000, seed=4)
    ref = hp.Hopper().physics(state, action, mode="f32", trig="det")
    q, v = state[:4], state[4:]
    tq = lg.torques(action, 1)
    for _ in range(hp.SUBSTEPS):
        q, v = lg.substep(q, v, tq, 1, iters=1, mode="f32", hopper_sum=True)
    np.testing.assert_array_equal(np.concatenate([q, v]), ref)
    assert not np.array_equal(lg.Legged(1, iters=1, mode="f32").physics(state, action), ref)


def standing_drift(c, iters, substeps=400, mode="f32"):
    """test_legged.py:29-38."""
    pose = lg.static_pose(c)
    d = 3 + c
    q = pose[:d].astype(np.float32)[:, None]
    v = np.zeros((d, 1), dtype=np.float32)
    tq = [np.zeros(1, dtype=np.float32)] * c
    for _ in range(substeps):
        q, v = lg.substep(q, v, tq, c, iters=iters, mode=mode)
    return float(np.abs(q[:, 0] - pose[:d]).max())


def test_standing_on_two_legs_converges_with_iterations():
    """test_legged.py:41-46, literally in the reference arithmetic: exact at 256 sweeps.
    In float32 the creep falls the same way down to a floor of ~2.3e-4 rad (the legs
    splay by float32 rounding of the balance), which bounds the f32 assertion instead."""
    drifts = [standing_drift(2, k, mode="reference") for k in (1, 4, lg.ITERS, 32, 256)]
    assert all(a > b for a, b in zip(drifts, drifts[1:])), drifts
    assert drifts[-1] < 1e-6 and drifts[2] < 1e-2, drifts
    f32 = [standing_drift(2, k) for k in (1, 4, lg.ITERS, 32)]
    assert all(a > b for a, b in zip(f32, f32[1:])), f32
    assert f32[-1] < 1e-3 and f32[2] < 1e-2, f32


def test_redundant_contacts_converge_too():
    """test_legged.py:49-55 (four legs as two coincident pairs), float32 arithmetic."""
    drifts = [standing_drift(4, k) for k in (1, lg.ITERS, 64)]
    assert all(a > b for a, b in zip(drifts, drifts[1:])), drifts
    assert drifts[-1] < 5e-3 and drifts[1] < 2e-2, drifts


def test_drop_on_two_legs_lands_without_bounce():
    """test_legged.py:58-66."""
    stand = lg.stand_pose(2)
    q = stand[:5].astype(np.float32)[:, None].copy()
    q[1] += 0.4
    v = np.zeros((5, 1), dtype=np.float32)
    tq = [np.zeros(1, dtype=np.float32)] * 2
    min_foot = 0.0
    for _ in range(300):
        q, v = lg.substep(q, v, tq, 2, mode="f32")
        min_foot = min(min_foot, (q[1] - lg.L * np.cos(q[2] + q[3:5])).min())
    assert min_foot > -0.03 and abs(q[1, 0] - stand[1]) < 0.02 and abs(v[1, 0]) < 1e-2


def visited_states(c, n=400, steps=50, seed=0):
    """test_legged.py:69-76: states a random policy reaches from the reset."""
    from oracle import rng

    body = lg.Legged(c)
    state = body.reset(n, seed=seed)
    for t in range(1, steps + 1):
        state, _, _ = body.step(state, rng.uniform_actions(t, n, 3**c), seed=t)
    return state, rng.uniform_actions(steps + 1, n, 3**c)


def test_gauss_seidel_converges_on_visited_states():
    """test_legged.py:79-95."""
    c = 4
    state, action = visited_states(c)
    q, v = state[:7], state[7:]
    tq = lg.torques(action, c)
    _, ref_v = lg.substep(q, v, tq, c, iters=1024, mode="f32")
    p99 = []
    for k in (1, 2, 4, 8, 16, 32):
        _, vk = lg.substep(q, v, tq, c, iters=k, mode="f32")
        err = np.abs(vk - ref_v).max(axis=0)
        p99.append(np.percentile(err, 99))
    assert all(a > b for a, b in zip(p99, p99[1:])), p99
    assert p99[3] < 0.1 and p99[4] < 1e-2 and p99[5] < 1e-3, p99
    assert (err > 1e-2).mean() < 0.02


@pytest.mark.parametrize("c", [1, 2, 4])
def test_test_states_mix_regimes_and_f32_tracks_the_literal_reference(c):
    """test_legged.py:98-110's mixed states: the float32 program against the literal
    (float64-promoting) reference, within the reference's own 1e-3 gate, p99 within 1e-5."""
    state, action = legged_states(c, 300, seed=c)
    ref = lg.Legged(c, mode="reference").physics(state, action)
    out = lg.Legged(c, mode="f32").physics(state, action)
    assert ref.dtype == np.float64 and out.dtype == np.float32
    np.testing.assert_allclose(out, ref, rtol=1e-3, atol=1e-3)
    rel = np.abs(out - ref) / (np.abs(ref) + 1e-3)
    assert np.percentile(rel, 99) < 1e-5
    touching = ((state[1] - lg.L * np.cos(state[2] + state[3:3 + c])) <= 0).mean()
    assert 0.2 < touching < 0.8


def test_random_policy_stays_finite_above_the_floor():
    """test_legged.py:113-122."""
    from oracle import rng

    for c in (2, 4):
        body = lg.Legged(c)
        state = body.reset(512, seed=0)
        worst = 0.0
        for t in range(1, 201):
            state, reward, done = body.step(state, rng.uniform_actions(t, 512, 3**c), seed=t)
            worst = min(worst, (state[1] - lg.L * np.cos(state[2] + state[3:3 + c])).min())
        assert np.isfinite(state).all() and worst > -0.08, (c, worst)
        assert state.dtype == np.float32 and reward.dtype == np.float32
