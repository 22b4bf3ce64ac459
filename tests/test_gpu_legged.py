"""Legged step and fused legged ES rollout kernels vs the oracle, through the C ABI (GPU).

Bar: bit-exact against the oracle's float32 restatement of legged_np (the
arithmetic of the reference's Metal kernel). The literal reference promotes to
float64 inside contact_impulse; the oracle tests bound that gap separately.
"""

import numpy as np
import pytest
import torch

from oracle import es as oes
from oracle import legged as olg
from oracle import rng
from test_oracle_legged import legged_states

pytestmark = pytest.mark.gpu


def to_np(t):
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("c", [1, 2, 3, 4])
@pytest.mark.parametrize("iters", [1, 8])
def test_step_matches_oracle(dev, c, iters):
    from hipenvs import legged

    state, action = legged_states(c, 300, seed=c)
    body = legged.Legged(c, iters)
    body.reseed(3)
    ns, rew, done = body.step(torch.from_numpy(state).to(dev), torch.from_numpy(action.astype(np.int32)).to(dev))
    ens, erew, edone = olg.Legged(c, iters).step(state, action, seed=4)
    np.testing.assert_array_equal(to_np(ns), ens)
    np.testing.assert_array_equal(to_np(rew), erew)
    np.testing.assert_array_equal(to_np(done), edone)


def test_step_at_the_benchmark_size(dev):
    """C = 4, 8 sweeps at N = 65,536, the reference's legged step benchmark shape."""
    from hipenvs import legged

    state, action = legged_states(4, 1 << 16, seed=16)
    state[1, :2000] = 0.4  # torsos below the fall height: these terminate and reset
    state[2, 2000:4000] = 1.3  # and tilted past the fall angle
    body = legged.Legged(4, 8)
    body.reseed(5)
    ns, rew, done = body.step(torch.from_numpy(state).to(dev), torch.from_numpy(action.astype(np.int32)).to(dev))
    ens, erew, edone = olg.Legged(4, 8).step(state, action, seed=6)
    np.testing.assert_array_equal(to_np(done), edone)
    np.testing.assert_array_equal(to_np(ns), ens)
    np.testing.assert_array_equal(to_np(rew), erew)
    assert 0 < edone.sum() < len(edone)


@pytest.mark.parametrize("c", [2, 4])
def test_step_with_assist_matches_oracle(dev, c):
    from hipenvs import legged

    state, action = legged_states(c, 200, seed=10 + c)
    body = legged.Legged(c)
    body.reseed(0)
    ns, rew, done = body.step(torch.from_numpy(state).to(dev), torch.from_numpy(action.astype(np.int32)).to(dev), 20.0)
    ens, erew, edone = olg.Legged(c).step(state, action, seed=1, assist=20.0)
    np.testing.assert_array_equal(to_np(ns), ens)
    np.testing.assert_array_equal(to_np(done), edone)


@pytest.mark.parametrize("c", [2, 4])
def test_free_running_chain_identical_flags(dev, c):
    """Reset, then 40 steps of uniform random actions: identical flags every step."""
    from hipenvs import legged

    n = 512
    body, ref = legged.Legged(c), olg.Legged(c)
    s_dev = body.reset(n, seed=1, device=dev)
    s_ref = ref.reset(n, seed=1)
    np.testing.assert_array_equal(to_np(s_dev), s_ref)
    body.reseed(100)
    for t in range(101, 141):
        a = rng.uniform_actions(t, n, 3**c)
        s_dev, _, d_dev = body.step(s_dev, torch.from_numpy(a).to(dev))
        s_ref, _, d_ref = ref.step(s_ref, a, seed=t)
        np.testing.assert_array_equal(to_np(d_dev), d_ref, err_msg=f"step {t}")
    np.testing.assert_array_equal(to_np(s_dev), s_ref)


def _population(p, c, hidden, scale, seed):
    from hipenvs import legged_rollout

    r = np.random.default_rng(seed)
    return (r.standard_normal((p, legged_rollout.n_params(hidden, c))) * scale).astype(np.float32)


@pytest.mark.parametrize("iters", [4, 8, 16])
@pytest.mark.parametrize("c,hidden,p,horizon", [(1, 8, 128, 60), (2, 16, 256, 100), (2, 64, 96, 40),
                                                 (3, 32, 96, 40), (4, 64, 96, 40)])
def test_rollout_matches_oracle_both_layouts(dev, c, hidden, p, horizon, iters):
    """Every schedule at the benchmark's sweep counts S = 4, 8, 16, including the biped and
    the quadruped at H = 64."""
    from hipenvs import legged, legged_rollout

    theta = _population(p, c, hidden, 0.3, c)
    state = olg.Legged(c).reset(p, seed=7)
    st, th = torch.from_numpy(state).to(dev), torch.from_numpy(theta).to(dev)
    fk, sk = legged_rollout.rollout(st, th, hidden, horizon, c, iters=iters)
    ef, es_ = olg.rollout_fused(state, theta, hidden, horizon, c, iters=iters)
    np.testing.assert_array_equal(to_np(fk), ef)
    np.testing.assert_array_equal(to_np(sk), es_)
    fc, sc = legged_rollout.rollout(st, th.T.contiguous(), hidden, horizon, c, schedule="columns", iters=iters)
    np.testing.assert_array_equal(to_np(fc), ef)
    np.testing.assert_array_equal(to_np(sc), es_)
    fr, sr = legged_rollout.rollout(st, th, hidden, horizon, c, schedule="rows", iters=iters)
    np.testing.assert_array_equal(to_np(fr), ef)
    np.testing.assert_array_equal(to_np(sr), es_)
    # the chunked schedule from (D, P) columns as well as from the rows above
    fq, sq = legged_rollout.rollout(st, None, hidden, horizon, c, iters=iters, theta_cols=th.T.contiguous())
    np.testing.assert_array_equal(to_np(fq), ef)
    np.testing.assert_array_equal(to_np(sq), es_)
    assert 1 <= es_.mean() <= horizon


@pytest.mark.parametrize("c", [1, 2, 3, 4])
def test_chunked_rows_at_any_alignment_and_ragged_p(dev, c):
    """The chunked schedule reading the caller's (P, D) rows in its first chunk: populations
    that are views 4, 8 and 12 bytes into a larger buffer (rows at every 4-byte alignment,
    read in place through the C ABI), and P off multiples of 64; equal to the columns form
    and the one-lane static schedule."""
    from hipenvs import _lib, legged_rollout

    hidden, horizon = 64, 48
    for p, off in ((1, 1), (63, 2), (130, 3), (130, 0)):
        d = legged_rollout.n_params(hidden, c)
        theta = torch.from_numpy(_population(p, c, hidden, 0.3, 50 + p)).to(dev)
        buf = torch.zeros(p * d + 4, device=dev)
        buf[off:off + p * d] = theta.reshape(-1)
        view = buf[off:off + p * d].view(p, d)
        assert view.data_ptr() % 16 == 4 * off
        st = torch.from_numpy(olg.Legged(c).reset(p, seed=60 + p)).to(dev)
        fr, sr = legged_rollout.rollout(st, view, hidden, horizon, c)
        fc, sc = legged_rollout.rollout(st, None, hidden, horizon, c, theta_cols=theta.T.contiguous())
        fs, ss = legged_rollout.rollout(st, theta, hidden, horizon, c, schedule="rows")
        assert torch.equal(fr, fc) and torch.equal(sr, sc) and torch.equal(fr, fs) and torch.equal(sr, ss), (c, p)
        # the C ABI directly, on the unaligned view: the same results
        nbytes = _lib.lib().hipenvs_legged_es_rollout_workspace_bytes(c, hidden, p)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        fa, sa = torch.empty_like(fr), torch.empty_like(sr)
        rc = _lib.lib().hipenvs_legged_es_rollout_chunked_rows(c, hidden, 8, 32, _lib.ptr(st), _lib.ptr(view), p,
                                                              horizon, 1.0, 0.0, 0.0, 0.0, _lib.ptr(fa), _lib.ptr(sa),
                                                              _lib.ptr(ws), nbytes, _lib.stream_of(dev))
        assert rc == 0
        assert torch.equal(fa, fc) and torch.equal(sa, sc), (c, p, off)


def test_chunked_schedule_at_scale_equals_static(dev):
    """Populations larger than the resident grid (grid-stride loops), chunk lengths that do
    and do not divide the horizon, and horizon 0 / 1: the compacting schedule equals the
    one-member-per-lane kernel member for member."""
    from hipenvs import legged, legged_rollout

    c, hidden = 4, 16
    for p, horizon, chunk in ((300_001, 70, 16), (300_001, 70, 32), (1000, 0, 32), (1000, 1, 32), (1, 30, 7),
                              (4099, 200, 1)):
        theta = torch.from_numpy(_population(p, c, hidden, 0.3, p % 97)).to(dev)
        state = legged.Legged(c).reset(p, seed=3, device=dev)
        fq, sq = legged_rollout.rollout(state, theta, hidden, horizon, c, schedule="chunked", chunk_steps=chunk)
        fs, ss = legged_rollout.rollout(state, theta, hidden, horizon, c, schedule="rows")
        assert torch.equal(fq, fs) and torch.equal(sq, ss), (p, horizon, chunk)
    # assist keeps bodies up for the whole horizon: every member survives every chunk
    theta = torch.from_numpy(_population(4096, c, hidden, 0.0, 1)).to(dev)
    state = legged.Legged(c).reset(4096, seed=4, device=dev)
    fq, sq = legged_rollout.rollout(state, theta, hidden, 100, c, assist=20.0, schedule="chunked", chunk_steps=16)
    fs, ss = legged_rollout.rollout(state, theta, hidden, 100, c, assist=20.0, schedule="rows")
    assert torch.equal(fq, fs) and torch.equal(sq, ss)


@pytest.mark.parametrize("c,hidden,iters", [(1, 4, 8), (1, 64, 8), (2, 8, 8), (2, 32, 8), (3, 16, 8), (3, 64, 8),
                                            (4, 4, 8), (4, 64, 8), (2, 64, 4), (2, 64, 16), (4, 64, 4), (4, 64, 16)])
def test_group_tail_equals_static(dev, c, hidden, iters):
    """Populations that the compacting schedule hands to its group tail (a lane group per
    member) after the first chunk, at every leg count and hidden width the group code
    distinguishes (one to four hidden units per lane, 2C + 1 solve lanes, 3C head lanes),
    with assisted members that stay up for the whole horizon: member for member equal to
    the one-member-per-lane kernel."""
    from hipenvs import legged, legged_rollout

    p, horizon = 3001, 150
    theta = torch.from_numpy(_population(p, c, hidden, 0.3, 11 * c + hidden)).to(dev)
    state = legged.Legged(c).reset(p, seed=5, device=dev)
    for assist in (0.0, 20.0):
        fq, sq = legged_rollout.rollout(state, theta, hidden, horizon, c, assist=assist, schedule="chunked",
                                        chunk_steps=8, iters=iters)
        fs, ss = legged_rollout.rollout(state, theta, hidden, horizon, c, assist=assist, schedule="rows",
                                        iters=iters)
        assert torch.equal(fq, fs) and torch.equal(sq, ss), (c, hidden, assist)
        assert ss.max().item() > 8  # members outlived the first chunk


@pytest.mark.parametrize("c,hidden,iters,above", [(1, 4, 8, 8), (2, 32, 8, 8), (3, 64, 8, 8), (4, 64, 8, 8),
                                                  (2, 64, 4, 8), (4, 64, 16, 8), (4, 4, 8, 8), (4, 32, 8, 8),
                                                  (4, 64, 8, 44), (2, 64, 8, 28)])
def test_group_chunk_equals_static(dev, c, hidden, iters, above):
    """Populations `above` members per CU over the group tail's bound (16 per CU at C = 4, 32
    at C <= 2, where the tail runs two waves per SIMD), within 64 per CU. Later chunks run in
    the group form (4 lanes per member: the solves, Delassus blocks and heads spread over the
    quad, the Gauss-Seidel sweeps split over it) and append their survivors until the count
    falls to the tail's bound: member for member equal to the one-lane kernel."""
    from hipenvs import legged, legged_rollout

    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    tail_per_cu = 16 if c > 2 else 32
    p, horizon = (tail_per_cu + above) * cus, 60
    state = legged.Legged(c).reset(p, seed=6, device=dev)
    past_first = 0
    for assist, scale in ((0.0, 0.3), (20.0, 0.0)):
        theta = torch.from_numpy(_population(p, c, hidden, scale, 7 * c + hidden)).to(dev)
        fq, sq = legged_rollout.rollout(state, theta, hidden, horizon, c, assist=assist, schedule="chunked",
                                        chunk_steps=8, iters=iters)
        fs, ss = legged_rollout.rollout(state, theta, hidden, horizon, c, assist=assist, schedule="rows",
                                        iters=iters)
        assert torch.equal(fq, fs) and torch.equal(sq, ss), (c, hidden, assist)
        past_first = max(past_first, int((ss > 8).sum().item()))
    assert past_first > tail_per_cu * cus  # the second chunk ran above the tail's bound


def test_shaped_reward_and_assist_match_oracle(dev):
    """test_es.py:71-104's variants: alive 0.1 + fall penalty 20 (some fitness negative),
    and the assist spring with a gate."""
    from hipenvs import legged_rollout

    c, hidden, p, horizon = 2, 16, 256, 80
    theta = _population(p, c, hidden, 0.3, 11)
    state = olg.Legged(c).reset(p, seed=2)
    st, th = torch.from_numpy(state).to(dev), torch.from_numpy(theta).to(dev)
    fk, sk = legged_rollout.rollout(st, th, hidden, horizon, c, alive_bonus=0.1, fall_penalty=20.0)
    ef, es_ = olg.rollout_fused(state, theta, hidden, horizon, c, alive_bonus=0.1, fall_penalty=20.0)
    np.testing.assert_array_equal(to_np(fk), ef)
    np.testing.assert_array_equal(to_np(sk), es_)
    assert (ef < 0).any()
    fa, sa = legged_rollout.rollout(st, th, hidden, horizon, c, alive_bonus=0.0, height_gate=0.85, assist=20.0)
    efa, esa = olg.rollout_fused(state, theta, hidden, horizon, c, alive_bonus=0.0, height_gate=0.85, assist=20.0)
    np.testing.assert_array_equal(to_np(fa), efa)
    np.testing.assert_array_equal(to_np(sa), esa)
    assert esa.mean() > 1.5 * es_.mean() or esa.mean() > 0.9 * horizon


def test_fused_rollout_close_to_the_oracle_loop(dev):
    """test_es.py:60-69 for the legged body: the fused kernel against es.loop_fitness over the
    step (reward - 1 in float32, auto-reset), within the reference's tolerance."""
    from hipenvs import legged_rollout

    c, hidden, p, horizon = 2, 16, 256, 60
    theta = _population(p, c, hidden, 0.3, 5)
    state = olg.Legged(c).reset(p, seed=5)
    fk, sk = legged_rollout.rollout(torch.from_numpy(state).to(dev), torch.from_numpy(theta).to(dev), hidden, horizon, c)
    params = oes.unflatten(theta, hidden, 5 + 2 * c, 3 * c)
    body = olg.Legged(c)

    def logits(s, *prm):
        return olg.policy_logits(s[:3 + c], s[3 + c:], *prm, c)

    def action_of(lg_):
        return oes.legged_action(lg_.T, c)

    fl, sl = oes.loop_fitness(body.step, logits, action_of, state, params, horizon, seed0=1)
    fk, sk = to_np(fk), to_np(sk)
    close = np.abs(fk - fl) <= 1e-3 * np.maximum(np.abs(fl), 1.0) + 1e-2
    assert close.mean() > 0.95 and (sk == sl).mean() > 0.95, (close.mean(), (sk == sl).mean())
    assert 5 < sl.mean() < 200


@pytest.mark.parametrize("c", [2, 4])
@pytest.mark.parametrize("iters", [4, 8, 16])
def test_config4_population_matches_oracle(dev, c, iters):
    """The benchmark's population at small P: H = 64, sigma 0.03 antithetic around
    theta0 = 0.1 N(0, 1), alive bonus 1 + forward velocity, S = 4/8/16, for the biped and the
    quadruped: the seeded rollout against the oracle's fused restatement on the oracle's own
    perturbation, member for member."""
    from hipenvs import legged_rollout
    from oracle import es_noise as oen

    p, hidden, horizon = 128, 64, 120
    d = legged_rollout.n_params(hidden, c)
    theta = (np.random.default_rng(2024 + c).standard_normal(d) * 0.1).astype(np.float32)
    pop = oen.perturb(theta, p, 31 + iters, 0.03)
    state = olg.Legged(c).reset(p, seed=9)
    print(f"config-4 population c={c} iters={iters}", flush=True)
    fk, sk = legged_rollout.rollout_seeded(torch.from_numpy(state).to(dev), torch.from_numpy(theta).to(dev),
                                           31 + iters, 0.03, hidden, horizon, c, iters=iters)
    ef, es_ = olg.rollout_fused(state, pop, hidden, horizon, c, iters=iters)
    np.testing.assert_array_equal(to_np(sk), es_)
    np.testing.assert_array_equal(to_np(fk), ef)
    assert es_.min() < es_.max()


@pytest.mark.parametrize("c", [2, 4])
def test_horizon_1000_against_oracle(dev, c):
    """The whole config-4 horizon at small P: 256 members of the benchmark's population
    (H = 64, sigma 0.03 around theta0 = 0.1 N(0, 1), S = 8) with a torso-assist spring of 5,
    so that some members stand for all 1,000 steps. After the first 32-step chunk the
    survivors run in the group tail (16 lanes per member) to the end of their episodes; the
    drop-in rollout and the seeded rollout each equal the oracle's fused restatement member
    for member."""
    from hipenvs import legged_rollout
    from oracle import es_noise as oen

    p, hidden, horizon, assist = 256, 64, 1000, 5.0
    d = legged_rollout.n_params(hidden, c)
    theta = (np.random.default_rng(77 + c).standard_normal(d) * 0.1).astype(np.float32)
    pop = oen.perturb(theta, p, 91, 0.03)
    state = olg.Legged(c).reset(p, seed=13)
    print(f"horizon 1000 c={c}: oracle", flush=True)
    ef, es_ = olg.rollout_fused(state, pop, hidden, horizon, c, iters=8, assist=assist)
    assert (es_ >= horizon).sum() >= 4 and es_.min() < 32  # members in the first chunk only and to the end
    st = torch.from_numpy(state).to(dev)
    print(f"horizon 1000 c={c}: drop-in rollout", flush=True)
    fk, sk = legged_rollout.rollout(st, torch.from_numpy(pop).to(dev), hidden, horizon, c, assist=assist)
    np.testing.assert_array_equal(to_np(sk), es_)
    np.testing.assert_array_equal(to_np(fk), ef)
    print(f"horizon 1000 c={c}: seeded rollout", flush=True)
    fs, ss = legged_rollout.rollout_seeded(st, torch.from_numpy(theta).to(dev), 91, 0.03, hidden, horizon, c,
                                           assist=assist)
    np.testing.assert_array_equal(to_np(ss), es_)
    np.testing.assert_array_equal(to_np(fs), ef)
