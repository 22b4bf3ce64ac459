"""Seeded ES generation through the C ABI (GPU): the perturbation and update kernels
against the oracle bit for bit, and each seeded rollout against the rollout of the
perturbed population, member for member.
"""

import numpy as np
import pytest
import torch

from oracle import es as oes
from oracle import es_noise as oen

pytestmark = pytest.mark.gpu


def to_np(t):
    return t.detach().cpu().numpy()


def theta0(d, seed):
    return (np.random.default_rng(seed).standard_normal(d) * 0.1).astype(np.float32)


@pytest.mark.parametrize("p,d", [(2, 1), (6, 7), (64, 226), (130, 323), (512, 1676)])
def test_perturb_rows_and_columns_match_oracle(dev, p, d):
    from hipenvs import es_noise

    theta = theta0(d, d)
    expect = oen.perturb(theta, p, 1000 + p, 0.03)
    t = torch.from_numpy(theta).to(dev)
    rows = es_noise.perturb(t, p, 1000 + p, 0.03)
    cols = es_noise.perturb(t, p, 1000 + p, 0.03, layout="columns")
    np.testing.assert_array_equal(to_np(rows), expect)
    np.testing.assert_array_equal(to_np(cols), expect.T)


@pytest.mark.parametrize("p,d", [(2, 3), (4096, 226), (4096, 323), (40_000, 12), (2000, 1676)])
def test_update_matches_oracle(dev, p, d):
    """Includes a population above 2 * 16384 members, where each partial sum covers 128 pairs."""
    from hipenvs import es_noise

    rng = np.random.default_rng(p)
    theta = theta0(d, p + d)
    fit = rng.standard_normal(p).astype(np.float32)
    ranks = oes.centered_ranks(fit).astype(np.float32)
    expect = oen.update(theta, ranks, 77, 0.1, 0.05)
    got = es_noise.update(torch.from_numpy(theta).to(dev), torch.from_numpy(ranks).to(dev), 77, 0.1, 0.05)
    np.testing.assert_array_equal(to_np(got), expect)


def test_update_may_write_in_place(dev):
    from hipenvs import _lib

    d, p = 226, 256
    theta = torch.from_numpy(theta0(d, 5)).to(dev)
    ranks = torch.linspace(-0.5, 0.5, p, device=dev)
    expect = oen.update(to_np(theta), to_np(ranks), 3, 0.1, 0.1)
    nbytes = _lib.lib().hipenvs_es_update_workspace_bytes(d, p)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    _lib.call("hipenvs_es_update", _lib.ptr(theta), _lib.ptr(ranks), d, p, _lib.u32(3), 0.1, 0.1, _lib.ptr(theta),
              _lib.ptr(ws), nbytes, _lib.stream_of(dev))
    np.testing.assert_array_equal(to_np(theta), expect)


@pytest.mark.parametrize("p", [512, 20_000])
@pytest.mark.parametrize("hidden", [8, 32])
def test_cartpole_and_acrobot_seeded_rollouts(dev, p, hidden):
    """Lane-group populations (512) and one member per lane (20,000)."""
    from hipenvs import acrobot, acrobot_rollout, cartpole, cartpole_rollout, es_noise

    for env, mod, d, horizon in ((cartpole, cartpole_rollout, 7 * hidden + 2, 300),
                                 (acrobot, acrobot_rollout, 10 * hidden + 3, 100)):
        theta = torch.from_numpy(theta0(d, hidden)).to(dev)
        state = env.reset(p, seed=9, device=dev)
        got = mod.rollout_steps_seeded(state, theta, 4242, 0.1, hidden, horizon)
        expect = mod.rollout_steps(state, es_noise.perturb(theta, p, 4242, 0.1), hidden, horizon)
        assert torch.equal(got, expect), mod.__name__
        assert expect.max().item() > 0


@pytest.mark.parametrize("c,hidden,p", [(4, 64, 640), (4, 16, 20_000), (3, 64, 3000), (3, 32, 5_002),
                                         (2, 32, 3000), (2, 16, 16_446), (1, 8, 130), (1, 8, 8_322)])
def test_legged_seeded_rollout(dev, c, hidden, p):
    """Populations the group tail takes whole (640, 130, 3000: at most 16 members per CU at
    C >= 3, 32 at C <= 2) and ones that run a first chunk over antithetic pairs and then
    compacted chunks (20,000, 5,002, 16,446, 8,322; the last pair tile of each partly
    filled), with and without the assist spring."""
    from hipenvs import es_noise, legged, legged_rollout

    d = legged_rollout.n_params(hidden, c)
    theta = torch.from_numpy(theta0(d, c * hidden)).to(dev)
    state = legged.Legged(c).reset(p, seed=6, device=dev)
    longest = 0.0
    for assist in (0.0, 20.0):
        fs, ss = legged_rollout.rollout_seeded(state, theta, 99, 0.03, hidden, 120, c, assist=assist, chunk_steps=16)
        pop = es_noise.perturb(theta, p, 99, 0.03)
        fr, sr = legged_rollout.rollout(state, pop, hidden, 120, c, assist=assist, schedule="rows")
        assert torch.equal(fs, fr) and torch.equal(ss, sr), (c, hidden, p, assist)
        longest = max(longest, sr.max().item())
    assert longest > 16  # members outlived the first chunk


@pytest.mark.parametrize("horizon", [1, 10, 33])
def test_legged_seeded_short_horizon(dev, horizon):
    """Horizons inside and just past the first chunk (32 steps at C = 4) on the pairs path."""
    from hipenvs import es_noise, legged, legged_rollout

    c, hidden, p = 4, 16, 20_002
    d = legged_rollout.n_params(hidden, c)
    theta = torch.from_numpy(theta0(d, 77)).to(dev)
    state = legged.Legged(c).reset(p, seed=8, device=dev)
    fs, ss = legged_rollout.rollout_seeded(state, theta, 5, 0.03, hidden, horizon, c)
    fr, sr = legged_rollout.rollout(state, es_noise.perturb(theta, p, 5, 0.03), hidden, horizon, c, schedule="rows")
    assert torch.equal(fs, fr) and torch.equal(ss, sr), horizon
    assert sr.max().item() == horizon


def test_legged_seeded_zero_horizon(dev):
    from hipenvs import legged, legged_rollout

    theta = torch.zeros(legged_rollout.n_params(16, 2), device=dev)
    state = legged.Legged(2).reset(64, seed=1, device=dev)
    f, s = legged_rollout.rollout_seeded(state, theta, 1, 0.1, 16, 0, 2)
    assert torch.count_nonzero(f).item() == 0 and torch.count_nonzero(s).item() == 0


def test_seeded_generation_is_rollout_ranks_update(dev):
    """es.SeededBackend.generation is the seeded rollout, the centered ranks and the update
    with one seed, and a few generations of CartPole improve the population's fitness."""
    from hipenvs import cartpole_rollout, es, es_noise

    cfg = es.Config(task="cartpole", pop=256, sigma=0.1, lr=0.1, horizon=200)
    backend = es.SeededBackend(es.TASKS["cartpole"], 3, dev)
    theta = torch.from_numpy(theta0(226, 1)).to(dev)
    probe = es.SeededBackend(es.TASKS["cartpole"], 3, dev)
    seed = probe.next_noise_seed()
    state = probe.reset(cfg.pop)
    fit = cartpole_rollout.rollout_steps_seeded(state, theta, seed, cfg.sigma, 32, cfg.horizon)
    expect = es_noise.update(theta, es.centered_ranks(fit), seed, cfg.sigma, cfg.lr)
    got, fit_b, _ = es.generation(backend, theta, cfg, 32)
    assert torch.equal(fit_b, fit) and torch.equal(got, expect)
    means = [fit_b.mean().item()]
    for gen in range(2, 12):
        got, fit_b, _ = es.generation(backend, got, cfg, 32, gen)
        means.append(fit_b.mean().item())
    assert max(means[-3:]) > means[0]


def test_bad_populations_are_rejected(dev):
    from hipenvs import _lib, es_noise

    theta = torch.zeros(10, device=dev)
    with pytest.raises(ValueError):
        es_noise.perturb(theta, 7, 0, 0.1)
    null = _lib.ptr(None)
    l = _lib.lib()
    assert l.hipenvs_es_perturb(_lib.ptr(theta), 10, 3, 0, 0.1, 0, _lib.ptr(theta), null) == _lib.E_ARG
    assert l.hipenvs_es_perturb(_lib.ptr(theta), 10, 4, 0, 0.1, 2, _lib.ptr(theta), null) == _lib.E_ARG
    assert l.hipenvs_es_update_workspace_bytes(10, 5) == -1
    assert l.hipenvs_cartpole_es_rollout_seeded(null, null, 4, 0, 0.1, 32, 10, null, null, 0, null) == _lib.E_ARG


@pytest.mark.parametrize("c,iters", [(4, 4), (4, 8), (4, 16), (2, 4), (2, 8), (2, 16), (3, 8), (1, 8)])
def test_config4_full_size_schedules_agree(dev, c, iters):
    """At the benchmark's full shape (N = 262,144, H = 64, horizon 1,000, sigma 0.03 around
    0.1 N(0, 1)) for the quadruped and the biped at S = 4, 8, 16, and for three legs and one
    at S = 8: the seeded rollout, the
    chunked rollout of the perturbed columns, the chunked rollout of the perturbed rows (the
    drop-in call) and the one-member-per-lane rollout of the rows agree member for member."""
    from hipenvs import es_noise, legged, legged_rollout

    p, hidden = 262_144, 64
    print(f"config-4 full size c={c} iters={iters}", flush=True)
    theta = torch.from_numpy(theta0(legged_rollout.n_params(hidden, c), 2024)).to(dev)
    state = legged.Legged(c).reset(p, seed=0, device=dev)
    fs, ss = legged_rollout.rollout_seeded(state, theta, 5, 0.03, hidden, 1000, c, iters=iters)
    cols = es_noise.perturb(theta, p, 5, 0.03, layout="columns")
    fc, sc = legged_rollout.rollout(state, None, hidden, 1000, c, theta_cols=cols, iters=iters)
    del cols
    rows = es_noise.perturb(theta, p, 5, 0.03)
    fr, sr = legged_rollout.rollout(state, rows, hidden, 1000, c, schedule="rows", iters=iters)
    # the drop-in call: the chunked schedule reading the (P, D) rows in its first chunk
    fd, sd = legged_rollout.rollout(state, rows, hidden, 1000, c, iters=iters)
    assert torch.equal(fs, fc) and torch.equal(ss, sc)
    assert torch.equal(fs, fr) and torch.equal(ss, sr)
    assert torch.equal(fs, fd) and torch.equal(ss, sd)
    # the benchmark's bodies have a long tail that reaches the group phase; every body
    # outlives the first chunk
    assert sr.max().item() > (300 if c in (2, 4) else 32)
