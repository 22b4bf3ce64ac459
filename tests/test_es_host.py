"""hipenvs.es host logic without a GPU: layout, ranks, actions, policy forward (CPU)."""

import numpy as np
import torch

from hipenvs import es
from oracle import cartpole as oc
from oracle import es as oes

CP, AC = es.TASKS["cartpole"], es.TASKS["acrobot"]


def test_unflatten_layout_is_consistent():
    """test_es.py:11-18."""
    for task in (CP, AC):
        h, p = 8, 3
        theta = torch.arange(p * es.n_params(h, task), dtype=torch.float32).reshape(p, -1)
        w1, b1, w2, b2 = es.unflatten(theta, h, task)
        i, o = task.obs_dim, task.n_out
        assert w1.shape == (p, i, h) and b1.shape == (p, h) and w2.shape == (p, h, o) and b2.shape == (p, o)
        assert w1[1, 2, 3] == theta[1, 2 * h + 3] and b2[2, o - 1] == theta[2, -1]


def test_centered_ranks_golden_vector_and_ties():
    """test_es.py:21-25, and index tie-break identical to the oracle's."""
    v = torch.tensor([3.0, 1.0, 2.0, 10.0])
    torch.testing.assert_close(es.centered_ranks(v), torch.tensor([1 / 6, -0.5, -1 / 6, 0.5]), atol=1e-6, rtol=0)
    r = np.random.default_rng(0).integers(0, 5, 1000).astype(np.float32)
    np.testing.assert_array_equal(es.centered_ranks(torch.from_numpy(r)).numpy(), oes.centered_ranks(r))


def test_legged_action_composes_per_leg_heads():
    """test_es.py:28-31."""
    logits = torch.tensor([[0, 5, 0, 9, 0, 0], [7, 0, 0, 0, 0, 3]], dtype=torch.float32)
    assert es.legged_action(2)(logits).tolist() == [1, 6]


def test_population_forward_matches_mean_policy():
    """test_es.py:34-43: P copies of one row act like the single policy, on every task."""
    g = torch.Generator().manual_seed(0)
    for task in (CP, AC):
        h, p = task.hidden, 64
        theta = torch.randn(es.n_params(h, task), generator=g)
        obs = torch.randn(p, task.obs_dim, generator=g)
        batched = task.action(es.population_logits(obs, es.unflatten(theta.expand(p, -1).contiguous(), h, task)))
        single = task.action(es.mean_policy(theta, h, task)(obs))
        assert torch.equal(batched, single), task.name


def test_torch_policy_close_to_the_oracle_policy():
    """The loop backend's torch forward vs the fused kernels' sequential order (oracle)."""
    r = np.random.default_rng(1)
    h, p = 32, 256
    theta = r.standard_normal((p, 7 * h + 2)).astype(np.float32) * 0.5
    state = oc.reset(p, seed=2) * 10
    ref = oc.policy_logits(state, *oes.unflatten(theta, h, 4, 2))
    got = es.population_logits(torch.from_numpy(state.T.copy()), es.unflatten(torch.from_numpy(theta), h, CP))
    np.testing.assert_allclose(got.numpy().T, ref, rtol=1e-5, atol=1e-5)


def test_curriculum_anneals():
    """test_es.py:87-88."""
    cfg = es.Config(task="cartpole", assist_k0=20.0, start_velocity=0.3, anneal_gens=100)
    assert es.curriculum(cfg, 1) == (20.0, 0.3) and es.curriculum(cfg, 51) == (10.0, 0.15)
    assert es.curriculum(cfg, 101) == (0.0, 0.0)


def test_command_line_matches_the_reference_defaults():
    """es.py:357-371: the same flags and defaults (task cartpole, pop 1,024, backend metal,
    seed 0, lr 0.1, sigma 0.1, 120 s, 500 generations, no curricula, anneal 300); the
    reference's backend names map onto this package's backends."""
    cfg, backend, seed = es.parse_args([])
    assert (cfg.task, cfg.pop, backend, seed, cfg.lr, cfg.sigma) == ("cartpole", 1024, "fused", 0, 0.1, 0.1)
    assert (cfg.time_budget, cfg.max_generations, cfg.assist_k0, cfg.start_velocity, cfg.anneal_gens) == \
        (120.0, 500, 0.0, 0.0, 300)
    assert cfg == es.Config()
    cfg, backend, seed = es.parse_args(["--task", "legged4", "--pop", "256", "--backend", "mlx", "--seed", "3",
                                        "--assist", "20", "--start-velocity", "0.3", "--anneal", "100",
                                        "--lr", "0.05", "--sigma", "0.03", "--time-budget", "9",
                                        "--max-generations", "7"])
    assert backend == "loop" and seed == 3
    assert (cfg.task, cfg.pop, cfg.assist_k0, cfg.start_velocity, cfg.anneal_gens) == ("legged4", 256, 20.0, 0.3, 100)
    assert (cfg.lr, cfg.sigma, cfg.time_budget, cfg.max_generations) == (0.05, 0.03, 9.0, 7)
    assert es.parse_args(["--backend", "seeded"])[1] == "seeded"
    for name in ("metal", "mlx", "fused", "loop", "seeded"):
        assert es.BACKEND_ALIASES.get(name, name) in es.BACKENDS
