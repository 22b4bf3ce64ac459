"""hipenvs.es on the GPU: generations, backends agreeing, learning (GPU)."""

import numpy as np
import pytest
import torch

from hipenvs import es

pytestmark = pytest.mark.gpu
CP, AC = es.TASKS["cartpole"], es.TASKS["acrobot"]


def _kernel_vs_loop(dev, task, scale, horizon=200, pop=1024):
    g = torch.Generator(device=dev).manual_seed(0)
    theta_pop = torch.randn((pop, es.n_params(task.hidden, task)), generator=g, device=dev) * scale
    state = task.env.reset(pop, seed=123, device=dev)
    fit_k, steps_k = task.rollout(state, theta_pop, task.hidden, horizon)
    backend = es.LoopBackend(task, 0, dev)
    fit_l, steps_l = es.loop_fitness(backend, es.unflatten(theta_pop, task.hidden, task), horizon, state=state)
    return fit_k.cpu().numpy(), steps_k.cpu().numpy(), fit_l.cpu().numpy(), steps_l.cpu().numpy()


def test_fused_kernels_match_the_torch_loop(dev):
    """test_es.py:60-69: same population and initial states; the fused kernel and the loop
    backend (torch policy + HIP step kernel) agree for >95% of members (they evaluate the
    policy's tanh and sums in different orders, so chaotic members may part)."""
    for task, scale in ((CP, 0.5), (AC, 0.5)):
        fk, sk, fl, sl = _kernel_vs_loop(dev, task, scale)
        close = np.abs(fk - fl) <= 1e-3 * np.maximum(np.abs(fl), 1.0) + 1e-2
        assert close.mean() > 0.95 and (sk == sl).mean() > 0.95, (task.name, close.mean(), (sk == sl).mean())


def test_generation_uses_antithetic_pairs_and_moves_theta(dev):
    """test_es.py:107-113."""
    cfg = es.Config(pop=8, horizon=5)
    backend = es.FusedBackend(CP, 0, dev)
    theta = torch.zeros(es.n_params(4, CP), device=dev)
    new_theta, fit, steps = es.generation(backend, theta, cfg, 4)
    assert fit.shape == (8,) and float(steps.max()) <= 5
    assert not torch.allclose(new_theta, torch.zeros_like(new_theta))


def test_es_learns_cartpole(dev):
    """test_es.py:116-121 (fused backend): the greedy mean policy reaches 150."""
    r = es.train(es.Config(pop=256, time_budget=30.0, solved_at=150.0, max_generations=200), "fused", seed=0, device=dev)
    assert r.score >= 150.0, r


def test_es_learns_acrobot(dev):
    r = es.train(es.Config(task="acrobot", pop=4096, time_budget=30.0, solved_at=-250.0, max_generations=100),
                 "fused", seed=0, device=dev)
    assert r.score >= -250.0, r


@pytest.mark.parametrize("backend", ["fused", "seeded"])
def test_es_learns_to_stay_up_on_two_legs(dev, backend):
    """test_es.py:124-131: a random biped falls in about 20 steps (training fitness ~20 under
    the alive bonus); within 60 generations of 1,024 members the population's training
    fitness reaches 300 (standing is worth about 500)."""
    last = []
    es.train(es.Config(task="legged2", pop=1024, time_budget=30.0, max_generations=60), backend, seed=0,
             device=dev, log=lambda gen, steps, secs, fit, score: last.append(fit))
    assert last[-1] >= 300.0, last
