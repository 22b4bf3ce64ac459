"""ES pieces of the oracle against the reference's test_es.py (CPU)."""

import numpy as np

from oracle import acrobot, cartpole, es


def test_unflatten_layout_is_consistent():
    """test_es.py:11-18."""
    for obs_dim, n_out in ((4, 2), (6, 3), (9, 6)):
        h, p = 8, 3
        theta = np.arange(p * es.n_params(h, obs_dim, n_out), dtype=np.float32).reshape(p, -1)
        w1, b1, w2, b2 = es.unflatten(theta, h, obs_dim, n_out)
        assert w1.shape == (p, obs_dim, h) and b1.shape == (p, h) and w2.shape == (p, h, n_out) and b2.shape == (p, n_out)
        assert w1[1, 2, 3] == theta[1, 2 * h + 3] and b2[2, n_out - 1] == theta[2, -1]


def test_centered_ranks_golden_vector():
    """test_es.py:21-25: [3, 1, 2, 10] -> [1/6, -1/2, -1/6, 1/2]."""
    v = np.array([3.0, 1.0, 2.0, 10.0], dtype=np.float32)
    np.testing.assert_allclose(es.centered_ranks(v), np.array([1 / 6, -0.5, -1 / 6, 0.5], dtype=np.float32), atol=1e-6)


def test_centered_ranks_ties_by_index():
    v = np.array([5.0, 5.0, 1.0, 5.0], dtype=np.float32)
    np.testing.assert_allclose(es.centered_ranks(v), np.array([1 / 3, 2 / 3, 0.0, 1.0]) - 0.5, atol=1e-6)


def test_legged_action_composes_per_leg_heads():
    """test_es.py:28-31."""
    logits = np.array([[0, 5, 0, 9, 0, 0], [7, 0, 0, 0, 0, 3]], dtype=np.float32)
    assert es.legged_action(logits, 2).tolist() == [1, 6]


def test_population_forward_matches_single_policy():
    """test_es.py:34-43: P copies of one row act exactly like the single policy."""
    r = np.random.default_rng(0)
    h, p = 32, 64
    theta = r.standard_normal(es.n_params(h, 4, 2)).astype(np.float32)
    obs = r.standard_normal((4, p)).astype(np.float32)
    batched = cartpole.policy_logits(obs, *es.unflatten(np.broadcast_to(theta, (p, theta.size)).copy(), h, 4, 2))
    for i in range(0, p, 9):
        single = cartpole.policy_logits(obs[:, i:i + 1], *es.unflatten(theta[None, :], h, 4, 2))
        np.testing.assert_array_equal(batched[:, i:i + 1], single)


def _rollout_vs_loop(env, obs_dim, n_out, sign, scale, horizon=200, p=256, hidden=32):
    r = np.random.default_rng(0)
    theta_pop = (r.standard_normal((p, es.n_params(hidden, obs_dim, n_out))) * scale).astype(np.float32)
    state = env.reset(p, seed=5)
    params = es.unflatten(theta_pop, hidden, obs_dim, n_out)
    fused = env.rollout_survived(state, theta_pop, hidden, horizon) if env is cartpole else \
        env.rollout_steps(state, theta_pop, hidden, horizon)
    fit_k, steps_k = es.steps_fitness(fused, horizon, sign)
    if env is cartpole:
        action_of = lambda lg: (lg[1] > lg[0]).astype(np.int32)
    else:
        action_of = es.first_argmax
    fit_l, steps_l = es.loop_fitness(env.step, env.policy_logits, action_of, state, params, horizon, seed0=1)
    return fit_k, steps_k, fit_l, steps_l


def test_fused_rollout_equals_the_step_loop():
    """test_es.py:46-69, exactly: the fused early-exit semantics and es.loop_fitness's masked
    auto-reset loop agree on every member (the reference allowed 5% chaotic mismatches)."""
    for env, obs_dim, n_out, sign in ((cartpole, 4, 2, 1.0), (acrobot, 6, 3, -1.0)):
        fk, sk, fl, sl = _rollout_vs_loop(env, obs_dim, n_out, sign, 0.5, horizon=120)
        np.testing.assert_array_equal(fk, fl)
        np.testing.assert_array_equal(sk, sl)
        assert 0 < sk.mean() <= 120


def test_generation_update_moves_theta_along_ranked_noise():
    r = np.random.default_rng(1)
    d, p = 10, 8
    half = r.standard_normal((p // 2, d)).astype(np.float32)
    eps = np.concatenate([half, -half])
    fit = np.arange(p, dtype=np.float32)
    new = es.generation_update(np.zeros(d, np.float32), eps, fit, 0.1, 0.1)
    ranks = np.arange(p) / (p - 1) - 0.5
    np.testing.assert_allclose(new, 0.1 * (ranks[:, None] * eps).sum(0) / (p * 0.1), rtol=1e-5, atol=1e-7)
