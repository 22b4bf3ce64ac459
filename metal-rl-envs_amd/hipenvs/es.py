"""Evolution strategies on the batched HIP environments: the caller of the fused rollouts.

A torch restatement of the reference's learner ``es.py`` (Salimans et al.
2017): each population member is a small MLP with its own weights, the whole
population runs against the batched environment for a horizon, and the update
is a rank-weighted sum of antithetic perturbations, once per generation.

Kept from the reference:

* the task registry and per-task policy shapes (``es.py:47-132``);
* the (P, D) parameter-row layout of ``n_params``/``unflatten``
  (``es.py:152-164``): w1 (I, H), b1 (H), w2 (H, O), b2 (O), row-major;
* ``loop_fitness``'s accounting (``es.py:174-193``), ``push``/``curriculum``
  (``es.py:196-211``), ``centered_ranks`` (``es.py:214-215``, with ties broken
  by index: a stable sort), ``generation`` (``es.py:218-227``), ``evaluate``
  (``es.py:308-322``) and the stopping rule of ``train`` (``es.py:334-354``).

Backends (``es.py:230-299``): ``"fused"`` runs the whole rollout as one HIP
launch per generation (the reference's ``metal`` backend); ``"loop"`` runs the
policy in torch and steps the HIP step kernel once per iteration (its ``mlx``
backend). The reference's ``numpy`` backend is the CPU oracle, which this
package does not import. For these two, sampling, ranking and the update are
torch ops on the GPU, as in the reference. ``"seeded"`` keeps the same
generation but regenerates the antithetic noise from a counter-RNG seed inside
the rollout and update kernels (``es_noise``), so neither the (P, D) noise nor
the population is ever a tensor; ranking stays a torch sort.
"""

import time
from dataclasses import dataclass
from typing import Any, Callable

import torch

from . import acrobot, acrobot_rollout, cartpole, cartpole_rollout, es_noise, legged, legged_rollout


@dataclass(frozen=True)
class Task:
    name: str
    obs_dim: int
    n_out: int
    hidden: int
    solved_at: float
    env: Any                   # step module/object: reset(n, seed=None, device=None), step(state, action[, assist])
    obs: Callable              # state (D, P) -> (P, obs_dim)
    action: Callable           # logits (P, n_out) -> action index (P,) int32
    rollout: Callable          # (state, theta_pop, hidden, horizon[, assist]) -> (fitness, steps taken)
    rollout_seeded: Callable | None = None  # (state, theta, seed, sigma, hidden, horizon[, assist]) -> same
    alive_bonus: float = 1.0
    fall_penalty: float = 0.0
    eval_bonus: float = 1.0
    height_gate: float = 0.0
    xdot_row: int | None = None
    assistable: bool = False
    evaluate_policy: Callable | None = None  # (state, theta, hidden, steps) -> per-env score, one launch


def argmax_action(logits):
    return torch.argmax(logits, dim=-1).to(torch.int32)


def cartpole_obs(state):
    return state.T


def acrobot_obs(state):
    th1, th2, dth1, dth2 = state
    return torch.stack([torch.cos(th1), torch.sin(th1), torch.cos(th2), torch.sin(th2), dth1, dth2], dim=1)


def legged_obs(state):
    """Everything but x: the policy is translation-invariant (``es.py:81-83``)."""
    return state[1:].T


def legged_action(c):
    """Per-leg argmax of each three-way head, composed as sum_k a_k 3**k (``es.py:86-93``)."""
    def action(logits):
        out = torch.zeros(logits.shape[0], dtype=torch.int32, device=logits.device)
        for k in range(c):
            out = out + torch.argmax(logits[:, 3 * k:3 * k + 3], dim=-1).to(torch.int32) * 3**k
        return out
    return action


def steps_fitness(kernel, sign):
    """CartPole's and Acrobot's fused kernels return steps survived; fitness is that with the
    task's sign and steps taken counts the terminating step, capped at the horizon (``es.py:96-103``)."""
    def rollout(state, theta_pop, hidden, horizon):
        steps = kernel(state, theta_pop, hidden, horizon)
        return sign * steps, torch.clamp(steps + 1, max=horizon)
    return rollout


def steps_fitness_seeded(kernel, sign):
    """``steps_fitness`` for the seeded kernels, which take (theta, seed, sigma) for the population."""
    def rollout(state, theta, seed, sigma, hidden, horizon):
        steps = kernel(state, theta, seed, sigma, hidden, horizon)
        return sign * steps, torch.clamp(steps + 1, max=horizon)
    return rollout


TASKS = {
    "cartpole": Task("cartpole", 4, 2, 32, 475.0, cartpole, cartpole_obs, argmax_action,
                     steps_fitness(cartpole_rollout.rollout_steps, 1.0),
                     steps_fitness_seeded(cartpole_rollout.rollout_steps_seeded, 1.0),
                     evaluate_policy=cartpole_rollout.evaluate),
    "acrobot": Task("acrobot", 6, 3, 32, -100.0, acrobot, acrobot_obs, argmax_action,
                    steps_fitness(acrobot_rollout.rollout_steps, -1.0),
                    steps_fitness_seeded(acrobot_rollout.rollout_steps_seeded, -1.0),
                    evaluate_policy=acrobot_rollout.evaluate),
}


def legged_task(c, name, alive=1.0, fall=0.0, gate=0.0, hidden=16, iters=legged.ITERS):
    """``es.py:106-114``: training fitness forward velocity (above the gate) + `alive` per step,
    minus `fall` at a fall; canonical score forward distance until the first fall (threshold 100)."""
    env = legged.Legged(c, iters)

    def rollout(state, theta_pop, hidden_, horizon, assist=0.0):
        return legged_rollout.rollout(state, theta_pop, hidden_, horizon, c, alive, fall, gate, assist, iters)

    def rollout_seeded(state, theta, seed, sigma, hidden_, horizon, assist=0.0):
        return legged_rollout.rollout_seeded(state, theta, seed, sigma, hidden_, horizon, c, alive, fall, gate,
                                             assist, iters)

    def evaluate_policy(state, theta, hidden_, steps):
        return legged_rollout.evaluate(state, theta, hidden_, steps, c, iters, eval_bonus=0.0)

    return Task(f"legged{c}{name}", 5 + 2 * c, 3 * c, hidden, 100.0, env, legged_obs, legged_action(c), rollout,
                rollout_seeded, alive, fall, 0.0, gate, 3 + c, True, evaluate_policy)


for _c, _name, _kw in ((2, "", {}), (4, "", {}), (2, "_distance", {"alive": 0.0}), (4, "_distance", {"alive": 0.0}),
                       (2, "_alive10", {"alive": 0.1}), (2, "_fall", {"alive": 0.0, "fall": 20.0}),
                       (2, "_alive10_fall", {"alive": 0.1, "fall": 20.0}), (4, "_alive10", {"alive": 0.1}),
                       (2, "_gated", {"alive": 0.0, "gate": 0.85})):
    TASKS[f"legged{_c}{_name}"] = legged_task(_c, _name, **_kw)


def register(task):
    TASKS[task.name] = task
    return task


@dataclass
class Config:
    task: str = "cartpole"
    pop: int = 1024
    hidden: int | None = None
    sigma: float = 0.1
    lr: float = 0.1
    horizon: int = 500
    solved_at: float | None = None
    max_generations: int = 500
    time_budget: float = 120.0
    assist_k0: float = 0.0
    start_velocity: float = 0.0
    anneal_gens: int = 300


def n_params(hidden, task):
    return task.obs_dim * hidden + hidden + hidden * task.n_out + task.n_out


def unflatten(theta_pop, hidden, task):
    """(P, D) rows to (w1 (P, I, H), b1 (P, H), w2 (P, H, O), b2 (P, O)) views."""
    p, h, i, o = theta_pop.shape[0], hidden, task.obs_dim, task.n_out
    k = 0
    w1 = theta_pop[:, k:k + i * h].reshape(p, i, h); k += i * h
    b1 = theta_pop[:, k:k + h]; k += h
    w2 = theta_pop[:, k:k + h * o].reshape(p, h, o); k += h * o
    b2 = theta_pop[:, k:k + o]
    return w1, b1, w2, b2


def population_logits(obs, params):
    """Every member runs its own policy (``es.py:167-171``), as elementwise products summed
    over the input axis (float32 throughout)."""
    w1, b1, w2, b2 = params
    h = torch.tanh((obs[:, :, None] * w1).sum(dim=1) + b1)
    return (h[:, :, None] * w2).sum(dim=1) + b2


def push(task, state, start_velocity):
    """The starting-push curriculum: a forward velocity added to every initial state (``es.py:196-205``)."""
    if not start_velocity or task.xdot_row is None:
        return state
    state = state.clone()
    state[task.xdot_row] += start_velocity
    return state


def curriculum(cfg, gen):
    """Assistance stiffness and starting push at generation `gen` (``es.py:208-211``)."""
    ramp = max(0.0, 1.0 - (gen - 1) / cfg.anneal_gens) if cfg.anneal_gens > 0 else 0.0
    return cfg.assist_k0 * ramp, cfg.start_velocity * ramp


def centered_ranks(values):
    """argsort(argsort(v)) / (P - 1) - 0.5 with index tie-break (``es.py:214-215``)."""
    order = torch.argsort(values, stable=True)
    ranks = torch.empty_like(order)
    ranks[order] = torch.arange(values.shape[0], device=values.device)
    return ranks.to(values.dtype) / (values.shape[0] - 1) - 0.5


class FusedBackend:
    """One HIP launch per generation for the whole rollout (the reference's ``metal`` backend)."""

    name = "fused"

    def __init__(self, task, seed, device=None):
        self.task = task
        self.device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.gen = torch.Generator(device=self.device)
        self.gen.manual_seed(seed)
        self.reset_counter = (seed * 0x01000193) & 0x7FFFFFFF
        env = task.env
        (env.reseed if hasattr(env, "reseed") else lambda s: None)(seed)

    def normal(self, shape):
        return torch.randn(shape, generator=self.gen, device=self.device, dtype=torch.float32)

    def reset(self, n):
        self.reset_counter += 1
        return self.task.env.reset(n, seed=0xC0000000 + self.reset_counter, device=self.device)

    def step(self, state, action, assist=None):
        if assist is None:
            return self.task.env.step(state, action)
        return self.task.env.step(state, action, float(assist))

    def rollout(self, theta_pop, hidden, horizon, assist=0.0, start_velocity=0.0):
        state = push(self.task, self.reset(theta_pop.shape[0]), start_velocity)
        if self.task.assistable:
            return self.task.rollout(state, theta_pop, hidden, horizon, assist)
        return self.task.rollout(state, theta_pop, hidden, horizon)


class LoopBackend(FusedBackend):
    """Policy in torch, one HIP step launch per iteration (the reference's ``mlx`` backend)."""

    name = "loop"

    def rollout(self, theta_pop, hidden, horizon, assist=0.0, start_velocity=0.0):
        return loop_fitness(self, unflatten(theta_pop, hidden, self.task), horizon, assist, start_velocity)


class SeededBackend(FusedBackend):
    """Fused rollouts on a population regenerated from a counter-RNG seed (``es_noise``): one
    seed per generation drives both the rollout's population and the update's noise."""

    name = "seeded"

    def __init__(self, task, seed, device=None):
        if task.rollout_seeded is None:
            raise ValueError(f"task {task.name} has no seeded rollout")
        super().__init__(task, seed, device)
        self.noise_counter = (seed * 0x9E3779B9) & 0xFFFFFFFF

    def next_noise_seed(self):
        self.noise_counter = (self.noise_counter + 1) & 0xFFFFFFFF
        return self.noise_counter

    def rollout_seeded(self, theta, seed, sigma, pop, hidden, horizon, assist=0.0, start_velocity=0.0):
        state = push(self.task, self.reset(pop), start_velocity)
        if self.task.assistable:
            return self.task.rollout_seeded(state, theta, seed, sigma, hidden, horizon, assist)
        return self.task.rollout_seeded(state, theta, seed, sigma, hidden, horizon)

    def generation(self, theta, cfg, hidden, gen=1):
        """``es.py:218-227`` with the noise of one seed: rollout, centered ranks, update."""
        seed = self.next_noise_seed()
        assist, start_velocity = curriculum(cfg, gen)
        fit, steps = self.rollout_seeded(theta, seed, cfg.sigma, cfg.pop, hidden, cfg.horizon, assist,
                                         start_velocity)
        theta = es_noise.update(theta, centered_ranks(fit), seed, cfg.sigma, cfg.lr)
        return theta, fit, steps


BACKENDS = {"fused": FusedBackend, "loop": LoopBackend, "seeded": SeededBackend}


def loop_fitness(backend, params, horizon, assist=0.0, start_velocity=0.0, state=None):
    """(reward sum until first termination, steps taken) per member, stepping the whole
    population once per iteration with auto-reset (``es.py:174-193``)."""
    task = backend.task
    p = params[0].shape[0]
    if state is None:
        state = push(task, backend.reset(p), start_velocity)
    alive = torch.ones(p, dtype=torch.bool, device=state.device)
    fit = torch.zeros(p, device=state.device)
    steps = torch.zeros(p, device=state.device)
    for _ in range(horizon):
        action = task.action(population_logits(task.obs(state), params))
        state, reward, done = backend.step(state, action, assist) if task.assistable else backend.step(state, action)
        steps = steps + alive.to(steps.dtype)
        fell = alive & done
        alive = alive & ~done
        if task.height_gate:
            forward = (reward - 1.0) * (state[1] >= task.height_gate).to(fit.dtype)
        else:
            forward = reward - 1.0
        fit = fit + (forward + task.alive_bonus) * alive.to(fit.dtype) - task.fall_penalty * fell.to(fit.dtype)
    return fit, steps


def generation(backend, theta, cfg, hidden, gen=1):
    """One ES generation (``es.py:218-227``): antithetic noise, rollout, ranks, update."""
    if isinstance(backend, SeededBackend):
        return backend.generation(theta, cfg, hidden, gen)
    half = backend.normal((cfg.pop // 2, theta.shape[0]))
    eps = torch.cat([half, -half], dim=0)
    assist, start_velocity = curriculum(cfg, gen)
    fit, steps = backend.rollout(theta[None, :] + cfg.sigma * eps, hidden, cfg.horizon, assist, start_velocity)
    grad = (centered_ranks(fit)[:, None] * eps).sum(dim=0) / (cfg.pop * cfg.sigma)
    return theta + cfg.lr * grad, fit, steps


def mean_policy(theta, hidden, task):
    """The unperturbed policy as an actor on (n, obs_dim) observations (``es.py:302-305``)."""
    w1, b1, w2, b2 = (p[0] for p in unflatten(theta[None, :], hidden, task))
    return lambda obs: torch.tanh(obs @ w1 + b1) @ w2 + b2


def evaluate(task, actor, n=2048, steps=500, device=None, seed=0x7FFF0000):
    """Canonical score of a greedy actor over n fresh episodes: the environment's reward minus
    one plus ``task.eval_bonus``, summed to the first termination (``es.py:308-322``)."""
    device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    state = task.env.reset(n, seed=seed, device=device)
    alive = torch.ones(n, dtype=torch.bool, device=device)
    fit = torch.zeros(n, device=device)
    for _ in range(steps):
        action = task.action(actor(task.obs(state)))
        state, reward, done = task.env.step(state, action)
        alive = alive & ~done
        fit = fit + (reward - 1.0 + task.eval_bonus) * alive.to(torch.float32)
    return fit.mean().item()


def evaluate_theta(task, theta, hidden, n=2048, steps=500, device=None, seed=0x7FFF0000):
    """``evaluate(task, mean_policy(theta, hidden, task), n, steps)`` (``es.py:302-322``) as one
    launch of the task's fused evaluation kernel when it has one; the per-env sums are the
    reference's, with the policy summed in the fused rollouts' order instead of a matmul's."""
    if task.evaluate_policy is None:
        return evaluate(task, mean_policy(theta, hidden, task), n, steps, device, seed)
    device = torch.device(device) if device is not None else theta.device
    state = task.env.reset(n, seed=seed, device=device)
    return task.evaluate_policy(state, theta, hidden, steps).mean().item()


@dataclass
class Result:
    solved: bool
    generations: int
    env_steps: int
    train_seconds: float
    score: float


@dataclass
class GenerationLog:
    generation: int
    env_steps: int        # steps taken so far, summed over members and generations
    train_seconds: float  # device time of the generations so far
    pop_fitness: float    # mean training fitness of this generation's population
    score: float          # the mean policy's canonical score after this generation


class Trainer:
    """One ES run: its backend, the current parameters and the running totals. ``advance()``
    runs a generation between two device synchronisations (the training clock) and scores
    the updated mean policy after the clock stops."""

    def __init__(self, cfg, backend_name, seed, device=None):
        if cfg.pop % 2:
            raise ValueError("the population must be even (antithetic pairs)")
        self.cfg = cfg
        self.task = TASKS[cfg.task]
        self.hidden = self.task.hidden if cfg.hidden is None else cfg.hidden
        self.threshold = self.task.solved_at if cfg.solved_at is None else cfg.solved_at
        self.backend = BACKENDS[backend_name](self.task, seed, device)
        self.theta = self.backend.normal((n_params(self.hidden, self.task),)) * 0.1   # initial policy (es.py:340)
        self.history = []
        self._seconds, self._steps = 0.0, 0

    def advance(self):
        gen = len(self.history) + 1
        dev = self.backend.device
        torch.cuda.synchronize(dev)
        start = time.perf_counter()
        self.theta, fit, steps = generation(self.backend, self.theta, self.cfg, self.hidden, gen)
        torch.cuda.synchronize(dev)
        self._seconds += time.perf_counter() - start
        self._steps += int(steps.sum().item())
        score = evaluate_theta(self.task, self.theta, self.hidden, device=dev)
        record = GenerationLog(gen, self._steps, self._seconds, float(fit.mean().item()), score)
        self.history.append(record)
        return record

    @property
    def solved(self):
        return bool(self.history) and self.history[-1].score >= self.threshold

    @property
    def exhausted(self):
        return len(self.history) >= self.cfg.max_generations or self._seconds >= self.cfg.time_budget


def train(cfg, backend_name, seed, log=None, device=None):
    """Generations until the mean policy's score reaches the task's threshold, the generation
    cap or the training-time budget (the reference's ``train``, ``es.py:334-354``).
    ``log(generation, env_steps, train_seconds, pop_fitness, score)`` is called after each."""
    trainer = Trainer(cfg, backend_name, seed, device)
    while True:
        rec = trainer.advance()
        if log is not None:
            log(rec.generation, rec.env_steps, rec.train_seconds, rec.pop_fitness, rec.score)
        if trainer.solved or trainer.exhausted:
            return Result(trainer.solved, rec.generation, rec.env_steps, rec.train_seconds, rec.score)


# The reference's backend names on the command line: its fused Metal rollout is the
# "fused" backend here and its MLX step loop the "loop" backend; its numpy backend is the
# CPU oracle, which this package does not run.
BACKEND_ALIASES = {"metal": "fused", "mlx": "loop"}


def parse_args(argv=None):
    """(Config, backend name, seed) from the reference's command line (``es.py:357-371``):
    the same flags with the same defaults, plus ``--hidden`` and ``--horizon`` and the
    "seeded" backend, which the reference does not have."""
    import argparse

    p = argparse.ArgumentParser(prog="python -m hipenvs.es", description=__doc__,
                                formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--task", choices=sorted(TASKS), default="cartpole")
    p.add_argument("--pop", type=int, default=1024)
    p.add_argument("--backend", choices=sorted(BACKENDS) + sorted(BACKEND_ALIASES), default="metal")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--lr", type=float, default=0.1)
    p.add_argument("--sigma", type=float, default=0.1)
    p.add_argument("--time-budget", type=float, default=120.0)
    p.add_argument("--max-generations", type=int, default=500)
    p.add_argument("--assist", type=float, default=0.0,
                   help="torso-assist spring stiffness at generation 1, annealed to zero")
    p.add_argument("--start-velocity", type=float, default=0.0,
                   help="forward push at episode start, annealed to zero")
    p.add_argument("--anneal", type=int, default=300, help="generation by which both curricula reach zero")
    p.add_argument("--hidden", type=int, default=None, help="hidden units (default: the task's)")
    p.add_argument("--horizon", type=int, default=500)
    a = p.parse_args(argv)
    cfg = Config(task=a.task, pop=a.pop, hidden=a.hidden, sigma=a.sigma, lr=a.lr, horizon=a.horizon,
                 max_generations=a.max_generations, time_budget=a.time_budget, assist_k0=a.assist,
                 start_velocity=a.start_velocity, anneal_gens=a.anneal)
    return cfg, BACKEND_ALIASES.get(a.backend, a.backend), a.seed


def main(argv=None):
    """The reference's ``python es.py ...`` (``es.py:357-382``): train and print each
    generation, then the result."""
    cfg, backend, seed = parse_args(argv)
    result = train(cfg, backend, seed, log=lambda gen, es_, secs, fit, score: print(
        f"gen {gen:4d}  env_steps {es_:>13,}  train {secs:7.2f}s  pop fitness {fit:8.1f}  score {score:8.1f}",
        flush=True))
    print(result)
    return result


if __name__ == "__main__":
    main()
