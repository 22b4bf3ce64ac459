"""hipenvs: batched RL environments and fused ES rollouts as HIP kernels for MI355X.

A drop-in for the Metal hot path of metal-rl-envs: the step modules
(``cartpole``, ``acrobot``, ``pendulum_aba.Pendulum``, ``legged.Legged``) keep
the reference's ``reset``/``step``/``reseed`` surface over (D, N) float32 SoA
state tensors, the rollout modules (``cartpole_rollout``, ``acrobot_rollout``,
``legged_rollout``) keep its ``rollout_steps``/``rollout`` calls, and ``es``
is the ES loop that drives them. Every
computation runs in ``libhipenvs.so`` (built by ``metal-rl-envs_amd/build.py``);
there is no host fallback.
"""

from ._lib import HipEnvsError, version  # noqa: F401
