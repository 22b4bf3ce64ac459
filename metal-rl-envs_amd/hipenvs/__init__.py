"""hipenvs: batched RL environments and fused ES rollouts as HIP kernels for MI355X.

A drop-in for the Metal hot path of metal-rl-envs: the step modules
(``cartpole``, and the other bodies as they land) keep the reference's
``reset``/``step``/``reseed`` surface over (D, N) float32 SoA state tensors,
and the rollout modules keep its ``rollout_steps``/``rollout`` calls. Every
computation runs in ``libhipenvs.so`` (built by ``metal-rl-envs_amd/build.py``);
there is no host fallback.
"""

from ._lib import HipEnvsError, version  # noqa: F401
