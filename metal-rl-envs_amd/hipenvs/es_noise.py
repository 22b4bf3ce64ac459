"""Seeded ES generation: antithetic perturbations regenerated from a counter RNG.

The reference's ``generation`` (``es.py:218-227``) draws ``half`` (P/2, D)
normals, materialises ``eps = [half; -half]`` and the population
``theta + sigma * eps``, and reduces ``sum(ranks[:, None] * eps, 0) / (P sigma)``.
Here the noise is a function of (seed, member pair, weight pair), evaluated in
the kernels that need it:

* ``perturb``: the population ``theta + sigma * [eps; -eps]``, rows (P, D) or
  columns (D, P), for callers that want it (the loop backend, tests);
* the ``rollout_steps_seeded`` / ``rollout_seeded`` functions of the rollout
  modules write the population into their own workspace (the legged one
  straight into its packed member tiles) and never return it;
* ``update``: ``theta + lr * sum_m ranks[m] eps[m] / (P sigma)``, regenerating
  eps on the fly; ranks come from ``es.centered_ranks`` as in the reference.

The generator (member key, Box-Muller on 24-bit fixed point with float32 ln,
sin and cos written as elementary operations) is defined in the library's
``csrc/es_noise.h``. Member ``m + P/2`` carries ``-eps[m]``.
"""

import torch

from . import _lib

LAYOUTS = {"rows": 0, "columns": 1}


def perturb(theta, p, seed, sigma, layout="rows"):
    """theta + sigma * [eps; -eps] for p (even) members: (p, d) for "rows", (d, p) for "columns"."""
    if layout not in LAYOUTS:
        raise ValueError(f"layout must be one of {tuple(LAYOUTS)}")
    p = _lib.check_population(p)
    if not isinstance(theta, torch.Tensor) or theta.dim() != 1:
        raise TypeError("theta must be a 1-D torch.Tensor")
    d = theta.shape[0]
    theta = _lib.check_theta_vector(theta, d, theta.device)
    shape = (p, d) if layout == "rows" else (d, p)
    out = torch.empty(shape, dtype=torch.float32, device=theta.device)
    with _lib.on(theta.device):
        _lib.call("hipenvs_es_perturb", _lib.ptr(theta), d, p, _lib.u32(seed), float(sigma), LAYOUTS[layout],
                  _lib.ptr(out), _lib.stream_of(theta.device))
    return out


def _update_args(theta, ranks):
    if not isinstance(theta, torch.Tensor) or theta.dim() != 1:
        raise TypeError("theta must be a 1-D torch.Tensor")
    d = theta.shape[0]
    theta = _lib.check_theta_vector(theta, d, theta.device)
    if not isinstance(ranks, torch.Tensor) or ranks.dim() != 1:
        raise TypeError("ranks must be a 1-D torch.Tensor")
    p = _lib.check_population(ranks.shape[0])
    ranks = _lib.as_f32_vector(ranks, p, theta.device, "ranks")
    return theta, ranks, d, p


def update_static(theta, ranks, seed, sigma, lr, out):
    """``update`` into the caller's ``out`` (d,) with no device allocation: the partial sums
    live in the library's static 2 MiB device array (d <= 2048 at any population), which
    calls on one GPU share, so overlapping calls race. For capture and serving loops."""
    theta, ranks, d, p = _update_args(theta, ranks)
    out_ok = (isinstance(out, torch.Tensor) and out.dtype == torch.float32 and out.shape == (d,)
              and out.device == theta.device and out.is_contiguous())
    if not out_ok:
        raise ValueError(f"out must be a contiguous float32 ({d},) tensor on {theta.device}")
    with _lib.on(theta.device):
        _lib.call("hipenvs_es_update_static", _lib.ptr(theta), _lib.ptr(ranks), d, p, _lib.u32(seed), float(sigma),
                  float(lr), _lib.ptr(out), _lib.stream_of(theta.device))
    return out


def update(theta, ranks, seed, sigma, lr):
    """theta + lr * (sum_m ranks[m] eps[m]) / (P sigma) with the noise of ``seed``; ranks (P,) float32."""
    theta, ranks, d, p = _update_args(theta, ranks)
    nbytes = _lib.lib().hipenvs_es_update_workspace_bytes(d, p)
    if nbytes < 0:
        raise _lib.HipEnvsError(f"hipenvs_es_update: unsupported population ({p}, {d})")
    workspace = torch.empty(nbytes, dtype=torch.uint8, device=theta.device)
    out = torch.empty_like(theta)
    with _lib.on(theta.device):
        _lib.call("hipenvs_es_update", _lib.ptr(theta), _lib.ptr(ranks), d, p, _lib.u32(seed), float(sigma),
                  float(lr), _lib.ptr(out), _lib.ptr(workspace), nbytes, _lib.stream_of(theta.device))
    return out
