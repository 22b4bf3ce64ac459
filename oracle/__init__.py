"""CPU oracle for the hipenvs HIP library.

TEST INFRASTRUCTURE, NOT PRODUCT CODE. This package is a numpy restatement of
the reference's numpy environments and ES loop (metal-rl-envs:
``cartpole_np.py``, ``acrobot_np.py``, ``pendulum_np.py``,
``pendulum_aba_np.py``, ``hopper_np.py``, ``legged_np.py``, ``es.py``), each
function citing the reference lines it follows. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it, and only to check results against or as the timed CPU baseline; the library under
``metal-rl-envs_amd/`` never imports, links or runs anything here, and fails
loudly when its HIP library is missing.

Shared conventions that make oracle and kernels agree bit for bit:

* the same float32 operation order as the reference's numpy code;
* no fused multiply-add anywhere (the HIP library is compiled with
  ``-ffp-contract=off``);
* deterministic transcendentals (``detmath``) and a counter RNG (``rng``)
  evaluated identically on both sides.

Which checks pin which function (the reference's own closed forms, golden
fixtures, invariants) is listed in the module docstrings and in the tests.
"""
