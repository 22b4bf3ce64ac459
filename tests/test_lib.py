"""The C-ABI library without a GPU: it loads, exports what the header declares, and
its compiled-in constants are the float32 values of the reference's constants (CPU)."""

import ctypes
import math
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "hipenvs.h"
CSRC = ROOT / "metal-rl-envs_amd" / "csrc"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(hipenvs_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_exports_every_declared_symbol():
    from hipenvs import _lib

    assert _lib.LIB_PATH.exists(), "run python metal-rl-envs_amd/build.py"
    handle = ctypes.CDLL(str(_lib.LIB_PATH))
    names = declared_functions()
    assert len(names) >= 7
    for name in names:
        assert hasattr(handle, name), name


def test_python_binding_covers_the_header():
    from hipenvs import _lib

    status_fns = set(declared_functions()) - {"hipenvs_version", "hipenvs_last_hip_error"} - set(_lib.VALUE_SIGNATURES)
    assert status_fns == set(_lib.SIGNATURES)
    assert _lib.lib().hipenvs_legged_es_rollout_workspace_bytes(4, 64, 1000) > 1000 * 1676 * 4
    # two sets of 1,024 slots x (2 x 6 state rows + D = 1,353 weights + 4), plus the counters
    assert _lib.lib().hipenvs_legged_es_rollout_workspace_bytes(3, 64, 1000) == 2 * (12 + 1353 + 4) * 1024 * 4 + 64
    assert _lib.lib().hipenvs_legged_es_rollout_workspace_bytes(5, 64, 1000) == -1
    assert _lib.lib().hipenvs_legged_es_rollout_workspace_bytes(0, 64, 1000) == -1
    assert _lib.lib().hipenvs_legged_es_rollout_workspace_bytes(4, 12, 1000) == -1
    assert _lib.version().startswith("hipenvs ")
    assert _lib.lib().hipenvs_last_hip_error() == 0


def test_bad_arguments_are_rejected_before_any_launch():
    """The C ABI validates sizes and pointers; none of these reach the GPU."""
    from hipenvs import _lib

    l = _lib.lib()
    null = ctypes.c_void_p(0)
    assert l.hipenvs_cartpole_step(null, null, 0, null, null, null, 16, null) == _lib.E_ARG
    assert l.hipenvs_cartpole_step(null, null, 0, null, null, null, -1, null) == _lib.E_ARG
    assert l.hipenvs_cartpole_step(null, null, 0, null, null, null, 0, null) == _lib.OK
    assert l.hipenvs_sample_actions(null, 8, 0, 0, null) == _lib.E_ARG
    assert l.hipenvs_sample_actions(null, 8, 257, 0, null) == _lib.E_ARG


def test_legged_rollout_entry_points_check_their_shapes_on_the_host():
    """The chunked rollouts return before any launch for a misaligned rows pointer, a rows
    array past the 32-bit byte offsets, a short workspace, an odd or tiny seeded population
    and an unsupported leg count. The addresses are never dereferenced."""
    from hipenvs import _lib

    l = _lib.lib()
    p_ = ctypes.c_void_p
    ok, odd = p_(1 << 20), p_((1 << 20) + 2)
    args = (1.0, 0.0, 0.0, 0.0, ok, ok)
    need = l.hipenvs_legged_es_rollout_workspace_bytes(4, 64, 4096)
    rows = l.hipenvs_legged_es_rollout_chunked_rows
    assert rows(4, 64, 8, 32, ok, odd, 4096, 10, *args, ok, need, None) == _lib.E_ARG
    assert rows(4, 64, 8, 32, ok, ok, 4096, 10, *args, ok, need - 1, None) == _lib.E_ARG
    big = (1 << 31) // (1676 * 4) + 1  # p * D * 4 >= 2^31 at C = 4, H = 64
    assert rows(4, 64, 8, 32, ok, ok, big, 10, *args, ok, 1 << 62, None) == _lib.E_UNSUPPORTED
    assert rows(5, 64, 8, 32, ok, ok, 4096, 10, *args, ok, 1 << 62, None) == _lib.E_UNSUPPORTED
    seeded = l.hipenvs_legged_es_rollout_seeded
    assert seeded(4, 64, 8, 32, ok, ok, 4097, 1, 0.03, 10, *args, ok, 1 << 62, None) == _lib.E_ARG
    assert seeded(4, 64, 8, 32, ok, ok, 1, 1, 0.03, 10, *args, ok, 1 << 62, None) == _lib.E_ARG
    assert seeded(4, 64, 8, 32, ok, ok, 4096, 1, 0.03, 10, *args, ok, need - 1, None) == _lib.E_ARG


def test_python_wrappers_check_tensors():
    import torch

    from hipenvs import cartpole

    with pytest.raises(TypeError):
        cartpole.step(np.zeros((4, 8), np.float32), torch.zeros(8, dtype=torch.int32))
    with pytest.raises(TypeError):
        cartpole.step(torch.zeros((4, 8), dtype=torch.float64), torch.zeros(8, dtype=torch.int32))
    with pytest.raises(ValueError):
        cartpole.step(torch.zeros((3, 8)), torch.zeros(8, dtype=torch.int32))
    with pytest.raises(ValueError):
        cartpole.step(torch.zeros((4, 8)), torch.zeros(8, dtype=torch.int32))   # CPU tensor: not on a GPU


def kernel_constants():
    """(name, value, expression) for every `constexpr float NAME = HEX;  // float32(EXPR)` line."""
    out = []
    for path in sorted(CSRC.glob("*.hip")):
        for m in re.finditer(r"constexpr float (\w+) = (-?0x[0-9a-fA-F.]+p[+-]?\d+)f;\s*// float32\((.+)\)", path.read_text()):
            out.append((f"{path.name}:{m.group(1)}", float.fromhex(m.group(2)), m.group(3)))
    return out


def test_kernel_constants_are_float32_of_the_reference_values():
    consts = kernel_constants()
    assert len(consts) >= 11
    for name, value, expr in consts:
        expect = float(np.float32(eval(expr, {"pi": math.pi, "np": np})))
        assert value == expect, (name, expr, value, expect)


def test_unsupported_shapes_are_rejected_on_the_host():
    from hipenvs import pendulum_aba

    with pytest.raises(ValueError):
        pendulum_aba.Pendulum(5)
