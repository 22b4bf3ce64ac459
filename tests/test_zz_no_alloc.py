"""The no-allocation ES update (hipenvs_es_update_static, GPU): partial sums in the
library's static device array instead of a caller workspace. Called through the C ABI
and compared bit for bit with hipenvs_es_update and with the oracle, on two calls in a
row (the second smaller, so stale partials of the first call sit beyond what it reads),
plus the size limit and the in-place form.
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle import es as oes
from oracle import es_noise as oen

pytestmark = pytest.mark.gpu


def to_np(t):
    return t.detach().cpu().numpy()


def case(dev, d, p, seed):
    rng = np.random.default_rng(seed)
    theta = (rng.standard_normal(d) * 0.1).astype(np.float32)
    ranks = oes.centered_ranks(rng.standard_normal(p).astype(np.float32)).astype(np.float32)
    return theta, ranks, torch.from_numpy(theta).to(dev), torch.from_numpy(ranks).to(dev)


def with_workspace(theta, ranks, d, p, seed, sigma, lr):
    from hipenvs import _lib

    nbytes = _lib.lib().hipenvs_es_update_workspace_bytes(d, p)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=theta.device)
    out = torch.empty_like(theta)
    _lib.call("hipenvs_es_update", _lib.ptr(theta), _lib.ptr(ranks), d, p, _lib.u32(seed), sigma, lr, _lib.ptr(out),
              _lib.ptr(ws), nbytes, _lib.stream_of(theta.device))
    return out


def static(theta, ranks, d, p, seed, sigma, lr, out=None):
    from hipenvs import _lib

    out = torch.empty_like(theta) if out is None else out
    rc = _lib.lib().hipenvs_es_update_static(_lib.ptr(theta), _lib.ptr(ranks), d, p, _lib.u32(seed), sigma, lr,
                                             _lib.ptr(out), _lib.stream_of(theta.device))
    assert rc == _lib.OK, rc
    return out


def test_two_calls_in_a_row_match_the_workspace_entry_point(dev):
    """legged4 H = 64 at P = 262,144 (256 partial rows of D = 1,676, the largest config),
    then CartPole H = 32 at P = 4,096 (64 rows of D = 226) on the same static array."""
    print("no-alloc update: (1676, 262144) then (226, 4096)", flush=True)
    for d, p, seed in ((1676, 262144, 11), (226, 4096, 12)):
        theta_np, ranks_np, theta, ranks = case(dev, d, p, seed)
        got = static(theta, ranks, d, p, seed, 0.03, 0.1)
        want = with_workspace(theta, ranks, d, p, seed, 0.03, 0.1)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(to_np(got), to_np(want))
        if p <= 4096:
            np.testing.assert_array_equal(to_np(got), oen.update(theta_np, ranks_np, seed, 0.03, 0.1))


def test_repeated_calls_and_in_place(dev):
    """The same call twice gives the same bits, and theta_out may alias theta."""
    d, p = 323, 2000
    theta_np, ranks_np, theta, ranks = case(dev, d, p, 5)
    first = static(theta, ranks, d, p, 9, 0.1, 0.05)
    second = static(theta, ranks, d, p, 9, 0.1, 0.05)
    expect = oen.update(theta_np, ranks_np, 9, 0.1, 0.05)
    np.testing.assert_array_equal(to_np(first), expect)
    np.testing.assert_array_equal(to_np(second), expect)
    static(theta, ranks, d, p, 9, 0.1, 0.05, out=theta)
    np.testing.assert_array_equal(to_np(theta), expect)


def test_python_wrapper(dev):
    from hipenvs import es_noise

    d, p = 1030, 8192
    theta_np, ranks_np, theta, ranks = case(dev, d, p, 21)
    out = torch.empty_like(theta)
    es_noise.update_static(theta, ranks, 4, 0.03, 0.1, out)
    np.testing.assert_array_equal(to_np(out), to_np(es_noise.update(theta, ranks, 4, 0.03, 0.1)))


def test_shapes_beyond_the_static_array_are_rejected(dev):
    """d = 2049 at a population with 256 partial rows needs 2,098,176 bytes > 2 MiB: rejected
    on the host before any launch; the same d with few rows fits."""
    from hipenvs import _lib

    null = ctypes.c_void_p(0)
    l = _lib.lib()
    assert l.hipenvs_es_update_workspace_bytes(2049, 32768) > _lib.ES_UPDATE_STATIC_BYTES
    dummy = torch.zeros(1, device=dev)
    p_ = _lib.ptr(dummy)
    assert l.hipenvs_es_update_static(p_, p_, 2049, 32768, 0, 0.1, 0.1, p_, null) == _lib.E_SCRATCH
    assert l.hipenvs_es_update_static(p_, p_, 2048, 32768, 0, 0.1, 0.1, null, null) == _lib.E_ARG
    theta_np, ranks_np, theta, ranks = case(dev, 2049, 64, 3)
    got = static(theta, ranks, 2049, 64, 3, 0.1, 0.1)
    np.testing.assert_array_equal(to_np(got), oen.update(theta_np, ranks_np, 3, 0.1, 0.1))


CAPTURE_CHILD = r"""
import sys
sys.path[:0] = [sys.argv[1], sys.argv[2]]
import numpy as np
import torch
from hipenvs import _lib

dev = torch.device("cuda", 0)
d, p, seed, sigma, lr = 1676, 8192, 17, 0.03, 0.1
rng = np.random.default_rng(seed)
theta = torch.from_numpy((rng.standard_normal(d) * 0.1).astype(np.float32)).to(dev)
ranks = torch.from_numpy(((np.argsort(np.argsort(rng.standard_normal(p), kind="stable"), kind="stable")
                           / (p - 1)) - 0.5).astype(np.float32)).to(dev)
out = torch.zeros_like(theta)
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
side = torch.cuda.Stream(device=dev)
side.wait_stream(torch.cuda.current_stream(dev))
with torch.cuda.stream(side):
    with torch.cuda.graph(g, stream=side):
        # the library's first call on this device: its static array's address is looked up here
        rc = _lib.lib().hipenvs_es_update_static(_lib.ptr(theta), _lib.ptr(ranks), d, p, _lib.u32(seed), sigma, lr,
                                                 _lib.ptr(out), _lib.stream_of(dev))
torch.cuda.synchronize()
print("captured, status", rc, flush=True)
assert rc == _lib.OK, rc
nbytes = _lib.lib().hipenvs_es_update_workspace_bytes(d, p)
ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
want = torch.empty_like(theta)
_lib.call("hipenvs_es_update", _lib.ptr(theta), _lib.ptr(ranks), d, p, _lib.u32(seed), sigma, lr, _lib.ptr(want),
          _lib.ptr(ws), nbytes, _lib.stream_of(dev))
torch.cuda.synchronize()
for r in range(3):
    out.fill_(float(r + 7))               # eager work between replays
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, want), f"replay {r} differs from hipenvs_es_update"
    print(f"replay {r} equal", flush=True)
print("capture ok", flush=True)
"""


def test_first_call_under_graph_capture(dev):
    """A fresh process whose first call of the library on the device is made under HIP graph
    capture (torch.cuda.graph, global capture mode): the static array's address is looked up
    inside the capture, the captured update is replayed three times with eager work and
    synchronisations between the replays, and every replay equals hipenvs_es_update's result."""
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    print("no-alloc update under graph capture (child process)", flush=True)
    r = subprocess.run([sys.executable, "-c", CAPTURE_CHILD, str(root), str(root / "metal-rl-envs_amd")],
                       capture_output=True, text=True, timeout=240)
    assert r.returncode == 0 and "capture ok" in r.stdout, (r.returncode, r.stdout[-2000:], r.stderr[-2000:])
