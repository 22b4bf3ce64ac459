"""Benchmark of the hipenvs hot path on one MI355X; prints ONE JSON line on stdout
(progress goes to stderr).

Headline (`value`): the batched CartPole step at N = 2**18 environments under the
reference's timing rule (bench.py:48-61, README:135-172): every iteration samples the
actions on the device (Bernoulli(0.5) from the counter RNG, hipenvs_sample_actions)
and then steps (hipenvs_cartpole_step, the cartpole_metal.step API), and every step's
reward and done rows are kept, as the reference's harness materialises them. The
`--steps` iterations are captured once into a HIP graph outside the clock; a timed
region replays that graph `repeats_per_region` times back to back between two device
synchronisations (enough replays for a region of about 0.25 s, so short `--steps`
runs still measure the steady state); env-steps/s = N x steps x replays / wall
seconds, median of `--repeats` regions; `ms_per_step` = wall / (steps x replays).

`roofline` (the dominant kernel, cp::step_kernel): achieved = 41 algorithmic bytes
per env-step (16 B state in, 4 B action, 16 B state out, 4 B reward, 1 B done) x N /
the kernel's average duration in the rocprofv3 kernel trace of this command
(profiles/cartpole_step_n262144.md; the tracer runs every dispatch on its own);
`achieved_events` / `frac_events` are the same bytes over the back-to-back launch
time measured live here with HIP events on the replay stream, on a graph of the
step alone with pre-drawn actions; `traffic` is the counter-measured HBM bytes per
launch (FETCH_SIZE + WRITE_SIZE, scaled by a copy of known size).

`cpu_baseline`: the CPU oracle's numpy CartPole step (the reference's algorithm
and op order with np.sin/np.cos, one process) at the same N for a bounded
sample of about `--cpu-seconds` seconds on this host.

`extra` holds the rest of the workload list, measured in the same run:
* `legged4_es_rollout`, `legged2_es_rollout`: the fused legged ES rollout at
  N = 262,144 members, C = 4 legs (quadruped) and C = 2 (biped), H = 64, sigma 0.03
  antithetic around theta0 = 0.1 N(0, 1), alive bonus 1 + forward velocity,
  horizon 1,000, S = 4/8/16 Gauss-Seidel sweeps:
  compacting chunked schedule, env-steps (steps taken) per second, a VALU roofline from the algorithmic
  FLOP count of the kernel source, and the numpy reference path (oracle in
  the reference's literal arithmetic: einsum policy + legged_np step) timed
  on a bounded sample of steps at the same N;
* `cartpole_step_kernel_only`: the step alone on actions drawn before the clock (the
  previous headline form), and `cartpole_module_api`: the drop-in module calls
  (hipenvs.cartpole.sample_actions + hipenvs.cartpole.step) from a Python loop, the
  rate a caller of the reference's API sees without graph capture;
* `cartpole_step_n1048576`, `cartpole_step_n16777216`: the step alone at 2^20 and at
  2^24 (a working set far beyond the 256 MB last-level cache: HBM-bound);
* `cartpole_fused_k32`: the K = 32 fused CartPole step, in-kernel and array actions;
* `es_config2`: CartPole and Acrobot fused ES rollouts, P = 4,096, H = 32, horizon 500,
  with a VALU roofline from the kernel source's FLOP count per step taken, and the
  reference's numpy ES loop (all members stepped every iteration) timed beside them in
  member-steps/s, to compare with the GPU's P x horizon rate;
* `aba_euler`: the K-link pendulum, semi-implicit Euler dt 0.01, N = 65,536,
  K = 4/16/64, 1,000 graph-replayed steps with the U[-1, 1] root torque drawn in the
  kernel, with its HBM roofline (16K + 5 B: state in and out, reward, done) and the
  numpy ABA Euler step timed beside it;
* `es_generation`: one whole ES generation (noise, rollout, centered ranks,
  update) two ways: "materialised" is the reference's generation (es.py:218-227)
  in torch around the fused rollout ((P/2, D) randn, concatenated noise,
  population, rank-weighted sum); "seeded" regenerates the noise from a
  counter-RNG seed inside the rollout and update kernels. Wall time (median of
  repeats) and peak allocated device memory, for CartPole and Acrobot at
  P = 4,096, H = 32, horizon 500 and legged4 at N = 262,144, H = 64, S = 8,
  horizon 1,000;
* `step_bodies`: single-step kernels graph-replayed for 1,000 steps with actions drawn on
  the device: the mass-matrix K-link pendulum (K = 2/4/8/16, RK4 dt 0.02) and the hopper at
  N = 65,536; the Acrobot step at N = 262,144; the legged C = 4 step with 8 sweeps at
  N = 65,536 (uniform actions in [0, 81)) -- the reference's own step benchmarks' shapes --
  and the same legged step in the reference's precision (float64 state);
* `es_evaluate`: the learner's greedy evaluation of the mean policy (es.py:308-322,
  2,048 envs x 500 steps): the fused one-launch kernel against the reference's
  loop (torch mean policy + one env-step launch per iteration); wall time, median
  of repeats, and both scores. CartPole, Acrobot and legged4 from theta = 0.1 N(0, 1);
  legged4_standing from a policy whose bodies stand for all 500 steps, as a trained
  one's do;

Usage: python bench.py [--gpus 1] [--steps 1000] [--warmup 16] [--repeats 3] [--sweep] [--skip-cpu]
                      [--only cartpole|legged|aba|steps|generation]
"""

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (str(ROOT), str(ROOT / "metal-rl-envs_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "env-steps/s at N=2^18 (CartPole, legged-4c ES rollout); % HBM/VALU roofline"
HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3           # MI355X FP32 vector, packed (published)
FP32_UNPACKED_TFLOPS = 78.6        # one FMA per lane per cycle
CARTPOLE_BYTES = 41
# HBM bytes per launch: rocprofv3 --pmc FETCH_SIZE and then WRITE_SIZE (one counter per run)
# over `bench.py --only cartpole --skip-cpu --steps 32 --warmup 2 --repeats 1 --region-seconds
# 0.0001 --copy-mib 256`, `bench.py --only aba --skip-cpu --copy-mib 256` (`--only steps` for the
# step bodies) and `bench.py --only legged --skip-cpu --repeats 1 --copy-mib 256`, in KiB per
# dispatch. The same counters read
# 131085.3-131085.4 and 262144.0 KiB for the 256 MiB device copy in the same process, so FETCH_SIZE is
# scaled by 2.000 and WRITE_SIZE by 1.000. Algorithmic bytes: 41 x N for the CartPole step.
# Tables and commands: profiles/cartpole_step_n262144.md, profiles/aba_euler_n65536.md,
# profiles/legged_es_rollout_n262144.md, profiles/step_bodies_and_evaluate.md.
CARTPOLE_TRAFFIC = {1 << 18: 10793034, 1 << 20: 43187100, 1 << 24: 689700249}
ABA_TRAFFIC = {4: 4649746, 16: 17437438, 64: 99818014}
ABA_RK4_TRAFFIC = {4: 5102694, 16: 18511667, 32: 37387878, 64: 405806592}  # profiles/aba_rk4_n65536.md
# The reference's articulated-body kernel (RK4, eval every 32) at N = 65,536 on its M3 Pro,
# results/aba.csv:137,222,307,392,460 (K = 4, 8, 16, 32, 64).
ABA_RK4_REFERENCE = {4: 450437382, 8: 184284347, 16: 68215640, 32: 17807725, 64: 3961767}
STEP_BODY_TRAFFIC = {"pendulum_k2": 2833253, "pendulum_k4": 5104345, "pendulum_k8": 9586116,
                     "pendulum_k16": 19185779, "hopper": 4889324, "acrobot": 10906005, "legged4_s8": 8227360,
                     "legged4_s8_reference": 16402468}
# per rollout of the drop-in call on (P, D) rows (every chunk, group-chunk and tail kernel of
# one rollout), keyed by (C, S)
LEGGED_ROLLOUT_TRAFFIC = {(4, 4): 89099891712, (4, 8): 101928242176, (4, 16): 110521539584,
                          (2, 4): 44110212710, (2, 8): 46772397466, (2, 16): 62815717376}


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def parse_args():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=1000)
    p.add_argument("--warmup", type=int, default=16)
    p.add_argument("--n", type=int, default=1 << 18)
    p.add_argument("--repeats", type=int, default=3)
    p.add_argument("--region-seconds", type=float, default=0.25,
                   help="length of a timed region of the headline: graph replays back to back")
    p.add_argument("--fused-k", type=int, default=32)
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--legged-cpu-seconds", type=float, default=12.0)
    p.add_argument("--skip-cpu", action="store_true")
    p.add_argument("--only", choices=["cartpole", "legged", "aba", "steps", "generation"], default=None,
                   help="run one block: the CartPole headline, the legged rollouts (then the line's value is the "
                        "legged4 S = 8 rollout), the ABA Euler step, the ABA Euler step and the other step "
                        "bodies, or the whole ES generations (the last three for counter collection; no line)")
    p.add_argument("--legged-n", type=int, default=262144)
    p.add_argument("--legged-horizon", type=int, default=1000)
    p.add_argument("--sweep", action="store_true", help="also run the CartPole N = 2^0..2^24 sweep")
    p.add_argument("--sweep-out", default=None)
    p.add_argument("--copy-mib", type=int, default=0,
                   help="first run a plain device-to-device copy of this many MiB three times (a known-size "
                        "kernel that scales hardware byte counters)")
    return p.parse_args()


# ---------------------------------------------------------------------------
# CartPole step
# ---------------------------------------------------------------------------

class CartPoleRun:
    """Preallocated buffers and raw C-ABI launches for the CartPole step benchmark."""

    def __init__(self, n, steps, dev, seed0=1):
        import torch

        from hipenvs import _lib, cartpole

        self.torch, self.lib, self.n, self.steps, self.dev = torch, _lib, n, steps, dev
        self.bufs = [cartpole.reset(n, seed=0, device=dev), torch.empty((4, n), dtype=torch.float32, device=dev)]
        self.actions = torch.empty((steps, n), dtype=torch.int32, device=dev)
        for t in range(steps):
            cartpole.sample_actions(n, seed=seed0 + t, device=dev, out=self.actions[t])
        self.rewards = torch.empty((steps, n), dtype=torch.float32, device=dev)
        self.dones = torch.empty((steps, n), dtype=torch.bool, device=dev)
        self.seed0 = seed0
        self.fn = _lib.lib().hipenvs_cartpole_step
        self.fn_k = _lib.lib().hipenvs_cartpole_step_k
        torch.cuda.synchronize()

    def launch_step(self, t, stream):
        P = self.lib.ptr
        rc = self.fn(P(self.bufs[t % 2]), P(self.actions[t]), self.seed0 + t, P(self.bufs[(t + 1) % 2]),
                     P(self.rewards[t]), P(self.dones[t]), self.n, stream)
        if rc != 0:
            raise RuntimeError(f"hipenvs_cartpole_step failed: {rc}")

    def launch_fused(self, t0, k, stream, array_actions):
        P = self.lib.ptr
        acts = P(self.actions[t0]) if array_actions else P(None)
        j = t0 // k
        rc = self.fn_k(P(self.bufs[j % 2]), acts, self.seed0 + t0, k, P(self.bufs[(j + 1) % 2]),
                       P(self.rewards[t0]), P(self.dones[t0]), self.n, stream)
        if rc != 0:
            raise RuntimeError(f"hipenvs_cartpole_step_k failed: {rc}")

    def graph_single(self):
        return capture_graph(self.dev, lambda s: [self.launch_step(t, s) for t in range(self.steps)])

    def graph_sampled(self):
        """Per iteration: the device sampler draws step t's actions into one (N,) row, then the
        step consumes them (the reference's loop samples inside the timed region)."""
        P = self.lib.ptr
        sampler = self.lib.lib().hipenvs_sample_actions
        row = self.torch.empty(self.n, dtype=self.torch.int32, device=self.dev)

        def body(stream):
            for t in range(self.steps):
                rc = sampler(P(row), self.n, 2, self.seed0 + t, stream)
                if rc != 0:
                    raise RuntimeError(f"hipenvs_sample_actions failed: {rc}")
                rc = self.fn(P(self.bufs[t % 2]), P(row), self.seed0 + t, P(self.bufs[(t + 1) % 2]),
                             P(self.rewards[t]), P(self.dones[t]), self.n, stream)
                if rc != 0:
                    raise RuntimeError(f"hipenvs_cartpole_step failed: {rc}")

        self.sample_row = row
        return capture_graph(self.dev, body)

    def graph_fused(self, k, array_actions):
        def body(s):
            t = 0
            while t < self.steps:
                kk = min(k, self.steps - t)
                self.launch_fused(t, kk, s, array_actions)
                t += kk
        return capture_graph(self.dev, body)


def capture_graph(dev, body):
    """A HIP graph of the launches `body(stream)` enqueues on a side stream."""
    import torch

    from hipenvs import _lib

    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            body(_lib.stream_of(dev))
    torch.cuda.synchronize()
    return g


def time_replay(g, repeats, per_region=1):
    """(median wall s, median HIP-event s) of timed regions, each `per_region` graph replays
    back to back between two device synchronisations; events on the replay's stream."""
    import torch

    g.replay()
    torch.cuda.synchronize()
    walls, events = [], []
    for _ in range(repeats):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        start.record()
        for _ in range(per_region):
            g.replay()
        end.record()
        torch.cuda.synchronize()
        walls.append(time.perf_counter() - t0)
        events.append(start.elapsed_time(end) / 1e3)
    return statistics.median(walls), statistics.median(events)


def replays_for(g, seconds):
    """Graph replays that fill a timed region of about `seconds` (at least one)."""
    wall, _ = time_replay(g, 1)
    return max(1, int(round(seconds / max(wall, 1e-9))))


def bench_cartpole(args, dev):
    """The headline: device action sampler + step per iteration (the reference's rule), then
    the step alone on pre-drawn actions and the K-fused step."""
    import torch

    from hipenvs import _lib

    n, steps, warmup = args.n, args.steps, args.warmup
    run = CartPoleRun(n, steps, dev)
    stream = _lib.stream_of(dev)
    for t in range(warmup):
        run.launch_step(t % steps, stream)
    torch.cuda.synchronize()
    g = run.graph_sampled()
    per_region = replays_for(g, args.region_seconds)
    wall, ev = time_replay(g, args.repeats, per_region)
    iterations = steps * per_region
    value = n * iterations / wall
    log(f"cartpole sampler + step N={n}: {value:,.0f} env-steps/s; {wall / iterations * 1e6:.3f} us per iteration "
        f"({per_region} replays of {steps} steps per region)")
    gk1 = run.graph_single()
    wall1, ev1 = time_replay(gk1, args.repeats, per_region)
    launch = ev1 / iterations
    kernel_only = {"env_steps_per_s": n * iterations / wall1, "us_per_launch_events": launch * 1e6,
                   "achieved_gbs_events": CARTPOLE_BYTES * n / launch / 1e9}
    log(f"cartpole_step alone (actions drawn before the clock) N={n}: {kernel_only['env_steps_per_s']:,.0f} "
        f"env-steps/s; {launch * 1e6:.3f} us per launch -> {kernel_only['achieved_gbs_events']:.1f} GB/s")
    gk = run.graph_fused(args.fused_k, False)
    wk, evk = time_replay(gk, args.repeats)
    gka = run.graph_fused(args.fused_k, True)
    wka, evka = time_replay(gka, args.repeats)
    k = args.fused_k
    launches = -(-steps // k)
    fused = {
        "k": k,
        "inkernel_actions_env_steps_per_s": n * steps / wk,
        "array_actions_env_steps_per_s": n * steps / wka,
        "inkernel_us_per_launch": evk / launches * 1e6,
        "array_us_per_launch": evka / launches * 1e6,
        "array_actions_algorithmic_gbs": (32 / k + 9) * n * steps / evka / 1e9,
        "inkernel_actions_algorithmic_gbs": (32 / k + 5) * n * steps / evk / 1e9,
    }
    log(f"cartpole fused K={k}: in-kernel actions {fused['inkernel_actions_env_steps_per_s']:,.0f}, "
        f"array actions {fused['array_actions_env_steps_per_s']:,.0f} env-steps/s")
    del g, gk1, gk, gka, run
    return {"value": value, "wall": wall, "iterations": iterations, "per_region": per_region,
            "us_per_iteration": wall / iterations * 1e6, "kernel_only": kernel_only, "fused": fused}


def module_api_rate(n, steps, dev):
    """The drop-in modules called from a Python loop (no graph): per iteration
    hipenvs.cartpole.sample_actions then hipenvs.cartpole.step, every reward and done kept
    until one synchronisation at the end (the reference's mlx_rollout, bench.py:48-61)."""
    import torch

    from hipenvs import cartpole

    def loop(count, seed0):
        state = cartpole.reset(n, seed=0, device=dev)
        pending = []
        for t in range(count):
            state, reward, done = cartpole.step(state, cartpole.sample_actions(n, seed=seed0 + t, device=dev))
            pending += [reward, done]
        return state, pending

    loop(16, 1)
    torch.cuda.synchronize()
    walls = []
    for r in range(3):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        loop(steps, 100 + r * steps)
        torch.cuda.synchronize()
        walls.append(time.perf_counter() - t0)
    wall = statistics.median(walls)
    out = {"n_envs": n, "steps": steps, "env_steps_per_s": n * steps / wall, "us_per_iteration": wall / steps * 1e6}
    log(f"cartpole module API loop N={n}: {out['env_steps_per_s']:,.0f} env-steps/s, "
        f"{out['us_per_iteration']:.2f} us per iteration")
    return out


# Average duration of cp::step_kernel per dispatch in the rocprofv3 kernel trace of the
# default command (`bench.py`, all of whose step launches at a given N are traced: the
# headline loop, the step alone and the bounded sweep's graphs), in ns;
# profiles/cartpole_step_n262144.md tabulates them. The tracer runs each dispatch on its own,
# so these include the per-dispatch ramp and drain that back-to-back launches overlap.
CARTPOLE_TRACE_NS = {1 << 18: 3433.3, 1 << 20: 8353.0, 1 << 24: 110188.9}
# sha256 (first 16 hex digits) of the sources the traced kernel was built from,
# csrc/cartpole.hip then csrc/hipenvs_device.h: when the sources differ, the trace no longer
# describes this build, and cartpole_roofline falls back to the run's own HIP-event figure.
CARTPOLE_TRACE_SOURCE_SHA = "5bda771dbf5c067d"
CARTPOLE_TRACE_SOURCES = ("metal-rl-envs_amd/csrc/cartpole.hip", "metal-rl-envs_amd/csrc/hipenvs_device.h")


def cartpole_source_sha():
    import hashlib

    h = hashlib.sha256()
    for rel in CARTPOLE_TRACE_SOURCES:
        h.update((ROOT / rel).read_bytes())
    return h.hexdigest()[:16]


def cartpole_roofline(n, kernel_only):
    """HBM roofline of cp::step_kernel at N: primary from the kernel trace's average duration,
    secondary from this run's back-to-back HIP-event launch time."""
    bytes_launch = CARTPOLE_BYTES * n
    events_gbs = kernel_only["achieved_gbs_events"]
    current = cartpole_source_sha() == CARTPOLE_TRACE_SOURCE_SHA
    trace_ns = CARTPOLE_TRACE_NS.get(n) if current else None
    achieved = bytes_launch / (trace_ns * 1e-9) / 1e9 if trace_ns else events_gbs
    return {"bound": "hbm", "kernel": "cp::step_kernel", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS, "traffic": CARTPOLE_TRAFFIC.get(n) if current else None,
            "frac_source": "kernel trace" if trace_ns else "hip events (this run)",
            "trace_matches_sources": current,
            "algorithmic_bytes_per_launch": bytes_launch, "avg_launch_ns_trace": trace_ns,
            "avg_launch_ns_events": kernel_only["us_per_launch_events"] * 1e3,
            "achieved_events": events_gbs, "frac_events": events_gbs / HBM_PEAK_GBS}


def copy_floor(n, steps, repeats, dev):
    """The step's back-to-back launch time against the floor for moving its bytes, at N: an
    elementwise kernel (torch.neg) that reads and writes 41 B x N / 2 each, replayed
    `steps` times in a graph like the step, with resident buffers; and the step itself with
    resident buffers (every launch on action row 0 and reward/done row 0)."""
    import torch

    elems = CARTPOLE_BYTES * n // 8  # float32 elements: 41 N / 2 bytes read, as many written
    src = torch.ones(elems, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    g = capture_graph(dev, lambda s: [torch.neg(src, out=dst) for _ in range(steps)])
    _, ev_copy = time_replay(g, repeats)
    run = CartPoleRun(n, 1, dev)
    P = run.lib.ptr

    def body(stream):
        for t in range(steps):
            rc = run.fn(P(run.bufs[t % 2]), P(run.actions[0]), run.seed0 + t, P(run.bufs[(t + 1) % 2]),
                        P(run.rewards[0]), P(run.dones[0]), n, stream)
            if rc != 0:
                raise RuntimeError(f"hipenvs_cartpole_step failed: {rc}")

    gs = capture_graph(dev, body)
    _, ev_step = time_replay(gs, repeats)
    out = {"n_envs": n, "bytes_per_launch": CARTPOLE_BYTES * n, "copy_us_per_launch": ev_copy / steps * 1e6,
           "step_resident_us_per_launch": ev_step / steps * 1e6}
    log(f"N={n}: elementwise copy of the step's bytes {out['copy_us_per_launch']:.3f} us, step with resident "
        f"buffers {out['step_resident_us_per_launch']:.3f} us per launch")
    del g, gs, run, src, dst
    return out


def bench_cartpole_at(n, steps, repeats, dev):
    """The step alone (pre-drawn actions), graph-replayed, at another N (the 2**20 and 2**24
    points of the step sweep)."""
    run = CartPoleRun(n, steps, dev)
    wall, ev = time_replay(run.graph_single(), repeats)
    launch = ev / steps
    gbs = CARTPOLE_BYTES * n / launch / 1e9
    log(f"cartpole_step N={n}: {n * steps / wall:,.0f} env-steps/s; {launch * 1e6:.3f} us per launch -> {gbs:.1f} GB/s")
    del run
    return {"n_envs": n, "steps": steps, "env_steps_per_s": n * steps / wall, "us_per_launch": launch * 1e6,
            "roofline": cartpole_roofline(n, {"us_per_launch_events": launch * 1e6, "achieved_gbs_events": gbs})}


def cpu_baseline_cartpole(n, seconds):
    """numpy CartPole step (reference algorithm, np.sin/np.cos) on one process; env-steps/s."""
    from oracle import cartpole as oc
    from oracle import rng

    state = oc.reset(n, seed=0)
    actions = [rng.action_bits(t, n) for t in range(1, 9)]
    for t in range(2):
        state, _, _ = oc.step(state, actions[t], seed=t + 1, trig="numpy")
    steps, t0 = 0, time.perf_counter()
    while True:
        state, _, _ = oc.step(state, actions[steps % 8], seed=steps + 3, trig="numpy")
        steps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return n * steps / el, steps


def cpu_rate_cartpole(n, seconds):
    """numpy CartPole env-steps/s at N (the oracle's step with np.sin/np.cos, one process)."""
    from oracle import cartpole as oc
    from oracle import rng

    state = oc.reset(n, seed=0)
    actions = [rng.action_bits(t, n) for t in range(1, 5)]
    state, _, _ = oc.step(state, actions[0], seed=1, trig="numpy")
    steps, t0 = 0, time.perf_counter()
    while True:
        state, _, _ = oc.step(state, actions[steps % 4], seed=steps + 2, trig="numpy")
        steps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            return n * steps / el


def sweep(dev, steps0, k, out_path, cpu_seconds=0.25, region_seconds=0.0):
    """Config-1 sweep: single-step and K-fused rates at N = 2^0..2^20 (and 2^22, 2^24), with the
    numpy rate at each N unless cpu_seconds is 0; the crossover is the first N where the
    single-step GPU rate passes numpy's. Every form is a HIP graph of `steps0` iterations
    (128 past 2^20), replayed back to back in 3 timed regions of about `region_seconds` (at
    least one replay each): the step alone on pre-drawn actions, the device sampler + step per
    iteration (the reference's rule), and the K-fused step with in-kernel or array actions."""
    rows = []
    for e in list(range(0, 21)) + [22, 24]:
        n = 1 << e
        steps = steps0 if n <= (1 << 20) else 128  # keep the (steps, N) buffers a few GB
        run = CartPoleRun(n, steps, dev)
        g1 = run.graph_single()
        reps = replays_for(g1, region_seconds) if region_seconds > 0 else 1
        w1, ev1 = time_replay(g1, 3, reps)
        ws, _ = time_replay(run.graph_sampled(), 3, reps)
        wk, _ = time_replay(run.graph_fused(k, False), 3, reps)
        wka, _ = time_replay(run.graph_fused(k, True), 3, reps)
        its = steps * reps
        launch = ev1 / its
        row = dict(n=n, steps=steps, replays=reps, single=n * its / w1, sampled=n * its / ws,
                   fused_inkernel=n * its / wk, fused_array=n * its / wka, launch_us=launch * 1e6,
                   single_gbs=CARTPOLE_BYTES * n / launch / 1e9)
        if cpu_seconds > 0:
            row["numpy"] = cpu_rate_cartpole(n, cpu_seconds)
        rows.append(row)
        log(f"N=2^{e:<2d} single {row['single']:>16,.0f}  sampler+step {row['sampled']:>16,.0f}  fused(in-kernel) "
            f"{row['fused_inkernel']:>16,.0f}  fused(array) {row['fused_array']:>16,.0f} env-steps/s  launch "
            f"{row['launch_us']:7.2f} us {row['single_gbs']:8.1f} GB/s"
            + (f"  numpy {row['numpy']:>14,.0f}" if "numpy" in row else ""))
        del run, g1
    crossover = next((r["n"] for r in rows if "numpy" in r and r["single"] > r["numpy"]), None)
    crossover_sampled = next((r["n"] for r in rows if "numpy" in r and r["sampled"] > r["numpy"]), None)
    out = {"rows": rows, "crossover_n": crossover, "crossover_n_sampler_and_step": crossover_sampled,
           "steps_per_graph": steps0, "numpy_seconds_per_n": cpu_seconds}
    if out_path:
        Path(out_path).write_text(json.dumps(out, indent=1))
    return out


# ---------------------------------------------------------------------------
# Legged ES rollout
# ---------------------------------------------------------------------------

def legged_flops_per_step(c, sweeps, hidden):
    """Algorithmic FP32 operations per env-step of the fused legged rollout, counted from the
    kernel source (add, sub, mul, div, sqrt = 1 each; no FMA; comparisons, selects and sign
    flips not counted; sin/cos/tanh counted separately). N = 3 + C generalised coordinates.
    Per substep: feet 10C, foot sums 9(C-1)+3, mass matrix 3C+4, forces 5C+11, Cholesky
    N(N+1)(2N+1)/6, (1+2C) solves of 2N^2, free velocity 2N, Delassus 16C^2 + 8C, per sweep
    and contact 25 (exact contact) + 6(C-1) + 2(C-2) + 2 (coupling sums), update 4CN + 2N.
    Per step: 4 substeps + policy 2*OBS*H + 2*H*OUT + 3 for the reward bookkeeping."""
    n = 3 + c
    coupling = (6 * (c - 1) + 2 * max(c - 2, 0) + 2) if c > 1 else 0
    sub = (10 * c + 9 * (c - 1) + 3 + 3 * c + 4 + 5 * c + 11 + n * (n + 1) * (2 * n + 1) // 6
           + (1 + 2 * c) * 2 * n * n + 2 * n + 16 * c * c + 8 * c + sweeps * c * (25 + coupling) + 4 * c * n + 2 * n)
    obs, out = 5 + 2 * c, 3 * c
    policy = 2 * obs * hidden + 2 * hidden * out
    return 4 * sub + policy + 3


def legged_population(dev, p, c, hidden, sigma=0.03, seed=0):
    """(P, D) rows: theta0 + sigma * [half; -half] around theta0 = 0.1 N(0, 1)."""
    import torch

    from hipenvs import legged_rollout

    d = legged_rollout.n_params(hidden, c)
    g = torch.Generator(device=dev).manual_seed(seed)
    theta0 = torch.randn(d, generator=g, device=dev) * 0.1
    half = torch.randn((p // 2, d), generator=g, device=dev)
    return theta0[None, :] + sigma * torch.cat([half, -half], dim=0)


def time_rollout(state, theta, hidden, horizon, c, sweeps, schedule, repeats, alive_at=()):
    """(median wall s, median HIP-event s, steps taken, mean fitness) of full rollouts, and
    with alive_at the members still alive after each of those step counts. schedule
    "dropin" is the drop-in call: the chunked schedule on the caller's (P, D) rows;
    "chunked" the same schedule on (D, P) columns; "rows"/"columns" one member per lane."""
    import torch

    from hipenvs import legged_rollout

    cols = schedule in ("columns", "chunked")
    small = theta[:, :64].contiguous() if cols else theta[:64].contiguous()
    sched = "chunked" if schedule == "dropin" else schedule
    kw = {"theta_cols": small} if schedule == "chunked" else {}
    legged_rollout.rollout(state[:, :64].contiguous(), None if kw else small, hidden, 4, c, iters=sweeps,
                           schedule=sched, **kw)
    torch.cuda.synchronize()
    walls, evs, taken, fit = [], [], None, None
    for _ in range(repeats):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        start.record()
        kw = {"theta_cols": theta} if schedule == "chunked" else {}
        fit, steps = legged_rollout.rollout(state, None if kw else theta, hidden, horizon, c, iters=sweeps,
                                            schedule=sched, **kw)
        end.record()
        torch.cuda.synchronize()
        walls.append(time.perf_counter() - t0)
        evs.append(start.elapsed_time(end) / 1e3)
        taken = float(steps.double().sum().item())
    out = (statistics.median(walls), statistics.median(evs), taken, float(fit.mean().item()))
    if alive_at:
        alive = {t: int((steps > t).sum().item()) for t in alive_at}
        alive["steps_in_first_32"] = int(torch.clamp(steps, max=32).double().sum().item())
        return out + (alive,)
    return out


# step counts at which the legged benchmark reports how many members are still alive
ALIVE_AT = (32, 64, 96, 128, 160, 192, 224, 256, 512, 999)


def bench_legged(args, dev, c=4, sweeps_list=(4, 8, 16)):
    import torch

    from hipenvs import legged, legged_rollout

    hidden, p, horizon = 64, args.legged_n, args.legged_horizon
    theta = legged_population(dev, p, c, hidden)
    theta_cols = theta.T.contiguous()
    state = legged.Legged(c).reset(p, seed=0, device=dev)
    d = legged_rollout.n_params(hidden, c)
    first = ", the first 16" if c <= 2 else ""
    out = {"n_envs": p, "c": c, "hidden": hidden, "horizon": horizon, "sigma": 0.03, "alive_bonus": 1.0,
           "schedule": f"chunked ({legged_rollout.CHUNK_STEPS} steps{first}), the drop-in call on the caller's "
                       f"(P, D) rows", "by_sweeps": {}}
    for s in sweeps_list:
        wall, ev, taken, fit_mean, alive = time_rollout(state, theta, hidden, horizon, c, s, "dropin",
                                                        args.repeats, alive_at=ALIVE_AT)
        flops = legged_flops_per_step(c, s, hidden)
        achieved_tf = taken * flops / ev / 1e12
        rec = {
            "env_steps_per_s": taken / wall,
            "steps_taken": taken,
            "mean_episode": taken / p,
            "wall_s": wall,
            "kernel_event_s": ev,
            "flops_per_env_step": flops,
            "roofline": {"bound": "valu", "achieved": achieved_tf, "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": achieved_tf / FP32_PEAK_TFLOPS,
                         "frac_of_unpacked_peak": achieved_tf / FP32_UNPACKED_TFLOPS,
                         "traffic": LEGGED_ROLLOUT_TRAFFIC.get((c, s))},
            "weight_bytes_per_env_step": 4 * d,
            "weight_stream_gbs": taken * 4 * d / ev / 1e9,
            "fitness_mean": fit_mean,
            "alive_after_steps": {str(t): n for t, n in alive.items()},
        }
        out["by_sweeps"][str(s)] = rec
        log(f"legged{c} ES rollout N={p} H={hidden} S={s} (drop-in rows): {rec['env_steps_per_s']:,.0f} env-steps/s "
            f"(mean episode {taken / p:.1f} steps, {ev * 1e3:.1f} ms), {achieved_tf:.2f} TFLOP/s algorithmic, "
            f"weights read at {rec['weight_stream_gbs']:.0f} GB/s")
        log(f"  alive after t steps: {', '.join(f'{t}: {n:,}' for t, n in alive.items() if t in ALIVE_AT)}; "
            f"member-steps in the first 32 steps: {alive['steps_in_first_32']:,}")
    # the same schedule on pre-transposed (D, P) columns, whose first chunk reads weight d of
    # 64 members as one 256-byte row
    wall, ev, taken, _ = time_rollout(state, theta_cols, hidden, horizon, c, 8, "chunked", args.repeats)
    rows_rec = out["by_sweeps"].get("8")
    out["columns_s8"] = {"env_steps_per_s": taken / wall, "wall_s": wall, "kernel_event_s": ev,
                         "same_steps_as_rows": rows_rec is None or taken == rows_rec["steps_taken"]}
    log(f"legged{c} chunked rollout on (D, P) columns, S=8: {taken / wall:,.0f} env-steps/s, {ev * 1e3:.1f} ms")
    if c == 4:
        wall, ev, taken, _ = time_rollout(state, theta, hidden, horizon, c, 8, "rows", 1)
        out["static_rows_s8_env_steps_per_s"] = taken / wall
        del theta
        wall, ev, taken, _ = time_rollout(state, theta_cols, hidden, horizon, c, 8, "columns", 1)
        out["static_columns_s8_env_steps_per_s"] = taken / wall
        log(f"legged4 one member per lane, S=8: rows {out['static_rows_s8_env_steps_per_s']:,.0f}, "
            f"columns {out['static_columns_s8_env_steps_per_s']:,.0f} env-steps/s")
    del theta_cols
    return out


def cpu_baseline_es(task, seconds, p=4096, hidden=32):
    """The reference's numpy ES path for config 2 (es.py:174-193 with the numpy backend):
    every iteration runs the einsum policy (es.py:167-171) and the numpy env step over all P
    members. Returns member-steps per second (P x iterations / s) and the iterations timed."""
    import numpy as np

    from oracle import acrobot as oa
    from oracle import cartpole as oc
    from oracle import es as oes

    obs_dim, n_out, env = (4, 2, oc) if task == "cartpole" else (6, 3, oa)
    r = np.random.default_rng(0)
    d = oes.n_params(hidden, obs_dim, n_out)
    theta0 = r.standard_normal(d, dtype=np.float32) * np.float32(0.1)
    half = r.standard_normal((p // 2, d), dtype=np.float32)
    w1, b1, w2, b2 = oes.unflatten(theta0[None, :] + np.float32(0.1) * np.concatenate([half, -half]), hidden,
                                   obs_dim, n_out)
    state = env.reset(p, seed=0)

    def obs(st):
        if task == "cartpole":
            return st.T
        th1, th2, dth1, dth2 = st
        return np.stack([np.cos(th1), np.sin(th1), np.cos(th2), np.sin(th2), dth1, dth2], axis=1)

    def one(t, st):
        h = np.tanh(np.einsum("pi,pih->ph", obs(st), w1) + b1)
        action = np.argmax(np.einsum("ph,pho->po", h, w2) + b2, axis=-1).astype(np.int32)
        return env.step(st, action, t, trig="numpy")[0]

    state = one(1, state)
    steps, t0 = 0, time.perf_counter()
    while True:
        state = one(steps + 2, state)
        steps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return p * steps / el, steps


def cpu_baseline_aba(k, seconds, n=65536):
    """The numpy ABA (the oracle's restatement of pendulum_aba_np.aba_accelerations with np.sin/
    np.cos) stepped by semi-implicit Euler at N envs, one process; env-steps per second."""
    from oracle import pendulum_aba as opa

    body = opa.Pendulum(k, trig="numpy")
    state = body.reset_euler(n, seed=0)
    state = body.step_euler(state, None, 1)[0]
    steps, t0 = 0, time.perf_counter()
    while True:
        state = body.step_euler(state, None, steps + 2)[0]
        steps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return n * steps / el, steps


def cpu_baseline_legged(n, seconds, c=4, hidden=64, sweeps=8):
    """The reference's numpy ES path at N members: einsum policy (es.py:167-171), per-leg
    argmax (es.py:86-93), legged_np step in its literal arithmetic; steps per second."""
    import numpy as np

    from oracle import es as oes
    from oracle import legged as olg

    body = olg.Legged(c, sweeps, mode="reference")
    state = body.reset(n, seed=0)
    r = np.random.default_rng(0)
    d = oes.n_params(hidden, 5 + 2 * c, 3 * c)
    theta0 = (r.standard_normal(d, dtype=np.float32) * np.float32(0.1))
    half = r.standard_normal((n // 2, d), dtype=np.float32)
    theta = theta0[None, :] + np.float32(0.03) * np.concatenate([half, -half])
    del half
    w1, b1, w2, b2 = oes.unflatten(theta, hidden, 5 + 2 * c, 3 * c)

    def one(t, state):
        obs = state[1:].T
        h = np.tanh(np.einsum("pi,pih->ph", obs, w1) + b1)
        logits = np.einsum("ph,pho->po", h, w2) + b2
        return body.step(state, oes.legged_action(logits, c), seed=t)[0]

    state = one(1, state)  # warm-up
    steps, t0 = 0, time.perf_counter()
    while True:
        state = one(steps + 2, state)
        steps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return n * steps / el, steps


# ---------------------------------------------------------------------------
# ES config 2 and ABA config 3
# ---------------------------------------------------------------------------

def bench_es_generation(dev, repeats, legged_n, legged_horizon):
    import torch

    from hipenvs import (acrobot, acrobot_rollout, cartpole, cartpole_rollout, es, es_noise, legged,
                         legged_rollout)

    cases = (
        ("cartpole", 4096, 32, 500, 0.1, cartpole.reset,
         lambda st, pop: cartpole_rollout.rollout_steps(st, pop, 32, 500),
         lambda st, th, sd: cartpole_rollout.rollout_steps_seeded(st, th, sd, 0.1, 32, 500)),
        ("acrobot", 4096, 32, 500, 0.1, acrobot.reset,
         lambda st, pop: acrobot_rollout.rollout_steps(st, pop, 32, 500),
         lambda st, th, sd: acrobot_rollout.rollout_steps_seeded(st, th, sd, 0.1, 32, 500)),
        ("legged4", legged_n, 64, legged_horizon, 0.03, legged.Legged(4).reset,
         lambda st, pop: legged_rollout.rollout(st, pop, 64, legged_horizon, 4)[0],
         lambda st, th, sd: legged_rollout.rollout_seeded(st, th, sd, 0.03, 64, legged_horizon, 4)[0]),
    )
    out = {}
    for name, p, hidden, horizon, sigma, reset, roll, roll_seeded in cases:
        d = {"cartpole": 7 * hidden + 2, "acrobot": 10 * hidden + 3}.get(name) or legged_rollout.n_params(hidden, 4)
        g = torch.Generator(device=dev)
        g.manual_seed(0)
        theta = torch.randn(d, generator=g, device=dev) * 0.1
        state = reset(p, seed=0, device=dev)
        lr = 0.1

        def materialised():
            half = torch.randn((p // 2, d), generator=g, device=dev)
            eps = torch.cat([half, -half])
            fit = roll(state, theta[None, :] + sigma * eps)
            grad = (es.centered_ranks(fit)[:, None] * eps).sum(dim=0) / (p * sigma)
            return theta + lr * grad

        def seeded():
            fit = roll_seeded(state, theta, 7)
            return es_noise.update(theta, es.centered_ranks(fit), 7, sigma, lr)

        rec = {"P": p, "D": d, "hidden": hidden, "horizon": horizon}
        for label, fn in (("materialised", materialised), ("seeded", seeded)):
            fn()
            torch.cuda.synchronize()
            torch.cuda.reset_peak_memory_stats(dev)
            walls = []
            for _ in range(repeats):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                fn()
                torch.cuda.synchronize()
                walls.append(time.perf_counter() - t0)
            rec[label] = {"generation_ms": statistics.median(walls) * 1e3,
                          "peak_alloc_gib": torch.cuda.max_memory_allocated(dev) / 2**30}
        log(f"ES generation {name} P={p} D={d}: materialised {rec['materialised']['generation_ms']:.2f} ms "
            f"({rec['materialised']['peak_alloc_gib']:.2f} GiB), seeded {rec['seeded']['generation_ms']:.2f} ms "
            f"({rec['seeded']['peak_alloc_gib']:.2f} GiB)")
        out[name] = rec
        del state, theta
    return out


def bench_es_evaluate(dev, repeats):
    import torch

    from hipenvs import es

    out = {}
    # legged4_standing: small weights and head biases that pick each leg's zero-torque action,
    # a policy that stands for the whole evaluation as a trained one does (long episodes)
    for name, hidden in (("cartpole", 32), ("acrobot", 32), ("legged4", 64), ("legged4_standing", 64)):
        task = es.TASKS[name.replace("_standing", "")]
        g = torch.Generator(device=dev)
        g.manual_seed(1)
        theta = torch.randn(es.n_params(hidden, task), generator=g, device=dev) * 0.1
        if name.endswith("_standing"):
            c = 4
            obs, outs = 5 + 2 * c, 3 * c
            theta = theta * 0.2
            b2 = obs * hidden + hidden + hidden * outs
            theta[b2 + 1:b2 + outs:3] = 1.0
        rec = {"n": 2048, "steps": 500, "hidden": hidden}
        for label, fn in (("fused", lambda: es.evaluate_theta(task, theta, hidden, device=dev)),
                          ("loop", lambda: es.evaluate(task, es.mean_policy(theta, hidden, task), device=dev))):
            score = fn()
            walls = []
            for _ in range(repeats):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                fn()
                torch.cuda.synchronize()
                walls.append(time.perf_counter() - t0)
            rec[label] = {"ms": statistics.median(walls) * 1e3, "score": score}
        log(f"ES evaluate {name}: fused {rec['fused']['ms']:.2f} ms (score {rec['fused']['score']:.3f}), "
            f"loop {rec['loop']['ms']:.2f} ms (score {rec['loop']['score']:.3f})")
        out[name] = rec
    return out


def es_flops_per_step(task, hidden):
    """Algorithmic FP32 operations per step taken of the config-2 fused rollouts, counted from
    the kernel source as legged_flops_per_step counts (add, sub, mul, div = 1; selects,
    compares, floor and sign flips not counted; tanh, sin and cos counted separately).
    CartPole: per hidden unit 4 mul + 4 add and two heads' mul + add (12 H); physics 26
    (temp 5, angular acceleration 9, cart acceleration 4, Euler 8); plus H tanh and one
    sin/cos pair. Acrobot: per hidden unit 6 mul + 6 add and three heads' mul + add (18 H);
    RK4 of four derivative evaluations of 35 each, three stage inputs of 8, the combination
    28, two wraps of 4, and the termination's 2 (202); plus H tanh and 22 sin/cos."""
    return 12 * hidden + 26 if task == "cartpole" else 18 * hidden + 202


def bench_es_config2(dev, repeats):
    import torch

    from hipenvs import acrobot, acrobot_rollout, cartpole, cartpole_rollout

    out = {}
    for name, env, mod, d_of in (("cartpole", cartpole, cartpole_rollout, lambda h: 7 * h + 2),
                                 ("acrobot", acrobot, acrobot_rollout, lambda h: 10 * h + 3)):
        p, hidden, horizon = 4096, 32, 500
        g = torch.Generator(device=dev).manual_seed(0)
        theta0 = torch.randn(d_of(hidden), generator=g, device=dev) * 0.1
        half = torch.randn((p // 2, d_of(hidden)), generator=g, device=dev)
        theta = theta0[None, :] + 0.1 * torch.cat([half, -half])
        state = env.reset(p, seed=0, device=dev)
        mod.rollout_steps(state, theta, hidden, horizon)
        walls, survived = [], None
        for _ in range(repeats):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            survived = mod.rollout_steps(state, theta, hidden, horizon)
            torch.cuda.synchronize()
            walls.append(time.perf_counter() - t0)
        wall = statistics.median(walls)
        taken = float(torch.clamp(survived + 1, max=horizon).sum().item())
        flops = es_flops_per_step(name, hidden)
        achieved_tf = taken * flops / wall / 1e12
        out[name] = {"P": p, "hidden": hidden, "horizon": horizon, "rollout_s": wall,
                     "steps_taken_per_s": taken / wall, "p_x_horizon_per_s": p * horizon / wall,
                     "mean_steps_survived": float(survived.mean().item()), "flops_per_step_taken": flops,
                     "roofline": {"bound": "valu", "achieved": achieved_tf, "peak": FP32_PEAK_TFLOPS,
                                  "unit": "TFLOP/s", "frac": achieved_tf / FP32_PEAK_TFLOPS,
                                  "frac_of_unpacked_peak": achieved_tf / FP32_UNPACKED_TFLOPS, "traffic": None}}
        log(f"ES {name} P={p} H={hidden}: {taken / wall:,.0f} steps-taken/s, {p * horizon / wall:,.0f} PxH/s "
            f"({wall * 1e3:.2f} ms per rollout)")
    return out


def bench_aba(dev, steps=1000, n=65536, ks=(4, 16, 64)):
    import torch

    from hipenvs import _lib, pendulum_aba

    out = {}
    for k in ks:
        p = pendulum_aba.Pendulum(k)
        bufs = [p.reset(n, seed=0, device=dev, zero_velocity=True), torch.empty((2 * k, n), device=dev)]
        reward = torch.empty(n, device=dev)
        done = torch.empty(n, dtype=torch.bool, device=dev)
        fn = _lib.lib().hipenvs_pendulum_aba_step_euler
        P = _lib.ptr

        def body(s):
            for t in range(steps):
                rc = fn(k, P(bufs[t % 2]), P(None), t + 1, P(bufs[(t + 1) % 2]), P(reward), P(done), n, s)
                if rc != 0:
                    raise RuntimeError(f"aba step failed: {rc}")

        g = capture_graph(dev, body)
        wall, ev = time_replay(g, 3)
        launch = ev / steps
        bytes_step = 16 * k + 5  # 2K floats in and out, reward, done; the torque is drawn in the kernel
        achieved = bytes_step * n / launch / 1e9
        out[str(k)] = {"n_envs": n, "steps": steps, "env_steps_per_s": n * steps / wall, "us_per_launch": launch * 1e6,
                       "bytes_per_env_step": bytes_step,
                       "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                    "frac": achieved / HBM_PEAK_GBS, "traffic": ABA_TRAFFIC.get(k)}}
        log(f"ABA Euler K={k} N={n}: {n * steps / wall:,.0f} env-steps/s, {launch * 1e6:.2f} us per launch, "
            f"{achieved:.0f} GB/s algorithmic")
        del g, bufs
    return out


def bench_aba_rk4(dev, steps=64, n=65536, ks=(4, 16, 32, 64), region_seconds=0.1):
    """The reference's own ABA benchmark (bench_aba.py:26-37 through bench.py:48-61): the RK4
    drop-in step (dt 0.02, torque (a - 1) for a in {0, 1, 2}) at N = 65,536 from the reset
    distribution (all 2K rows U[+-0.1]), every iteration drawing its actions on the device and
    stepping, every reward and done kept; `steps` iterations per HIP graph, replayed back to back.
    Also the step alone on actions drawn before the clock (HIP events on the replay stream),
    with its HBM roofline at 16K + 9 algorithmic bytes per env-step."""
    import torch

    from hipenvs import _lib, cartpole, pendulum_aba

    P = _lib.ptr
    fn = _lib.lib().hipenvs_pendulum_aba_step
    sampler = _lib.lib().hipenvs_sample_actions
    out = {}
    for k in ks:
        body_ = pendulum_aba.Pendulum(k)
        bufs = [body_.reset(n, seed=0, device=dev), torch.empty((2 * k, n), device=dev)]
        rewards = torch.empty((steps, n), device=dev)
        dones = torch.empty((steps, n), dtype=torch.bool, device=dev)
        row = torch.empty(n, dtype=torch.int32, device=dev)
        actions = torch.empty((steps, n), dtype=torch.int32, device=dev)
        for t in range(steps):
            cartpole.sample_actions(n, m=3, seed=1 + t, device=dev, out=actions[t])

        def sampled(s):
            for t in range(steps):
                rc = sampler(P(row), n, 3, 1 + t, s)
                if rc != 0:
                    raise RuntimeError(f"hipenvs_sample_actions failed: {rc}")
                rc = fn(k, P(bufs[t % 2]), P(row), t + 1, P(bufs[(t + 1) % 2]), P(rewards[t]), P(dones[t]), n, s)
                if rc != 0:
                    raise RuntimeError(f"aba rk4 step failed: {rc}")

        def alone(s):
            for t in range(steps):
                rc = fn(k, P(bufs[t % 2]), P(actions[t]), t + 1, P(bufs[(t + 1) % 2]), P(rewards[t]), P(dones[t]), n,
                        s)
                if rc != 0:
                    raise RuntimeError(f"aba rk4 step failed: {rc}")

        g = capture_graph(dev, sampled)
        per_region = replays_for(g, region_seconds)
        wall, _ = time_replay(g, 3, per_region)
        its = steps * per_region
        ga = capture_graph(dev, alone)
        _, ev = time_replay(ga, 3, per_region)
        launch = ev / its
        bytes_step = 16 * k + 9  # 2K floats in and out, action, reward, done
        achieved = bytes_step * n / launch / 1e9
        out[str(k)] = {"n_envs": n, "steps_per_graph": steps, "replays_per_region": per_region,
                       "env_steps_per_s": n * its / wall, "us_per_iteration": wall / its * 1e6,
                       "step_alone_us_per_launch": launch * 1e6, "bytes_per_env_step": bytes_step,
                       "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                    "frac": achieved / HBM_PEAK_GBS, "traffic": ABA_RK4_TRAFFIC.get(k)},
                       "reference_m3pro_env_steps_per_s": ABA_RK4_REFERENCE.get(k)}
        log(f"ABA RK4 K={k} N={n}: {n * its / wall:,.0f} env-steps/s (sampler + step), step alone "
            f"{launch * 1e6:.2f} us per launch, {achieved:.0f} GB/s algorithmic")
        del g, ga, bufs, rewards, dones, actions
    return out


# The reference's legged step (its chained kernel, eval every 32) at N = 65,536 on its M3 Pro
# by Gauss-Seidel sweeps, README.md:1605-1612.
LEGGED_STEP_REFERENCE = {2: {1: 148587531, 2: 130199428, 4: 130241539, 8: 112607332, 16: 85876189, 32: 58376177},
                         4: {1: 27656704, 2: 27492110, 4: 26196758, 8: 24300548, 16: 21181268, 32: 17752265}}


def bench_legged_step_sweep(dev, steps=200, n=65536, region_seconds=0.05):
    """The reference's price list of the legged step by sweeps (README.md:1605-1612): the
    float32 step at C = 2 and 4, S = 1/2/4/8/16/32, N = 65,536 from the stand reset, every
    iteration drawing uniform actions in [0, 3^C) on the device and stepping, `steps`
    iterations per HIP graph replayed back to back."""
    import torch

    from hipenvs import _lib, legged

    P = _lib.ptr
    fn = _lib.lib().hipenvs_legged_step
    sampler = _lib.lib().hipenvs_sample_actions
    out = {}
    for c in (2, 4):
        body_ = legged.Legged(c, 8)
        rows = 2 * (3 + c)
        stand = body_.stand_on(dev)
        reward = torch.empty(n, device=dev)
        done = torch.empty(n, dtype=torch.bool, device=dev)
        row = torch.empty(n, dtype=torch.int32, device=dev)
        for s_ in (1, 2, 4, 8, 16, 32):
            bufs = [body_.reset(n, seed=0, device=dev), torch.empty((rows, n), device=dev)]

            def sampled(st, s_=s_, bufs=bufs):
                for t in range(steps):
                    rc = sampler(P(row), n, 3 ** c, 1 + t, st)
                    if rc != 0:
                        raise RuntimeError(f"hipenvs_sample_actions failed: {rc}")
                    rc = fn(c, s_, 0.0, P(bufs[t % 2]), P(row), t + 1, P(stand), P(bufs[(t + 1) % 2]), P(reward),
                            P(done), n, st)
                    if rc != 0:
                        raise RuntimeError(f"legged step failed: {rc}")

            g = capture_graph(dev, sampled)
            per_region = replays_for(g, region_seconds)
            wall, ev = time_replay(g, 3, per_region)
            its = steps * per_region
            rate = n * its / wall
            ref = LEGGED_STEP_REFERENCE[c][s_]
            out[f"c{c}_s{s_}"] = {"n_envs": n, "env_steps_per_s": rate, "us_per_iteration": wall / its * 1e6,
                                  "reference_m3pro_env_steps_per_s": ref}
            log(f"legged C={c} step S={s_} N={n}: {rate:,.0f} env-steps/s (sampler + step, "
                f"{wall / its * 1e6:.2f} us per iteration); reference M3 Pro {ref:,}")
            del g, bufs
    return out


def bench_step_bodies(dev, steps=1000, n=65536, ks=(2, 4, 8, 16)):
    """The reference's remaining step modules: the mass-matrix K-link pendulum (RK4, actions
    drawn per step on the device) and the hopper, graph-replayed like the ABA step."""
    import torch

    from hipenvs import _lib, acrobot, cartpole, hopper, legged, pendulum

    P = _lib.ptr
    out = {}
    cases = [(f"pendulum_k{k}", 2 * k, 16 * k + 9, k, n) for k in ks] + [("hopper", 8, 73, "hopper", n),
                                                                         ("acrobot", 4, 41, "acrobot", 262144),
                                                                         ("legged4_s8", 14, 121, "legged", n),
                                                                         ("legged4_s8_reference", 14, 233,
                                                                          "legged_ref", n)]
    for name, rows, bytes_step, k, n in cases:
        if k == "hopper":
            bufs = [hopper.Hopper().reset(n, seed=0, device=dev), torch.empty((rows, n), device=dev)]
            fn = _lib.lib().hipenvs_hopper_step
            call = lambda t, s, a: fn(P(bufs[t % 2]), P(a), t + 1, P(bufs[(t + 1) % 2]), P(reward), P(done), n, s)
        elif k == "acrobot":
            bufs = [acrobot.reset(n, seed=0, device=dev), torch.empty((rows, n), device=dev)]
            fn = _lib.lib().hipenvs_acrobot_step
            call = lambda t, s, a: fn(P(bufs[t % 2]), P(a), t + 1, P(bufs[(t + 1) % 2]), P(reward), P(done), n, s)
        elif k == "legged":
            body = legged.Legged(4, 8)
            bufs = [body.reset(n, seed=0, device=dev), torch.empty((rows, n), device=dev)]
            stand = body.stand_on(dev)
            fn = _lib.lib().hipenvs_legged_step
            call = lambda t, s, a: fn(4, 8, 0.0, P(bufs[t % 2]), P(a), t + 1, P(stand), P(bufs[(t + 1) % 2]), P(reward),
                                      P(done), n, s)
        elif k == "legged_ref":
            # the reference's precision: float64 state in and out (legged_np's dtype after its first step)
            body = legged.Legged(4, 8)
            bufs = [body.reset(n, seed=0, device=dev).double(), torch.empty((rows, n), dtype=torch.float64, device=dev)]
            stand = body.stand_on(dev)
            fn = _lib.lib().hipenvs_legged_step_reference
            call = lambda t, s, a: fn(4, 8, 0.0, P(bufs[t % 2]), 1, P(a), t + 1, P(stand), P(bufs[(t + 1) % 2]),
                                      P(reward), P(done), n, s)
        else:
            bufs = [pendulum.Pendulum(k).reset(n, seed=0, device=dev), torch.empty((rows, n), device=dev)]
            fn = _lib.lib().hipenvs_pendulum_step
            call = lambda t, s, a, k=k: fn(k, P(bufs[t % 2]), P(a), t + 1, P(bufs[(t + 1) % 2]), P(reward), P(done),
                                           n, s)
        reward = torch.empty(n, device=dev)
        done = torch.empty(n, dtype=torch.bool, device=dev)
        actions = torch.empty((steps, n), dtype=torch.int32, device=dev)
        n_actions = 81 if k in ("legged", "legged_ref") else 3
        for t in range(steps):
            cartpole.sample_actions(n, m=n_actions, seed=1 + t, device=dev, out=actions[t])

        def body(s):
            for t in range(steps):
                rc = call(t, s, actions[t])
                if rc != 0:
                    raise RuntimeError(f"{name} step failed: {rc}")

        g = capture_graph(dev, body)
        wall, ev = time_replay(g, 3)
        launch = ev / steps
        achieved = bytes_step * n / launch / 1e9
        out[name] = {"n_envs": n, "steps": steps, "env_steps_per_s": n * steps / wall, "us_per_launch": launch * 1e6,
                     "bytes_per_env_step": bytes_step,
                     "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                  "frac": achieved / HBM_PEAK_GBS, "traffic": STEP_BODY_TRAFFIC.get(name)}}
        log(f"{name} step N={n}: {n * steps / wall:,.0f} env-steps/s, {launch * 1e6:.2f} us per launch")
        del g, bufs, actions
    return out


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported: the hot path has no "
              f"cross-GPU work (every environment and member is independent)", file=sys.stderr)
        sys.exit(2)
    import torch

    from hipenvs import _lib

    dev = torch.device("cuda", 0)
    log(f"hipenvs: {_lib.version()} on {torch.cuda.get_device_name(dev)}; host os.cpu_count()={os.cpu_count()}")
    extra = {}
    if args.copy_mib:
        src = torch.ones(args.copy_mib << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"calibration copy: {args.copy_mib} MiB x 3")
        del src, dst
    head = None
    if args.only in (None, "cartpole"):
        head = bench_cartpole(args, dev)
        extra["cartpole_step_kernel_only"] = head["kernel_only"]
        extra["cartpole_fused_k32"] = head["fused"]
        extra["cartpole_module_api"] = module_api_rate(args.n, min(args.steps, 1000), dev)
        if args.n != 1 << 20:
            extra["cartpole_step_n1048576"] = bench_cartpole_at(1 << 20, args.steps, args.repeats, dev)
        extra["cartpole_step_n16777216"] = bench_cartpole_at(1 << 24, 64, args.repeats, dev)
        extra["cartpole_copy_floor"] = [copy_floor(m, args.steps, args.repeats, dev) for m in (args.n, 1 << 20)]
        # config 1: the full sweep with --sweep; a bounded one (64 iterations per graph, regions of
        # about 20 ms, 0.05 s of numpy per N) in the default run
        if args.sweep:
            extra["cartpole_sweep"] = sweep(dev, args.steps, args.fused_k, args.sweep_out,
                                            0.0 if args.skip_cpu else 0.25)
        elif args.only is None:
            extra["cartpole_sweep"] = sweep(dev, 64, args.fused_k, args.sweep_out, 0.0 if args.skip_cpu else 0.05,
                                            region_seconds=0.02)
    if args.only in (None, "legged"):
        for c in (4, 2):
            legged = bench_legged(args, dev, c)
            if not args.skip_cpu:
                rate, csteps = cpu_baseline_legged(args.legged_n, args.legged_cpu_seconds, c=c)
                legged["cpu_baseline"] = {
                    "value": rate, "unit": "env-steps/s", "cores": 1, "kind": "port",
                    "sample": f"numpy ES step (einsum policy + legged step in the reference's literal arithmetic), "
                              f"N={args.legged_n}, C={c}, H=64, S=8, {csteps} timed steps after 1 warm-up"}
                legged["speedup_vs_cpu_s8"] = legged["by_sweeps"]["8"]["env_steps_per_s"] / rate
                log(f"legged{c} numpy baseline: {rate:,.0f} env-steps/s -> GPU/CPU "
                    f"{legged['speedup_vs_cpu_s8']:,.0f}x")
            extra[f"legged{c}_es_rollout"] = legged
    if args.only in ("aba", "steps"):
        extra["aba_euler"] = bench_aba(dev)
        extra["aba_rk4"] = bench_aba_rk4(dev)
        if args.only == "steps":
            extra["step_bodies"] = bench_step_bodies(dev)
            extra["legged_step_sweeps"] = bench_legged_step_sweep(dev)
        print(json.dumps(extra), flush=True)
        return
    if args.only == "generation":
        extra["es_generation"] = bench_es_generation(dev, args.repeats, args.legged_n, args.legged_horizon)
        print(json.dumps(extra), flush=True)
        return
    if args.only is None:
        extra["es_config2"] = bench_es_config2(dev, args.repeats)
        if not args.skip_cpu:
            for task in ("cartpole", "acrobot"):
                rate, its = cpu_baseline_es(task, 2.0)
                rec = extra["es_config2"][task]
                rec["cpu_baseline"] = {"value": rate, "unit": "member-steps/s", "cores": 1, "kind": "port",
                                       "sample": f"numpy ES loop (einsum policy + numpy {task} step over all 4,096 "
                                                 f"members per iteration, es.py:174-193), {its} iterations"}
                rec["speedup_p_x_horizon_vs_cpu"] = rec["p_x_horizon_per_s"] / rate
                log(f"ES {task} numpy loop: {rate:,.0f} member-steps/s -> GPU P x H rate "
                    f"{rec['speedup_p_x_horizon_vs_cpu']:,.0f}x")
        extra["es_generation"] = bench_es_generation(dev, args.repeats, args.legged_n, args.legged_horizon)
        extra["es_evaluate"] = bench_es_evaluate(dev, args.repeats)
        extra["aba_euler"] = bench_aba(dev)
        if not args.skip_cpu:
            for k, rec in extra["aba_euler"].items():
                rate, its = cpu_baseline_aba(int(k), 1.5)
                rec["cpu_baseline"] = {"value": rate, "unit": "env-steps/s", "cores": 1, "kind": "port",
                                       "sample": f"numpy ABA Euler step (np.sin/np.cos) at N=65,536, K={k}, "
                                                 f"{its} steps"}
                rec["speedup_vs_cpu"] = rec["env_steps_per_s"] / rate
                log(f"ABA K={k} numpy: {rate:,.0f} env-steps/s -> GPU {rec['speedup_vs_cpu']:,.0f}x")
        extra["aba_rk4"] = bench_aba_rk4(dev)
        extra["step_bodies"] = bench_step_bodies(dev)
        extra["legged_step_sweeps"] = bench_legged_step_sweep(dev)

    cpu = None
    if not args.skip_cpu and args.only in (None, "cartpole"):
        rate, csteps = cpu_baseline_cartpole(args.n, args.cpu_seconds)
        cpu = {"value": rate, "unit": "env-steps/s", "cores": 1, "kind": "port",
               "sample": f"numpy CartPole step (reference op order, np.sin/np.cos), N={args.n}, {csteps} steps, "
                         f"single process on a host with os.cpu_count()={os.cpu_count()}"}
        log(f"cartpole numpy baseline: {rate:,.0f} env-steps/s over {csteps} steps")

    if head is None:  # --only legged: the legged rollout is the line
        rec = extra["legged4_es_rollout"]["by_sweeps"]["8"]
        value, wall = rec["env_steps_per_s"], rec["wall_s"]
        roofline = rec["roofline"]
        cpu = extra["legged4_es_rollout"].get("cpu_baseline")
        config = {"workload": f"legged4 ES rollout (the drop-in call on (P, D) rows), N={args.legged_n}, H=64, S=8, "
                              f"horizon {args.legged_horizon}",
                  "n_envs": args.legged_n}
        ms = wall * 1e3
        steps = args.legged_horizon
    else:
        value = head["value"]
        roofline = cartpole_roofline(args.n, head["kernel_only"])
        config = {"workload": f"cartpole: device action sampler + cartpole_step per iteration, N={args.n}, "
                              f"{args.steps} iterations per HIP graph, {head['per_region']} graph replays per timed "
                              f"region, every reward and done row kept",
                  "n_envs": args.n, "repeats_per_region": head["per_region"], "timed_regions": args.repeats,
                  "parallelism": "single GPU, one thread per env"}
        ms = head["wall"] * 1e3 / head["iterations"]
        steps = args.steps
    line = {
        "metric": METRIC, "value": value, "unit": "env-steps/s", "n_gpus": 1, "steps": steps, "warmup": args.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32", "data": "synthetic (counter-RNG states and actions, seeded Gaussian ES populations)",
        "config": config, "roofline": roofline, "cpu_baseline": cpu, "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
