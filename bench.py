"""Benchmark of the hipenvs hot path on one MI355X; prints ONE JSON line.

Headline workload: the batched CartPole step at N = 2**18 environments, the
reference's step kernel API (one launch per env step, cartpole_metal.step),
over `--steps` steps (default 1,000) after `--warmup` untimed steps. The launches
of the timed steps are captured once into a HIP graph (outside the clock) and
replayed, so the clock measures the kernels, not Python. Inputs (state, the
pre-drawn Bernoulli(0.5) actions of every step) are resident in HBM before the
clock starts; every step's reward and done rows are written to a (steps, N)
rollout buffer, as the reference's harness materialises them (bench.py:48-61).

Timing rule (the reference's, bench.py:75-82 / README:135-172): env-steps/s =
N x timed steps / wall seconds, device synchronised before and after the timed
region, median of `--repeats` repeats.

Roofline: `achieved` = 41 algorithmic bytes per env-step x N / the average
launch duration, which is the HIP-event time of the timed replay (events on the
replay's stream) divided by the launches in it. Also measured in the same run
and reported under "extra": the K = 32 fused kernel (in-kernel and array
actions).

`cpu_baseline`: the CPU oracle's numpy CartPole step (the reference's
algorithm, np.sin/np.cos, single process) on the same N for a bounded sample
of about `--cpu-seconds` seconds on this host.

Usage: python bench.py [--gpus 1] [--steps 1000] [--warmup 16] [--sweep]
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
CARTPOLE_BYTES = 41  # 16 B state in + 4 B action + 16 B state out + 4 B reward + 1 B done


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def parse_args():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=1000)
    p.add_argument("--warmup", type=int, default=16)
    p.add_argument("--n", type=int, default=1 << 18)
    p.add_argument("--repeats", type=int, default=3)
    p.add_argument("--fused-k", type=int, default=32)
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--skip-cpu", action="store_true")
    p.add_argument("--sweep", action="store_true", help="also run the N = 2^0..2^24 sweep (to stderr and --sweep-out)")
    p.add_argument("--sweep-out", default=None)
    return p.parse_args()


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

    def capture(self, body):
        """A HIP graph of the launches `body(stream)` enqueues."""
        torch = self.torch
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream(device=self.dev)
        side.wait_stream(torch.cuda.current_stream(self.dev))
        with torch.cuda.stream(side):
            with torch.cuda.graph(g, stream=side):
                body(self.lib.stream_of(self.dev))
        torch.cuda.synchronize()
        return g

    def graph_single(self):
        return self.capture(lambda s: [self.launch_step(t, s) for t in range(self.steps)])

    def graph_fused(self, k, array_actions):
        def body(s):
            t = 0
            while t < self.steps:
                kk = min(k, self.steps - t)
                self.launch_fused(t, kk, s, array_actions)
                t += kk
        return self.capture(body)

    def time_graph(self, g, repeats):
        """Median wall seconds of a replay, and the HIP-event time of the same replays."""
        torch = self.torch
        g.replay()
        torch.cuda.synchronize()
        walls, events = [], []
        for _ in range(repeats):
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            start.record()
            g.replay()
            end.record()
            torch.cuda.synchronize()
            walls.append(time.perf_counter() - t0)
            events.append(start.elapsed_time(end) / 1e3)
        return statistics.median(walls), statistics.median(events)


def cpu_baseline_cartpole(n, seconds):
    """numpy CartPole step (reference algorithm, np.sin/np.cos) on one process; env-steps/s."""
    import numpy as np

    from oracle import cartpole as oc
    from oracle import rng

    state = oc.reset(n, seed=0)
    actions = [rng.action_bits(t, n) for t in range(1, 9)]
    for t in range(2):  # warm-up
        state, _, _ = oc.step(state, actions[t], seed=t + 1, trig="numpy")
    steps, t0 = 0, time.perf_counter()
    while True:
        state, _, _ = oc.step(state, actions[steps % 8], seed=steps + 3, trig="numpy")
        steps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return n * steps / el, steps


def sweep(dev, steps, k, out_path):
    rows = []
    for e in list(range(0, 21)) + [22, 24]:
        n = 1 << e
        steps = steps if n <= (1 << 20) else 128  # keep the (steps, N) action and reward buffers a few GB
        run = CartPoleRun(n, steps, dev)
        g1 = run.graph_single()
        w1, ev1 = run.time_graph(g1, 3)
        gk = run.graph_fused(k, False)
        wk, _ = run.time_graph(gk, 3)
        gka = run.graph_fused(k, True)
        wka, _ = run.time_graph(gka, 3)
        launch = ev1 / steps
        row = dict(n=n, single=n * steps / w1, fused_inkernel=n * steps / wk, fused_array=n * steps / wka,
                   launch_us=launch * 1e6, single_gbs=CARTPOLE_BYTES * n / launch / 1e9)
        rows.append(row)
        log(f"N=2^{e:<2d} single {row['single']:>16,.0f}  fused(in-kernel) {row['fused_inkernel']:>16,.0f}  "
            f"fused(array) {row['fused_array']:>16,.0f} env-steps/s  launch {row['launch_us']:7.2f} us "
            f"{row['single_gbs']:8.1f} GB/s")
        del run, g1, gk, gka
    if out_path:
        Path(out_path).write_text(json.dumps(rows, indent=1))
    return rows


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported (the hot path has no "
              f"cross-GPU work; see the sharding note in the design document)", file=sys.stderr)
        sys.exit(2)
    import torch

    from hipenvs import _lib

    dev = torch.device("cuda", 0)
    n, steps, warmup = args.n, args.steps, args.warmup
    log(f"hipenvs: {_lib.version()} on {torch.cuda.get_device_name(dev)}; N={n} steps={steps} warmup={warmup}")

    run_t = CartPoleRun(n, steps, dev)
    stream = _lib.stream_of(dev)
    for t in range(warmup):  # untimed eager steps: module load, clocks, caches
        run_t.launch_step(t % steps, stream)
    torch.cuda.synchronize()
    g = run_t.graph_single()
    wall, ev = run_t.time_graph(g, args.repeats)
    value = n * steps / wall
    log(f"single-step kernel, graph replay: {value:,.0f} env-steps/s ({wall * 1e3:.3f} ms for {steps} steps)")
    launch = ev / steps  # average launch duration: HIP events around the timed replay, on its stream
    achieved = CARTPOLE_BYTES * n / launch / 1e9
    log(f"cartpole_step: {launch * 1e6:.3f} us per launch (HIP events over the timed region) "
        f"-> {achieved:.1f} GB/s algorithmic")
    gk = run_t.graph_fused(args.fused_k, False)
    wk, _ = run_t.time_graph(gk, args.repeats)
    gka = run_t.graph_fused(args.fused_k, True)
    wka, _ = run_t.time_graph(gka, args.repeats)
    log(f"fused K={args.fused_k}: in-kernel actions {n * steps / wk:,.0f}, array actions {n * steps / wka:,.0f} env-steps/s")

    extra = {
        "single_step_timed_region_event_s": ev,
        "cartpole_step_us_per_launch": launch * 1e6,
        f"fused_k{args.fused_k}_inkernel_actions_env_steps_per_s": n * steps / wk,
        f"fused_k{args.fused_k}_array_actions_env_steps_per_s": n * steps / wka,
        f"fused_k{args.fused_k}_array_actions_algorithmic_gbs": (32 / args.fused_k + 9) * n * steps / wka / 1e9,
    }
    if args.sweep:
        extra["sweep"] = sweep(dev, steps, args.fused_k, args.sweep_out)

    cpu = None
    if not args.skip_cpu:
        rate, csteps = cpu_baseline_cartpole(n, args.cpu_seconds)
        cpu = {"value": rate, "unit": "env-steps/s", "cores": 1, "kind": "port",
               "sample": f"numpy CartPole step (reference op order, np.sin/np.cos), N={n}, {csteps} steps, "
                         f"single process on a host with os.cpu_count()={os.cpu_count()}"}
        log(f"cpu baseline: {rate:,.0f} env-steps/s over {csteps} steps")

    line = {
        "metric": METRIC, "value": value, "unit": "env-steps/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": wall * 1e3 / steps, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32", "data": "synthetic (counter-RNG states and Bernoulli(0.5) actions)",
        "config": {"workload": f"cartpole_step, N={n}, {steps} steps, one launch per step (HIP graph replay)",
                   "n_envs": n, "parallelism": "single GPU, one thread per 4 envs"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
