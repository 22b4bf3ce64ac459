"""The measured constants bench.py reports (kernel-trace durations and counter traffic) are
the figures tabulated in profiles/, so every roofline field of the bench line can be
recomputed from a committed profile."""

import ast
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def bench_constants():
    """Literal dict constants at bench.py's top level, without importing it (no torch)."""
    tree = ast.parse((ROOT / "bench.py").read_text())
    out = {}
    for node in tree.body:
        if isinstance(node, ast.Assign) and len(node.targets) == 1 and isinstance(node.targets[0], ast.Name):
            name = node.targets[0].id
            if name.endswith("_TRACE_NS") or name.endswith("_TRAFFIC"):
                out[name] = eval(compile(ast.Expression(node.value), "bench.py", "eval"))  # literals and shifts only
    return out


def numbers(text):
    """Every number in a profile, thousands separators dropped, exponent forms kept."""
    return {float(m.replace(",", "")) for m in re.findall(r"\d[\d,]*\.?\d*(?:e[+-]?\d+)?", text)}


def profile(name):
    return (ROOT / "profiles" / name).read_text()


def test_cartpole_trace_and_traffic_are_tabulated():
    c = bench_constants()
    text = numbers(profile("cartpole_step_n262144.md"))
    for ns in c["CARTPOLE_TRACE_NS"].values():
        assert ns in text, ns
    for b in c["CARTPOLE_TRAFFIC"].values():
        assert float(b) in text, b


def test_aba_and_step_body_traffic_are_tabulated():
    c = bench_constants()
    aba = numbers(profile("aba_euler_n65536.md"))
    for b in c["ABA_TRAFFIC"].values():
        assert float(b) in aba, b
    rk4 = numbers(profile("aba_rk4_n65536.md"))
    for b in c["ABA_RK4_TRAFFIC"].values():
        assert float(b) in rk4, b
    bodies = numbers(profile("step_bodies_and_evaluate.md"))
    for name, b in c["STEP_BODY_TRAFFIC"].items():
        assert float(b) in bodies, (name, b)


def test_legged_rollout_traffic_is_tabulated():
    c = bench_constants()
    text = profile("legged_es_rollout_n262144.md")
    # the table gives bytes per rollout to five significant figures, e.g. 1.2569e11
    tabulated = {float(m) for m in re.findall(r"\d\.\d{4}e1\d", text)}
    for key, b in c["LEGGED_ROLLOUT_TRAFFIC"].items():
        assert float(f"{b:.4e}") in tabulated, (key, b)


def test_cartpole_trace_matches_the_kernel_sources():
    """CARTPOLE_TRACE_NS describes the build whose sources hash to CARTPOLE_TRACE_SOURCE_SHA;
    a change to the CartPole kernel or the shared device header fails here until the kernel is
    traced again (bench.py meanwhile reports its HIP-event figure as `frac`)."""
    import hashlib

    tree = ast.parse((ROOT / "bench.py").read_text())
    consts = {}
    for node in tree.body:
        if isinstance(node, ast.Assign) and len(node.targets) == 1 and isinstance(node.targets[0], ast.Name):
            if node.targets[0].id in ("CARTPOLE_TRACE_SOURCE_SHA", "CARTPOLE_TRACE_SOURCES"):
                consts[node.targets[0].id] = ast.literal_eval(node.value)
    h = hashlib.sha256()
    for rel in consts["CARTPOLE_TRACE_SOURCES"]:
        h.update((ROOT / rel).read_bytes())
    assert h.hexdigest()[:16] == consts["CARTPOLE_TRACE_SOURCE_SHA"]
    assert consts["CARTPOLE_TRACE_SOURCE_SHA"] in profile("cartpole_step_n262144.md")
