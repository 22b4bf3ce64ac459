"""Build libhipenvs.so for gfx950 in-tree with hipcc.

Usage: python metal-rl-envs_amd/build.py [--jobs N] [--verbose]

Every .hip file under csrc/ is compiled to an object with the flags below and
the objects are linked into hipenvs/libhipenvs.so. The flags are part of the
library's contract:

* ``-ffp-contract=off``: no multiply-add fusion, so each ``a * b + c`` rounds
  twice exactly as numpy does; the kernels reproduce the reference's float32
  arithmetic bit for bit.
* no fast-math: IEEE division and square root (HIP's default correctly rounded
  fp32 divide and sqrt), denormals kept.
* ``-Xclang -target-feature -Xclang -packed-fp32-ops``: no packed FP32
  (v_pk_*_f32) instructions are emitted.
"""

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OUT_DIR = HERE / "hipenvs"
LIB_NAME = "libhipenvs.so"
BUILD_DIR = HERE / "_build"

ARCH = "gfx950"
COMMON_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP library cannot be built")


def compile_one(src, verbose):
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stdout}\n{r.stderr}")
    warn = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip())
    if warn and verbose:
        print(warn, file=sys.stderr)
    return obj


def build(jobs=None, verbose=False):
    """Compile every csrc/*.hip and link hipenvs/libhipenvs.so; returns the library path."""
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    jobs = jobs or min(8, os.cpu_count() or 1)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: compile_one(s, verbose), sources))
    lib = OUT_DIR / LIB_NAME
    tmp = OUT_DIR / (LIB_NAME + ".tmp")
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, lib)
    return lib


def main():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--jobs", type=int, default=None)
    p.add_argument("--verbose", action="store_true")
    a = p.parse_args()
    print(build(a.jobs, a.verbose))


if __name__ == "__main__":
    main()
