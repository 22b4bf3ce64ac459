"""bench.py's command line on the CPU: --gpus above 1 exits with a message before any GPU
or torch work (one GPU is the whole measurement)."""

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_exits_with_a_message():
    for n in ("2", "8"):
        r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", n], capture_output=True, text=True,
                           timeout=60, cwd=ROOT)
        assert r.returncode == 2, r.stderr
        assert "one GPU only" in r.stderr and f"--gpus {n}" in r.stderr
        assert r.stdout == ""  # no JSON line
