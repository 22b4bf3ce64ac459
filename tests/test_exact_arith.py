"""Exactness of the kernels' arithmetic shortcuts, proved on the CPU.

* ``div_const(x, 1 / (double)c)`` (``hipenvs_device.h``) replaces the IEEE float32
  division ``x / c`` by a float32 constant ``c`` (CartPole's ``/ total_mass``,
  cartpole_np.py:65-72; the angle wrap's ``/ (2 pi)``, acrobot_np.py:64). Every divisor
  the kernels pass to it is checked against IEEE division over all 2^32 float32 inputs
  by a small C program (``tests/csrc/div_const_check.c``), so the substitution cannot
  change a bit of any kernel output.
* ``DivRecip`` (``hipenvs_device.h``) divides by a divisor used many times (the legged
  body's Cholesky pivots, Delassus determinants and cone denominators) through its float64
  reciprocal, and marks nonzero subnormal quotients for an IEEE redo;
  ``tests/csrc/div_recip_check.c`` checks the marking key over all 2^32 bit patterns, the
  quotient against IEEE division on random, special and near-midpoint operand pairs, and
  that the exact subnormal midpoints it gets wrong are all marked.
* ``uniform_pm`` evaluates ``((h >> 8) * 2^-24 * 2 - 1) * bound``
  (cartpole_metal.py:47-50) as ``((h >> 8) - 2^23) * (bound * 2^-23)``; checked here
  for all 2^24 values of ``h >> 8`` against the literal float32 expression.
"""

import re
import shutil
import subprocess

import numpy as np
import pytest

from conftest import PKG, ROOT

CSRC = PKG / "csrc"
HEX_FLOAT = r"(-?0x[0-9a-fA-F.]+p[+-]?\d+)f"


def div_const_divisors():
    """{INV_name: hex literal of c} for every `constexpr double INV_X = 1.0 / (double)X;`."""
    found = {}
    for src in sorted(CSRC.glob("*.hip")):
        text = src.read_text()
        for inv, name in re.findall(r"constexpr double (INV_\w+) = 1\.0 / \(double\)(\w+);", text):
            m = re.search(rf"constexpr float {name} = {HEX_FLOAT};", text)
            assert m, f"{src.name}: {name} has no float32 hex literal"
            found.setdefault(inv, set()).add(m.group(1))
    return found


def test_every_div_const_divisor_is_declared():
    """Every div_const call names an INV_ constant whose divisor the exhaustive test covers."""
    declared = div_const_divisors()
    assert {"INV_TOTAL_MASS", "INV_TWO_PI"} <= set(declared)
    for src in sorted(CSRC.glob("*.hip")):
        for arg in re.findall(r"div_const\([^;]*?,\s*(\w+)\)", src.read_text()):
            assert arg in declared, f"{src.name}: div_const with unchecked divisor {arg}"


@pytest.fixture(scope="module")
def div_check_bin(tmp_path_factory):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    exe = tmp_path_factory.mktemp("divchk") / "div_const_check"
    subprocess.run([gcc, "-O2", "-fopenmp", "-ffp-contract=off", "-o", str(exe),
                    str(ROOT / "tests" / "csrc" / "div_const_check.c"), "-lm"], check=True)
    return exe


@pytest.mark.parametrize("literal", sorted({v for vs in div_const_divisors().values() for v in vs}))
def test_div_const_equals_ieee_division_for_all_floats(div_check_bin, literal):
    out = subprocess.run([str(div_check_bin), literal], capture_output=True, text=True, timeout=600)
    assert out.returncode == 0 and "mismatches=0" in out.stdout, out.stdout + out.stderr


def test_div_const_check_catches_a_wrong_reciprocal(tmp_path):
    """The exhaustive check is not vacuous: a float32 reciprocal (one extra rounding) fails it."""
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    src = (ROOT / "tests" / "csrc" / "div_const_check.c").read_text()
    planted = src.replace("const double inv_c = 1.0 / (double)c;", "const double inv_c = (float)(1.0 / (double)c);")
    assert planted != src
    (tmp_path / "planted.c").write_text(planted)
    exe = tmp_path / "planted"
    subprocess.run([gcc, "-O2", "-fopenmp", "-ffp-contract=off", "-o", str(exe), str(tmp_path / "planted.c"), "-lm"],
                   check=True)
    out = subprocess.run([str(exe), "0x1.19999ap+0"], capture_output=True, text=True, timeout=600)
    assert out.returncode == 1 and "mismatches=0" not in out.stdout


def _build(tmp_path, source_text, name):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    src = tmp_path / f"{name}.c"
    src.write_text(source_text)
    exe = tmp_path / name
    subprocess.run([gcc, "-O2", "-fopenmp", "-ffp-contract=off", "-o", str(exe), str(src), "-lm"], check=True)
    return exe


DIV_RECIP_SRC = ROOT / "tests" / "csrc" / "div_recip_check.c"


def test_div_recip_matches_ieee_except_marked_subnormals(tmp_path):
    exe = _build(tmp_path, DIV_RECIP_SRC.read_text(), "div_recip_check")
    out = subprocess.run([str(exe), "20000000"], capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "key_mismatches=0" in out.stdout and " mismatches=0" in out.stdout, out.stdout


def test_div_recip_check_catches_unmarked_subnormals(tmp_path):
    """Not vacuous: taking the marked subnormal quotients as final answers fails it (the exact
    subnormal midpoints come out wrong)."""
    text = DIV_RECIP_SRC.read_text()
    planted = text.replace("if (is_subnormal_nonzero(q)) { ++flagged; continue; }", "").replace(
        "if (!is_subnormal_nonzero(q)) {", "if (1) {")
    assert planted.count("is_subnormal_nonzero(q)") == text.count("is_subnormal_nonzero(q)") - 2
    exe = _build(tmp_path, planted, "planted")
    out = subprocess.run([str(exe), "20000000"], capture_output=True, text=True, timeout=600)
    assert out.returncode == 1 and " mismatches=0" not in out.stdout, out.stdout


@pytest.mark.parametrize("bound", [np.float32(0.05), np.float32(0.1), np.float32(1.0), np.float32(0.03),
                                   np.float32(3.0)])
def test_uniform_pm_rewrite_is_exact(bound):
    k = np.arange(1 << 24, dtype=np.uint32)
    f32 = np.float32
    literal = ((k.astype(f32) * f32(1.0 / 16777216.0)) * f32(2.0) - f32(1.0)) * bound
    rewritten = (k.astype(np.int32) - 0x800000).astype(f32) * (bound * f32(2.0**-23))
    np.testing.assert_array_equal(literal.view(np.uint32), rewritten.view(np.uint32))
