"""Host check that the single-FMA dequantization predicate is sound.

Every kernel takes the fast path (one v_fma_mix per weight, constants
c0 = b - 1024 s and c1 = b - 64 s) only for groups that
cider_press_amd/csrc/kernels/fastpath.hpp accepts, and the slow path
(fmaf(s, q, b) directly) otherwise.  fastpath_check.cpp enumerates (s, b)
pairs over every sign and exponent of bf16 and f16 with a spread of
significands and checks, for each accepted pair and every q, that the fast
path's fp32 value equals fmaf(s, q, b) bit for bit (signed zeros included),
and that the packed many-groups check the kernels run first accepts only
pairs the exact predicate accepts.
The planted variants below are wrong predicates the check must reject.
"""
import pathlib
import shutil
import subprocess

import pytest

HERE = pathlib.Path(__file__).resolve().parent
HEADER = HERE.parent / "cider_press_amd" / "csrc" / "kernels" / "fastpath.hpp"
SRC = HERE / "fastpath_check.cpp"

pytestmark = pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")


def _build_and_run(tmp_path, header):
    exe = tmp_path / "fastpath_check"
    subprocess.run(["g++", "-O2", "-ffp-contract=off", "-std=c++17", f'-DCPQ_FASTPATH_HEADER="{header}"',
                    "-o", str(exe), str(SRC)], check=True, capture_output=True, text=True, timeout=300)
    return subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)


def test_fast_path_predicate_is_exact(tmp_path):
    r = _build_and_run(tmp_path, HEADER)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.startswith("ok "), r.stdout


@pytest.mark.parametrize("old,new,why", [
    ("eb - es + 5u <= 26u", "eb - es + 5u <= 30u", "bf16 exponent gap too wide (c1 inexact)"),
    ("eb - es + 5u <= 26u", "eb - es + 9u <= 30u", "bf16 negative gap too wide (c0 inexact)"),
    ("eb - 27u < 227u", "eb - 27u < 228u", "bf16 bias at the top binade (c0 overflows)"),
    ("eb - es + 2u <= 20u", "eb - es + 2u <= 24u", "f16 exponent gap too wide"),
    ("const bool z_ok = !(", "const bool z_ok = true || !(", "signed-zero result not excluded"),
    ("(240u - 27u) << 7, (253u - 27u) << 7, 26u << 7", "(240u - 27u) << 7, (253u - 27u) << 7, 28u << 7",
     "packed bf16 check: exponent gap too wide"),
    ("(240u - 27u) << 7, (253u - 27u) << 7", "(240u - 27u) << 7, (254u - 27u) << 7",
     "packed bf16 check: bias at the top binade"),
    ("29u << 10, 29u << 10, 20u << 10", "29u << 10, 29u << 10, 22u << 10", "packed f16 check: exponent gap too wide"),
])
def test_check_rejects_unsound_predicates(tmp_path, old, new, why):
    text = HEADER.read_text()
    assert old in text
    bad = tmp_path / "fastpath_bad.hpp"
    bad.write_text(text.replace(old, new, 1))
    r = _build_and_run(tmp_path, bad)
    assert r.returncode != 0 and "MISMATCH" in r.stdout, f"planted error not caught: {why}\n{r.stdout}"
