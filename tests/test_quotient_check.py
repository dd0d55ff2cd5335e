"""The FP8 quantiser's one-correction quotient is exact for bf16 / fp16 inputs (CPU only).

tests/quotient_check.c compares the kernel's q1 = RN(q0 + RN(x - s*q0) * r), q0 = RN(x * r),
r = RN(1 / s) against the correctly rounded quotient from exact integer division.  bf16 (8
significant bits) runs over every significand pair (2^30 cases); fp16 (11 bits) over every x
significand and every 16th s significand here (the full 2^33 run, like 12 bits, also gave no
mismatch).  The same program shows that the uncorrected q0 is wrong in about a quarter of the
cases, so the check can fail.
"""

from __future__ import annotations

import os
import re
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    cc = shutil.which("gcc")
    if cc is None:
        pytest.skip("gcc not available")
    exe = tmp_path_factory.mktemp("quot") / "quotient_check"
    src = os.path.join(HERE, "quotient_check.c")
    # OpenMP only spreads the loop over cores; without libgomp the pragma is ignored.
    for flags in (["-fopenmp"], []):
        built = subprocess.run([cc, "-O3", *flags, "-ffp-contract=off", "-o", str(exe), src, "-lm"],
                               capture_output=True, text=True)
        if built.returncode == 0:
            return str(exe)
    raise AssertionError(f"gcc could not build quotient_check.c:\n{built.stderr}")


@pytest.mark.parametrize("bits,stride", [(8, 1), (11, 16)])
def test_one_correction_quotient_is_correctly_rounded(checker, bits, stride):
    out = subprocess.run([checker, str(bits), str(stride)], check=True, capture_output=True, text=True).stdout
    m = re.search(r"cases=(\d+) one_step_mismatches=(\d+) no_correction_mismatches=(\d+)", out)
    assert m, out
    cases, bad, bad0 = map(int, m.groups())
    assert cases == (1 << (bits - 1)) * ((1 << 23) // stride)
    assert bad == 0, out
    assert bad0 > cases // 10, out  # the uncorrected product is often wrong: the comparison has teeth
