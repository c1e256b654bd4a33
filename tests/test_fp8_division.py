"""The fp8 requantisation's division, checked exhaustively on the CPU.

The kernel computes y / k_scale with Markstein's correction (two fmas after a multiply
by the rounded reciprocal) and relies on it equalling the correctly rounded quotient.
tests/fp8_division_check.c walks every fp32 y in the range that matters at a few
scales from the K-scale range [0.01, 0.1]; this test builds and runs it with gcc.
"""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_markstein_division_is_correctly_rounded(tmp_path):
    exe = str(tmp_path / "fp8_division_check")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math",
                    os.path.join(HERE, "fp8_division_check.c"), "-o", exe, "-lm"], check=True)
    # the K scales of the fp8 tests, and both ends of the range they are drawn from
    out = subprocess.run([exe, "0.01", "0.037", "0.081", "0.1"], capture_output=True,
                         text=True, timeout=300)
    assert out.returncode == 0, out.stdout
    assert out.stdout.strip().endswith(" 0 mismatches"), out.stdout
