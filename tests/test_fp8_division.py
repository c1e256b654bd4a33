"""The fp8 requantisation's division, checked exhaustively on the CPU.

The kernel computes y / k_scale without a division per element
(marathon_amd/csrc/fp8_e4m3.h): q0 = y * rz + RN(y * rlo), from the reciprocal split in
two, is within one ulp of the quotient, and one Markstein correction with r = RN(1/s)
then gives the correctly rounded quotient, which the oracle computes by an IEEE
division.  tests/fp8_division_check.c repeats the kernel's operations and walks, at
every K scale the fp8 workloads and the GPU tests use and at scales whose reciprocal
rounds up, down or not at all, every fp32 y whose quotient can change an e4m3fn code
(2^-12 <= |y/s| < 2^10, both signs: 3.7e8 quotients per scale), plus 3e8 random
(scale, y) pairs over 41 binades of scale.
"""

from __future__ import annotations

import os
import shutil
import subprocess

import numpy as np
import pytest

from marathon_amd import workloads as W

HERE = os.path.dirname(os.path.abspath(__file__))

# fixed K scales of the fp8 GPU tests (tests/test_gpu_spans.py, test_gpu_fp8_codec.py)
# and both ends of the range the random ones are drawn from
TEST_SCALES = [0.01, 0.1, 0.021, 0.031, 0.037, 0.044, 0.05, 0.066, 0.072, 0.081]


def _hex(scales) -> list:
    return [f"{int(b):08x}" for b in np.asarray(scales, np.float32).view(np.uint32)]


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    exe = str(tmp_path_factory.mktemp("fp8div") / "fp8_division_check")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math",
                    os.path.join(HERE, "fp8_division_check.c"), "-o", exe, "-lm", "-lpthread"],
                   check=True)
    return exe


def _run(exe, args, timeout=600):
    out = subprocess.run([exe, *args], capture_output=True, text=True, timeout=timeout)
    assert out.returncode == 0, out.stdout[-2000:]
    assert out.stdout.strip().endswith(" 0 mismatches"), out.stdout[-2000:]
    return out.stdout


def test_every_k_scale_of_the_fp8_qwen3_14b_workload(checker):
    k_scale, _ = W.fp8_layer_scales(4, 40)  # the fp8 multi-span shift's 40 layers
    out = _run(checker, _hex(k_scale))
    assert out.count("scale ") == 40


def test_the_fixed_scales_of_the_fp8_gpu_tests(checker):
    _run(checker, _hex(TEST_SCALES))


def test_random_scales_over_41_binades(checker):
    _run(checker, ["random", "300000000"])


def test_scales_by_how_their_reciprocal_rounds(checker):
    # 0.125: exact reciprocal (rlo = 0); 0.1, 3.0: RN(1/s) above 1/s (rz is its
    # predecessor); 0.01: below; the largest and smallest significands, where a single
    # correction from RN(y * r) has the least margin
    out = _run(checker, _hex([0.125, 0.1, 3.0, 0.01]) + ["3fffffff", "3f800001", "3f7fffff"])
    assert out.count("scale ") == 7


def test_both_ends_of_the_scale_range(checker):
    # the quotient is correctly rounded for K scales in [2^-90, 2^100]: walk both ends
    out = _run(checker, _hex([2.0 ** -90, 1.7 * 2.0 ** -90, 1.9 * 2.0 ** 99, 2.0 ** 100]))
    assert out.count("scale ") == 4


def test_the_walk_finds_a_wrong_quotient(checker):
    # planted mistake: RN(y * r) with no correction is one ulp off for many y
    out = subprocess.run([checker, "plain", *_hex([0.1])], capture_output=True, text=True,
                         timeout=600)
    assert out.returncode == 1
    bad = int(out.stdout.strip().rsplit(" ", 2)[-2])
    assert bad > 1000, out.stdout
