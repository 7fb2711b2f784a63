"""The sampler's FMA division (moat_amd/csrc/sample.hip, div_markstein) is the
correctly rounded quotient: checked against IEEE float division on the CPU
(gcc, fmaf) for the divisors it meets -- the exp table's step, the sums of
probabilities -- hard significands and random ones, over a whole binade of
dividends each.  A plain reciprocal multiply fails the same check."""

import os
import shutil
import subprocess

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    exe = str(tmp_path_factory.mktemp("markstein") / "check")
    subprocess.run([gcc, "-O2", "-ffp-contract=off", os.path.join(HERE, "markstein_check.c"), "-o", exe, "-lm"],
                   check=True)
    return exe


def test_fma_division_is_correctly_rounded(checker):
    step = float(np.float32(10.0 / 32767))  # the table's step as the kernel gets it
    divisors = [step, 0.7, 8.419368, 1.0, 1.99999988, 1.00000012, 1.5, 3.0, 32000.0, 1e-5]
    proc = subprocess.run([checker, "24", *[repr(d) for d in divisors]], capture_output=True, text=True,
                          timeout=600)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert " 0 mismatches" in proc.stdout and proc.stdout.startswith(str(34 * (1 << 23)))


def test_reciprocal_multiply_alone_is_not(checker, tmp_path):
    """The check has teeth: RN(a * RN(1/b)) differs from RN(a/b) for some a."""
    a = np.arange(0x3F800000, 0x3F800000 + (1 << 20), dtype=np.uint32).view(np.float32)
    b = np.float32(0.7)
    r = np.float32(np.float32(1.0) / b)
    assert np.any((a * r).astype(np.float32) != (a / b).astype(np.float32))
