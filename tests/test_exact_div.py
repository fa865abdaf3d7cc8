"""The division the HIP encoder uses for fp16 inputs (three fma: Markstein's
correction of x * RN(1/den)) equals IEEE fp32 division.  The C checker runs a
strided sample of the significand pairs here (the stride-1 run covers all
2^33 pairs of fp16 x significand and fp32 den significand in both quotient
binades and both signs: `exact_div_check 1`); its naive mode, the quotient
without the correction step, is a planted mistake that must fail."""
import shutil
import subprocess
from pathlib import Path

import pytest

SRC = Path(__file__).resolve().parent / "exact_div_check.c"


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    exe = tmp_path_factory.mktemp("divcheck") / "exact_div_check"
    subprocess.run([gcc, "-O2", "-mfma", "-ffp-contract=off", "-fopenmp", "-o", str(exe), str(SRC), "-lm"],
                   check=True)
    return exe


def test_markstein_division_matches_ieee(checker):
    r = subprocess.run([str(checker), "61"], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout
    assert " 0 mismatches" in r.stdout


def test_uncorrected_quotient_fails(checker):
    r = subprocess.run([str(checker), "61", "naive"], capture_output=True, text=True)
    assert r.returncode == 1 and " 0 mismatches" not in r.stdout
