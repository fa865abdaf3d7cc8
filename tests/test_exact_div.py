"""The encoder's division shortcuts equal IEEE fp32 division where it matters.

* ``exact_div_check.c``: d = x / den for fp16 x (three fma: Markstein's
  correction of x * RN(1/den)) equals IEEE fp32 division.  Here a strided
  sample of the significand pairs; the stride-1 run covers all 2^34 pairs of
  fp16 x significand and fp32 den significand in both quotient binades and both
  signs (`exact_div_check 1`).
* ``exact_code_check.c``: the half-even code of RN(t * yh + RN(t * yl)) with
  yh + yl = 1/s equals that of RN32(t / s).  Here every third scale
  significand; the stride-1 run (every fp32 significand of s, every 3-, 4- and
  5-bit level, 5.5e9 pairs, about 5 s on 8 threads) finds no mismatch.

Each checker's naive mode, the quotient without its correction, is a planted
mistake that must fail."""
import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


def _build(tmp_path_factory, name):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    exe = tmp_path_factory.mktemp(name) / name
    subprocess.run([gcc, "-O2", "-mfma", "-ffp-contract=off", "-fopenmp", "-o", str(exe), str(HERE / f"{name}.c"),
                    "-lm"], check=True)
    return exe


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    return _build(tmp_path_factory, "exact_div_check")


@pytest.fixture(scope="module")
def code_checker(tmp_path_factory):
    return _build(tmp_path_factory, "exact_code_check")


def test_markstein_division_matches_ieee(checker):
    r = subprocess.run([str(checker), "61"], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout
    assert " 0 mismatches" in r.stdout


def test_uncorrected_quotient_fails(checker):
    r = subprocess.run([str(checker), "61", "naive"], capture_output=True, text=True)
    assert r.returncode == 1 and " 0 mismatches" not in r.stdout


def test_two_term_reciprocal_codes_match_ieee(code_checker):
    r = subprocess.run([str(code_checker), "3"], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout
    assert " 0 code mismatches" in r.stdout


def test_high_part_alone_gives_wrong_codes(code_checker):
    r = subprocess.run([str(code_checker), "61", "naive"], capture_output=True, text=True)
    assert r.returncode == 1 and " 0 code mismatches" not in r.stdout
