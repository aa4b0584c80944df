"""The quotient of the quantisation kernels (multiply by 1 / s, one FMA correction) gives the codes of
the correctly rounded x / s: tests/quant_division_check.c over a sample of amax values (every 61st of
the 32,639 finite positive bf16 values plus the largest, all x with |x| <= amax, both signs, int8 and
e4m3). Run the program with amax_stride 1 for the full check (1.07e9 pairs per qmax, 0 mismatches).
The uncorrected product x * r must fail the same check, so the check itself is shown to catch errors."""

from __future__ import annotations

import pathlib
import re
import shutil
import subprocess

import pytest

SRC = pathlib.Path(__file__).with_name("quant_division_check.c")


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    if shutil.which("gcc") is None:
        pytest.skip("gcc is not available")
    exe = tmp_path_factory.mktemp("qdc") / "quant_division_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), str(SRC), "-lm"], check=True)
    return exe


def _counts(stdout: str) -> dict[str, tuple[int, int]]:
    found = re.findall(r"qmax (\d+): (\d+) pairs, (\d+) code mismatches", stdout)
    return {q: (int(p), int(m)) for q, p, m in found}


def test_corrected_quotient_codes_match_division(checker):
    out = subprocess.run([str(checker), "61"], capture_output=True, text=True, timeout=120)
    counts = _counts(out.stdout)
    assert out.returncode == 0, out.stdout
    assert set(counts) == {"127", "448"}
    for pairs, mismatches in counts.values():
        assert pairs > 10_000_000 and mismatches == 0


def test_uncorrected_product_fails_the_check(checker):
    out = subprocess.run([str(checker), "61", "uncorrected"], capture_output=True, text=True, timeout=120)
    counts = _counts(out.stdout)
    assert out.returncode == 1
    assert counts["127"][1] > 0 and counts["448"][1] > 0
