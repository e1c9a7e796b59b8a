"""The quantizers' fast division (y = x*r, e = fma(-y, s, x), q = fma(e, r, y)
with r = RN(1/s)) against IEEE division, on the CPU.  The full check over all
2^46 significand pairs is tests/cpu/division_check.c with the range
0 8388608 (about 4.5 CPU hours; it found no mismatch); this test compiles it
and runs slices that include both ends of the significand range, every s
whose significand is all ones or has one zero bit, and a spread of others."""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "cpu", "division_check.c")


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    cc = shutil.which("gcc")
    if cc is None:
        pytest.skip("no C compiler")
    exe = str(tmp_path_factory.mktemp("div") / "division_check")
    res = subprocess.run([cc, "-O3", "-mavx2", "-mfma", "-o", exe, SRC, "-lpthread", "-lm"], capture_output=True,
                         text=True)
    if res.returncode != 0:
        pytest.skip(f"cannot build the checker: {res.stderr[:200]}")
    return exe


@pytest.mark.parametrize("lo,hi", [(0, 256), ((1 << 23) - 256, 1 << 23), (1 << 22, (1 << 22) + 128),
                                   (3141592, 3141592 + 128), (6000000, 6000128)])
def test_fast_division_equals_ieee_division(checker, lo, hi):
    res = subprocess.run([checker, str(lo), str(hi), str(min(8, os.cpu_count() or 1))], capture_output=True,
                         text=True, timeout=300)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "0 mismatching pairs" in res.stdout


def test_fast_division_near_all_ones_significands(checker):
    """s significands with at most one zero bit: the reciprocal's hardest cases."""
    masks = [(1 << 23) - 1] + [((1 << 23) - 1) ^ (1 << b) for b in range(23)]
    for m in masks:
        res = subprocess.run([checker, str(m), str(m + 1), "1"], capture_output=True, text=True, timeout=60)
        assert res.returncode == 0, res.stdout + res.stderr
