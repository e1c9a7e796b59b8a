"""The hardware fp8 pack-convert agrees with the software e4m3 rounding.

The quantizers round to e4m3 with v_cvt_pk_fp8_f32 on tiles without NaN.  The
test program tests/hip/fp8_cvt_probe (built by __graft_entry__.build()) runs
both conversions on every fp32 bit pattern with |v| <= 448 and every NaN; the
only allowed differences are NaN inputs (the hardware writes 0xFF for +NaN),
which the quantizers route to the software path."""

from __future__ import annotations

import os
import re
import subprocess

import pytest

from conftest import ROOT

pytestmark = pytest.mark.gpu

PROBE = os.path.join(ROOT, "tests", "hip", "fp8_cvt_probe")


def test_hw_fp8_convert_matches_software_rounding(gpu_device):
    if not os.path.exists(PROBE):
        pytest.fail("tests/hip/fp8_cvt_probe is not built; run __graft_entry__.build()")
    res = subprocess.run([PROBE], capture_output=True, text=True, timeout=120)
    line = res.stdout.splitlines()[0]
    assert line.startswith("status=no error"), res.stdout
    fields = dict(re.findall(r"(\w+)=(\d+)", line))
    assert int(fields["checked"]) > 2_000_000_000
    assert int(fields["non_nan_mismatches"]) == 0, res.stdout
    assert res.returncode == 0


BF16_PROBE = os.path.join(ROOT, "tests", "hip", "bf16_cvt_probe")


def test_hw_bf16_convert_matches_software_rounding(gpu_device):
    """The dequant-fused GEMMs round weights to bf16 with v_cvt_pk_bf16_f32;
    every non-NaN fp32 input must round exactly as f32_to_bf16_bits (RNE) and
    every NaN must stay a NaN."""
    if not os.path.exists(BF16_PROBE):
        pytest.fail("tests/hip/bf16_cvt_probe is not built; run __graft_entry__.build()")
    res = subprocess.run([BF16_PROBE], capture_output=True, text=True, timeout=120)
    line = res.stdout.splitlines()[0]
    assert line.startswith("status=no error"), res.stdout
    fields = dict(re.findall(r"(\w+)=(\d+)", line))
    assert int(fields["checked"]) == 1 << 32
    assert int(fields["non_nan_mismatches"]) == 0, res.stdout
    assert int(fields["nan_not_nan"]) == 0, res.stdout
    assert res.returncode == 0


SR_PROBE = os.path.join(ROOT, "tests", "hip", "fp8_sr_cvt_probe")


def test_hw_fp8_stochastic_convert_matches_software_rule(gpu_device):
    """The stochastic-rounding tile paths round to e4m3 with v_cvt_sr_fp8_f32;
    its rounding must be e4m3_sr's (and the oracle's) for every fp32 |v| <=
    448, with random words and with the words at and just below the carry
    threshold."""
    if not os.path.exists(SR_PROBE):
        pytest.fail("tests/hip/fp8_sr_cvt_probe is not built; run __graft_entry__.build()")
    res = subprocess.run([SR_PROBE], capture_output=True, text=True, timeout=120)
    line = res.stdout.splitlines()[0]
    assert line.startswith("status=no error"), res.stdout
    fields = dict(re.findall(r"(\w+)=(\d+)", line))
    assert int(fields["checked"]) > 8_000_000_000
    assert int(fields["mismatches"]) == 0, res.stdout
    assert res.returncode == 0
