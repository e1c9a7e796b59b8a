"""Register, scratch and occupancy bounds of the built kernels, from the
compiler's kernel-resource-usage report that nano-train_amd/build.py keeps next
to the objects.  The HBM-bound quantizers depend on occupancy: a change that
grows their register count (a reordered loop did, from 59 to 83 VGPRs on the
128x128 pass, which halved the resident workgroups and cost 25% of its
bandwidth) fails here on the CPU before any GPU run."""

from __future__ import annotations

import json
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REPORT = os.path.join(ROOT, "nano-train_amd", "_build", "kernel_resources.json")


@pytest.fixture(scope="module")
def resources():
    if not os.path.exists(REPORT):
        pytest.skip("no kernel resource report: run nano-train_amd/build.py first")
    with open(REPORT) as fh:
        return json.load(fh)


def _matching(resources, needle):
    got = {k: v for k, v in resources.items() if needle in k}
    assert got, f"no kernel matching {needle}"
    return got


def test_no_kernel_uses_scratch_memory(resources):
    """No scratch and no VGPR spills (both go to memory).  SGPR spills, which
    the stochastic-rounding variants have, go to VGPR lanes instead."""
    bad = {k: (v.get("ScratchSize [bytes/lane]"), v.get("VGPRs Spill"))
           for k, v in resources.items() if v.get("ScratchSize [bytes/lane]", 0) or v.get("VGPRs Spill", 0)}
    assert not bad, bad


# (mangled-name fragment, most VGPRs): the round-to-nearest variants without a
# dq output that the configurations time, bf16 input
# quant_block_128x128_fast<IN_DT=bf16, GRID, SR=false, DQ=false>: 8 waves per SIMD
# quant_tile_1x128_fast<bf16, GRID, RN, no dq, no fan-out> and the fan-out form
# quant_tile_128x1_t_fast<bf16, GRID, RN, no dq, single or dual output>
BOUNDS = [
    ("quant_block_128x128_fastILi1ELi1ELb0ELb0E", 64),
    ("quant_block_128x128_fastILi1ELi0ELb0ELb0E", 64),
    ("quant_tile_1x128_fastILi1ELi1ELb0ELb0ELb0E", 48),
    ("quant_tile_1x128_fastILi1ELi0ELb0ELb0ELb0E", 48),
    ("quant_tile_1x128_fastILi1ELi1ELb0ELb0ELb1E", 48),
    ("quant_tile_128x1_t_fastILi1ELi1ELb0ELb0ELb0E", 64),
    ("quant_tile_128x1_t_fastILi1ELi1ELb0ELb0ELb1E", 104),
]


@pytest.mark.parametrize("needle,max_vgprs", BOUNDS)
def test_quantizer_register_bounds(resources, needle, max_vgprs):
    for name, v in _matching(resources, needle).items():
        assert v["VGPRs"] + v["AGPRs"] <= max_vgprs, (name, v["VGPRs"], v["AGPRs"])


def test_gemms_fit_two_waves_per_simd(resources):
    """The 512-thread GEMM workgroups run two waves per SIMD: 256 registers
    per lane at most, with the 160 KB of LDS shared by one workgroup."""
    for needle in ("gemm_blockscaled_kernel", "gemm_dq_kernel", "gemm_lowbit_fused_kernel"):
        for name, v in _matching(resources, needle).items():
            assert v["VGPRs"] + v["AGPRs"] <= 256, name
            assert v["Occupancy [waves/SIMD]"] >= 2, name
            assert v["LDS Size [bytes/block]"] <= 160 * 1024, name
