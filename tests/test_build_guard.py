"""The kernels whose main loops issue loads as inline assembly and wait for
them by count must compile without scratch or register spills (a spilled
register saved between a load and its wait would hold stale data).  The
figures are the compiler's own resource-usage remarks for our sources."""
from __future__ import annotations

import subprocess

import pytest

from r9v_amd import build as B

GUARDED = {"gemm.hip": ["gemm3_kernel"], "moe_gemm.hip": ["moe_gu_m3_kernel", "moe_dn_m3_kernel"]}


def _resources(src: str) -> dict:
    cmd = [B.HIPCC, *B.FLAGS, "-Rpass-analysis=kernel-resource-usage", "--offload-device-only", "-S",
           str(B.CSRC / src), "-o", "/dev/null"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return B.parse_resources(r.stderr)


@pytest.mark.parametrize("src", sorted(GUARDED))
def test_asm_pipelined_kernels_are_spill_free(src):
    res = _resources(src)
    for kernel in GUARDED[src]:
        found = {name: r for name, r in res.items() if kernel in name}
        assert found, f"{kernel} not built from {src}"
        for name, r in found.items():
            assert r.get("scratch") == 0 and r.get("vgpr_spill") == 0 and r.get("sgpr_spill") == 0, (name, r)
            assert r.get("vgpr", 999) <= 256, (name, r)  # two waves per SIMD
    assert not B.spill_problems(res)


def test_guard_parser_flags_a_spill():
    text = ("x.hip:1:1: remark: Function Name: _ZN12_GLOBAL__N_116moe_gu_m3_kernelILi23EEEvNS_11GroupedArgsE "
            "[-Rpass-analysis=kernel-resource-usage]\n"
            "x.hip:1:1: remark:     VGPRs: 256 [-Rpass-analysis=kernel-resource-usage]\n"
            "x.hip:1:1: remark:     ScratchSize [bytes/lane]: 12 [-Rpass-analysis=kernel-resource-usage]\n"
            "x.hip:1:1: remark:     VGPRs Spill: 2 [-Rpass-analysis=kernel-resource-usage]\n")
    res = B.parse_resources(text)
    assert list(res.values())[0]["vgpr_spill"] == 2
    assert len(B.spill_problems(res)) == 1
