"""Builds libr9vx.so (all HIP kernels + the C ABI) for gfx950 with hipcc.

    python -m r9v_amd.build        # compile every source, link r9v_amd/libr9vx.so

Objects go to r9v_amd/_build/; the library is written in-tree so it travels
with the repository snapshot to the GPU box.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import pathlib
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT = PKG / "libr9vx.so"
BUILD = PKG / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # strict IEEE: no contraction unless written as fmaf(); no fast math;
    # correctly rounded f32 divide (HIP's default), exact transcendentals
    "-ffp-contract=off",
    "-fno-fast-math",
    "-fno-gpu-approx-transcendentals",
    # no packed-FP32 instructions anywhere in the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


# Kernels whose main loops issue loads as inline assembly and wait for them by
# count (r9vx_mma2.h, r9vx_mma3.h): a register the compiler spills between a
# load and its wait would be saved before the data arrives, so these must be
# spill-free (no scratch at all).
SPILL_FREE = ("gemm2_kernel", "moe_gu_mfma_kernel", "moe_dn_mfma_kernel", "moe_gu_m3_kernel",
              "moe_dn_m3_kernel", "gemm3_kernel")
RESOURCES = BUILD / "kernel_resources.txt"

_FIELDS = {"VGPRs": "vgpr", "AGPRs": "agpr", "ScratchSize [bytes/lane]": "scratch", "VGPRs Spill": "vgpr_spill",
           "SGPRs Spill": "sgpr_spill", "Occupancy [waves/SIMD]": "occupancy", "LDS Size [bytes/block]": "lds"}


def parse_resources(text: str) -> dict:
    """Per-kernel figures from hipcc's -Rpass-analysis=kernel-resource-usage
    remarks on our own sources: {mangled name: {field: int}}."""
    out, cur = {}, None
    for line in text.splitlines():
        if "remark:" not in line:
            continue
        body = line.split("remark:", 1)[1].split("[-Rpass-analysis", 1)[0].strip()
        if body.startswith("Function Name:"):
            cur = out.setdefault(body.split(":", 1)[1].strip(), {})
            continue
        if cur is None or ":" not in body:
            continue
        key, val = body.rsplit(":", 1)
        if key.strip() in _FIELDS:
            try:
                cur[_FIELDS[key.strip()]] = int(val.strip())
            except ValueError:
                pass
    return out


def spill_problems(res: dict) -> list:
    """Kernels of SPILL_FREE that use scratch or spill registers."""
    bad = []
    for name, r in sorted(res.items()):
        if any(k in name for k in SPILL_FREE) and (r.get("scratch", 0) or r.get("vgpr_spill", 0)
                                                   or r.get("sgpr_spill", 0)):
            bad.append(f"{name}: scratch {r.get('scratch')} B/lane, {r.get('vgpr_spill')} VGPR / "
                       f"{r.get('sgpr_spill')} SGPR spills")
    return bad


def sources():
    return sorted(CSRC.glob("*.hip"))


def _compile(src: pathlib.Path):
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *FLAGS, "-Rpass-analysis=kernel-resource-usage", "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed on {src.name}")
    return obj, parse_resources(r.stderr)


def build(verbose: bool = True) -> pathlib.Path:
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        done = list(ex.map(_compile, srcs))
    objs = [o for o, _ in done]
    res = {}
    for _, r in done:
        res.update(r)
    with open(RESOURCES, "w") as f:
        f.write("kernel vgpr agpr scratch vgpr_spill sgpr_spill occupancy lds\n")
        for name, r in sorted(res.items()):
            f.write(" ".join([name] + [str(r.get(k, "-")) for k in ("vgpr", "agpr", "scratch", "vgpr_spill",
                                                                     "sgpr_spill", "occupancy", "lds")]) + "\n")
    bad = spill_problems(res)
    if bad:
        raise RuntimeError("kernels with asm-pipelined loads must be spill-free:\n  " + "\n  ".join(bad))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("link of libr9vx.so failed")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT} from {len(srcs)} sources; per-kernel registers in {RESOURCES}")
    return OUT


if __name__ == "__main__":
    build()
