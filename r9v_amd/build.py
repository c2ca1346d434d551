"""Builds libr9vx.so (all HIP kernels + the C ABI) for gfx950 with hipcc.

    python -m r9v_amd.build        # compile every source, link r9v_amd/libr9vx.so
    python -m r9v_amd.build --changed   # only sources newer than their object (or
                                        # with a newer header), then link

Objects go to r9v_amd/_build/; the library is written in-tree so it travels
with the repository snapshot to the GPU box.
"""
from __future__ import annotations

import concurrent.futures as cf
import json
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
# count (r9vx_mma3.h): a register the compiler spills between a
# load and its wait would be saved before the data arrives, so these must be
# spill-free (no scratch at all).
SPILL_FREE = ("moe_gu_m3_kernel", "moe_dn_m3_kernel", "gemm3_kernel")
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


def _inputs_stamp(src: pathlib.Path) -> float:
    """Newest modification time of the source and every header it could include."""
    return max(p.stat().st_mtime for p in [src, *CSRC.glob("*.h"), *(ROOT / "include").glob("*.h")])


def _compile(src: pathlib.Path):
    obj = BUILD / (src.stem + ".o")
    stamp = _inputs_stamp(src)  # taken before the compiler reads the inputs
    cmd = [HIPCC, *FLAGS, "-Rpass-analysis=kernel-resource-usage", "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed on {src.name}")
    res = parse_resources(r.stderr)
    obj.with_suffix(".res").write_text(json.dumps({"stamp": stamp, "res": res}))
    return obj, res


def _up_to_date(src: pathlib.Path) -> bool:
    """The object was compiled from inputs no older than the current ones."""
    obj, res = BUILD / (src.stem + ".o"), BUILD / (src.stem + ".res")
    if not (obj.exists() and res.exists()):
        return False
    try:
        stamp = json.loads(res.read_text())["stamp"]
    except (ValueError, KeyError, TypeError):
        return False
    return _inputs_stamp(src) <= stamp


def _reuse(src: pathlib.Path):
    obj = BUILD / (src.stem + ".o")
    return obj, json.loads(obj.with_suffix(".res").read_text())["res"]


def build(verbose: bool = True, changed_only: bool = False) -> pathlib.Path:
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    stale = [s for s in srcs if not (changed_only and _up_to_date(s))]
    with cf.ThreadPoolExecutor(max_workers=max(1, min(8, len(stale)))) as ex:
        fresh = dict(zip(stale, ex.map(_compile, stale)))
    done = [fresh[s] if s in fresh else _reuse(s) for s in srcs]
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
        print(f"built {OUT} from {len(srcs)} sources ({len(stale)} compiled); per-kernel registers in {RESOURCES}")
    return OUT


if __name__ == "__main__":
    build(changed_only="--changed" in sys.argv[1:])
