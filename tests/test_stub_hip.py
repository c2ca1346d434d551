"""libr9vx on a HIP runtime without a usable device, and on one that lacks a
symbol the library imports (the failure paths the reference's stub runtime
exercises, crates/r9v-hip/tests/fixtures/stub_hip.c:60-75): a stand-in
libamdhip64.so.7 built here from tests/fixtures/stub_amdhip64.c is put first
on the loader path of a child process.  No device is touched."""
from __future__ import annotations

import json
import os
import pathlib
import shutil
import subprocess
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
LIB = ROOT / "r9v_amd" / "libr9vx.so"
STUB_SRC = ROOT / "tests" / "fixtures" / "stub_amdhip64.c"
SYMBOLS = ["__hipRegisterFatBinary", "__hipUnregisterFatBinary", "__hipRegisterFunction", "__hipRegisterVar",
           "__hipPushCallConfiguration", "__hipPopCallConfiguration", "hipLaunchKernel", "hipGetDevice",
           "hipDeviceGetAttribute", "hipGetLastError", "hipGetErrorString", "hipGetSymbolAddress",
           "hipMemcpyAsync", "hipMemcpy2DAsync", "hipMemcpyFromSymbolAsync", "hipStreamSynchronize"]

pytestmark = pytest.mark.skipif(not LIB.exists() or shutil.which("gcc") is None,
                                reason="needs the built libr9vx.so and gcc")


def _stub(tmp_path, *defines):
    d = tmp_path / ("stub" + "".join(defines))
    d.mkdir()
    vs = d / "hip.map"
    vs.write_text("hip_4.2 {\n  global:\n" + "".join(f"    {s};\n" for s in SYMBOLS) + "  local: *;\n};\n")
    out = d / "libamdhip64.so.7"
    subprocess.run(["gcc", "-shared", "-fPIC", "-O1", *defines, "-Wl,-soname,libamdhip64.so.7",
                    f"-Wl,--version-script={vs}", "-o", str(out), str(STUB_SRC)], check=True)
    return d


def _child(stub_dir, code):
    env = dict(os.environ, LD_LIBRARY_PATH=str(stub_dir), PYTHONPATH=str(ROOT))
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout.strip().splitlines()[-1])


NO_DEVICE = r'''
import ctypes, json
from r9v_amd import ffi
L = ffi.load()
maps = open("/proc/self/maps").read().split()
out = {"abi": L.r9vx_abi_version(), "hip": sorted({m for m in maps if m.endswith("libamdhip64.so.7")})}
fake = ctypes.c_void_p(1 << 20)  # 256-byte aligned and never dereferenced: no kernel can run
def call(fn, *a):
    rc = fn(*a)
    return [rc, L.r9vx_last_error().decode()]
st = ffi.matmul_static(n=64, k=256, w_scheme=ffi.Q4_K, in_dtype=ffi.BF16, out_dtype=ffi.F32, m_bucket=1)
args = ffi.MatmulArgs(fake, None, None, fake, None, None, None, fake, None, 1, 0)
out["matmul"] = call(L.r9vx_matmul_launch, ctypes.byref(st), ctypes.byref(args), None)
rst = ffi.route_static(e=64, k=4, t_bucket=8)
rargs = ffi.MoeRouteArgs(fake, None, fake, fake, 2, 0)
out["route"] = call(L.r9vx_moe_route_launch, ctypes.byref(rst), ctypes.byref(rargs), None)
out["route_ex"] = call(L.r9vx_moe_route_launch_ex, ctypes.byref(rst), ctypes.byref(rargs), fake, None)
fst = ffi.ffn_static(t_bucket=4, e=8, k=2, dm=256, dff=256)
fargs = ffi.MoeFfnArgs(fake, fake, fake, fake, None, fake, None, fake, fake, 4, 0)
out["ffn"] = call(L.r9vx_moe_ffn_launch, ctypes.byref(fst), ctypes.byref(fargs), None)
s = ctypes.c_uint32(7)
out["ffn_status"] = call(L.r9vx_moe_ffn_status, ctypes.byref(fst), fake, ctypes.byref(s), None) + [s.value]
fargs.sort_workspace = None
out["ffn_noalloc"] = call(L.r9vx_moe_ffn_launch_noalloc, ctypes.byref(fst), ctypes.byref(fargs), None, None)
out["refusal"] = call(L.r9vx_moe_ffn_launch, None, ctypes.byref(fargs), None)
print(json.dumps(out))
'''


def test_no_device_paths_return_hip_errors(tmp_path):
    """Every launch that reaches the runtime returns its error code (100,
    hipErrorNoDevice) with the op named in r9vx_last_error, outputs are left
    alone, and host refusals still come first."""
    stub = _stub(tmp_path)
    out = _child(stub, NO_DEVICE)
    assert out["hip"] == [str(stub / "libamdhip64.so.7")]  # the stand-in, not the installed runtime
    assert out["abi"] == 3
    for op in ("matmul", "route", "route_ex", "ffn", "ffn_status", "ffn_noalloc"):
        rc, msg = out[op][:2]
        assert rc == 100, (op, rc, msg)
        assert "hipErrorNoDevice" in msg, (op, msg)
    assert out["ffn_status"][2] == 7  # the status word was not written
    assert out["refusal"][0] == -3  # a NULL static is refused before the runtime is asked


MISSING = r'''
import json
from r9v_amd import ffi
try:
    ffi.load()
    print(json.dumps({"loaded": True}))
except ffi.R9vxError as e:
    print(json.dumps({"loaded": False, "code": e.code, "msg": str(e)}))
'''


def test_missing_runtime_symbol_fails_loudly(tmp_path):
    out = _child(_stub(tmp_path, "-DSTUB_WITHOUT_LAUNCH"), MISSING)
    assert out["loaded"] is False and out["code"] == -100
    assert "hipLaunchKernel" in out["msg"] and "cannot load" in out["msg"]
