"""The GGUF reader under AddressSanitizer and UndefinedBehaviorSanitizer.

r9v_amd/csrc/gguf.hip is host code that reads untrusted bytes.  Here it is
compiled for the host only, with -fsanitize=address,undefined and no
recovery, into tests/fixtures/gguf_scan.cpp (HIP calls go to the stand-in
runtime of tests/fixtures/stub_amdhip64.c), and run over the reference's
fixtures, every prefix of their header and tables, and the same 2,400 seeded
byte mutations tests/test_gguf.py checks against the oracle.  Any
out-of-bounds access or undefined operation aborts the scanner with a
report; each record's result must equal the unsanitized library's."""
from __future__ import annotations

import ctypes
import pathlib
import random
import shutil
import struct
import subprocess

import pytest

from golden_io import gguf_fixture
from oracle import gguf_oracle as GO
from r9v_amd import ffi

ROOT = pathlib.Path(__file__).resolve().parents[1]
HIPCC = "/opt/rocm/bin/hipcc"
FIXTURES = ["a25_standard", "a25_split-00001-of-00002", "a25_split-00002-of-00002", "llama_tiny_q80"]
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"]

pytestmark = pytest.mark.skipif(not (pathlib.Path(HIPCC).exists() and shutil.which("g++") and shutil.which("gcc")),
                                reason="needs hipcc, g++ and gcc")


@pytest.fixture(scope="module")
def scanner(tmp_path_factory):
    d = tmp_path_factory.mktemp("gguf_san")
    inc = [f"-I{ROOT / 'include'}", f"-I{ROOT / 'r9v_amd' / 'csrc'}"]
    host_san = [f for s in SAN for f in ("-Xarch_host", s)]
    steps = [
        [HIPCC, "--cuda-host-only", "-x", "hip", "-std=c++17", "-O1", "-g", "-fPIC", *host_san, *inc, "-c",
         str(ROOT / "r9v_amd" / "csrc" / "gguf.hip"), "-o", str(d / "gguf.o")],
        ["g++", "-std=c++17", "-O1", "-g", *SAN, *inc, "-c", str(ROOT / "tests" / "fixtures" / "gguf_scan.cpp"), "-o",
         str(d / "scan.o")],
        ["gcc", "-O1", "-g", "-fsanitize=address", "-c", str(ROOT / "tests" / "fixtures" / "stub_amdhip64.c"), "-o",
         str(d / "stub.o")],
        ["g++", *SAN, str(d / "gguf.o"), str(d / "scan.o"), str(d / "stub.o"), "-o", str(d / "gguf_scan")],
    ]
    for cmd in steps:
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-3000:]
    return d / "gguf_scan"


def corpus():
    recs = []
    for name in FIXTURES:
        b = gguf_fixture(name)
        table_end = GO.parse(b)["ranges"][5]
        recs.append(b)
        recs += [b[:n] for n in range(table_end + 1)]
        rng = random.Random(0x6767 + len(b))  # the mutation stream of tests/test_gguf.py
        for _ in range(600):
            m = bytearray(b)
            pos = rng.randrange(table_end)
            m[pos] = rng.choice([0, 1, 2, 0x7F, 0x80, 0xFF, m[pos] ^ (1 << rng.randrange(8))])
            recs.append(bytes(m))
    return recs


def library_result(lib, data):
    out = ctypes.c_void_p()
    buf = (ctypes.c_uint8 * max(len(data), 1)).from_buffer_copy(data or b"\0")
    rc = lib.r9vx_gguf_parse(ctypes.cast(buf, ctypes.c_void_p), len(data), ctypes.byref(out))
    kinds = lib.r9vx_gguf_last_problems()
    if rc == 0:
        lib.r9vx_gguf_free(out)
    return rc, kinds


def test_reader_is_clean_under_asan_and_ubsan(scanner, tmp_path):
    recs = corpus()
    path = tmp_path / "corpus.bin"
    with open(path, "wb") as f:
        for r in recs:
            f.write(struct.pack("<Q", len(r)))
            f.write(r)
    r = subprocess.run([str(scanner), str(path)], capture_output=True, text=True, timeout=600,
                       env={"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=0", "UBSAN_OPTIONS": "print_stacktrace=1"})
    assert r.returncode == 0, r.stderr[-4000:]
    lines = r.stdout.splitlines()
    assert len(lines) == len(recs)
    lib = ffi.load()
    accepted = 0
    for data, line in zip(recs, lines):
        rc, kinds, _ = (int(x) for x in line.split())
        assert (rc, kinds) == library_result(lib, data)
        accepted += rc == 0
    assert 0 < accepted < len(recs)
