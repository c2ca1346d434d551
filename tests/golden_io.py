"""Parsers for the reference's golden fixture files under tests/golden."""
from __future__ import annotations

import pathlib

import numpy as np

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


def _records(path):
    cases, cur = [], None
    for line in path.read_text().splitlines():
        if not line or line.startswith("#"):
            continue
        key, val = line.split(" ", 1)
        if key == "case":
            if cur:
                cases.append(cur)
            cur = {"name": val}
        else:
            cur[key] = val
    if cur:
        cases.append(cur)
    return cases


def q4k_cases():
    """crates/r9v-format/tests/schemes.rs:49-133 (load_q4k_reference) format:
    block hex, d/dmin bits, sc/mn decimals, q = 256 logical nibbles, y = 256
    f32 words as 8-hex-digit big-endian numbers."""
    out = []
    for c in _records(GOLDEN / "q4k_reference.txt"):
        y = c["y"]
        out.append({
            "name": c["name"],
            "block": np.frombuffer(bytes.fromhex(c["block"]), dtype=np.uint8),
            "d_bits": int(c["d_bits"], 16),
            "dmin_bits": int(c["dmin_bits"], 16),
            "sc": [int(v) for v in c["sc"].split()],
            "mn": [int(v) for v in c["mn"].split()],
            "q": [int(ch, 16) for ch in c["q"]],
            "y_bits": np.array([int(y[i:i + 8], 16) for i in range(0, len(y), 8)], dtype=np.uint32),
        })
    assert len(out) == 6
    return out


def iq4_cases():
    """crates/r9v-format/tests/iq.rs:51-109 format: n, k, wire hex, y = f32 LE bytes hex."""
    out = {}
    for c in _records(GOLDEN / "iq4_reference.txt"):
        out[c["name"]] = {
            "n": int(c["n"]),
            "k": int(c["k"]),
            "wire": np.frombuffer(bytes.fromhex(c["wire"]), dtype=np.uint8),
            "y_bits": np.frombuffer(bytes.fromhex(c["y"]), dtype="<u4"),
        }
    return out


def gguf_fixture(name: str) -> bytes:
    """A whole GGUF file from tests/golden/gguf/<name>.hex (the reference's
    crates/r9v-format/tests/fixtures/r9v-format/<name>.hex; '#' lines are the
    provenance header)."""
    text = (GOLDEN / "gguf" / f"{name}.hex").read_text()
    return bytes.fromhex("".join(l for l in text.splitlines() if not l.startswith("#")))


def a23_cases():
    """crates/r9v-format/tests/gguf.rs:44-90 (load_reference) format: n, k, wire
    hex, y = f32 LE bytes hex (gguf-py 0.19.0 dequantize); Q8_0, Q4_K, Q6_K."""
    out = {}
    for c in _records(GOLDEN / "gguf_a23_reference.txt"):
        out[c["name"]] = {
            "n": int(c["n"]),
            "k": int(c["k"]),
            "wire": np.frombuffer(bytes.fromhex(c["wire"]), dtype=np.uint8),
            "y_bits": np.frombuffer(bytes.fromhex(c["y"]), dtype="<u4"),
        }
    return out
