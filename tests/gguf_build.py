"""GGUF file builder for tests: the layout rules of gguf-py 0.19.0's writer,
which produced the reference's fixtures (crates/r9v-format/tests/container.rs:4-8):
header, metadata entries, tensor-info rows with each offset the running sum of
alignment-padded entry sizes, zero padding to the alignment, then each entry's
bytes followed by zero padding to the alignment.  Also the raw encoder of the
reference's corrupt-input tests (`Raw`, container.rs:934-1000).

Values are (type, value) pairs or (ARRAY, elem, items), the shape
oracle/gguf_oracle.py returns, so a parsed file re-emits byte for byte.
"""
from __future__ import annotations

import struct

_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 10: "<Q", 11: "<q", 12: "<d"}


def _str(s) -> bytes:
    raw = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(raw)) + raw


def _scalar(t: int, v) -> bytes:
    if t == 7:
        return bytes([1 if v else 0])
    if t == 8:
        return _str(v)
    return struct.pack(_SCALAR[t], v)


def encode_value(v) -> bytes:
    if v[0] == 9:
        _, elem, items = v
        return struct.pack("<IIQ", 9, elem, len(items)) + b"".join(_scalar(elem, x) for x in items)
    return struct.pack("<I", v[0]) + _scalar(v[0], v[1])


def build(kvs, tensors, alignment: int = 32, version: int = 3) -> bytes:
    """kvs: [(key, value)]; tensors: [(name, dims innermost-first, type code, data bytes)]."""
    out = bytearray(b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs)))
    for key, v in kvs:
        out += _str(key) + encode_value(v)
    offset = 0
    for name, dims, dtype, data in tensors:
        out += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", dtype, offset)
        offset += (len(data) + alignment - 1) // alignment * alignment
    out += bytes(-len(out) % alignment)
    for _, _, _, data in tensors:
        out += bytes(data) + bytes(-len(data) % alignment)
    return bytes(out)


def rebuild(parsed: dict, blob: bytes) -> bytes:
    """Re-emits a file the oracle parsed, from its tables and entry bytes."""
    start = parsed["data_start"]
    tensors = [(t["name"], t["dims"], t["dtype"], blob[start + t["offset"]:start + t["offset"] + t["nbytes"]])
               for t in parsed["tensors"]]
    return build(parsed["kvs"], tensors, alignment=parsed["alignment"], version=parsed["version"])


class Raw:
    """Hand encoder that bypasses every validity rule (corrupt-input tests)."""

    def __init__(self, n_tensors: int, n_kv: int, version: int = 3):
        self.bytes = bytearray(b"GGUF" + struct.pack("<IQQ", version, n_tensors, n_kv))

    def str_raw(self, s: bytes):
        self.bytes += struct.pack("<Q", len(s)) + s

    def kv(self, key: str, ty: int, value: bytes):
        self.str_raw(key.encode())
        self.bytes += struct.pack("<I", ty) + value

    def u32_kv(self, key: str, v: int):
        self.kv(key, 4, struct.pack("<I", v))

    def tensor(self, name: str, dims, ty: int, offset: int):
        self.str_raw(name.encode())
        self.bytes += struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        self.bytes += struct.pack("<IQ", ty, offset)

    def pad_to(self, align: int):
        self.bytes += bytes(-len(self.bytes) % align)

    def data(self, n: int):
        self.bytes += bytes(n)
