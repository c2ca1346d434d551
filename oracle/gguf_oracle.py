"""CPU oracle for GGUF ingestion -- TEST INFRASTRUCTURE ONLY.

Only tests/ may import this module, as the checker of the C++ reader in
libr9vx (include/r9vx_gguf.h); nothing in the product calls it.

A plain-Python restatement of crates/r9v-format/src/container.rs for standard
GGUF v2/v3 files:
  - decode: parse_internal (:952-1025) over the checked cursor (:737-880):
    magic, version in {2, 3}, u64 tensor and KV counts, KV entries (u64-length
    UTF-8 key, u32 type 0..12, value; arrays are u32 element type + u64 count
    + scalars, nested arrays malformed; BOOL bytes other than 0/1 malformed),
    tensor-info rows (name, u32 n_dims, u64 dims, u32 type, u64 offset);
  - validate (:1046-1470): duplicate keys / tensors, general.alignment a
    nonzero power-of-two UINT32, coherent split.* keys, data_start =
    align_up(end of tensor-info table), each offset a multiple of alignment,
    each tensor sized by TensorType::data_nbytes (:673-700, sizes from
    gguf-py GGML_QUANT_SIZES :572-612), each range inside the file, no two
    ranges overlapping (sorted sweep);
  - ShardSet::open (:3476-3575).
Native R9V containers (r9v.* keys or type ids 1001-1022) are reported as the
single problem "Native", the boundary the C++ reader draws.

Parity pins: the reference tests' own fixtures and expectations
(crates/r9v-format/tests/container.rs:72-330, 897-930, 1058-1175, 1801-1900),
re-emission of those fixtures byte for byte by the gguf-py layout rules, and
differential runs against the C++ reader on truncated and mutated files.
"""
from __future__ import annotations

import struct

# problem kinds, named as the FormatError variants of crates/r9v-format/src/error.rs
TRUNCATED, BAD_MAGIC, BAD_VERSION, MALFORMED = "Truncated", "BadMagic", "UnsupportedVersion", "Malformed"
DUP_KEY, DUP_TENSOR, BAD_ALIGN, KV_TYPE = "DuplicateKey", "DuplicateTensor", "InvalidAlignment", "KvTypeMismatch"
MISSING_KEY, UNKNOWN_TYPE, BAD_RANGE, OVERFLOW, NATIVE = ("MissingKey", "UnknownTensorType", "BadTensorRange",
                                                          "Overflow", "Native")

# (block_len, block_bytes) per GGUF tensor type code (container.rs:572-612)
QUANT_SIZES = {
    0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 9: (32, 40),
    10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 15: (256, 292),
    16: (256, 66), 17: (256, 74), 18: (256, 98), 19: (256, 50), 20: (32, 18), 21: (256, 110),
    22: (256, 82), 23: (256, 136), 24: (1, 1), 25: (1, 2), 26: (1, 4), 27: (1, 8), 28: (1, 8),
    29: (256, 56), 30: (1, 2), 34: (256, 54), 35: (256, 66), 39: (32, 17), 40: (64, 36), 41: (128, 18),
}
U64_MAX = (1 << 64) - 1

# scalar KV codes -> struct format (container.rs:834-860)
_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 10: "<Q", 11: "<q", 12: "<d"}


class OracleError(Exception):
    def __init__(self, kinds, texts):
        super().__init__("; ".join(texts))
        self.kinds = set(kinds)
        self.texts = list(texts)


class _Stop(Exception):
    def __init__(self, kind, text):
        self.kind, self.text = kind, text


class _Cursor:
    def __init__(self, b):
        self.b, self.pos = b, 0

    def take(self, n, what):
        if n > len(self.b) - self.pos:
            raise _Stop(TRUNCATED, f"truncated at {self.pos}: need {n} for {what}")
        out = self.b[self.pos:self.pos + n]
        self.pos += n
        return out

    def num(self, fmt, what):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt), what))[0]

    def text(self, what):
        at = self.pos
        n = self.num("<Q", "string length")
        raw = self.take(n, what)
        try:
            return raw.decode("utf-8", errors="strict")
        except UnicodeDecodeError:
            raise _Stop(MALFORMED, f"invalid UTF-8 in {what} at {at}")

    def kv_type(self, what):
        at = self.pos
        t = self.num("<I", what)
        if t > 12:
            raise _Stop(MALFORMED, f"unknown GGUF metadata type code {t} at {at}")
        return t

    def scalar(self, t):
        if t == 7:
            at = self.pos
            v = self.num("<B", "bool value")
            if v > 1:
                raise _Stop(MALFORMED, f"BOOL value {v} is not 0 or 1 at {at}")
            return bool(v)
        if t == 8:
            return self.text("string value")
        if t == 9:
            raise _Stop(MALFORMED, "nested arrays are not valid GGUF metadata")
        return self.num(_SCALAR[t], "value")


def data_nbytes(dtype, dims):
    """TensorType::data_nbytes (container.rs:673-700): None when unsizable."""
    if dtype not in QUANT_SIZES or not dims or any(d == 0 for d in dims):
        return None
    bl, bb = QUANT_SIZES[dtype]
    if dims[0] % bl:
        return None
    elems = 1
    for d in dims:
        elems *= d
    out = elems // bl * bb
    return out if elems <= U64_MAX and out <= U64_MAX else None


def parse(b: bytes, file_size: int | None = None) -> dict:
    """Parsed shard as a dict, or OracleError naming every problem kind."""
    explicit = file_size is not None
    c = _Cursor(b)
    try:
        magic = c.num("<I", "magic")
        if magic != 0x46554747:
            raise _Stop(BAD_MAGIC, f"bad magic {magic:#010x}")
        version = c.num("<I", "version")
        if version not in (2, 3):
            raise _Stop(BAD_VERSION, f"unsupported version {version}")
        n_tensors = c.num("<Q", "tensor count")
        n_kv = c.num("<Q", "metadata count")
        header_end = c.pos
        kvs = []
        for _ in range(n_kv):
            key = c.text("metadata key")
            t = c.kv_type("metadata type")
            if t == 9:
                elem = c.kv_type("array element type")
                count = c.num("<Q", "array length")
                items = []
                for _ in range(count):
                    items.append(c.scalar(elem))
                kvs.append((key, (9, elem, tuple(items))))
            else:
                kvs.append((key, (t, c.scalar(t))))
        kv_end = c.pos
        tensors = []
        for _ in range(n_tensors):
            name = c.text("tensor name")
            nd = c.num("<I", "tensor dimension count")
            dims = tuple(c.num("<Q", "tensor dimension") for _ in range(nd))
            dtype = c.num("<I", "tensor type")
            offset = c.num("<Q", "tensor offset")
            tensors.append({"name": name, "dims": dims, "dtype": dtype, "offset": offset})
        ti_end = c.pos
    except _Stop as e:
        raise OracleError([e.kind], [e.text])

    if any(k.startswith("r9v.") for k, _ in kvs) or any(1001 <= t["dtype"] <= 1022 for t in tensors):
        raise OracleError([NATIVE], ["native R9V container"])

    size = file_size if explicit else len(b)
    probs = []
    kv_map, t_map = {}, {}
    for k, v in kvs:
        if k in kv_map:
            probs.append((DUP_KEY, f"duplicate metadata key {k!r}"))
        else:
            kv_map[k] = v
    for i, t in enumerate(tensors):
        if t["name"] in t_map:
            probs.append((DUP_TENSOR, f"duplicate tensor name {t['name']!r}"))
        else:
            t_map[t["name"]] = i

    align = 32
    if "general.alignment" in kv_map:
        v = kv_map["general.alignment"]
        if v[0] != 4:
            probs.append((KV_TYPE, "general.alignment is not UINT32"))
        elif v[1] == 0 or v[1] & (v[1] - 1):
            probs.append((BAD_ALIGN, f"invalid alignment {v[1]}"))
        else:
            align = v[1]

    if any(k.startswith("split.") for k in kv_map):
        want = {"split.no": 2, "split.count": 2, "split.tensors.count": 5}
        got = {}
        for key, code in want.items():
            if key not in kv_map:
                probs.append((MISSING_KEY, f"missing {key}"))
            elif kv_map[key][0] != code:
                probs.append((KV_TYPE, f"{key} has the wrong type"))
            else:
                got[key] = kv_map[key][1]
        if len(got) == 3:
            no, count, tc = got["split.no"], got["split.count"], got["split.tensors.count"]
            if count == 0:
                probs.append((MALFORMED, "split.count must be >= 1"))
            elif no >= count:
                probs.append((MALFORMED, f"split.no {no} must be < split.count {count}"))
            if tc < 0:
                probs.append((MALFORMED, "split.tensors.count < 0"))
            elif count == 1:
                if no != 0:
                    probs.append((MALFORMED, "single-shard split.no != 0"))
                if tc != len(tensors):
                    probs.append((MALFORMED, "split.tensors.count != tensors"))
            elif len(tensors) > tc:
                probs.append((MALFORMED, "shard tensor count exceeds split.tensors.count"))

    data_start = ti_end
    if ti_end + align - 1 > U64_MAX:
        probs.append((OVERFLOW, "data_start"))
    else:
        data_start = (ti_end + align - 1) // align * align
    if explicit and size < data_start:
        probs.append((MALFORMED, "logical file size below data start"))
        raise OracleError([k for k, _ in probs], [t for _, t in probs])

    spans = []
    for i, t in enumerate(tensors):
        start = data_start + t["offset"]
        if start > U64_MAX:
            probs.append((BAD_RANGE, f"{t['name']}: start overflows"))
            continue
        if t["offset"] % align:
            probs.append((BAD_RANGE, f"{t['name']}: offset not a multiple of alignment {align}"))
        if t["dtype"] not in QUANT_SIZES:
            probs.append((UNKNOWN_TYPE, f"unknown tensor type code {t['dtype']} for {t['name']!r}"))
            continue
        n = data_nbytes(t["dtype"], t["dims"])
        if n is None:
            probs.append((MALFORMED, f"{t['name']}: unsizable dims {t['dims']}"))
            continue
        t["nbytes"] = n
        end = start + n
        if end > U64_MAX:
            probs.append((BAD_RANGE, f"{t['name']}: end overflows"))
            continue
        if end > size:
            probs.append((BAD_RANGE, f"{t['name']}: range end {end} beyond file size {size}"))
            continue
        spans.append((start, end, i))
    spans.sort()
    if spans:
        wide = spans[0]
        for s in spans[1:]:
            if s[0] < wide[1]:
                probs.append((BAD_RANGE, f"{tensors[s[2]]['name']} overlaps {tensors[wide[2]]['name']}"))
            if s[1] > wide[1]:
                wide = s
    if probs:
        raise OracleError([k for k, _ in probs], [t for _, t in probs])
    return {"version": version, "alignment": align, "kvs": kvs, "kv": kv_map, "tensors": tensors,
            "data_start": data_start, "file_size": size,
            "ranges": (0, header_end, header_end, kv_end, kv_end, ti_end)}


def tensor_bytes(f: dict, name: str, b: bytes) -> bytes:
    """GgufFile::tensor_bytes (container.rs:2074-2116)."""
    t = next(t for t in f["tensors"] if t["name"] == name)
    start = f["data_start"] + t["offset"]
    if start + t["nbytes"] > len(b):
        raise OracleError([BAD_RANGE], [f"{name}: beyond buffer"])
    return b[start:start + t["nbytes"]]


def open_shards(shards: list) -> list:
    """ShardSet::open (container.rs:3476-3575): merged (shard, tensor index) order."""
    if not shards:
        raise OracleError([MALFORMED], ["split shard set is empty"])
    probs, seen, order = [], {}, []
    for si, f in enumerate(shards):
        for ti, t in enumerate(f["tensors"]):
            if t["name"] in seen:
                probs.append((DUP_TENSOR, f"{t['name']} (shards {seen[t['name']]} and {si})"))
            else:
                seen[t["name"]] = si
                order.append((si, ti))
    if len(shards) > 1 or any(k.startswith("split.") for f in shards for k in f["kv"]):
        for si, f in enumerate(shards):
            for key, code, want in (("split.count", 2, len(shards)), ("split.no", 2, si),
                                    ("split.tensors.count", 5, len(seen))):
                v = f["kv"].get(key)
                if v is None:
                    probs.append((MISSING_KEY, key))
                elif v[0] != code:
                    probs.append((KV_TYPE, key))
                elif v[1] != want:
                    probs.append((MALFORMED, f"shard {si}: {key} is {v[1]}, expected {want}"))
    if probs:
        raise OracleError([k for k, _ in probs], [t for _, t in probs])
    return order
