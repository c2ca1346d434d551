"""CPU tests of GGUF ingestion (include/r9vx_gguf.h, r9v_amd/gguf.py).

The C++ reader in libr9vx is checked three ways: against the reference's own
fixtures and the facts its tests assert about them
(crates/r9v-format/tests/container.rs), against the Python oracle
(oracle/gguf_oracle.py) on every truncation and on seeded byte mutations of
those fixtures, and, for XXH3, against the xxhash package (libxxhash 0.8.2,
python-xxhash 3.x), an implementation independent of this one.  No test here
touches a GPU: parsing, validation and hashing are host code.
"""
from __future__ import annotations

import ctypes

import random
import struct

import pytest

from golden_io import gguf_fixture
from gguf_build import Raw, build, rebuild
from oracle import gguf_oracle as GO
from r9v_amd import ffi, gguf

FIXTURES = ["a25_standard", "a25_split-00001-of-00002", "a25_split-00002-of-00002", "llama_tiny_q80"]


def parse_kinds(data, file_size=None):
    """(C++ result kinds or None, oracle kinds or None)."""
    try:
        if file_size is None:
            gguf.GgufFile.parse(data)
        else:
            gguf.GgufFile.parse_metadata_only(data, file_size)
        got = None
    except gguf.GgufError as e:
        got = e.kinds
    try:
        GO.parse(bytes(data), file_size)
        want = None
    except GO.OracleError as e:
        want = e.kinds
    return got, want


def same_tables(f: gguf.GgufFile, o: dict):
    assert f.version() == o["version"]
    assert f.alignment() == o["alignment"]
    assert f.data_start() == o["data_start"]
    assert f.file_size() == o["file_size"]
    assert f.header_range() + f.kv_range() + f.ti_range() == o["ranges"]
    kvs = f.kvs()
    assert [k for k, _ in kvs] == [k for k, _ in o["kvs"]]
    for (_, v), (_, ov) in zip(kvs, o["kvs"]):
        if ov[0] == 9:
            assert (v.type, v.elem) == (9, ov[1])
            assert list(v.value) == list(ov[2]) or all(
                (a != a and b != b) or a == b for a, b in zip(v.value, ov[2]))
        else:
            assert v.type == ov[0]
            assert v.value == ov[1] or (v.value != v.value and ov[1] != ov[1])
    rows = f.tensors()
    assert [(t.name, t.dims, t.dtype, t.offset, t.nbytes) for t in rows] == [
        (t["name"], t["dims"], t["dtype"], t["offset"], t["nbytes"]) for t in o["tensors"]]


# ------------------------------------------------ reference fixture facts

def test_standard_fixture_metadata_covers_all_kv_types():
    """crates/r9v-format/tests/container.rs:72-155."""
    b = gguf_fixture("a25_standard")
    f = gguf.GgufFile.parse(b)
    assert f.version() == 3 and f.alignment() == 32
    assert len(f.kvs()) == 28 and len(f.tensors()) == 12
    assert f.is_standard_gguf() and not f.is_native()
    kv = f.kv
    assert kv("general.architecture") == gguf.KvValue(gguf.STR, "llama")
    assert kv("general.name") == gguf.KvValue(gguf.STR, "a2.5-standard-fixture")
    assert kv("a25.u8") == gguf.KvValue(gguf.U8, 200)
    assert kv("a25.i8") == gguf.KvValue(gguf.I8, -5)
    assert kv("a25.u16") == gguf.KvValue(gguf.U16, 60000)
    assert kv("a25.i16") == gguf.KvValue(gguf.I16, -3000)
    assert kv("a25.u32") == gguf.KvValue(gguf.U32, 3_000_000_000)
    assert kv("a25.i32") == gguf.KvValue(gguf.I32, -2_000_000_000)
    assert kv("a25.f32") == gguf.KvValue(gguf.F32, 0.5)
    assert kv("a25.bool_true") == gguf.KvValue(gguf.BOOL, True)
    assert kv("a25.bool_false") == gguf.KvValue(gguf.BOOL, False)
    assert kv("a25.str") == gguf.KvValue(gguf.STR, "r9v-a2.5 ☃")
    assert kv("a25.u64") == gguf.KvValue(gguf.U64, (1 << 63) + 123)
    assert kv("a25.i64") == gguf.KvValue(gguf.I64, -(1 << 62))
    f64 = kv("a25.f64")
    assert f64.type == gguf.F64 and struct.pack("<d", f64.value) == struct.pack("<Q", 0x4005_BF0A_8B14_5769)
    assert kv("tokenizer.ggml.tokens") == gguf.KvValue(gguf.ARRAY, ("<unk>", "<s>", "hello"), gguf.STR)
    assert kv("a25.arr_i32_small") == gguf.KvValue(gguf.ARRAY, (1, 2, 3), gguf.I32)
    assert kv("a25.arr_bytes") == gguf.KvValue(gguf.ARRAY, (1, 2, 3), gguf.U8)
    assert kv("a25.arr_u64") == gguf.KvValue(gguf.ARRAY, (1 << 40, 1 << 63), gguf.U64)
    arr_f64 = kv("a25.arr_f64")
    assert arr_f64.elem == gguf.F64 and len(arr_f64.value) == 1
    assert kv("missing.key") is None


def test_standard_fixture_tensor_table_matches_writer_layout():
    """crates/r9v-format/tests/container.rs:157-201."""
    b = gguf_fixture("a25_standard")
    f = gguf.GgufFile.parse(b)
    expected = [
        ("bias_f32", (16,), 0, 64), ("norm_f16", (32, 16), 1, 1024), ("w_q80", (32, 16), 8, 544),
        ("w_q40", (32, 16), 2, 288), ("w_q41", (32, 16), 3, 320), ("w_q50", (32, 16), 6, 352),
        ("w_q51", (32, 16), 7, 384), ("w_q2k", (256, 16), 10, 1344), ("w_q3k", (256, 16), 11, 1760),
        ("w_q4k", (256, 16), 12, 2304), ("w_q5k", (256, 16), 13, 2816), ("w_q6k", (256, 16), 14, 3360),
    ]
    offset = 0
    assert len(f.tensors()) == len(expected)
    for t, (name, dims, code, nbytes) in zip(f.tensors(), expected):
        assert (t.name, t.dims, t.dtype, t.offset) == (name, dims, code, offset)
        assert len(f.tensor_bytes(name, b)) == nbytes == t.nbytes
        offset += -(-nbytes // 32) * 32
    assert f.data_start() % 32 == 0 and f.data_start() > f.ti_range()[1]
    assert f.tensor("w_q4k").type_name == "Q4_K"


def test_real_llamacpp_metadata_and_tensor_table():
    """crates/r9v-format/tests/container.rs:255-330 (a llama-quantize Q8_0 file)."""
    xxhash = pytest.importorskip("xxhash")
    b = gguf_fixture("llama_tiny_q80")
    f = gguf.GgufFile.parse(b)
    assert f.version() == 3 and len(f.tensors()) == 4 and f.is_standard_gguf()
    assert f.kv("general.architecture").value == "llama"
    assert f.kv("general.name").value == "tiny-llama"
    for key, v in (("llama.context_length", 32), ("llama.embedding_length", 32), ("llama.block_count", 1)):
        assert f.kv(key) == gguf.KvValue(gguf.U32, v)
    assert f.data_start() == 960
    for name, dtype, dims, offset, nbytes in (
            ("output.weight", 8, (32, 3), 0, 102), ("token_embd.weight", 8, (32, 3), 128, 102),
            ("blk.0.attn_norm.weight", 0, (32,), 256, 128), ("blk.0.attn_q.weight", 8, (32, 32), 384, 1088)):
        t = f.tensor(name)
        assert (t.dtype, t.dims, t.offset) == (dtype, dims, offset)
        data = f.tensor_bytes(name, b)
        assert len(data) == nbytes
        assert f.entry_xxh3(name, b) == xxhash.xxh3_64_intdigest(data)


def test_split_shards_merge_in_table_order():
    """crates/r9v-format/tests/container.rs:897-916."""
    a, b = gguf_fixture("a25_split-00001-of-00002"), gguf_fixture("a25_split-00002-of-00002")
    fa, fb = gguf.GgufFile.parse(a), gguf.GgufFile.parse(b)
    assert fa.kv("split.no") == gguf.KvValue(gguf.U16, 0)
    assert fb.kv("split.no") == gguf.KvValue(gguf.U16, 1)
    assert fa.kv("split.count") == gguf.KvValue(gguf.U16, 2)
    assert fa.kv("split.tensors.count") == gguf.KvValue(gguf.I32, 3)
    s = gguf.ShardSet.open([fa, fb])
    assert len(s) == 3 and not s.is_empty()
    assert [s.tensor_at(i)[1].name for i in range(len(s))] == ["shard.a_q80", "shard.b_f16", "shard.c_q40"]
    assert s.tensor("shard.c_q40")[0] == 1
    assert s.tensor("absent") is None and s.tensor_at(99) is None
    assert GO.open_shards([GO.parse(a), GO.parse(b)]) == [(0, 0), (0, 1), (1, 0)]


def test_split_mismatch_reports_every_problem():
    """crates/r9v-format/tests/container.rs:918-932."""
    a = gguf_fixture("a25_split-00001-of-00002")
    fa = gguf.GgufFile.parse(a)
    with pytest.raises(gguf.GgufError) as e:
        gguf.ShardSet.open([fa, gguf.GgufFile.parse(a)])
    assert len(str(e.value).split("; ")) >= 3
    assert {"DuplicateTensor", "Malformed"} <= e.value.kinds
    with pytest.raises(GO.OracleError) as o:
        GO.open_shards([GO.parse(a), GO.parse(a)])
    assert o.value.kinds == e.value.kinds and len(o.value.texts) == len(str(e.value).split("; "))
    with pytest.raises(gguf.GgufError):
        gguf.ShardSet.open([])
    fb = gguf.GgufFile.parse(gguf_fixture("a25_split-00002-of-00002"))
    assert len(fb.tensors()) == 1 and fb.tensor("shard.c_q40").dtype == 2


# ---------------------------------------------------- refusals

def expect(data, kinds, file_size=None, text=None):
    got, want = parse_kinds(data, file_size)
    assert got == set(kinds), (got, kinds)
    assert want == got, (want, got)
    if text is not None:
        with pytest.raises(gguf.GgufError) as e:
            gguf.GgufFile.parse(data)
        assert text in str(e.value), str(e.value)


def test_corrupt_headers_fail_with_kinds():
    """crates/r9v-format/tests/container.rs:1058-1128."""
    expect(b"", {"Truncated"}, text="truncated GGUF at offset 0")
    expect(b"GG", {"Truncated"})
    expect(b"XXXX" + bytes(28), {"BadMagic"}, text="bad GGUF magic 0x58585858")
    r = Raw(0, 0)
    r.bytes[4:8] = struct.pack("<I", 99)
    expect(bytes(r.bytes), {"UnsupportedVersion"}, text="unsupported GGUF version 99")
    r = Raw(0, 1)
    r.kv("flag", 7, b"\x02")
    expect(bytes(r.bytes), {"Malformed"}, text="BOOL value 2 is not 0 or 1")
    r = Raw(0, 1)
    r.str_raw(b"arr")
    r.bytes += struct.pack("<IIQ", 9, 9, 1)
    expect(bytes(r.bytes), {"Malformed"}, text="nested arrays")
    r = Raw(0, 1)
    r.kv("X", 4, struct.pack("<I", 1))
    r.bytes[32] = 0xFF
    expect(bytes(r.bytes), {"Malformed"}, text="invalid UTF-8 in metadata key")
    r = Raw(0, 1)
    r.kv("mystery", 13, b"")
    expect(bytes(r.bytes), {"Malformed"}, text="unknown GGUF metadata type code 13")
    # a version-2 header is accepted (GGUF_VERSIONS_ACCEPTED, container.rs:34)
    assert gguf.GgufFile.parse(bytes(Raw(0, 0, version=2).bytes)).version() == 2


def test_every_prefix_of_every_fixture_is_refused_like_the_oracle():
    """Truncation at every byte (the reference checks every 7th,
    container.rs:1079-1097): never accepted short of the whole file, and the
    refusal kinds equal the oracle's."""
    allowed = {"Truncated", "BadMagic", "UnsupportedVersion", "Malformed", "BadTensorRange",
               "UnknownTensorType"}
    for name in FIXTURES:
        b = gguf_fixture(name)
        for i in range(len(b)):
            got, want = parse_kinds(b[:i])
            assert got is not None and got <= allowed, (name, i, got)
            assert got == want, (name, i, got, want)


def test_table_validation_collects_all_problems():
    """crates/r9v-format/tests/container.rs:1131-1176."""
    r = Raw(3, 3)
    r.u32_kv("dup", 1)
    r.u32_kv("dup", 2)
    r.u32_kv("general.alignment", 48)
    r.tensor("t", [32], 8, 0)
    r.tensor("t", [32], 8, 0)
    r.tensor("mystery", [4], 4, 0)
    r.data(64)
    with pytest.raises(gguf.GgufError) as e:
        gguf.GgufFile.parse(bytes(r.bytes))
    msg = str(e.value)
    for text in ("duplicate metadata key", "duplicate tensor name", "invalid alignment",
                 "unknown tensor type code 4"):
        assert text in msg, msg
    assert {"DuplicateKey", "DuplicateTensor", "InvalidAlignment", "UnknownTensorType"} <= e.value.kinds
    assert parse_kinds(bytes(r.bytes))[1] == e.value.kinds
    r = Raw(2, 0)
    r.tensor("first", [32], 8, 0)
    r.tensor("second", [32], 8, 16)
    r.data(128)
    expect(bytes(r.bytes), {"BadTensorRange"})
    with pytest.raises(gguf.GgufError) as e:
        gguf.GgufFile.parse(bytes(r.bytes))
    assert "overlaps" in str(e.value)


def test_wire_sizing_validates_dims():
    """crates/r9v-format/tests/container.rs:1801-1865: empty dims, a zero
    dimension and an indivisible innermost dimension are Malformed."""
    for dims in ([], [0, 32], [16, 1]):
        r = Raw(1, 0)
        r.tensor("bad", dims, 2, 0)
        r.data(64)
        expect(bytes(r.bytes), {"Malformed"})


def test_every_tensor_offset_alignment():
    """crates/r9v-format/tests/container.rs:1867-1900."""
    r = Raw(1, 0)
    r.tensor("misaligned", [32, 1], 2, 1)
    r.data(128)
    expect(bytes(r.bytes), {"BadTensorRange"}, text="not a multiple of alignment 32")
    r = Raw(1, 1)
    r.u32_kv("general.alignment", 64)
    r.tensor("misaligned64", [32, 1], 2, 32)
    r.data(256)
    expect(bytes(r.bytes), {"BadTensorRange"}, text="not a multiple of alignment 64")


def test_alignment_key_type_and_split_key_coherence():
    """general.alignment must be UINT32 (container.rs:1076-1090); split.*
    declarations must be present, typed and coherent (:1146-1240)."""
    r = Raw(0, 1)
    r.kv("general.alignment", 10, struct.pack("<Q", 64))
    expect(bytes(r.bytes), {"KvTypeMismatch"})
    r = Raw(0, 1)
    r.kv("split.no", 2, struct.pack("<H", 0))
    expect(bytes(r.bytes), {"MissingKey"})
    base = [("split.no", (2, 1)), ("split.count", (2, 1)), ("split.tensors.count", (5, 0))]
    expect(build(base, []), {"Malformed"})               # single shard with split.no 1
    base = [("split.no", (2, 0)), ("split.count", (2, 0)), ("split.tensors.count", (5, 0))]
    expect(build(base, []), {"Malformed"})               # split.count 0
    base = [("split.no", (2, 0)), ("split.count", (2, 2)), ("split.tensors.count", (5, -1))]
    expect(build(base, []), {"Malformed"})
    base = [("split.no", (2, 0)), ("split.count", (2, 1)), ("split.tensors.count", (5, 0))]
    assert len(gguf.GgufFile.parse(build(base, [])).kvs()) == 3


def test_native_containers_are_refused():
    r = Raw(0, 1)
    r.u32_kv("r9v.format_version", 1)
    expect(bytes(r.bytes), {"Native"})
    r = Raw(1, 0)
    r.tensor("w", [256, 4], 1003, 0)
    r.data(4096)
    expect(bytes(r.bytes), {"Native"})
    r = Raw(1, 0)
    r.tensor("w", [256, 4], 1023, 0)            # beyond the native range: unknown
    r.data(4096)
    expect(bytes(r.bytes), {"UnknownTensorType"})


def test_parse_metadata_only():
    """GgufFile::parse_metadata_only (container.rs:942): the tables alone,
    ranges checked against the given file size."""
    b = gguf_fixture("a25_standard")
    o = GO.parse(b)
    f = gguf.GgufFile.parse_metadata_only(b[:o["ranges"][5]], len(b))
    same_tables(f, o)
    expect(b[:o["ranges"][5]], {"BadTensorRange"}, file_size=len(b) - 32)
    expect(b[:o["ranges"][5]], {"Malformed"}, file_size=o["data_start"] - 1)


# ------------------------------------------------ differential and layout pins

@pytest.mark.parametrize("name", FIXTURES)
def test_fixture_tables_equal_oracle_and_rebuild_byte_for_byte(name):
    b = gguf_fixture(name)
    o = GO.parse(b)
    same_tables(gguf.GgufFile.parse(b), o)
    assert rebuild(o, b) == b


@pytest.mark.parametrize("name", FIXTURES)
def test_mutated_fixtures_agree_with_oracle(name):
    """Seeded single-byte mutations inside the header and tables: the C++
    reader accepts exactly what the oracle accepts, refuses with the same
    problem kinds, and reads the same tables."""
    b = gguf_fixture(name)
    table_end = GO.parse(b)["ranges"][5]
    rng = random.Random(0x6767 + len(b))
    accepted = refused = 0
    for _ in range(600):
        m = bytearray(b)
        pos = rng.randrange(table_end)
        m[pos] = rng.choice([0, 1, 2, 0x7F, 0x80, 0xFF, m[pos] ^ (1 << rng.randrange(8))])
        got, want = parse_kinds(bytes(m))
        assert got == want, (name, pos, got, want)
        if got is None:
            accepted += 1
            same_tables(gguf.GgufFile.parse(bytes(m)), GO.parse(bytes(m)))
        else:
            refused += 1
    assert refused > 0 and accepted > 0


# ---------------------------------------------------------------- hashing

def test_xxh3_64_matches_libxxhash():
    xxhash = pytest.importorskip("xxhash")
    rng = random.Random(7)
    data = bytes(rng.getrandbits(8) for _ in range(20000))
    lengths = list(range(0, 1100)) + [2047, 2048, 2049, 4096, 4160, 16383, 16384, 20000]
    for n in lengths:
        assert gguf.xxh3_64(data[:n]) == xxhash.xxh3_64_intdigest(data[:n]), n
    big = bytes(rng.getrandbits(8) for _ in range(1 << 20))
    assert gguf.xxh3_64(big) == xxhash.xxh3_64_intdigest(big)


# ---------------------------------------------------------------- binding

def test_type_table_matches_quant_sizes():
    lib = ffi.load()
    import ctypes
    for code in range(0, 1100):
        bl, bb = ctypes.c_uint32(), ctypes.c_uint32()
        rc = lib.r9vx_gguf_type_size(code, ctypes.byref(bl), ctypes.byref(bb))
        if code in GO.QUANT_SIZES:
            assert rc == 0 and (bl.value, bb.value) == GO.QUANT_SIZES[code]
        else:
            assert rc == -2  # R9VX_ERR_UNSUPPORTED
    assert gguf.type_name(12) == "Q4_K" and gguf.type_name(23) == "IQ4_XS" and gguf.type_name(5) == "UNKNOWN"


def _model_file():
    q4k = bytes((7 * i) & 0xFF for i in range(3 * 8 * 144))     # 3 rows x 8 blocks
    e, dff, dm = 3, 256, 512
    gate = bytes(e * dff * (dm // 256) * 136)
    down = bytes(e * dm * (dff // 256) * 144)
    tensors = [
        ("blk.0.attn_q.weight", (2048, 3), 12, q4k),
        ("blk.0.ffn_gate_exps.weight", (dm, dff, e), 23, gate),
        ("blk.0.ffn_up_exps.weight", (dm, dff, e), 23, gate),
        ("blk.0.ffn_gate_up_exps.weight", (dm, 2 * dff, e), 23, gate + gate),
        ("blk.0.ffn_down_exps.weight", (dff, dm, e), 12, down),
        ("token_embd.weight", (32, 3), 8, bytes(102)),
        ("blk.0.attn_k_f16.weight", (256, 2), 1, bytes(1024)),
        ("blk.0.attn_v.weight", (512, 2), 8, bytes(2 * 16 * 34)),
        ("blk.0.ffn_up_bad.weight", (dm, dff, e), 12, bytes(e * dff * (dm // 256) * 144)),
        ("blk.0.attn_o_iq3.weight", (512, 2), 21, bytes(2 * 2 * 110)),
        ("blk.0.ffn_gate_iq3_exps.weight", (dm, dff, e), 21, bytes(e * dff * (dm // 256) * 110)),
        ("blk.0.ffn_down_iq3_exps.weight", (dff, dm, e), 21, bytes(e * dm * (dff // 256) * 110)),
        ("blk.0.ffn_gate_q8_exps.weight", (dm, dff, e), 8, bytes(e * dff * (dm // 32) * 34)),
        ("blk.0.ffn_down_q6_exps.weight", (dff, dm, e), 14, bytes(e * dm * (dff // 256) * 210)),
        ("blk.0.ffn_down_f16_exps.weight", (dff, dm, e), 1, bytes(e * dm * dff * 2)),
    ]
    return build([("general.architecture", (8, "llama"))], tensors)


def test_matmul_and_moe_ffn_statics_from_a_checkpoint():
    f = gguf.GgufFile.parse(_model_file())
    st = f.matmul_static("blk.0.attn_q.weight", m_bucket=5)
    assert (st.n, st.k, st.w_scheme, st.m_bucket) == (3, 2048, ffi.Q4_K, 5)
    with pytest.raises(gguf.GgufError, match="K=32; the matmul kernels take K in multiples of 256"):
        f.matmul_static("token_embd.weight")
    with pytest.raises(gguf.GgufError, match="is F16"):
        f.matmul_static("blk.0.attn_k_f16.weight")
    st8 = f.matmul_static("blk.0.attn_v.weight")
    assert (st8.n, st8.k, st8.w_scheme) == (2, 512, ffi.Q8_0)
    with pytest.raises(gguf.GgufError, match="not a .K, N. matrix"):
        f.matmul_static("blk.0.ffn_gate_exps.weight")
    with pytest.raises(gguf.GgufError, match="no tensor named"):
        f.matmul_static("absent")
    s = f.moe_ffn_static("blk.0.ffn_gate_exps.weight", "blk.0.ffn_up_exps.weight",
                         "blk.0.ffn_down_exps.weight", t_bucket=8, k=2)
    # the file's GGUF types IQ4_XS (23) and Q4_K (12) become SchemeId codes I4Xs (15) and I4K (3)
    assert (s.e_local, s.dm, s.dff, s.gate_up.scheme, s.down.scheme, s.k_topk) == (3, 512, 256, 15, 3, 2)
    fused = f.moe_ffn_static("blk.0.ffn_gate_up_exps.weight", None, "blk.0.ffn_down_exps.weight", 8, 2)
    assert (fused.e_local, fused.dm, fused.dff) == (3, 512, 256)
    with pytest.raises(gguf.GgufError, match="must agree in dims and type"):
        f.moe_ffn_static("blk.0.ffn_gate_exps.weight", "blk.0.ffn_up_bad.weight", "blk.0.ffn_down_exps.weight",
                         8, 2)
    assert (st.w_dtype, st.w_layout) == (ffi.I4, ffi.LAYOUT_GGUF_WIRE)
    assert (st8.w_dtype, st8.w_layout) == (ffi.I8, ffi.LAYOUT_SPLIT)
    st3 = f.matmul_static("blk.0.attn_o_iq3.weight")
    assert (st3.n, st3.k, st3.w_scheme) == (2, 512, ffi.IQ3_S)
    assert (st3.w_dtype, st3.w_layout) == (ffi.I4, ffi.LAYOUT_IQ3S_112)
    s3 = f.moe_ffn_static("blk.0.ffn_gate_iq3_exps.weight", "blk.0.ffn_gate_iq3_exps.weight",
                          "blk.0.ffn_down_exps.weight", t_bucket=8, k=2)
    assert (s3.gate_up.scheme, s3.down.scheme) == (ffi.IQ3_S, ffi.Q4_K)
    assert (s3.gate_up.layout, s3.down.layout) == (ffi.LAYOUT_IQ3S_112, ffi.LAYOUT_GGUF_WIRE)
    assert (s.gate_up.layout, s.down.layout, s.gate_up.dtype) == (ffi.LAYOUT_GGUF_WIRE, ffi.LAYOUT_GGUF_WIRE, ffi.I4)
    s4 = f.moe_ffn_static("blk.0.ffn_gate_exps.weight", "blk.0.ffn_up_exps.weight",
                          "blk.0.ffn_down_iq3_exps.weight", 8, 2)
    assert (s4.down.scheme, s4.down.dtype, s4.down.layout) == (ffi.IQ3_S, ffi.I4, ffi.LAYOUT_IQ3S_112)
    s5 = f.moe_ffn_static("blk.0.ffn_gate_q8_exps.weight", "blk.0.ffn_gate_q8_exps.weight",
                          "blk.0.ffn_down_q6_exps.weight", 8, 2)
    assert (s5.gate_up.scheme, s5.gate_up.dtype, s5.gate_up.layout) == (ffi.Q8_0, ffi.I8, ffi.LAYOUT_SPLIT)
    assert (s5.down.scheme, s5.down.dtype, s5.down.layout) == (ffi.Q6_K, ffi.I8, ffi.LAYOUT_SPLIT)
    with pytest.raises(gguf.GgufError, match="experts must be Q4_K .12., IQ4_XS .23., IQ3_S .21., Q8_0 .8. or Q6_K"):
        f.moe_ffn_static("blk.0.ffn_gate_exps.weight", "blk.0.ffn_up_exps.weight",
                         "blk.0.ffn_down_f16_exps.weight", 8, 2)
    with pytest.raises(gguf.GgufError, match="must be \\{256, 512, 3\\}"):
        f.moe_ffn_static("blk.0.ffn_gate_exps.weight", "blk.0.ffn_up_exps.weight", "blk.0.ffn_gate_exps.weight",
                         8, 2)


def test_upload_sizes_iq3s_for_its_device_blocks():
    """An IQ3_S upload writes 112-byte device blocks, so a destination sized
    for the 110-byte file blocks is refused before anything is copied, and
    Q8_0 / Q6_K are pointed at the split upload (no device is touched)."""
    f = gguf.GgufFile.parse(_model_file())
    b = _model_file()
    lib = ffi.load()
    info = f.tensor("blk.0.attn_o_iq3.weight")
    ptr = ctypes.create_string_buffer(b, len(b))
    rc = lib.r9vx_gguf_upload(f._h, ptr, len(b), b"blk.0.attn_o_iq3.weight", ctypes.c_void_p(0x1000),
                              info.nbytes, None)
    msg = lib.r9vx_last_error().decode()
    assert rc == -1 and f"needs {info.nbytes // 110 * 112}" in msg and "112-byte IQ3_S device blocks" in msg, msg
    assert gguf.device_bytes(info) == info.nbytes // 110 * 112
    rc = lib.r9vx_gguf_upload(f._h, ptr, len(b), b"blk.0.attn_v.weight", ctypes.c_void_p(0x1000), 1 << 20, None)
    assert rc == -2 and "r9vx_gguf_upload_split" in lib.r9vx_last_error().decode()
