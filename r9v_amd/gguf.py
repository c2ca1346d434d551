"""GGUF ingestion: the host-side mirror of R9V's container API over libr9vx.

`GgufFile` and `ShardSet` keep the names and meaning of
crates/r9v-format/src/container.rs (GgufFile :902-2160, ShardSet :3469-3614):
`GgufFile.parse(bytes)` raises `GgufError` where the reference returns a
FormatError, `kv(key)` returns a `KvValue`, `tensors()` the tensor-info rows
in file order, `tensor_bytes(name, bytes)` the checked entry slice and
`entry_xxh3` its XXH3-64.  The parsing, validation and hashing all run in the
C++ library (include/r9vx_gguf.h); this module only converts values.

`load_matmul_weight` / `load_moe_experts` are the load step of this path: they
bind a checkpoint tensor to the variant key of the matmul / moe_ffn launch and
copy its GGUF wire blocks into device memory, which is the layout the kernels
read.
"""
from __future__ import annotations

import ctypes
import struct
from dataclasses import dataclass

from . import ffi

# problem kinds (R9VX_GGUF_P_*), one per FormatError variant
P_TRUNCATED, P_BAD_MAGIC, P_BAD_VERSION, P_MALFORMED = 1, 2, 4, 8
P_DUPLICATE_KEY, P_DUPLICATE_TENSOR, P_BAD_ALIGNMENT, P_KV_TYPE = 16, 32, 64, 128
P_MISSING_KEY, P_UNKNOWN_TYPE, P_BAD_RANGE, P_OVERFLOW, P_NATIVE = 256, 512, 1024, 2048, 4096
PROBLEM_NAMES = {
    P_TRUNCATED: "Truncated", P_BAD_MAGIC: "BadMagic", P_BAD_VERSION: "UnsupportedVersion",
    P_MALFORMED: "Malformed", P_DUPLICATE_KEY: "DuplicateKey", P_DUPLICATE_TENSOR: "DuplicateTensor",
    P_BAD_ALIGNMENT: "InvalidAlignment", P_KV_TYPE: "KvTypeMismatch", P_MISSING_KEY: "MissingKey",
    P_UNKNOWN_TYPE: "UnknownTensorType", P_BAD_RANGE: "BadTensorRange", P_OVERFLOW: "Overflow",
    P_NATIVE: "Native",
}

# KvType codes (container.rs:60-127)
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARRAY, U64, I64, F64 = range(13)
KV_TYPE_NAMES = ["UINT8", "INT8", "UINT16", "INT16", "UINT32", "INT32", "FLOAT32", "BOOL",
                 "STRING", "ARRAY", "UINT64", "INT64", "FLOAT64"]


class GgufError(ffi.R9vxError):
    """A refused parse / lookup; `kinds` names the FormatError variants found."""

    def __init__(self, code: int, message: str, problems: int = 0):
        super().__init__(code, message)
        self.problems = problems
        self.kinds = {name for bit, name in PROBLEM_NAMES.items() if problems & bit}


class _Value(ctypes.Structure):
    _fields_ = [("type", ctypes.c_uint32), ("_pad", ctypes.c_uint32), ("bits", ctypes.c_uint64),
                ("str", ctypes.c_void_p), ("str_len", ctypes.c_uint64)]


class _Tensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_void_p), ("name_len", ctypes.c_uint64),
                ("dims", ctypes.POINTER(ctypes.c_uint64)),
                ("n_dims", ctypes.c_uint32), ("type", ctypes.c_uint32), ("offset", ctypes.c_uint64),
                ("nbytes", ctypes.c_uint64), ("block_len", ctypes.c_uint32),
                ("block_bytes", ctypes.c_uint32)]


@dataclass(frozen=True)
class KvValue:
    """A decoded metadata value (KvValue, container.rs:178-212): `type` is the
    KvType code; arrays carry `elem` and a tuple `value`."""
    type: int
    value: object
    elem: int | None = None


@dataclass(frozen=True)
class TensorInfo:
    """One tensor-info row (TensorInfo, container.rs:701-728); `dims` in file
    order (innermost first), `shape` outer-first."""
    name: str
    dims: tuple
    dtype: int
    offset: int
    nbytes: int
    block_len: int
    block_bytes: int

    @property
    def shape(self) -> tuple:
        return tuple(reversed(self.dims))

    @property
    def type_name(self) -> str:
        return type_name(self.dtype)


def _raise(rc: int):
    lib = ffi.load()
    raise GgufError(rc, lib.r9vx_last_error().decode(errors="replace"), lib.r9vx_gguf_last_problems())


def _buf(data):
    """(pointer, length, keepalive) for bytes / bytearray / memoryview / numpy."""
    if isinstance(data, bytes):
        return ctypes.cast(ctypes.c_char_p(data), ctypes.c_void_p), len(data), data
    mv = memoryview(data).cast("B")
    if mv.readonly:
        raw = bytes(mv)
        return ctypes.cast(ctypes.c_char_p(raw), ctypes.c_void_p), len(raw), raw
    arr = (ctypes.c_uint8 * len(mv)).from_buffer(mv)
    return ctypes.cast(arr, ctypes.c_void_p), len(mv), (arr, mv)


def _decode_item(v: _Value):
    t = v.type
    if t == STR:
        return ctypes.string_at(v.str, v.str_len).decode("utf-8")
    b = v.bits
    if t == F32:
        return struct.unpack("<f", struct.pack("<I", b & 0xFFFFFFFF))[0]
    if t == F64:
        return struct.unpack("<d", struct.pack("<Q", b))[0]
    if t == BOOL:
        return bool(b)
    if t in (I8, I16, I32, I64):
        return b - (1 << 64) if b >= (1 << 63) else b
    return b


def type_name(code: int) -> str:
    return ffi.load().r9vx_gguf_type_name(code).decode()


def xxh3_64(data) -> int:
    ptr, n, _keep = _buf(data)
    return ffi.load().r9vx_xxh3_64(ptr, n)


class GgufFile:
    """One parsed GGUF shard (GgufFile, container.rs:902)."""

    def __init__(self, handle):
        self._h = handle
        self._tensors = None

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        if h:
            ffi.load().r9vx_gguf_free(h)

    @classmethod
    def parse(cls, data) -> "GgufFile":
        """GgufFile::parse (container.rs:930)."""
        ptr, n, _keep = _buf(data)
        h = ctypes.c_void_p()
        rc = ffi.load().r9vx_gguf_parse(ptr, n, ctypes.byref(h))
        if rc != 0:
            _raise(rc)
        return cls(h)

    @classmethod
    def parse_metadata_only(cls, data, file_size: int) -> "GgufFile":
        """GgufFile::parse_metadata_only (container.rs:942)."""
        ptr, n, _keep = _buf(data)
        h = ctypes.c_void_p()
        rc = ffi.load().r9vx_gguf_parse_table(ptr, n, file_size, ctypes.byref(h))
        if rc != 0:
            _raise(rc)
        return cls(h)

    @classmethod
    def parse_file(cls, path) -> "GgufFile":
        """GgufFile::parse_file (container.rs:1028): reads and parses `path`."""
        with open(path, "rb") as fh:
            return cls.parse(fh.read())

    # header
    def version(self) -> int:
        return ffi.load().r9vx_gguf_version(self._h)

    def alignment(self) -> int:
        return ffi.load().r9vx_gguf_alignment(self._h)

    def data_start(self) -> int:
        return ffi.load().r9vx_gguf_data_start(self._h)

    def file_size(self) -> int:
        return ffi.load().r9vx_gguf_file_size(self._h)

    def _ranges(self):
        out = (ctypes.c_uint64 * 6)()
        ffi.load().r9vx_gguf_ranges(self._h, out)
        return list(out)

    def header_range(self):
        return tuple(self._ranges()[0:2])

    def kv_range(self):
        return tuple(self._ranges()[2:4])

    def ti_range(self):
        return tuple(self._ranges()[4:6])

    def is_native(self) -> bool:
        return bool(ffi.load().r9vx_gguf_is_native(self._h))

    def is_standard_gguf(self) -> bool:
        return not self.is_native()

    # metadata
    def _kv_at(self, i: int):
        lib = ffi.load()
        key, klen = ctypes.c_void_p(), ctypes.c_uint64()
        t, elem, count = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint64()
        rc = lib.r9vx_gguf_kv_info(self._h, i, ctypes.byref(key), ctypes.byref(klen), ctypes.byref(t),
                                   ctypes.byref(elem), ctypes.byref(count))
        if rc != 0:
            _raise(rc)
        v = _Value()
        items = []
        for j in range(count.value):
            rc = lib.r9vx_gguf_kv_value(self._h, i, j, ctypes.byref(v))
            if rc != 0:
                _raise(rc)
            items.append(_decode_item(v))
        name = ctypes.string_at(key, klen.value).decode("utf-8")
        if t.value == ARRAY:
            return name, KvValue(ARRAY, tuple(items), elem.value)
        return name, KvValue(t.value, items[0])

    def kvs(self):
        """Metadata in file order as (key, KvValue) pairs."""
        return [self._kv_at(i) for i in range(ffi.load().r9vx_gguf_n_kv(self._h))]

    def kv(self, key: str):
        i = ffi.load().r9vx_gguf_find_kv(self._h, key.encode())
        return None if i < 0 else self._kv_at(i)[1]

    # tensors
    def tensors(self):
        if self._tensors is None:
            lib = ffi.load()
            rows = []
            t = _Tensor()
            for i in range(lib.r9vx_gguf_n_tensors(self._h)):
                rc = lib.r9vx_gguf_tensor_at(self._h, i, ctypes.byref(t))
                if rc != 0:
                    _raise(rc)
                rows.append(_info(t))
            self._tensors = rows
        return self._tensors

    def tensor(self, name: str):
        i = ffi.load().r9vx_gguf_find_tensor(self._h, name.encode())
        return None if i < 0 else self.tensors()[i]

    def tensor_bytes(self, name: str, data) -> bytes:
        """GgufFile::tensor_bytes (container.rs:2074): a copy of the entry."""
        ptr, n, _keep = _buf(data)
        out, nb = ctypes.c_void_p(), ctypes.c_uint64()
        rc = ffi.load().r9vx_gguf_tensor_bytes(self._h, name.encode(), ptr, n, ctypes.byref(out),
                                               ctypes.byref(nb))
        if rc != 0:
            _raise(rc)
        return ctypes.string_at(out, nb.value)

    def entry_xxh3(self, name: str, data) -> int:
        """GgufFile::entry_xxh3 (container.rs:2136)."""
        ptr, n, _keep = _buf(data)
        h = ctypes.c_uint64()
        rc = ffi.load().r9vx_gguf_entry_xxh3(self._h, name.encode(), ptr, n, ctypes.byref(h))
        if rc != 0:
            _raise(rc)
        return h.value

    def matmul_static(self, name: str, m_bucket: int = 8, in_dtype: int = ffi.BF16,
                      out_dtype: int = ffi.F32) -> ffi.MatmulStatic:
        """The matmul variant key for weight `name` ({K, N} Q4_K / IQ4_XS)."""
        st = ffi.matmul_static(256, 256, ffi.Q4_K, in_dtype, out_dtype, m_bucket=m_bucket)
        rc = ffi.load().r9vx_gguf_matmul_static(self._h, name.encode(), ctypes.byref(st))
        if rc != 0:
            _raise(rc)
        return st

    def moe_ffn_static(self, gate: str, up: str | None, down: str, t_bucket: int, k: int,
                       shared: int = 0) -> ffi.MoeFfnStatic:
        """The moe_ffn variant key for stacked expert tensors (up=None: fused gate_up)."""
        st = ffi.ffn_static(t_bucket, 1, k, 256, 256, shared=shared)
        rc = ffi.load().r9vx_gguf_moe_ffn_static(self._h, gate.encode(), None if up is None else up.encode(),
                                                 down.encode(), ctypes.byref(st))
        if rc != 0:
            _raise(rc)
        return st


def _info(t: _Tensor) -> TensorInfo:
    return TensorInfo(ctypes.string_at(t.name, t.name_len).decode("utf-8"), tuple(t.dims[i] for i in range(t.n_dims)), t.type, t.offset,
                      t.nbytes, t.block_len, t.block_bytes)


class ShardSet:
    """An ordered split set (ShardSet, container.rs:3469)."""

    def __init__(self, handle, shards):
        self._h = handle
        self._shards = list(shards)

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        if h:
            ffi.load().r9vx_gguf_shards_free(h)

    @classmethod
    def open(cls, shards) -> "ShardSet":
        shards = list(shards)
        arr = (ctypes.c_void_p * max(1, len(shards)))(*[s._h for s in shards])
        h = ctypes.c_void_p()
        rc = ffi.load().r9vx_gguf_shards_open(arr, len(shards), ctypes.byref(h))
        if rc != 0:
            _raise(rc)
        return cls(h, shards)

    def shards(self):
        return list(self._shards)

    def __len__(self) -> int:
        return ffi.load().r9vx_gguf_shards_len(self._h)

    def is_empty(self) -> bool:
        return len(self) == 0

    def tensor_at(self, i: int):
        """(shard index, TensorInfo) of merged row i, or None."""
        if i < 0 or i >= len(self):
            return None
        shard, t = ctypes.c_uint32(), _Tensor()
        rc = ffi.load().r9vx_gguf_shards_tensor_at(self._h, i, ctypes.byref(shard), ctypes.byref(t))
        if rc != 0:
            _raise(rc)
        return shard.value, _info(t)

    def tensor(self, name: str):
        """(shard index, TensorInfo) of `name`, or None."""
        i = ffi.load().r9vx_gguf_shards_find(self._h, name.encode())
        return None if i < 0 else (i, self._shards[i].tensor(name))


# ------------------------------------------------------------------ loading

def device_bytes(info: TensorInfo) -> int:
    """Bytes of a tensor in its device layout (IQ3_S: 112-byte blocks)."""
    return info.nbytes // 110 * ffi.IQ3S_DEV_BYTES if info.dtype == ffi.GGML_IQ3_S else info.nbytes


def upload(file: GgufFile, data, name: str, out=None, stream=None):
    """Loads tensor `name` into a device uint8 tensor (`out`, or a new one) in
    its device layout -- Q4_K / IQ4_XS / F32 bytes as stored, IQ3_S repacked
    into 112-byte blocks -- and returns it once the copy is done."""
    import torch

    info = file.tensor(name)
    if info is None:
        raise GgufError(-1, f"no tensor named {name!r}")
    if out is None:
        out = torch.empty(device_bytes(info), dtype=torch.uint8, device="cuda")
    ptr, n, _keep = _buf(data)
    rc = ffi.load().r9vx_gguf_upload(file._h, ptr, n, name.encode(), ctypes.c_void_p(out.data_ptr()),
                                     out.numel() * out.element_size(), ffi._stream(torch, stream))
    if rc != 0:
        _raise(rc)
    torch.cuda.current_stream().synchronize() if stream is None else stream.synchronize()
    return out


def upload_gate_up(gate_file: GgufFile, gate_data, gate: str, up_file: GgufFile, up_data, up: str,
                   out=None, stream=None):
    """Stacks gate and up expert tensors into w_gate_up [E, 2*Dff, Dm] on the device."""
    import torch

    info = gate_file.tensor(gate)
    if info is None:
        raise GgufError(-1, f"no tensor named {gate!r}")
    if out is None:
        out = torch.empty(2 * device_bytes(info), dtype=torch.uint8, device="cuda")
    gp, gn, _gk = _buf(gate_data)
    up_, un, _uk = _buf(up_data)
    rc = ffi.load().r9vx_gguf_upload_gate_up(gate_file._h, gp, gn, gate.encode(), up_file._h, up_, un,
                                             up.encode(), ctypes.c_void_p(out.data_ptr()),
                                             out.numel() * out.element_size(), ffi._stream(torch, stream))
    if rc != 0:
        _raise(rc)
    torch.cuda.current_stream().synchronize() if stream is None else stream.synchronize()
    return out


def upload_gate_up_split(gate_file: GgufFile, gate_data, gate: str, up_file: GgufFile, up_data, up: str,
                         stream=None):
    """Q8_0 / Q6_K gate and up expert tensors stacked into the split layout
    of w_gate_up [E, 2*Dff, Dm]: (body uint8, scales int16 of f16 d bits)."""
    import torch

    info = gate_file.tensor(gate)
    if info is None:
        raise GgufError(-1, f"no tensor named {gate!r}")
    nb = 2 * (info.nbytes // info.block_bytes)
    body = torch.empty(nb * (info.block_bytes - 2), dtype=torch.uint8, device="cuda")
    scales = torch.empty(nb, dtype=torch.int16, device="cuda")
    gp, gn, _gk = _buf(gate_data)
    up_, un, _uk = _buf(up_data)
    rc = ffi.load().r9vx_gguf_upload_gate_up_split(gate_file._h, gp, gn, gate.encode(), up_file._h, up_, un,
                                                   up.encode(), ctypes.c_void_p(body.data_ptr()), body.numel(),
                                                   ctypes.c_void_p(scales.data_ptr()), 2 * scales.numel(),
                                                   ffi._stream(torch, stream))
    if rc != 0:
        _raise(rc)
    return body, scales


def upload_split(file: GgufFile, data, name: str, stream=None):
    """A Q8_0 / Q6_K tensor in the split device layout: (body uint8, scales
    int16 holding the f16 d bits); non-finite scales are refused on the host."""
    import torch

    info = file.tensor(name)
    if info is None:
        raise GgufError(-1, f"no tensor named {name!r}")
    nb = info.nbytes // info.block_bytes
    body = torch.empty(nb * (info.block_bytes - 2), dtype=torch.uint8, device="cuda")
    scales = torch.empty(nb, dtype=torch.int16, device="cuda")
    ptr, n, _keep = _buf(data)
    rc = ffi.load().r9vx_gguf_upload_split(file._h, ptr, n, name.encode(), ctypes.c_void_p(body.data_ptr()),
                                           body.numel(), ctypes.c_void_p(scales.data_ptr()), 2 * scales.numel(),
                                           ffi._stream(torch, stream))
    if rc != 0:
        _raise(rc)
    return body, scales


def load_matmul_weight(file: GgufFile, data, name: str, m_bucket: int = 8, in_dtype: int = ffi.BF16,
                       out_dtype: int = ffi.F32, validate: bool = True):
    """(MatmulStatic, w, w_scales) on the device for weight `name`: Q4_K /
    IQ4_XS wire blocks (w_scales None), the Q8_0 / Q6_K split layout, or
    IQ3_S repacked on the host into 112-byte blocks (w_scales None).  With
    `validate` the load-time scale check (check_wire_f16,
    crates/r9v-format/src/ggml.rs:421) refuses a block with a non-finite scale
    (on the device for wire blocks; the split and IQ3_S uploads always check)."""
    st = file.matmul_static(name, m_bucket=m_bucket, in_dtype=in_dtype, out_dtype=out_dtype)
    if st.w_scheme in ffi.SPLIT_SCHEMES:
        w, w_scales = upload_split(file, data, name)
        return st, w, w_scales
    w = upload(file, data, name)
    if validate and st.w_scheme != ffi.IQ3_S:
        bad = ffi.validate_weights(w, st.w_scheme, st.n, st.k)
        if bad:
            raise GgufError(-1, f"{name}: {bad} block(s) carry a non-finite scale")
    return st, w, None


class MoeExperts(tuple):
    """(static, w_gate_up, w_down) -- unpacks as that triple -- plus the split
    layout's d arrays `w_gate_up_scales` / `w_down_scales` (None unless the
    projection is Q8_0 / Q6_K)."""

    def __new__(cls, st, w_gate_up, w_down, w_gate_up_scales=None, w_down_scales=None):
        self = super().__new__(cls, (st, w_gate_up, w_down))
        self.w_gate_up_scales, self.w_down_scales = w_gate_up_scales, w_down_scales
        return self


def load_moe_experts(file: GgufFile, data, gate: str, up: str | None, down: str, t_bucket: int,
                     k: int, validate: bool = True) -> MoeExperts:
    """The experts of one shard on the device from stacked expert tensors
    (up=None takes a fused ffn_gate_up_exps tensor): Q4_K / IQ4_XS wire
    blocks, IQ3_S repacked into 112-byte blocks, Q8_0 / Q6_K in the split
    layout (body + d array)."""
    st = file.moe_ffn_static(gate, up, down, t_bucket, k)
    gs = ds = None
    if st.gate_up.scheme in ffi.SPLIT_SCHEMES:
        w_gate_up, gs = (upload_split(file, data, gate) if up is None
                         else upload_gate_up_split(file, data, gate, file, data, up))
    elif up is None:
        w_gate_up = upload(file, data, gate)
    else:
        w_gate_up = upload_gate_up(file, data, gate, file, data, up)
    if st.down.scheme in ffi.SPLIT_SCHEMES:
        w_down, ds = upload_split(file, data, down)
    else:
        w_down = upload(file, data, down)
    if validate:  # IQ3_S and split blocks were checked on the host by their uploads
        bad = 0
        if st.gate_up.scheme in (ffi.Q4_K, ffi.IQ4_XS):
            bad += ffi.validate_weights(w_gate_up, st.gate_up.scheme, st.e_local * 2 * st.dff, st.dm)
        if st.down.scheme in (ffi.Q4_K, ffi.IQ4_XS):
            bad += ffi.validate_weights(w_down, st.down.scheme, st.e_local * st.dm, st.dff)
        if bad:
            raise GgufError(-1, f"{gate}/{down}: {bad} expert block(s) carry a non-finite scale")
    return MoeExperts(st, w_gate_up, w_down, gs, ds)


def load_router_weight(file: GgufFile, data, name: str):
    """(E, dm, device weight in the k4 layout of ffi.router_repack) for an F32
    router tensor (ffn_gate_inp, file dims {dm, E}), for ffi.moe_route_hidden."""
    import torch

    info = file.tensor(name)
    if info is None:
        raise GgufError(-1, f"no tensor named {name!r}")
    if info.dtype != 0 or len(info.dims) != 2:
        raise GgufError(-2, f"{name}: the router weight must be a 2-D F32 tensor, got {info.type_name} {info.dims}")
    dm, e = info.dims
    raw = upload(file, data, name)
    return e, dm, ffi.router_repack(raw.view(torch.float32).reshape(e, dm))
