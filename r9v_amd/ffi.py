"""ctypes binding of libr9vx.so (include/r9vx.h) with torch device-memory plumbing.

This is the host-side mirror of R9V's op surface for this path: `matmul`,
`moe_route` and `moe_ffn` take the same operands with the same meaning as the
T0 executors (crates/r9v-t0/src/lib.rs:280-348 execute_matmul_op,
crates/r9v-t0/src/moe_route.rs:89 moe_route, crates/r9v-t0/src/moe_ffn.rs:75
moe_ffn) and raise R9vxError where those return a T0Error.  All compute runs in
the HIP library; there is no CPU or PyTorch fallback: a missing library or GPU
raises.
"""
from __future__ import annotations

import ctypes
import pathlib
import struct

PKG = pathlib.Path(__file__).resolve().parent
LIB_PATH = PKG / "libr9vx.so"

# enums (include/r9vx.h)
F32, F16, BF16, I8, I4, U32 = 0, 1, 2, 5, 6, 8
LAYOUT_L0, LAYOUT_L1, LAYOUT_L1S = 1, 2, 3                      # the reference's layouts: refused
LAYOUT_GGUF_WIRE, LAYOUT_SPLIT, LAYOUT_IQ3S_112 = 0x100, 0x101, 0x102
# weight schemes: the reference's SchemeId codes (I4K, I4Xs, I6K, I8B32F, Iq3S;
# crates/r9v-format/src/scheme.rs:115-138), which the statics carry
Q4_K, IQ4_XS, Q6_K, Q8_0, IQ3_S = 3, 15, 11, 5, 17
# GGUF ggml type ids of the same formats (file data only: GgufFile tensor types)
GGML_Q4_K, GGML_IQ4_XS, GGML_Q6_K, GGML_Q8_0, GGML_IQ3_S = 12, 23, 14, 8, 21
SCHEME_OF_GGML = {GGML_Q4_K: Q4_K, GGML_IQ4_XS: IQ4_XS, GGML_Q6_K: Q6_K, GGML_Q8_0: Q8_0, GGML_IQ3_S: IQ3_S}
EPILOGUE_NONE, EPILOGUE_BIAS, EPILOGUE_RESIDUAL, EPILOGUE_SWIGLU = 0, 1, 2, 3
SCORING_SOFTMAX, SCORING_SIGMOID = 0, 1
ACT_SILU = 0
STATUS_NONFINITE, STATUS_DEGENERATE, STATUS_BAD_EXPERT = 1, 2, 4
BLOCK_BYTES = {Q4_K: 144, IQ4_XS: 136, Q6_K: 210, Q8_0: 34, IQ3_S: 110}
BLOCK_LEN = {Q4_K: 256, IQ4_XS: 256, Q6_K: 256, Q8_0: 32, IQ3_S: 256}
SPLIT_SCHEMES = (Q6_K, Q8_0)      # read in the split device layout (body + f16 d array)
IQ3S_DEV_BYTES = 112              # IQ3_S is read as repacked 112-byte blocks (one array)

_P = ctypes.c_void_p
_U32 = ctypes.c_uint32
_U64 = ctypes.c_uint64


class MatmulStatic(ctypes.Structure):
    _fields_ = [("m_bucket", _U32), ("n", _U32), ("k", _U32), ("w_dtype", _U32), ("w_scheme", _U32),
                ("w_layout", _U32), ("in_dtype", _U32), ("act_scheme", _U32), ("out_dtype", _U32),
                ("epilogue", _U32), ("residual_dtype", _U32), ("transpose_w", _U32), ("interleave", _U32),
                ("sparse", _U32)]


class MatmulArgs(ctypes.Structure):
    _fields_ = [("w", _P), ("w_scales", _P), ("w_indices", _P), ("x", _P), ("x_scale", _P),
                ("bias", _P), ("residual", _P), ("y", _P), ("workspace", _P), ("m", _U32),
                ("_tail_pad", _U32)]


class MoeRouteStatic(ctypes.Structure):
    _fields_ = [("t_bucket", _U32), ("e_total", _U32), ("top_k", _U32), ("scoring", _U32),
                ("renormalize", _U32), ("n_group", _U32), ("topk_group", _U32), ("scale_bits", _U32),
                ("has_bias", _U32)]


class MoeRouteArgs(ctypes.Structure):
    _fields_ = [("logits", _P), ("bias", _P), ("expert_ids", _P), ("weights", _P), ("t", _U32),
                ("_tail_pad", _U32)]


class MoeRouteHiddenArgs(ctypes.Structure):
    _fields_ = [("x", _P), ("w_router", _P), ("bias", _P), ("expert_ids", _P), ("weights", _P),
                ("workspace", _P), ("t", _U32), ("dm", _U32)]


class MoeFfnProj(ctypes.Structure):
    _fields_ = [("dtype", _U32), ("scheme", _U32), ("layout", _U32)]


class MoeFfnStatic(ctypes.Structure):
    _fields_ = [("t_bucket", _U32), ("e_local", _U32), ("k_topk", _U32), ("dm", _U32),
                ("dff", _U32), ("gate_up", MoeFfnProj), ("down", MoeFfnProj),
                ("in_dtype", _U32), ("act_scheme", _U32), ("act", _U32), ("out_dtype", _U32),
                ("shared_experts", _U32), ("placement_kind", _U32)]


class MoeFfnArgs(ctypes.Structure):
    _fields_ = [("x", _P), ("expert_ids", _P), ("weights", _P), ("w_gate_up", _P),
                ("w_gate_up_scales", _P), ("w_down", _P), ("w_down_scales", _P), ("y", _P),
                ("sort_workspace", _P), ("t", _U32), ("_tail_pad", _U32)]


# Every function include/r9vx.h declares: (name, argtypes, restype).
EXPORTS = [
    ("r9vx_matmul_launch", [_P, _P, _P], ctypes.c_int),
    ("r9vx_matmul_workspace_bytes", [_P], ctypes.c_size_t),
    ("r9vx_matmul_static_bytes", [_P, _U32], ctypes.c_uint64),
    ("r9vx_matmul_static_flops", [_P, _U32], ctypes.c_uint64),
    ("r9vx_moe_route_launch", [_P, _P, _P], ctypes.c_int),
    ("r9vx_moe_route_launch_ex", [_P, _P, _P, _P], ctypes.c_int),
    ("r9vx_moe_route_status", [_P, _P], ctypes.c_int),
    ("r9vx_status_read", [_P, _P, _P], ctypes.c_int),
    ("r9vx_moe_route_static_bytes", [_P, _U32], ctypes.c_uint64),
    ("r9vx_moe_route_static_flops", [_P, _U32], ctypes.c_uint64),
    ("r9vx_moe_route_hidden_launch", [_P, _P, _P], ctypes.c_int),
    ("r9vx_moe_route_hidden_workspace_bytes", [_P], ctypes.c_size_t),
    ("r9vx_moe_route_hidden_status", [_P, _P, _P, _P], ctypes.c_int),
    ("r9vx_router_repack_launch", [_P, _U32, _U32, _P, _P], ctypes.c_int),
    ("r9vx_moe_ffn_launch", [_P, _P, _P], ctypes.c_int),
    ("r9vx_moe_ffn_launch_noalloc", [_P, _P, _P, _P], ctypes.c_int),
    ("r9vx_moe_ffn_workspace_bytes", [_P], ctypes.c_size_t),
    ("r9vx_moe_ffn_status", [_P, _P, _P, _P], ctypes.c_int),
    ("r9vx_moe_ffn_static_flops", [_P, _U32], ctypes.c_uint64),
    ("r9vx_moe_ffn_static_bytes", [_P, _U32], ctypes.c_uint64),
    ("r9vx_moe_ffn_expert_bytes", [_P], ctypes.c_uint64),
    ("r9vx_moe_sort_launch", [_P, _P, _U32, _P, _P, _P, _P, _P], ctypes.c_int),
    ("r9vx_dequantize_launch", [_U32, _P, _U32, _U32, _P, _P], ctypes.c_int),
    ("r9vx_validate_weights_launch", [_U32, _P, _U32, _U32, _P, _P], ctypes.c_int),
    ("r9vx_repack_launch", [_U32, _P, _U32, _U32, _P, _P, _P], ctypes.c_int),
    ("r9vx_scheme_from_ggml_type", [_U32], _U32),
    ("r9vx_last_error", [], ctypes.c_char_p),
    ("r9vx_abi_version", [], _U32),
    # include/r9vx_probe.h
    ("r9vx_probe_stream_launch", [_P, ctypes.c_uint64, _P, _P], ctypes.c_int),
    ("r9vx_probe_stream_blocks", [ctypes.c_uint64], _U32),
    ("r9vx_probe_mfma_launch", [_U32, _U32, _P, _P], ctypes.c_int),
    ("r9vx_probe_moe_stage_launch", [_P, _P, _U32, _P], ctypes.c_int),
    ("r9vx_probe_expf_check_launch", [_U32, _U32, _P, _P, _P], ctypes.c_int),
    # include/r9vx_gguf.h
    ("r9vx_gguf_parse", [_P, _U64, _P], ctypes.c_int),
    ("r9vx_gguf_parse_table", [_P, _U64, _U64, _P], ctypes.c_int),
    ("r9vx_gguf_free", [_P], None),
    ("r9vx_gguf_last_problems", [], _U32),
    ("r9vx_gguf_version", [_P], _U32),
    ("r9vx_gguf_alignment", [_P], _U64),
    ("r9vx_gguf_data_start", [_P], _U64),
    ("r9vx_gguf_file_size", [_P], _U64),
    ("r9vx_gguf_ranges", [_P, _P], None),
    ("r9vx_gguf_n_kv", [_P], _U64),
    ("r9vx_gguf_find_kv", [_P, ctypes.c_char_p], ctypes.c_int64),
    ("r9vx_gguf_kv_info", [_P, _U64, _P, _P, _P, _P, _P], ctypes.c_int),
    ("r9vx_gguf_kv_value", [_P, _U64, _U64, _P], ctypes.c_int),
    ("r9vx_gguf_n_tensors", [_P], _U64),
    ("r9vx_gguf_find_tensor", [_P, ctypes.c_char_p], ctypes.c_int64),
    ("r9vx_gguf_tensor_at", [_P, _U64, _P], ctypes.c_int),
    ("r9vx_gguf_tensor_bytes", [_P, ctypes.c_char_p, _P, _U64, _P, _P], ctypes.c_int),
    ("r9vx_gguf_entry_xxh3", [_P, ctypes.c_char_p, _P, _U64, _P], ctypes.c_int),
    ("r9vx_gguf_is_native", [_P], ctypes.c_int),
    ("r9vx_gguf_type_size", [_U32, _P, _P], ctypes.c_int),
    ("r9vx_gguf_type_name", [_U32], ctypes.c_char_p),
    ("r9vx_xxh3_64", [_P, _U64], _U64),
    ("r9vx_gguf_shards_open", [_P, _U32, _P], ctypes.c_int),
    ("r9vx_gguf_shards_free", [_P], None),
    ("r9vx_gguf_shards_len", [_P], _U64),
    ("r9vx_gguf_shards_tensor_at", [_P, _U64, _P, _P], ctypes.c_int),
    ("r9vx_gguf_shards_find", [_P, ctypes.c_char_p], ctypes.c_int64),
    ("r9vx_gguf_matmul_static", [_P, ctypes.c_char_p, _P], ctypes.c_int),
    ("r9vx_gguf_moe_ffn_static", [_P, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, _P],
     ctypes.c_int),
    ("r9vx_gguf_upload", [_P, _P, _U64, ctypes.c_char_p, _P, _U64, _P], ctypes.c_int),
    ("r9vx_gguf_upload_split", [_P, _P, _U64, ctypes.c_char_p, _P, _U64, _P, _U64, _P], ctypes.c_int),
    ("r9vx_gguf_upload_gate_up", [_P, _P, _U64, ctypes.c_char_p, _P, _P, _U64, ctypes.c_char_p,
                                  _P, _U64, _P], ctypes.c_int),
    ("r9vx_gguf_upload_gate_up_split", [_P, _P, _U64, ctypes.c_char_p, _P, _P, _U64, ctypes.c_char_p,
                                        _P, _U64, _P, _U64, _P], ctypes.c_int),
]

_lib = None


class R9vxError(RuntimeError):
    """A refusal (code < 0) or HIP error (code > 0) from libr9vx."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


def load():
    """Loads libr9vx.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise R9vxError(-100, f"{LIB_PATH} is missing: run `python -m r9v_amd.build`")
        try:
            L = ctypes.CDLL(str(LIB_PATH))
        except OSError as e:  # e.g. the HIP runtime it links is absent or lacks a symbol
            raise R9vxError(-100, f"cannot load {LIB_PATH}: {e}") from None
        for name, argtypes, restype in EXPORTS:
            try:
                fn = getattr(L, name)
            except AttributeError:
                raise R9vxError(-100, f"{LIB_PATH} does not export {name}: rebuild it") from None
            fn.argtypes = argtypes
            fn.restype = restype
        _lib = L
    return _lib


def _check(rc: int):
    if rc != 0:
        raise R9vxError(rc, load().r9vx_last_error().decode(errors="replace"))


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(torch, stream):
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _need_gpu(*tensors):
    import torch

    if not torch.cuda.is_available():
        raise R9vxError(-101, "no HIP device: libr9vx has no CPU path")
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise R9vxError(-102, "operands must be device tensors")
    return torch


def _dtype_code(t):
    import torch

    return {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}[t.dtype]


# ---------------------------------------------------------------- matmul

def weight_dtype(scheme):
    """The weight element type a scheme's blocks are keyed with."""
    return I8 if scheme in SPLIT_SCHEMES else I4


def weight_layout(scheme):
    """The device layout this path reads a scheme in."""
    return LAYOUT_SPLIT if scheme in SPLIT_SCHEMES else LAYOUT_IQ3S_112 if scheme == IQ3_S else LAYOUT_GGUF_WIRE


def matmul_static(n, k, w_scheme, in_dtype, out_dtype, m_bucket=8, epilogue=EPILOGUE_NONE,
                  residual_dtype=F32, w_layout=None):
    return MatmulStatic(m_bucket, n, k, weight_dtype(w_scheme), w_scheme,
                        weight_layout(w_scheme) if w_layout is None else w_layout, in_dtype, 0, out_dtype,
                        epilogue, residual_dtype, 0, 0, 0)


def matmul(w, w_scheme, n, k, x, out_dtype=F32, bias=None, residual=None, y=None, workspace=None,
           stream=None, w_scales=None, swiglu=False, m_bucket=None):
    """y[m, n] = x[m, :] . w[n, :] (+ bias | + residual): T0 execute_matmul_op meaning.
    Q6_K / Q8_0 weights are a split body `w` plus its f16 d array `w_scales`,
    IQ3_S weights the repacked 112-byte blocks (see `repack`).  The variant's
    M bucket is `m_bucket` (default: m itself); it, not m, picks the kernels."""
    torch = _need_gpu(w, x, bias, residual, y, w_scales)
    m = x.shape[0]
    if y is None:
        y = torch.empty((m, n), dtype=torch.float32 if out_dtype == F32 else torch.bfloat16,
                        device=x.device)
    epi = EPILOGUE_BIAS if bias is not None else (EPILOGUE_RESIDUAL if residual is not None else EPILOGUE_NONE)
    if swiglu:  # w holds 2n rows: gate [0, n) then up [n, 2n); y = silu(gate) * up
        epi = EPILOGUE_SWIGLU
    st = matmul_static(n, k, w_scheme, _dtype_code(x), out_dtype, m_bucket=m_bucket or max(m, 1), epilogue=epi)
    if workspace is None:
        nbytes = matmul_workspace_bytes(st)
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=x.device) if nbytes else None
    args = MatmulArgs(_ptr(w), _ptr(w_scales), None, _ptr(x), None, _ptr(bias), _ptr(residual), _ptr(y),
                      _ptr(workspace), m, 0)
    _check(load().r9vx_matmul_launch(ctypes.byref(st), ctypes.byref(args), _stream(torch, stream)))
    return y


def matmul_workspace_bytes(st: MatmulStatic) -> int:
    return int(load().r9vx_matmul_workspace_bytes(ctypes.byref(st)))


def matmul_static_bytes(st: MatmulStatic, m: int) -> int:
    return int(load().r9vx_matmul_static_bytes(ctypes.byref(st), m))


# ---------------------------------------------------------------- decode

def dequantize(wire, scheme, n_rows, k, out=None, stream=None):
    torch = _need_gpu(wire, out)
    if out is None:
        out = torch.empty((n_rows, k), dtype=torch.float32, device=wire.device)
    _check(load().r9vx_dequantize_launch(scheme, _ptr(wire), n_rows, k, _ptr(out), _stream(torch, stream)))
    return out


def repack(wire, scheme, n_rows, k, stream=None):
    """Q8_0 / Q6_K wire blocks on the device -> (body uint8, scales int16 holding
    f16 bits); IQ3_S -> (112-byte blocks uint8, None)."""
    torch = _need_gpu(wire)
    nb = n_rows * (k // BLOCK_LEN[scheme])
    if scheme == IQ3_S:
        body = torch.empty(nb * IQ3S_DEV_BYTES, dtype=torch.uint8, device=wire.device)
        _check(load().r9vx_repack_launch(scheme, _ptr(wire), n_rows, k, _ptr(body), None,
                                         _stream(torch, stream)))
        return body, None
    body = torch.empty(nb * (BLOCK_BYTES[scheme] - 2), dtype=torch.uint8, device=wire.device)
    scales = torch.empty(nb, dtype=torch.int16, device=wire.device)
    _check(load().r9vx_repack_launch(scheme, _ptr(wire), n_rows, k, _ptr(body), _ptr(scales),
                                     _stream(torch, stream)))
    return body, scales


def validate_weights(wire, scheme, n_rows, k, stream=None) -> int:
    torch = _need_gpu(wire)
    bad = torch.zeros(1, dtype=torch.int32, device=wire.device)
    _check(load().r9vx_validate_weights_launch(scheme, _ptr(wire), n_rows, k, _ptr(bad),
                                               _stream(torch, stream)))
    return int(bad.item())


# ---------------------------------------------------------------- moe_route

def route_static(e, k, t_bucket, scoring=SCORING_SOFTMAX, renormalize=True, scale=1.0,
                 has_bias=False):
    scale_bits = struct.unpack("<I", struct.pack("<f", scale))[0]
    return MoeRouteStatic(t_bucket, e, k, scoring, int(renormalize), 0, 0, scale_bits, int(has_bias))


def moe_route(logits, k, bias=None, scoring=SCORING_SOFTMAX, renormalize=True, scale=1.0,
              ids=None, weights=None, stream=None, status=None):
    """T0 moe_route; with `status` (a device int32 tensor of one element) the
    launch owns that status word (r9vx_moe_route_launch_ex), otherwise the
    stream's plain-launch word (read with moe_route_status(stream))."""
    torch = _need_gpu(logits, bias, status)
    t, e = logits.shape
    if ids is None:
        ids = torch.empty((t, k), dtype=torch.int32, device=logits.device)
    if weights is None:
        weights = torch.empty((t, k), dtype=torch.float32, device=logits.device)
    st = route_static(e, k, max(t, 1), scoring, renormalize, scale, bias is not None)
    args = MoeRouteArgs(_ptr(logits), _ptr(bias), _ptr(ids), _ptr(weights), t, 0)
    if status is not None:
        _check(load().r9vx_moe_route_launch_ex(ctypes.byref(st), ctypes.byref(args), _ptr(status),
                                               _stream(torch, stream)))
    else:
        _check(load().r9vx_moe_route_launch(ctypes.byref(st), ctypes.byref(args), _stream(torch, stream)))
    return ids, weights


def status_read(word, stream=None) -> int:
    """The value of a device status word (of moe_route(status=...))."""
    torch = _need_gpu(word)
    s = ctypes.c_uint32(0)
    _check(load().r9vx_status_read(_ptr(word), ctypes.byref(s), _stream(torch, stream)))
    return s.value


def router_repack(w, stream=None):
    """f32 router weight [E, dm] -> the k4-interleaved device layout [dm/4][E][4]."""
    torch = _need_gpu(w)
    e, dm = w.shape
    out = torch.empty(e * dm, dtype=torch.float32, device=w.device)
    _check(load().r9vx_router_repack_launch(_ptr(w), e, dm, _ptr(out), _stream(torch, stream)))
    return out


def moe_route_hidden(x, w_router, k, bias=None, scoring=SCORING_SOFTMAX, renormalize=True, scale=1.0,
                     ids=None, weights=None, workspace=None, t_bucket=None, stream=None, e=None):
    """Routing from bf16 hidden states x [t, dm] and an f32 router weight
    (in the layout of `router_repack`; pass e= its expert count) in one
    launch (t <= 8), bit-exact with T0's matmul + moe_route.
    Returns (ids, weights, workspace); the workspace's first t*E floats are
    the router logits.  A workspace passed in must have been zero-filled once."""
    torch = _need_gpu(x, w_router, bias, ids, weights, workspace)
    t, dm = x.shape
    e = e if e is not None else w_router.numel() // dm
    st = route_static(e, k, t_bucket or max(t, 1), scoring, renormalize, scale, bias is not None)
    if workspace is None:
        workspace = torch.zeros(int(load().r9vx_moe_route_hidden_workspace_bytes(ctypes.byref(st))),
                                dtype=torch.uint8, device=x.device)
    if ids is None:
        ids = torch.empty((t, k), dtype=torch.int32, device=x.device)
    if weights is None:
        weights = torch.empty((t, k), dtype=torch.float32, device=x.device)
    args = MoeRouteHiddenArgs(_ptr(x), _ptr(w_router), _ptr(bias), _ptr(ids), _ptr(weights), _ptr(workspace),
                              t, dm)
    _check(load().r9vx_moe_route_hidden_launch(ctypes.byref(st), ctypes.byref(args), _stream(torch, stream)))
    return ids, weights, workspace


def moe_route_hidden_status(workspace, e, k, t_bucket, stream=None) -> int:
    """Status bits of the last moe_route_hidden launch with this workspace."""
    torch = _need_gpu(workspace)
    st = route_static(e, k, t_bucket)
    s = ctypes.c_uint32(0)
    _check(load().r9vx_moe_route_hidden_status(ctypes.byref(st), _ptr(workspace), ctypes.byref(s),
                                               _stream(torch, stream)))
    return s.value


def moe_route_status(stream=None) -> int:
    import torch

    s = ctypes.c_uint32(0)
    _check(load().r9vx_moe_route_status(ctypes.byref(s), _stream(torch, stream)))
    return s.value


# ---------------------------------------------------------------- moe_ffn

def ffn_static(t_bucket, e, k, dm, dff, shared=0, gate_up_scheme=IQ4_XS, down_scheme=Q4_K):
    def proj(s):
        return MoeFfnProj(weight_dtype(s), s, weight_layout(s))

    return MoeFfnStatic(t_bucket, e, k, dm, dff, proj(gate_up_scheme), proj(down_scheme), BF16, 0,
                        ACT_SILU, F32, shared, 0)


def ffn_workspace_bytes(st: MoeFfnStatic) -> int:
    return int(load().r9vx_moe_ffn_workspace_bytes(ctypes.byref(st)))


def moe_ffn(x, ids, weights, w_gate_up, w_down, e, dff, shared=0, gate_up_scheme=IQ4_XS,
            down_scheme=Q4_K, y=None, workspace=None, t_bucket=None, stream=None, w_gate_up_scales=None,
            w_down_scales=None):
    """y = moe_ffn(x, ids, weights): gate/up and down experts in the device
    layout of their schemes (GGUF blocks; IQ3_S 112-byte blocks and Q8_0 /
    Q6_K split bodies as repack() returns them, the split d arrays passed as
    the *_scales tensors)."""
    torch = _need_gpu(x, ids, weights, w_gate_up, w_down, y, workspace, w_gate_up_scales, w_down_scales)
    t, dm = x.shape
    k = ids.shape[1]
    st = ffn_static(t_bucket or max(t, 1), e, k, dm, dff, shared, gate_up_scheme, down_scheme)
    if workspace is None:
        workspace = torch.empty(ffn_workspace_bytes(st), dtype=torch.uint8, device=x.device)
    if y is None:
        y = torch.empty((t, dm), dtype=torch.float32, device=x.device)
    args = MoeFfnArgs(_ptr(x), _ptr(ids), _ptr(weights), _ptr(w_gate_up), _ptr(w_gate_up_scales), _ptr(w_down),
                      _ptr(w_down_scales), _ptr(y), _ptr(workspace), t, 0)
    _check(load().r9vx_moe_ffn_launch(ctypes.byref(st), ctypes.byref(args), _stream(torch, stream)))
    return y, workspace, st


NOALLOC_SCRATCH_BYTES = 16 << 20


def moe_ffn_noalloc(x, ids, weights, w_gate_up, w_down, e, dff, y, shared=0, gate_up_scheme=IQ4_XS,
                    down_scheme=Q4_K, status=None, t_bucket=None, stream=None):
    """moe_ffn through r9vx_moe_ffn_launch_noalloc: no workspace (the
    library's own per-GPU scratch), y given by the caller, optional device
    u32 `status` receiving the launch's status bits."""
    torch = _need_gpu(x, ids, weights, w_gate_up, w_down, y, status)
    t, dm = x.shape
    k = ids.shape[1]
    st = ffn_static(t_bucket or max(t, 1), e, k, dm, dff, shared, gate_up_scheme, down_scheme)
    args = MoeFfnArgs(_ptr(x), _ptr(ids), _ptr(weights), _ptr(w_gate_up), None, _ptr(w_down), None,
                      _ptr(y), None, t, 0)
    _check(load().r9vx_moe_ffn_launch_noalloc(ctypes.byref(st), ctypes.byref(args), _ptr(status),
                                              _stream(torch, stream)))
    return y


def moe_ffn_status(st, workspace, stream=None) -> int:
    import torch

    s = ctypes.c_uint32(0)
    _check(load().r9vx_moe_ffn_status(ctypes.byref(st), _ptr(workspace), ctypes.byref(s),
                                      _stream(torch, stream)))
    return s.value


def moe_sort(ids, e, dm=256, dff=256, workspace=None, stream=None):
    torch = _need_gpu(ids, workspace)
    t, k = ids.shape
    st = ffn_static(max(t, 1), e, k, dm, dff)
    if workspace is None:
        workspace = torch.empty(ffn_workspace_bytes(st), dtype=torch.uint8, device=ids.device)
    counts = torch.empty(e, dtype=torch.int32, device=ids.device)
    offsets = torch.empty(e + 1, dtype=torch.int32, device=ids.device)
    order = torch.empty(t * k, dtype=torch.int32, device=ids.device)
    _check(load().r9vx_moe_sort_launch(ctypes.byref(st), _ptr(ids), t, _ptr(workspace), _ptr(counts),
                                       _ptr(offsets), _ptr(order), _stream(torch, stream)))
    return counts, offsets, order


# ---------------------------------------------------------------- ceilings

def probe_stream(src, stream=None):
    """Streams src (a device tensor) once; returns the sink tensor."""
    torch = _need_gpu(src)
    nbytes = src.numel() * src.element_size()
    sink = torch.empty(load().r9vx_probe_stream_blocks(nbytes), dtype=torch.int32, device=src.device)
    _check(load().r9vx_probe_stream_launch(_ptr(src), nbytes, _ptr(sink), _stream(torch, stream)))
    return sink


def probe_mfma(blocks, iters, sink=None, stream=None):
    torch = _need_gpu(sink)
    if sink is None:
        sink = torch.empty(blocks * 256, dtype=torch.float32, device="cuda")
    _check(load().r9vx_probe_mfma_launch(blocks, iters, _ptr(sink), _stream(torch, stream)))
    return sink


def probe_moe_stage(x, ids, weights, w_gate_up, w_down, e, dff, stage, y, workspace, shared=0,
                    gate_up_scheme=IQ4_XS, down_scheme=Q4_K, t_bucket=None, stream=None):
    """Relaunches one stage (1 gate/up GEMM, 2 down GEMM, 3 combine) of the
    grouped moe_ffn path on a workspace a full moe_ffn call with the same
    operands filled."""
    torch = _need_gpu(x, ids, weights, w_gate_up, w_down, y, workspace)
    t, dm = x.shape
    k = ids.shape[1]
    st = ffn_static(t_bucket or max(t, 1), e, k, dm, dff, shared, gate_up_scheme, down_scheme)
    args = MoeFfnArgs(_ptr(x), _ptr(ids), _ptr(weights), _ptr(w_gate_up), None, _ptr(w_down), None,
                      _ptr(y), _ptr(workspace), t, 0)
    _check(load().r9vx_probe_moe_stage_launch(ctypes.byref(st), ctypes.byref(args), stage, _stream(torch, stream)))
