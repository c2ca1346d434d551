"""ctypes binding of the CPU oracle (oracle/liboracle.so) -- the checker.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this.
"""
from __future__ import annotations

import ctypes
import pathlib
import subprocess

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent.parent
LIB_PATH = ROOT / "oracle" / "liboracle.so"

# Schemes by the SchemeId codes the library's statics carry (r9v_amd.ffi); the
# C oracle restates ggml_dequantize and is keyed by GGUF ggml type ids, so
# every wrapper below translates with _gg.
Q4_K, IQ4_XS, Q6_K, Q8_0, IQ3_S = 3, 15, 11, 5, 17
_GGML = {Q4_K: 12, IQ4_XS: 23, Q6_K: 14, Q8_0: 8, IQ3_S: 21}
F32, BF16 = 0, 2


def _gg(scheme):
    """The oracle's GGUF type id of a scheme code (unknown codes pass through
    unchanged, so the oracle's own refusal of them is what a test sees)."""
    return _GGML.get(scheme, scheme)

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        P = ctypes.c_void_p
        U = ctypes.c_uint32
        I = ctypes.c_int
        L.rxo_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.rxo_f16_to_f32.restype = ctypes.c_float
        L.rxo_f32_to_bf16.argtypes = [ctypes.c_float]
        L.rxo_f32_to_bf16.restype = ctypes.c_uint16
        L.rxo_expf.argtypes = [ctypes.c_float]
        L.rxo_expf.restype = ctypes.c_float
        L.rxo_expf_fill.argtypes = [U, ctypes.c_uint64, P]
        L.rxo_expf_fill.restype = None
        L.rxo_set_rows_at_once.argtypes = [I]
        L.rxo_set_rows_at_once.restype = None
        L.rxo_q4k_unpack_scales.argtypes = [P, P, P]
        L.rxo_dequantize.argtypes = [I, P, U, U, P]
        L.rxo_matmul.argtypes = [I, P, U, U, I, P, U, P, P, I, P]
        L.rxo_matmul_mt.argtypes = [I, P, U, U, I, P, U, I, P, I]
        L.rxo_moe_expert_mt.argtypes = [I, P, P, U, U, U, I, P, I, P, P, I]
        L.rxo_router_logits.argtypes = [P, P, U, U, U, P]
        L.rxo_router_logits.restype = None
        L.rxo_act_mul_silu.argtypes = [P, P, ctypes.c_uint64, P]
        L.rxo_act_mul_silu.restype = None
        L.rxo_moe_route.argtypes = [P, P, U, U, U, ctypes.c_float, I, I, P, P]
        L.rxo_moe_sort.argtypes = [P, U, U, U, P, P, P]
        L.rxo_moe_ffn.argtypes = [I, P, U, U, U, U, U, U, P, P, I, P, I, P, I, P]
        L.rxo_moe_ffn_mt.argtypes = [I, P, U, U, U, U, U, U, P, P, I, P, I, P, I, P, I]
        L.rxo_moe_ffn_full.argtypes = [I, P, U, U, U, U, U, P, P, I, P, I, P, P]
        L.rxo_expert_ffn.argtypes = [I, P, U, U, U, I, P, I, P, I, P]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


class OracleError(RuntimeError):
    def __init__(self, code: int, what: str):
        super().__init__(f"{what}: oracle refused with code {code}")
        self.code = code


def _check(rc, what):
    if rc != 0:
        raise OracleError(rc, what)


def set_rows_at_once(n):
    """1: the dots walk one row at a time, as T0's loop does (the CPU
    baseline's timing form); 4 (default): four rows per pass over k.  The
    outputs are bit-identical."""
    lib().rxo_set_rows_at_once(n)


def expf_fill(first_bits, n, out=None):
    """libm expf of the floats whose bits are first_bits .. first_bits + n - 1."""
    out = np.empty(n, dtype=np.float32) if out is None else out
    lib().rxo_expf_fill(first_bits, n, _p(out))
    return out


def dequantize(scheme, wire, n, k):
    out = np.empty((n, k), dtype=np.float32)
    _check(lib().rxo_dequantize(_gg(scheme), _p(np.ascontiguousarray(wire)), n, k, _p(out)), "dequantize")
    return out


def matmul(scheme, w, n, k, x, x_dtype, y_dtype=F32, bias=None, residual=None, threads=0):
    x = np.ascontiguousarray(x)
    m = x.shape[0]
    y = np.empty((m, n), dtype=np.float32 if y_dtype == F32 else np.uint16)
    w = np.ascontiguousarray(w)
    if threads and bias is None and residual is None:  # the threaded oracle has no epilogue
        rc = lib().rxo_matmul_mt(_gg(scheme), _p(w), n, k, x_dtype, _p(x), m, y_dtype, _p(y), threads)
    else:
        rc = lib().rxo_matmul(_gg(scheme), _p(w), n, k, x_dtype, _p(x), m, _p(bias), _p(residual),
                              y_dtype, _p(y))
    _check(rc, "matmul")
    return y


def router_logits(x_bf16, w):
    x_bf16 = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.float32)
    t, dm = x_bf16.shape
    e = w.shape[0]
    out = np.empty((t, e), dtype=np.float32)
    lib().rxo_router_logits(_p(x_bf16), _p(w), t, e, dm, _p(out))
    return out


def act_mul_silu(g, u):
    g = np.ascontiguousarray(g, dtype=np.float32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    y = np.empty_like(g)
    lib().rxo_act_mul_silu(_p(g), _p(u), g.size, _p(y))
    return y


def matmul_swiglu(scheme, w, n, k, x, x_dtype):
    """T0's matmul over the stacked [gate; up] rows (f32 out), then act_mul."""
    gu = matmul(scheme, w, 2 * n, k, x, x_dtype)
    return act_mul_silu(gu[:, :n], gu[:, n:])


def moe_route(logits, k, bias=None, scale=1.0, renormalize=True, scoring=0):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    t, e = logits.shape
    ids = np.zeros((t, k), dtype=np.uint32)
    w = np.zeros((t, k), dtype=np.float32)
    _check(lib().rxo_moe_route(_p(logits), _p(bias), t, e, k, scale, int(renormalize), scoring,
                               _p(ids), _p(w)), "moe_route")
    return ids, w


def moe_sort(ids, e):
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    t, k = ids.shape
    counts = np.zeros(e, dtype=np.uint32)
    offsets = np.zeros(e + 1, dtype=np.uint32)
    sorted_ = np.zeros(t * k, dtype=np.uint32)
    _check(lib().rxo_moe_sort(_p(ids), t, k, e, _p(counts), _p(offsets), _p(sorted_)), "moe_sort")
    return counts, offsets, sorted_


def moe_ffn(x, x_dtype, ids, weights, e, dff, w_gate_up, w_down, scheme_gu=IQ4_XS,
            scheme_dn=Q4_K, shared=0, h_bf16=False, threads=0):
    """T0 moe_ffn; threads > 0 runs the expert FFNs on that many OpenMP
    threads (bit-identical result)."""
    x = np.ascontiguousarray(x)
    t, dm = x.shape
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    weights = np.ascontiguousarray(weights, dtype=np.float32)
    k = ids.shape[1]
    y = np.empty((t, dm), dtype=np.float32)
    args = (x_dtype, _p(x), t, dm, dff, e, shared, k, _p(ids), _p(weights), _gg(scheme_gu),
            _p(np.ascontiguousarray(w_gate_up)), _gg(scheme_dn), _p(np.ascontiguousarray(w_down)), int(h_bf16),
            _p(y))
    if threads:
        _check(lib().rxo_moe_ffn_mt(*args, threads), "moe_ffn")
    else:
        _check(lib().rxo_moe_ffn(*args), "moe_ffn")
    return y


def host_threads():
    """Threads for the oracle's parallel forms: the host's CPUs, at most 16
    (a GPU box's CPU share)."""
    import os

    return max(1, min(16, len(os.sched_getaffinity(0))))


def moe_ffn_full(x, x_dtype, ids, weights, e, dff, w_gate_up, w_down, scheme_gu=IQ4_XS,
                 scheme_dn=Q4_K):
    x = np.ascontiguousarray(x)
    t, dm = x.shape
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    weights = np.ascontiguousarray(weights, dtype=np.float32)
    k = ids.shape[1]
    y = np.empty((t, dm), dtype=np.float32)
    _check(lib().rxo_moe_ffn_full(x_dtype, _p(x), t, dm, dff, e, k, _p(ids), _p(weights),
                                  _gg(scheme_gu), _p(np.ascontiguousarray(w_gate_up)), _gg(scheme_dn),
                                  _p(np.ascontiguousarray(w_down)), _p(y)), "moe_ffn_full")
    return y


def expert_ffn(x, x_dtype, dff, w_gate_up, w_down, scheme_gu=IQ4_XS, scheme_dn=Q4_K,
               h_bf16=False):
    x = np.ascontiguousarray(x)
    rows, dm = x.shape
    out = np.empty((rows, dm), dtype=np.float32)
    _check(lib().rxo_expert_ffn(x_dtype, _p(x), rows, dm, dff, _gg(scheme_gu),
                                _p(np.ascontiguousarray(w_gate_up)), _gg(scheme_dn),
                                _p(np.ascontiguousarray(w_down)), int(h_bf16), _p(out)),
           "expert_ffn")
    return out


def moe_expert(x, x_dtype, tokens, dff, gu_expert, dn_expert, scheme_gu=IQ4_XS, scheme_dn=Q4_K, threads=1):
    """One expert's FFN over the rows `tokens` of x (the per-expert body of
    moe_ffn), rows split over `threads` OpenMP threads."""
    x = np.ascontiguousarray(x)
    dm = x.shape[1]
    tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
    out = np.empty((len(tokens), dm), dtype=np.float32)
    _check(lib().rxo_moe_expert_mt(x_dtype, _p(x), _p(tokens), len(tokens), dm, dff, _gg(scheme_gu),
                                   _p(np.ascontiguousarray(gu_expert)), _gg(scheme_dn),
                                   _p(np.ascontiguousarray(dn_expert)), _p(out), threads), "moe_expert")
    return out
