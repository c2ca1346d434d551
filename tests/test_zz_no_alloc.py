"""r9vx_moe_ffn_launch_noalloc (the moe_ffn launch that allocates nothing)
against r9vx_moe_ffn_launch on the same operands, through the C ABI:
bit-exact y and status on two calls in a row, the second with fewer tokens
(and the decode path instead of the grouped one), plus its refusals."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle_ffi as O
from r9v_amd import ffi, synth

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

E, K, DM, DFF, SHARED = 64, 4, 512, 256, 1
ERR_INVALID, ERR_UNSUPPORTED = -1, -2  # R9VX_ERR_INVALID, R9VX_ERR_UNSUPPORTED


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _operands(t, seed):
    logits = synth.zipf_logits(seed, t, E)
    ids, w = O.moe_route(logits, K)
    x = synth.normal_bf16(seed + 1, (t, DM))
    return dev(x.view(np.int16)).view(torch.bfloat16), dev(ids.view(np.int32)), dev(w)


@pytest.fixture(scope="module")
def weights():
    gu = synth.quant_weights(synth.IQ4_XS, 2101, (E + SHARED) * 2 * DFF, DM)
    dn = synth.quant_weights(synth.Q4_K, 2102, (E + SHARED) * DM, DFF)
    return dev(gu), dev(dn)


def _both(weights, x, ids, w):
    gu, dn = weights
    t = x.shape[0]
    ref, ws, st = ffi.moe_ffn(x, ids, w, gu, dn, E, DFF, shared=SHARED)
    ref_status = ffi.moe_ffn_status(st, ws)
    y = torch.full((t, DM), float("nan"), dtype=torch.float32, device="cuda")
    status = torch.full((1,), 0xFFFF, dtype=torch.int32, device="cuda")
    ffi.moe_ffn_noalloc(x, ids, w, gu, dn, E, DFF, y, shared=SHARED, status=status)
    torch.cuda.synchronize()
    return ref, ref_status, y, int(status.item())


def test_noalloc_matches_workspace_launch_twice(weights):
    # 40 tokens run the grouped path, then 5 tokens the decode path, both on
    # the scratch the first call left behind
    for t, seed in ((40, 2201), (5, 2211)):
        x, ids, w = _operands(t, seed)
        ref, ref_status, y, status = _both(weights, x, ids, w)
        assert ref_status == 0 and status == 0
        assert torch.equal(y.view(torch.int32), ref.view(torch.int32)), f"t={t}: y differs from moe_ffn"


def test_noalloc_status_of_a_refused_call(weights):
    x, ids, w = _operands(6, 2221)
    ids[2, 1] = E + SHARED + 3  # out of range: the device refuses the call
    ref, ref_status, y, status = _both(weights, x, ids, w)
    assert ref_status == status == ffi.STATUS_BAD_EXPERT
    assert torch.isnan(y).all(), "a refused call must leave y untouched"
    # the next good call on the same scratch is whole again
    x, ids, w = _operands(6, 2231)
    ref, ref_status, y, status = _both(weights, x, ids, w)
    assert status == 0 and torch.equal(y.view(torch.int32), ref.view(torch.int32))


def test_noalloc_refusals(weights):
    gu, dn = weights
    x, ids, w = _operands(4, 2241)
    y = torch.empty((4, DM), dtype=torch.float32, device="cuda")
    lib = ffi.load()
    st = ffi.ffn_static(4, E, K, DM, DFF, SHARED)
    ws = torch.empty(ffi.ffn_workspace_bytes(st), dtype=torch.uint8, device="cuda")
    args = ffi.MoeFfnArgs(ffi._ptr(x), ffi._ptr(ids), ffi._ptr(w), ffi._ptr(gu), None, ffi._ptr(dn), None,
                          ffi._ptr(y), ffi._ptr(ws), 4, 0)
    s = ffi._stream(torch, None)
    assert lib.r9vx_moe_ffn_launch_noalloc(ctypes.byref(st), ctypes.byref(args), None, s) == ERR_INVALID
    assert b"sort_workspace must be NULL" in lib.r9vx_last_error()
    big = ffi.ffn_static(8192, 512, 10, 2048, 512)
    assert ffi.ffn_workspace_bytes(big) > ffi.NOALLOC_SCRATCH_BYTES
    args.sort_workspace = None
    assert lib.r9vx_moe_ffn_launch_noalloc(ctypes.byref(big), ctypes.byref(args), None, s) == ERR_UNSUPPORTED
    assert b"exceeds the no-alloc scratch" in lib.r9vx_last_error()
