"""GPU parity of routing from hidden states (r9vx_moe_route_hidden_launch):
the router logits x . w_r^T accumulated in T0's matmul order and moe_route
in one launch.  Logits, ids and weights must equal the oracle's T0 pipeline
(router matmul in Branch-D order, then moe_route) bit for bit."""
from __future__ import annotations

import numpy as np
import pytest

import oracle_ffi as O
from gguf_build import build
from r9v_amd import ffi, gguf, synth

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def bf16_dev(bits):
    return dev(bits.view(np.int16)).view(torch.bfloat16)


def host(t):
    return t.cpu().numpy()


def case(t, e, dm, seed):
    x = synth.normal_bf16(seed, (t, dm))
    w = synth.normal_f32(seed + 1, (e, dm), 0.05)
    return x, w


def run(x, w, k, bias=None, scoring=0, renormalize=True, scale=1.0):
    ids, wts, ws = ffi.moe_route_hidden(bf16_dev(x), ffi.router_repack(dev(w)), k, bias=None if bias is None else dev(bias),
                                        scoring=scoring, renormalize=renormalize, scale=scale)
    torch.cuda.synchronize()
    t, e = x.shape[0], w.shape[0]
    logits = host(ws[:t * e * 4].view(torch.float32)).reshape(t, e)
    return host(ids).view(np.uint32), host(wts), logits, ffi.moe_route_hidden_status(ws, e, k, max(t, 1))


@pytest.mark.parametrize("t,e,dm,k", [(1, 512, 2048, 10), (5, 512, 2048, 10), (8, 512, 4096, 8),
                                      (3, 64, 1024, 2), (7, 160, 2048, 6), (2, 1024, 512, 32), (4, 128, 128, 1)])
def test_route_hidden_bit_exact(t, e, dm, k):
    x, w = case(t, e, dm, 100 + t + e)
    ids, wts, logits, status = run(x, w, k)
    assert status == 0
    ref_logits = O.router_logits(x, w)
    assert np.array_equal(logits.view(np.uint32), ref_logits.view(np.uint32))
    rid, rw = O.moe_route(ref_logits, k)
    assert np.array_equal(ids, rid.astype(np.uint32))
    assert np.array_equal(wts.view(np.uint32), rw.view(np.uint32))


def test_route_hidden_bias_sigmoid_scale():
    t, e, dm, k = 6, 256, 2048, 4
    x, w = case(t, e, dm, 77)
    bias = synth.normal_f32(79, (e,), 0.1)
    ref_logits = O.router_logits(x, w)
    for scoring, renorm, scale in ((1, True, 1.0), (0, False, 2.5), (1, False, 0.5)):
        ids, wts, _, status = run(x, w, k, bias=bias, scoring=scoring, renormalize=renorm, scale=scale)
        assert status == 0
        rid, rw = O.moe_route(ref_logits, k, bias=bias, scoring=scoring, renormalize=renorm, scale=scale)
        assert np.array_equal(ids, rid.astype(np.uint32)), (scoring, renorm, scale)
        assert np.array_equal(wts.view(np.uint32), rw.view(np.uint32)), (scoring, renorm, scale)


def test_route_hidden_back_to_back_and_refusal():
    """The completion counter is left at zero: consecutive launches on one
    workspace are each correct; a non-finite hidden state refuses the whole
    batch before any write (moe_route.rs:313-418)."""
    t, e, dm, k = 5, 512, 2048, 10
    st = ffi.route_static(e, k, t)
    import ctypes
    ws = torch.zeros(int(ffi.load().r9vx_moe_route_hidden_workspace_bytes(ctypes.byref(st))), dtype=torch.uint8,
                     device="cuda")
    for seed in (5, 6, 7):
        x, w = case(t, e, dm, seed)
        ids, wts, _ = ffi.moe_route_hidden(bf16_dev(x), ffi.router_repack(dev(w)), k, workspace=ws)
        torch.cuda.synchronize()
        rid, rw = O.moe_route(O.router_logits(x, w), k)
        assert np.array_equal(host(ids).view(np.uint32), rid.astype(np.uint32))
        assert np.array_equal(host(wts).view(np.uint32), rw.view(np.uint32))
    x, w = case(t, e, dm, 8)
    xb = x.copy()
    xb[3, 100] = 0x7FC0  # bf16 NaN
    ids = torch.full((t, k), 7, dtype=torch.int32, device="cuda")
    wts = torch.full((t, k), 0.5, dtype=torch.float32, device="cuda")
    ffi.moe_route_hidden(bf16_dev(xb), ffi.router_repack(dev(w)), k, ids=ids, weights=wts, workspace=ws)
    assert ffi.moe_route_hidden_status(ws, e, k, t) == ffi.STATUS_NONFINITE
    assert np.all(host(ids) == 7) and np.all(host(wts) == 0.5)
    x, w = case(t, e, dm, 9)
    ids, wts, _ = ffi.moe_route_hidden(bf16_dev(x), ffi.router_repack(dev(w)), k, workspace=ws)
    torch.cuda.synchronize()
    assert ffi.moe_route_hidden_status(ws, e, k, t) == 0
    rid, _ = O.moe_route(O.router_logits(x, w), k)
    assert np.array_equal(host(ids).view(np.uint32), rid.astype(np.uint32))


def test_router_repack_layout():
    e, dm = 96, 256
    w = synth.normal_f32(3, (e, dm))
    got = host(ffi.router_repack(dev(w)))
    assert np.array_equal(got.reshape(dm // 4, e, 4), w.reshape(e, dm // 4, 4).transpose(1, 0, 2))


def test_route_hidden_from_a_loaded_router_tensor():
    t, e, dm, k = 5, 512, 2048, 10
    x, w = case(t, e, dm, 55)
    b = build([], [("blk.0.ffn_gate_inp.weight", (dm, e), 0, w.tobytes())])
    f = gguf.GgufFile.parse(b)
    ne, ndm, wk4 = gguf.load_router_weight(f, b, "blk.0.ffn_gate_inp.weight")
    assert (ne, ndm) == (e, dm)
    ids, wts, _ = ffi.moe_route_hidden(bf16_dev(x), wk4, k, e=e)
    torch.cuda.synchronize()
    rid, rw = O.moe_route(O.router_logits(x, w), k)
    assert np.array_equal(host(ids).view(np.uint32), rid.astype(np.uint32))
    assert np.array_equal(host(wts).view(np.uint32), rw.view(np.uint32))
