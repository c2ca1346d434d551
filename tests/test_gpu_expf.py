"""The router's exp on the device equals the host libm expf bit for bit.

Routing is bit-exact with T0 only if the device exp (r9vx_expf.h) returns the
bits of the host expf that the reference's f32::exp lowers to.  The host
build of the same header is checked exhaustively on the CPU
(tests/expf_twin_check.c); this runs the device build of all three forms the
routing kernels call over every f32 in [-104, 0] (softmax: exp(s - max)) and
[0, 104] (sigmoid's exp(-s) of negative scores, through overflow), against
the oracle's libm values."""
from __future__ import annotations

import struct

import numpy as np
import pytest

import oracle_ffi as O
from r9v_amd import ffi

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def _bits(x):
    return struct.unpack("<I", struct.pack("<f", x))[0]


@pytest.mark.parametrize("lo,hi", [(-0.0, -104.0), (0.0, 104.0)], ids=["negative", "positive"])
def test_device_expf_matches_libm(lo, hi):
    first, last = _bits(lo), _bits(hi)  # bits grow with |x| on either side
    chunk = 1 << 26
    want_h = torch.empty(chunk, dtype=torch.float32, pin_memory=True)
    want_d = torch.empty(chunk, dtype=torch.float32, device="cuda")
    bad = torch.zeros(3, dtype=torch.int32, device="cuda")
    lib = ffi.load()
    stream = torch.cuda.current_stream()
    b = first
    total = 0
    while b <= last:
        n = min(chunk, last - b + 1)
        O.expf_fill(b, n, out=want_h.numpy())
        want_d[:n].copy_(want_h[:n], non_blocking=True)
        ffi._check(lib.r9vx_probe_expf_check_launch(b, n, ffi._ptr(want_d), ffi._ptr(bad),
                                                    ffi._stream(torch, stream)))
        torch.cuda.synchronize()  # want_h is refilled next
        total += n
        b += n
    assert total == last - first + 1
    counts = bad.cpu().numpy()
    assert counts.tolist() == [0, 0, 0], f"mismatches per form (expf, expf_tab, expf_tab_nb): {counts.tolist()}"
