"""GPU parity of the gated (SwiGLU) matmul epilogue: one launch computing
y = silu(x . w_gate) * (x . w_up) over stacked [gate; up] weights, against
T0's matmul (f32 out) followed by act_mul with SiLU
(crates/r9v-t0/src/act_mul.rs:86-99), at the north-star tolerance."""
from __future__ import annotations

import numpy as np
import pytest

import oracle_ffi as O
from gguf_build import build
from r9v_amd import ffi, gguf, synth
from tol import check_bf16_out, check_close

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

SCHEMES = [ffi.Q4_K, ffi.IQ4_XS, ffi.Q6_K, ffi.Q8_0]


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def bf16_dev(bits):
    return dev(bits.view(np.int16)).view(torch.bfloat16)


def host(t):
    return t.cpu().numpy()


def weights(scheme, seed, rows, k):
    wire = synth.quant_weights(scheme, seed, rows, k)
    if scheme in ffi.SPLIT_SCHEMES:
        body, scales = ffi.repack(dev(wire), scheme, rows, k)
        return wire, body, scales
    return wire, dev(wire), None


@pytest.mark.parametrize("scheme", SCHEMES)
@pytest.mark.parametrize("n,k,m", [(1024, 2048, 1), (1024, 2048, 5), (777, 4096, 3), (2560, 1024, 8),
                                   (96, 768, 2)])
def test_swiglu_gemv_parity(scheme, n, k, m):
    wire, w, ws = weights(scheme, 700 + n + m, 2 * n, k)
    x = synth.normal_bf16(800 + k + m, (m, k))
    y = host(ffi.matmul(w, scheme, n, k, bf16_dev(x), w_scales=ws, swiglu=True))
    check_close(y, O.matmul_swiglu(scheme, wire, n, k, x, O.BF16), f"scheme={scheme} n={n} k={k} m={m}")


@pytest.mark.parametrize("scheme", [ffi.Q4_K, ffi.Q6_K])
def test_swiglu_bf16_out_and_unfused_equivalence(scheme):
    """bf16 output is the RNE of the f32 result; and the gated launch equals
    the unfused pair (the plain matmul's f32 gate and up, then act_mul) to
    within the same bound."""
    n, k, m = 1536, 2048, 4
    wire, w, ws = weights(scheme, 91, 2 * n, k)
    x = synth.normal_bf16(92, (m, k))
    y32 = host(ffi.matmul(w, scheme, n, k, bf16_dev(x), w_scales=ws, swiglu=True))
    y16 = ffi.matmul(w, scheme, n, k, bf16_dev(x), w_scales=ws, swiglu=True, out_dtype=ffi.BF16)
    ref = O.matmul_swiglu(scheme, wire, n, k, x, O.BF16)
    got16 = host(y16.view(torch.int16)).view(np.uint16).astype(np.uint32) << 16
    check_bf16_out(got16.view(np.float32), y32, ref, "bf16 out")
    gu = host(ffi.matmul(w, scheme, 2 * n, k, bf16_dev(x), w_scales=ws))
    check_close(y32, O.act_mul_silu(gu[:, :n], gu[:, n:]), "unfused pair")


def test_swiglu_on_a_loaded_dense_ffn():
    """ffn_gate / ffn_up of a checkpoint uploaded into one stacked buffer."""
    n, k = 640, 2048
    gate = synth.quant_weights(ffi.Q4_K, 61, n, k)
    up = synth.quant_weights(ffi.Q4_K, 62, n, k)
    b = build([], [("blk.0.ffn_gate.weight", (k, n), 12, gate.tobytes()),
                   ("blk.0.ffn_up.weight", (k, n), 12, up.tobytes())])
    f = gguf.GgufFile.parse(b)
    w = torch.empty(2 * gate.size, dtype=torch.uint8, device="cuda")
    gguf.upload(f, b, "blk.0.ffn_gate.weight", out=w[:gate.size])
    gguf.upload(f, b, "blk.0.ffn_up.weight", out=w[gate.size:])
    x = synth.normal_bf16(63, (2, k))
    y = host(ffi.matmul(w, ffi.Q4_K, n, k, bf16_dev(x), swiglu=True))
    check_close(y, O.matmul_swiglu(ffi.Q4_K, np.concatenate([gate, up]), n, k, x, O.BF16), "loaded ffn")
