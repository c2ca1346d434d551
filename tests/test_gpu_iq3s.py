"""GPU parity of the IQ3_S path (GGUF IQ3_S experts and projections,
crates/r9v-format/src/iq.rs:698-722), through the C ABI.

- wire decode is bit-exact with the oracle and with the reference's golden
  case (iq_a24_reference.txt, gguf-py 0.19.0);
- the load-time repack (r9vx_repack_launch) writes the 112-byte device block
  (qs 64 | signs 32 | qh 8 | scales 4 | d 2 | 0 0) bit for bit;
- the decode GEMV, its SwiGLU form and the prefill GEMM on the repacked
  blocks meet the oracle (f32 decode, then the ascending-K dot of
  crates/r9v-t0/src/matmul.rs:1940-2414) at the north-star tolerance.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle_ffi as O
from golden_io import iq4_cases
from gguf_build import build
from r9v_amd import ffi, gguf, synth
from tol import check_bf16_out, check_close

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

IQ3_S = ffi.IQ3_S


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def bf16_dev(bits):
    return dev(bits.view(np.int16)).view(torch.bfloat16)


def host(t):
    return t.cpu().numpy()


def device_blocks_np(wire):
    """The 112-byte device block restated in numpy from the wire field offsets
    (d 0:2, qs 2:66, qh 66:74, signs 74:106, scales 106:110)."""
    b = wire.reshape(-1, 110)
    z = np.zeros((b.shape[0], 2), dtype=np.uint8)
    return np.concatenate([b[:, 2:66], b[:, 74:106], b[:, 66:74], b[:, 106:110], b[:, 0:2], z], axis=1).reshape(-1)


def test_dequantize_golden_case():
    c = iq4_cases()["IQ3_S"]
    got = host(ffi.dequantize(dev(np.ascontiguousarray(c["wire"])), IQ3_S, c["n"], c["k"]))
    assert np.array_equal(got.reshape(-1).view(np.uint32), c["y_bits"])


def test_dequantize_bit_exact_random():
    n, k = 41, 2048
    w = synth.quant_weights(IQ3_S, 919, n, k)
    got = host(ffi.dequantize(dev(w), IQ3_S, n, k))
    assert np.array_equal(got.view(np.uint32), O.dequantize(IQ3_S, w, n, k).view(np.uint32))


def test_validate_counts_nonfinite_d():
    n, k = 3, 1024
    w = synth.quant_weights(IQ3_S, 17, n, k).reshape(-1, 110).copy()
    for b, bits in ((0, 0x7C00), (7, 0xFE00), (11, 0xFC00)):
        w[b, 0:2] = np.frombuffer(np.uint16(bits).tobytes(), np.uint8)
    assert ffi.validate_weights(dev(w.reshape(-1)), IQ3_S, n, k) == 3


def test_repack_writes_the_device_block():
    n, k = 29, 1536
    w = synth.quant_weights(IQ3_S, 616, n, k)
    body, scales = ffi.repack(dev(w), IQ3_S, n, k)
    assert scales is None
    assert np.array_equal(host(body), device_blocks_np(w))


SHAPES = [(4096, 4096, 1), (1024, 4096, 5), (5120, 2048, 3), (333, 1280, 8), (64, 256, 2),
          (777, 3072, 4), (2048, 2048, 7), (2600, 14336, 1), (3000, 8192, 6)]


@pytest.mark.parametrize("n,k,m", SHAPES)
def test_gemv_parity(n, k, m):
    w = synth.quant_weights(IQ3_S, 1000 + n + m, n, k)
    x = synth.normal_bf16(2000 + k + m, (m, k))
    body, _ = ffi.repack(dev(w), IQ3_S, n, k)
    y = host(ffi.matmul(body, IQ3_S, n, k, bf16_dev(x)))
    check_close(y, O.matmul(IQ3_S, w, n, k, x, O.BF16, threads=8), f"n={n} k={k} m={m}")


def test_gemv_epilogues_and_bf16_out():
    n, k, m = 640, 2048, 3
    w = synth.quant_weights(IQ3_S, 31, n, k)
    x = synth.normal_bf16(32, (m, k))
    body, _ = ffi.repack(dev(w), IQ3_S, n, k)
    bias = synth.normal_f32(33, (n,))
    res = synth.normal_f32(34, (m, n))
    yb = host(ffi.matmul(body, IQ3_S, n, k, bf16_dev(x), bias=dev(bias)))
    check_close(yb, O.matmul(IQ3_S, w, n, k, x, O.BF16, bias=bias), "bias")
    yr = host(ffi.matmul(body, IQ3_S, n, k, bf16_dev(x), residual=dev(res)))
    check_close(yr, O.matmul(IQ3_S, w, n, k, x, O.BF16, residual=res), "residual")
    y16 = ffi.matmul(body, IQ3_S, n, k, bf16_dev(x), out_dtype=ffi.BF16)
    y32 = host(ffi.matmul(body, IQ3_S, n, k, bf16_dev(x)))
    got16 = host(y16.view(torch.int16)).view(np.uint16).astype(np.uint32) << 16
    check_bf16_out(got16.view(np.float32), y32, O.matmul(IQ3_S, w, n, k, x, O.BF16), "bf16 out")


@pytest.mark.parametrize("n,k,m", [(768, 2048, 1), (2816, 2048, 4), (512, 4096, 8)])
def test_gemv_swiglu_parity(n, k, m):
    w = synth.quant_weights(IQ3_S, 51 + n, 2 * n, k)
    x = synth.normal_bf16(52 + m, (m, k))
    body, _ = ffi.repack(dev(w), IQ3_S, 2 * n, k)
    y = host(ffi.matmul(body, IQ3_S, n, k, bf16_dev(x), swiglu=True))
    check_close(y, O.matmul_swiglu(IQ3_S, w, n, k, x, O.BF16), f"swiglu n={n} m={m}")


def test_gemv_row_and_batch_invariance():
    n, k = 1500, 2048
    w = synth.quant_weights(IQ3_S, 41, n, k)
    x = synth.normal_bf16(42, (6, k))
    body, _ = ffi.repack(dev(w), IQ3_S, n, k)
    full = host(ffi.matmul(body, IQ3_S, n, k, bf16_dev(x)))
    for r in range(6):
        one = host(ffi.matmul(body, IQ3_S, n, k, bf16_dev(x[r:r + 1])))
        assert np.array_equal(one.view(np.uint32), full[r:r + 1].view(np.uint32)), r


PREFILL = [(9, 320, 2048), (40, 1000, 4096), (300, 512, 2048), (129, 2304, 1024)]


@pytest.mark.parametrize("m,n,k", PREFILL)
def test_prefill_gemm_parity(m, n, k):
    w = synth.quant_weights(IQ3_S, 3000 + m + n, n, k)
    x = synth.normal_bf16(4000 + m + k, (m, k))
    body, _ = ffi.repack(dev(w), IQ3_S, n, k)
    y = host(ffi.matmul(body, IQ3_S, n, k, bf16_dev(x)))
    check_close(y, O.matmul(IQ3_S, w, n, k, x, O.BF16, threads=8), f"m={m} n={n} k={k}")


# m > 8 runs the 256 x 256 loop for every n (two threads per weight row, a
# thread's half K step one 32-weight group: its 8 grid indices, sign word and
# the block's side word, decoded through the signed grid table in LDS); these
# shapes reach its row-chunk plans with ragged row tiles and the bias
# epilogue.
@pytest.mark.parametrize("m,n,k", [(9, 256, 512), (700, 2560, 512), (1100, 5376, 512), (2048, 4096, 1024)])
def test_prefill_gemm_256_tile(m, n, k):
    w = synth.quant_weights(IQ3_S, 3400 + m, n, k)
    x = synth.normal_bf16(3500 + m, (m, k))
    b = synth.normal_f32(3600 + m, (n,))
    body, _ = ffi.repack(dev(w), IQ3_S, n, k)
    y = host(ffi.matmul(body, IQ3_S, n, k, bf16_dev(x), bias=dev(b)))
    rows = np.arange(m) if m * n <= 4_000_000 else np.unique(np.concatenate([np.arange(0, m, 7), [m - 1]]))
    ref = O.matmul(IQ3_S, w, n, k, np.ascontiguousarray(x[rows]), O.BF16, bias=b, threads=8)
    check_close(y[rows], ref, f"m={m} n={n} k={k}")


def test_prefill_gemm_large_sampled():
    m, n, k = 1024, 4096, 4096
    w = synth.quant_weights(IQ3_S, 5151, n, k)
    x = synth.normal_bf16(5152, (m, k))
    res = synth.normal_f32(5153, (m, n))
    body, _ = ffi.repack(dev(w), IQ3_S, n, k)
    y = host(ffi.matmul(body, IQ3_S, n, k, bf16_dev(x), residual=dev(res)))
    rows = np.array([0, 1, 127, 128, 511, 640, 1000, 1023])
    ref = O.matmul(IQ3_S, w, n, k, x[rows], O.BF16, residual=res[rows], threads=8)
    check_close(y[rows], ref, "sampled")


@pytest.mark.parametrize("t,shared,dn", [(3, 0, ffi.Q4_K), (8, 1, ffi.IQ4_XS), (300, 0, ffi.Q4_K),
                                         (300, 1, ffi.IQ4_XS)])
def test_moe_ffn_iq3s_gate_up_experts(t, shared, dn):
    """IQ3_S gate/up experts (repacked) with Q4_K / IQ4_XS down experts:
    t <= 8 runs the decode kernels, larger t the grouped MFMA GEMMs."""
    e, dm, dff, k = 6, 512, 256, 2
    ea = e + shared
    gu = synth.quant_weights(IQ3_S, 700 + t, ea * 2 * dff, dm)
    down = synth.quant_weights(dn, 800 + t, ea * dm, dff)
    logits = synth.normal_f32(31 + t, (t, e))
    ids, w = O.moe_route(logits, k)
    x = synth.normal_bf16(32 + t, (t, dm))
    gu_dev, _ = ffi.repack(dev(gu), IQ3_S, ea * 2 * dff, dm)
    y, ws, st = ffi.moe_ffn(bf16_dev(x), dev(ids.view(np.int32)), dev(w), gu_dev, dev(down), e, dff,
                            shared=shared, gate_up_scheme=IQ3_S, down_scheme=dn)
    torch.cuda.synchronize()
    assert ffi.moe_ffn_status(st, ws) == 0
    ref = O.moe_ffn(x, O.BF16, ids, w, e, dff, gu, down, scheme_gu=IQ3_S, scheme_dn=dn, shared=shared)
    check_close(host(y), ref, f"moe t={t} shared={shared}")


def test_gguf_loads_repack_iq3s_weights_and_experts():
    """IQ3_S tensors of a checkpoint: load_matmul_weight and load_moe_experts
    upload the wire blocks, check every d, and repack them on the device."""
    n, k = 320, 2048
    wq = synth.quant_weights(IQ3_S, 61, n, k)
    e, dm, dff = 4, 512, 256
    gate = synth.quant_weights(IQ3_S, 62, e * dff, dm)
    up = synth.quant_weights(IQ3_S, 63, e * dff, dm)
    down = synth.quant_weights(ffi.Q4_K, 64, e * dm, dff)
    b = build([("general.architecture", (8, "qwen3moe"))], [
        ("blk.0.attn_o.weight", (k, n), 21, wq.tobytes()),
        ("blk.0.ffn_gate_exps.weight", (dm, dff, e), 21, gate.tobytes()),
        ("blk.0.ffn_up_exps.weight", (dm, dff, e), 21, up.tobytes()),
        ("blk.0.ffn_down_exps.weight", (dff, dm, e), 12, down.tobytes())])
    f = gguf.GgufFile.parse(b)
    st, w, ws = gguf.load_matmul_weight(f, b, "blk.0.attn_o.weight", m_bucket=2)
    assert ws is None and st.w_scheme == IQ3_S
    assert np.array_equal(host(w), device_blocks_np(wq))
    x = synth.normal_bf16(65, (2, k))
    check_close(host(ffi.matmul(w, IQ3_S, n, k, bf16_dev(x))), O.matmul(IQ3_S, wq, n, k, x, O.BF16), "loaded")
    fst, w_gu, w_dn = gguf.load_moe_experts(f, b, "blk.0.ffn_gate_exps.weight", "blk.0.ffn_up_exps.weight",
                                            "blk.0.ffn_down_exps.weight", t_bucket=16, k=2)
    stacked = np.concatenate([gate.reshape(e, dff, -1), up.reshape(e, dff, -1)], axis=1).reshape(-1)
    assert np.array_equal(host(w_gu), device_blocks_np(stacked))
    assert (fst.gate_up.scheme, fst.down.scheme) == (IQ3_S, ffi.Q4_K)
    bad = wq.reshape(-1, 110).copy()
    bad[5, 0:2] = np.frombuffer(np.uint16(0x7C00).tobytes(), np.uint8)
    b2 = build([], [("w", (k, n), 21, bad.tobytes())])
    with pytest.raises(gguf.GgufError, match="1 block"):
        gguf.load_matmul_weight(gguf.GgufFile.parse(b2), b2, "w")
