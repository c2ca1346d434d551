"""GPU parity of the Q8_0 and Q6_K path (the other GGUF types on the model
path: Q8_0 projections, Q6_K heads and value/down projections of Q4_K_M
files), through the C ABI.

- wire decode is bit-exact with the oracle and with the reference's gguf-py
  golden vectors (gguf_a23_reference.txt);
- the load-time split (r9vx_repack_launch, and the host split of
  r9vx_gguf_upload_split) moves every wire byte to its place, bit for bit;
- the decode GEMV on the split layout meets the oracle (f32 decode then the
  ascending-K dot of matmul.rs:1940-2414) at the north-star tolerance, with
  every epilogue and output dtype.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle_ffi as O
from golden_io import a23_cases
from gguf_build import build
from r9v_amd import ffi, gguf, synth
from tol import check_bf16_out, check_close

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

SCHEMES = [ffi.Q6_K, ffi.Q8_0]


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def bf16_dev(bits):
    return dev(bits.view(np.int16)).view(torch.bfloat16)


def host(t):
    return t.cpu().numpy()


def split_np(wire, scheme):
    """The split layout restated in numpy: body = blocks without d, d array."""
    bb = ffi.BLOCK_BYTES[scheme]
    blocks = wire.reshape(-1, bb)
    o = synth.D_OFFSET[scheme]
    body = np.concatenate([blocks[:, :o], blocks[:, o + 2:]], axis=1).reshape(-1)
    return body, blocks[:, o:o + 2].copy().view(np.int16).reshape(-1)


@pytest.mark.parametrize("scheme", SCHEMES)
def test_dequantize_bit_exact_random(scheme):
    n, k = 37, 1024
    w = synth.quant_weights(scheme, 515, n, k)
    got = host(ffi.dequantize(dev(w), scheme, n, k))
    assert np.array_equal(got.view(np.uint32), O.dequantize(scheme, w, n, k).view(np.uint32))


def test_dequantize_golden_vectors():
    cases = a23_cases()
    for name, scheme in (("Q8_0", ffi.Q8_0), ("Q6_K", ffi.Q6_K), ("Q4_K", ffi.Q4_K)):
        c = cases[name]
        wire = np.ascontiguousarray(c["wire"])
        got = host(ffi.dequantize(dev(wire), scheme, c["n"], c["k"]))
        assert np.array_equal(got.reshape(-1).view(np.uint32), c["y_bits"]), name


@pytest.mark.parametrize("scheme", SCHEMES)
def test_repack_moves_every_byte(scheme):
    n, k = 29, 2048
    w = synth.quant_weights(scheme, 616, n, k)
    body, scales = ffi.repack(dev(w), scheme, n, k)
    want_body, want_scales = split_np(w, scheme)
    assert np.array_equal(host(body), want_body)
    assert np.array_equal(host(scales), want_scales)


@pytest.mark.parametrize("scheme", SCHEMES)
def test_validate_counts_nonfinite_wire_scales(scheme):
    n, k = 4, 512
    w = synth.quant_weights(scheme, 17, n, k).reshape(-1, ffi.BLOCK_BYTES[scheme]).copy()
    o = synth.D_OFFSET[scheme]
    for b, bits in ((1, 0x7C00), (5, 0xFE00), (6, 0xFC00)):
        w[b, o:o + 2] = np.frombuffer(np.uint16(bits).tobytes(), np.uint8)
    assert ffi.validate_weights(dev(w.reshape(-1)), scheme, n, k) == 3


SHAPES = [(4096, 4096, 1), (1024, 4096, 5), (5120, 2048, 3), (333, 1280, 8), (64, 256, 2),
          (777, 3072, 4), (2048, 2048, 7)]


@pytest.mark.parametrize("scheme", SCHEMES)
@pytest.mark.parametrize("n,k,m", SHAPES)
def test_gemv_split_layout_parity(scheme, n, k, m):
    w = synth.quant_weights(scheme, 1000 + n + m, n, k)
    x = synth.normal_bf16(2000 + k + m, (m, k))
    body, scales = ffi.repack(dev(w), scheme, n, k)
    y = host(ffi.matmul(body, scheme, n, k, bf16_dev(x), w_scales=scales))
    check_close(y, O.matmul(scheme, w, n, k, x, O.BF16), f"scheme={scheme} n={n} k={k} m={m}")


@pytest.mark.parametrize("scheme", SCHEMES)
def test_gemv_split_epilogues_and_bf16_out(scheme):
    n, k, m = 640, 2048, 3
    w = synth.quant_weights(scheme, 31, n, k)
    x = synth.normal_bf16(32, (m, k))
    body, scales = ffi.repack(dev(w), scheme, n, k)
    bias = synth.normal_f32(33, (n,))
    res = synth.normal_f32(34, (m, n))
    yb = host(ffi.matmul(body, scheme, n, k, bf16_dev(x), bias=dev(bias), w_scales=scales))
    check_close(yb, O.matmul(scheme, w, n, k, x, O.BF16, bias=bias), "bias")
    yr = host(ffi.matmul(body, scheme, n, k, bf16_dev(x), residual=dev(res), w_scales=scales))
    check_close(yr, O.matmul(scheme, w, n, k, x, O.BF16, residual=res), "residual")
    y16 = ffi.matmul(body, scheme, n, k, bf16_dev(x), out_dtype=ffi.BF16, w_scales=scales)
    y32 = host(ffi.matmul(body, scheme, n, k, bf16_dev(x), w_scales=scales))
    got16 = host(y16.view(torch.int16)).view(np.uint16).astype(np.uint32) << 16
    check_bf16_out(got16.view(np.float32), y32, O.matmul(scheme, w, n, k, x, O.BF16), "bf16 out")


@pytest.mark.parametrize("scheme", SCHEMES)
def test_gemv_split_row_and_batch_invariance(scheme):
    """A row's result does not depend on the other activation rows or on the
    other weight rows it shares a launch with (bit for bit)."""
    n, k = 1500, 2048
    w = synth.quant_weights(scheme, 41, n, k)
    x = synth.normal_bf16(42, (6, k))
    body, scales = ffi.repack(dev(w), scheme, n, k)
    full = host(ffi.matmul(body, scheme, n, k, bf16_dev(x), w_scales=scales))
    for r in range(6):
        one = host(ffi.matmul(body, scheme, n, k, bf16_dev(x[r:r + 1]), w_scales=scales))
        assert np.array_equal(one.view(np.uint32), full[r:r + 1].view(np.uint32)), r
    # a sub-matrix of rows, repacked on its own, gives the same values for those rows
    body2, scales2 = ffi.repack(dev(w[100:356]), scheme, 256, k)
    part = host(ffi.matmul(body2, scheme, 256, k, bf16_dev(x), w_scales=scales2))
    assert np.array_equal(part.view(np.uint32), full[:, 100:356].view(np.uint32))


def test_gguf_split_upload_runs_like_the_device_repack():
    n, k = 320, 2048
    wq6 = synth.quant_weights(ffi.Q6_K, 71, n, k)
    wq8 = synth.quant_weights(ffi.Q8_0, 72, 256, k)
    b = build([("general.architecture", (8, "llama"))],
              [("output.weight", (k, n), 14, wq6.tobytes()), ("blk.0.attn_v.weight", (k, 256), 8, wq8.tobytes())])
    f = gguf.GgufFile.parse(b)
    x = synth.normal_bf16(73, (2, k))
    for name, wire, scheme, rows in (("output.weight", wq6, ffi.Q6_K, n), ("blk.0.attn_v.weight", wq8, ffi.Q8_0, 256)):
        st, body, scales = gguf.load_matmul_weight(f, b, name, m_bucket=2)
        assert (st.n, st.k, st.w_scheme) == (rows, k, scheme)
        want_body, want_scales = split_np(wire, scheme)
        assert np.array_equal(host(body), want_body) and np.array_equal(host(scales), want_scales)
        y = host(ffi.matmul(body, scheme, rows, k, bf16_dev(x), w_scales=scales))
        check_close(y, O.matmul(scheme, wire, rows, k, x, O.BF16), name)
    bad = wq6.copy().reshape(-1, 210)
    bad[3, 208:210] = np.frombuffer(np.uint16(0x7C00).tobytes(), np.uint8)
    b2 = build([], [("w", (k, n), 14, bad.tobytes())])
    with pytest.raises(gguf.GgufError, match="1 block"):
        gguf.load_matmul_weight(gguf.GgufFile.parse(b2), b2, "w")


PREFILL = [(9, 320, 2048), (40, 1000, 4096), (300, 512, 2048), (129, 2304, 1024)]


@pytest.mark.parametrize("scheme", SCHEMES)
@pytest.mark.parametrize("m,n,k", PREFILL)
def test_prefill_gemm_split_layout_parity(scheme, m, n, k):
    """m > 8: the MFMA GEMM on the split layout (the 256 x 256 loop; a
    ragged n repeats row n - 1 in its last weight block)."""
    w = synth.quant_weights(scheme, 3000 + m + n, n, k)
    x = synth.normal_bf16(4000 + m + k, (m, k))
    body, scales = ffi.repack(dev(w), scheme, n, k)
    y = host(ffi.matmul(body, scheme, n, k, bf16_dev(x), w_scales=scales))
    check_close(y, O.matmul(scheme, w, n, k, x, O.BF16, threads=8), f"scheme={scheme} m={m} n={n} k={k}")


# Q8_0 / Q6_K run the 256 x 256 loop (every n) that decodes each
# weight tile once into LDS (two threads per weight row; a thread's half K
# step is one Q8_0 block, or 16 Q6_K ql bytes and their 16 qh bytes, loaded
# two steps ahead); these shapes reach its row-chunk plans (one block,
# uniform chunks in the XCD band order, two chunk counts, several rounds)
# with ragged last row tiles and the bias epilogue.
@pytest.mark.parametrize("scheme", SCHEMES)
@pytest.mark.parametrize("m,n,k", [(9, 256, 512), (700, 2560, 512), (1100, 5376, 512), (2048, 4096, 1024)])
def test_prefill_gemm_split_256_tile(scheme, m, n, k):
    w = synth.quant_weights(scheme, 3100 + m + scheme, n, k)
    x = synth.normal_bf16(3200 + m, (m, k))
    b = synth.normal_f32(3300 + m, (n,))
    body, scales = ffi.repack(dev(w), scheme, n, k)
    y = host(ffi.matmul(body, scheme, n, k, bf16_dev(x), bias=dev(b), w_scales=scales))
    rows = np.arange(m) if m * n <= 4_000_000 else np.unique(np.concatenate([np.arange(0, m, 7), [m - 1]]))
    ref = O.matmul(scheme, w, n, k, np.ascontiguousarray(x[rows]), O.BF16, bias=b, threads=8)
    check_close(y[rows], ref, f"scheme={scheme} m={m} n={n} k={k}")


@pytest.mark.parametrize("scheme", SCHEMES)
def test_prefill_gemm_split_large_sampled(scheme):
    """A 1024 x 4096 x 4096 launch (16 K tiles of rows, 16 column tiles):
    sampled rows against the oracle, residual epilogue and bf16 output."""
    m, n, k = 1024, 4096, 4096
    w = synth.quant_weights(scheme, 5151, n, k)
    x = synth.normal_bf16(5152, (m, k))
    res = synth.normal_f32(5153, (m, n))
    body, scales = ffi.repack(dev(w), scheme, n, k)
    y = host(ffi.matmul(body, scheme, n, k, bf16_dev(x), residual=dev(res), w_scales=scales))
    yb = ffi.matmul(body, scheme, n, k, bf16_dev(x), residual=dev(res), out_dtype=ffi.BF16, w_scales=scales)
    rows = np.array([0, 1, 127, 128, 511, 640, 1000, 1023])
    ref = O.matmul(scheme, w, n, k, x[rows], O.BF16, residual=res[rows], threads=8)
    check_close(y[rows], ref, f"scheme={scheme} sampled")
    got16 = host(yb.view(torch.int16))[rows].view(np.uint16).astype(np.uint32) << 16
    check_bf16_out(got16.view(np.float32), y[rows], ref, "bf16 out")
