"""GPU parity of the decode (bit-exact) and of the dequant-fused GEMV / GEMM
against the CPU oracle, through the C ABI."""
from __future__ import annotations

import numpy as np
import pytest

import oracle_ffi as O
from golden_io import iq4_cases, q4k_cases
from r9v_amd import ffi, synth
from tol import check_bf16_out, check_close

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def bf16_dev(bits):
    return dev(bits.view(np.int16)).view(torch.bfloat16)


def host(t):
    return t.cpu().numpy()


# ---------------------------------------------------------------- decode

@pytest.mark.parametrize("scheme", [O.Q4_K, O.IQ4_XS])
def test_dequantize_bit_exact_random(scheme):
    n, k = 61, 1024
    w = synth.quant_weights(scheme, 101, n, k)
    got = host(ffi.dequantize(dev(w), scheme, n, k))
    want = O.dequantize(scheme, w, n, k)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequantize_golden_vectors():
    for c in q4k_cases():
        got = host(ffi.dequantize(dev(c["block"]), O.Q4_K, 1, 256))[0]
        assert np.array_equal(got.view(np.uint32), c["y_bits"]), c["name"]
    c = iq4_cases()["IQ4_XS"]
    got = host(ffi.dequantize(dev(c["wire"]), O.IQ4_XS, c["n"], c["k"]))
    assert np.array_equal(got.reshape(-1).view(np.uint32), c["y_bits"])


def test_validate_weights_counts_nonfinite_blocks():
    w = synth.quant_weights(O.Q4_K, 5, 8, 512).copy()
    w[3, 2:4] = [0x00, 0x7C]  # dmin of block 6 = +inf
    w[5, 144:146] = [0x01, 0x7E]  # d of block 11 = nan
    assert ffi.validate_weights(dev(w), O.Q4_K, 8, 512) == 2
    assert ffi.validate_weights(dev(synth.quant_weights(O.IQ4_XS, 6, 8, 512)), O.IQ4_XS, 8, 512) == 0


# ---------------------------------------------------------------- GEMV

def _gemv_case(scheme, n, k, m, x_dtype, out_dtype=O.F32, seed=0, bias=False, residual=False):
    w = synth.quant_weights(scheme, seed + 1, n, k)
    if x_dtype == O.BF16:
        x = synth.normal_bf16(seed + 2, (m, k))
        xd = bf16_dev(x)
    else:
        x = synth.normal_f32(seed + 2, (m, k))
        xd = dev(x)
    b = synth.normal_f32(seed + 3, (n,)) if bias else None
    r = synth.normal_f32(seed + 4, (m, n)) if residual else None
    ref = O.matmul(scheme, w, n, k, x, x_dtype, bias=b, residual=r)
    y = ffi.matmul(dev(w), scheme, n, k, xd, out_dtype=out_dtype,
                   bias=None if b is None else dev(b), residual=None if r is None else dev(r))
    torch.cuda.synchronize()
    got = host(y.float()) if out_dtype == O.BF16 else host(y)
    return got, ref


def test_gemv_config0_q4k_f32():
    """Q4_K 4096x4096, x fp32 [1x4096], y fp32."""
    got, ref = _gemv_case(O.Q4_K, 4096, 4096, 1, O.F32, seed=1000)
    check_close(got, ref, "config0")


@pytest.mark.parametrize("m", [1, 5])
def test_gemv_config1_iq4xs_bf16(m):
    """IQ4_XS K=2048 N=5120, x bf16 [M x 2048], M in {1, 5}."""
    got, ref = _gemv_case(O.IQ4_XS, 5120, 2048, m, O.BF16, seed=2000 + m)
    check_close(got, ref, f"config1 m={m}")


@pytest.mark.parametrize("scheme", [O.Q4_K, O.IQ4_XS])
@pytest.mark.parametrize("x_dtype", [O.F32, O.BF16])
@pytest.mark.parametrize("m", [1, 2, 3, 5, 8])
def test_gemv_k_and_n_sweep(scheme, x_dtype, m):
    """Lanes-per-row widths 24 (K=768), 32, 64 with one and two chunks per lane."""
    for n, k in ((77, 768), (130, 1024), (1000, 2048), (33, 4096), (9, 8192)):
        got, ref = _gemv_case(scheme, n, k, m, x_dtype, seed=3500 + m + n)
        check_close(got, ref, f"n={n} k={k} m={m}")


@pytest.mark.parametrize("scheme", [O.Q4_K, O.IQ4_XS])
@pytest.mark.parametrize("n,k,m", [(4096, 14336, 1), (2600, 14336, 4), (6000, 8192, 2), (9000, 8192, 5),
                                   (14336, 4096, 8), (700, 4096, 6)])
def test_gemv_multi_segment_rows(scheme, n, k, m):
    """Rows of several 64-lane K segments (K = 14336 is seven, K = 8192 four,
    K = 4096 at M >= 5 two) at row counts where the launcher picks each
    number of rows per lane group."""
    w = synth.quant_weights(scheme, 7100 + n + m, n, k)
    x = synth.normal_bf16(7200 + k + m, (m, k))
    y = host(ffi.matmul(dev(w), scheme, n, k, bf16_dev(x)))
    check_close(y, O.matmul(scheme, w, n, k, x, O.BF16, threads=8), f"n={n} k={k} m={m}")


@pytest.mark.parametrize("scheme", [O.Q4_K, O.IQ4_XS])
@pytest.mark.parametrize("x_dtype", [O.BF16, O.F32])
@pytest.mark.parametrize("n,k", [(20001, 4096), (13000, 2048), (32768, 4096)])
def test_gemv_streaming_form(scheme, x_dtype, n, k):
    """m = 1 over n >= 12 x SIMDs rows takes the streaming kernel (persistent
    waves, two weight buffers); every output against the oracle, and each
    row bit-equal to the same row in an m = 2 launch (the one-shot kernel):
    the two forms share the per-row arithmetic.  n = 20001 leaves a ragged
    last row group."""
    w = synth.quant_weights(scheme, 7300 + n + k, n, k)
    x = synth.normal_bf16(7400 + k, (2, k)) if x_dtype == O.BF16 else synth.normal_f32(7400 + k, (2, k))
    xd = bf16_dev(x) if x_dtype == O.BF16 else dev(x)
    wd = dev(w)
    y1 = host(ffi.matmul(wd, scheme, n, k, xd[:1].contiguous(), m_bucket=8))
    y2 = host(ffi.matmul(wd, scheme, n, k, xd, m_bucket=8))
    assert np.array_equal(y1[0].view(np.int32), y2[0].view(np.int32)), "streaming and one-shot rows differ"
    check_close(y1, O.matmul(scheme, w, n, k, x[:1], x_dtype, threads=8), f"n={n} k={k}")


def test_gemv_graph_replays_match_eager():
    """GEMV launches captured in a HIP graph: every replay (with eager work
    between replays) equals the eager result bit for bit."""
    n, k, m = 5120, 2048, 5
    w = dev(synth.quant_weights(O.IQ4_XS, 3701, n, k))
    x = bf16_dev(synth.normal_bf16(3702, (m, k)))
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    ffi.matmul(w, O.IQ4_XS, n, k, x, y=y)
    want = host(y).copy()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ffi.matmul(w, O.IQ4_XS, n, k, x, y=y, stream=s)
        s.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for _ in range(3):
                ffi.matmul(w, O.IQ4_XS, n, k, x, y=y, stream=s)
    torch.cuda.synchronize()
    for _ in range(3):
        y.fill_(0.0)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(y), want)
        ffi.matmul(w, O.IQ4_XS, n, k, x)  # eager work between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("scheme", [O.Q4_K, O.IQ4_XS])
@pytest.mark.parametrize("x_dtype", [O.F32, O.BF16])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 6, 7, 8])
def test_gemv_all_m(scheme, x_dtype, m):
    got, ref = _gemv_case(scheme, 77, 1024, m, x_dtype, seed=3000 + m)
    check_close(got, ref, f"m={m}")


@pytest.mark.parametrize("scheme", [O.Q4_K, O.IQ4_XS])
@pytest.mark.parametrize("n,k", [(1, 256), (3, 512), (17, 768), (130, 2048), (33, 4096), (9, 8192)])
def test_gemv_ragged_shapes(scheme, n, k):
    got, ref = _gemv_case(scheme, n, k, 3, O.BF16, seed=4000 + n + k)
    check_close(got, ref, f"n={n} k={k}")
    got, ref = _gemv_case(scheme, n, k, 1, O.F32, seed=4100 + n + k)
    check_close(got, ref, f"f32 n={n} k={k}")


def test_gemv_epilogues_and_bf16_out():
    got, ref = _gemv_case(O.IQ4_XS, 96, 512, 4, O.BF16, seed=5000, bias=True)
    check_close(got, ref, "bias")
    got, ref = _gemv_case(O.Q4_K, 96, 512, 4, O.BF16, seed=5001, residual=True)
    check_close(got, ref, "residual")
    got, ref = _gemv_case(O.Q4_K, 96, 512, 2, O.BF16, out_dtype=O.BF16, seed=5002)
    got32, _ = _gemv_case(O.Q4_K, 96, 512, 2, O.BF16, out_dtype=O.F32, seed=5002)
    check_bf16_out(got, got32, ref, "bf16 out")


def test_gemv_batch_invariance():
    """Row m of a batched launch equals the same row launched alone (bit-equal),
    the T0 batch-invariance gate (crates/r9v-t0/src/harness.rs:910-950)."""
    n, k = 300, 2048
    w = dev(synth.quant_weights(O.IQ4_XS, 6001, n, k))
    x = bf16_dev(synth.normal_bf16(6002, (5, k)))
    yb = host(ffi.matmul(w, O.IQ4_XS, n, k, x))
    for r in range(5):
        y1 = host(ffi.matmul(w, O.IQ4_XS, n, k, x[r:r + 1].contiguous()))
        assert np.array_equal(y1[0], yb[r])
    y2 = host(ffi.matmul(w, O.IQ4_XS, n, k, x))
    assert np.array_equal(y2, yb)  # run-twice determinism


def test_matmul_refusals():
    w = dev(synth.quant_weights(O.Q4_K, 7, 4, 256))
    x = dev(np.zeros((1, 300), np.float32))
    with pytest.raises(ffi.R9vxError) as e:
        ffi.matmul(w, O.Q4_K, 4, 300, x)
    assert e.value.code == -1 and "k=300" in str(e.value)
    with pytest.raises(ffi.R9vxError):
        ffi.matmul(w, 99, 4, 256, dev(np.zeros((1, 256), np.float32)))


# ---------------------------------------------------------------- MFMA GEMM

def _gemm_case(scheme, n, k, m, seed, out_dtype=O.F32, bias=False, residual=False, rows=None, cols=None,
               oracle=True):
    """Full GPU GEMM; oracle on the sampled rows/cols (all when None)."""
    w = synth.quant_weights(scheme, seed + 1, n, k)
    x = synth.normal_bf16(seed + 2, (m, k))
    b = synth.normal_f32(seed + 3, (n,)) if bias else None
    r = synth.normal_f32(seed + 4, (m, n)) if residual else None
    y = ffi.matmul(dev(w), scheme, n, k, bf16_dev(x), out_dtype=out_dtype,
                   bias=None if b is None else dev(b), residual=None if r is None else dev(r))
    got = host(y.float())
    rows = np.arange(m) if rows is None else np.asarray(rows)
    cols = np.arange(n) if cols is None else np.asarray(cols)
    if not oracle:
        return got[np.ix_(rows, cols)], None
    ref = O.matmul(scheme, np.ascontiguousarray(w[cols]), len(cols), k, np.ascontiguousarray(x[rows]), O.BF16,
                   bias=None if b is None else np.ascontiguousarray(b[cols]),
                   residual=None if r is None else np.ascontiguousarray(r[np.ix_(rows, cols)]))
    return got[np.ix_(rows, cols)], ref


def test_gemm_config2_full():
    """x bf16 [2048 x 4096] . Q4_K [14336 x 4096]^T -> bf16; every
    one of the 2048 x 14336 outputs against the oracle (its OpenMP form on
    all host threads, bit-identical to the serial one)."""
    m, n, k = 2048, 14336, 4096
    w = synth.quant_weights(O.Q4_K, 7001, n, k)
    x = synth.normal_bf16(7002, (m, k))
    wd, xd = dev(w), bf16_dev(x)
    got = host(ffi.matmul(wd, O.Q4_K, n, k, xd, out_dtype=O.BF16).float())
    got32 = host(ffi.matmul(wd, O.Q4_K, n, k, xd, out_dtype=O.F32))
    ref = O.matmul(O.Q4_K, w, n, k, x, O.BF16, threads=O.host_threads())
    check_bf16_out(got, got32, ref, "config2 full")


@pytest.mark.parametrize("scheme", [O.Q4_K, O.IQ4_XS])
@pytest.mark.parametrize("m,n,k", [(9, 33, 256), (100, 300, 768), (257, 256, 512), (512, 513, 1024)])
def test_gemm_shapes(scheme, m, n, k):
    got, ref = _gemm_case(scheme, n, k, m, 7100 + m + n + k)
    check_close(got, ref, f"m={m} n={n} k={k}")


# Launches of many 256 x 256 tiles (gemm3_kernel, every n): ragged M and N
# tails (the last weight block past n decodes row n - 1 again and stores
# nothing past n) and the smallest K (one super-block).
@pytest.mark.parametrize("scheme", [O.Q4_K, O.IQ4_XS])
@pytest.mark.parametrize("m,n,k", [(1000, 16400, 256), (1024, 16384, 512), (770, 21760, 1280), (300, 65536, 256)])
def test_gemm_large_ragged_shapes(scheme, m, n, k):
    rows = np.unique(np.concatenate([np.arange(0, m, 37), [0, 255, 256, m - 1]]))
    cols = np.unique(np.concatenate([np.arange(0, n, 29), [0, 31, 32, 255, 256, n - 17, n - 1]]))
    got, ref = _gemm_case(scheme, n, k, m, 7300 + m + k, rows=rows, cols=cols)
    check_close(got, ref, f"m={m} n={n} k={k}")


# Epilogues and bf16 output with n a multiple of 256, with a ragged last
# block (n % 8 == 0: 16-byte rows), and with n % 8 != 0 (element stores).
@pytest.mark.parametrize("n", [28000, 28160, 1001])
def test_gemm_epilogues_ragged_n(n):
    m, k = 600, 256
    rows = np.arange(0, m, 7)
    cols = np.unique(np.concatenate([np.arange(0, n, 41), [n - 1]]))
    got, ref = _gemm_case(O.IQ4_XS, n, k, m, 7400, bias=True, rows=rows, cols=cols)
    check_close(got, ref, "bias")
    got, ref = _gemm_case(O.Q4_K, n, k, m, 7401, residual=True, rows=rows, cols=cols)
    check_close(got, ref, "residual")
    got, ref = _gemm_case(O.Q4_K, n, k, m, 7402, out_dtype=O.BF16, rows=rows, cols=cols)
    got32, _ = _gemm_case(O.Q4_K, n, k, m, 7402, out_dtype=O.F32, rows=rows, cols=cols, oracle=False)
    check_bf16_out(got, got32, ref, "bf16 out")


# The 256-column GEMM (gemm3_kernel) cuts each weight block's rows into
# chunks sized to fill whole rounds of the CUs; these shapes reach its plans:
# one block, one 32-row tile per chunk, every block with the same chunk
# count (the XCD band order), two chunk counts across blocks, several
# rounds, ragged last row tiles.
@pytest.mark.parametrize("scheme", [O.Q4_K, O.IQ4_XS])
@pytest.mark.parametrize("m,n", [(9, 256), (700, 2560), (2048, 4096), (1100, 5376), (2600, 14336)])
def test_gemm_row_chunk_plans(scheme, m, n):
    k = 512
    rows = np.arange(m) if m * n <= 4_000_000 else np.unique(np.concatenate([np.arange(0, m, 7), [m - 1]]))
    got, ref = _gemm_case(scheme, n, k, m, 7500 + m, rows=rows)
    check_close(got, ref, f"m={m} n={n}")


def test_gemm_rows_past_32_bit_activation_offsets():
    """m * k >= 2^31 (x16 past 4 GiB): the rows go in several launches (at
    most 149,792 rows at k = 14336); rows on both sides of the cut meet the
    oracle and equal, bit for bit, the same rows launched alone."""
    m, n, k = 150000, 256, 14336
    w_h = synth.quant_weights(O.Q4_K, 7701, n, k)
    w = dev(w_h)
    g = torch.Generator(device="cuda")
    g.manual_seed(7702)
    x = torch.randn((m, k), generator=g, device="cuda").to(torch.bfloat16)
    y = ffi.matmul(w, O.Q4_K, n, k, x)
    rows = [0, 149791, 149792, 149999]
    got = host(y[rows])
    del y
    alone = host(ffi.matmul(w, O.Q4_K, n, k, x[rows].contiguous(), m_bucket=16))
    assert np.array_equal(got.view(np.uint32), alone.view(np.uint32))
    xr = host(x[rows].view(torch.int16)).view(np.uint16)
    del x
    torch.cuda.empty_cache()
    check_close(got, O.matmul(O.Q4_K, w_h, n, k, xr, O.BF16, threads=8), "rows around the launch cut")


def test_gemm_row_chunk_plans_keep_row_bits():
    """The same rows under two chunk plans of one static (m = 1100 and 2600 at
    m_bucket 4096, n = 14336: one round of uniform chunks, three rounds of two
    chunk counts) come out bit-equal."""
    n, k = 14336, 512
    w = dev(synth.quant_weights(O.Q4_K, 7601, n, k))
    x = synth.normal_bf16(7602, (2600, k))
    big = host(ffi.matmul(w, O.Q4_K, n, k, bf16_dev(x), m_bucket=4096).view(torch.int32))
    small = host(ffi.matmul(w, O.Q4_K, n, k, bf16_dev(x[:1100]), m_bucket=4096).view(torch.int32))
    assert np.array_equal(small, big[:1100])


def test_gemm_epilogues_bf16_out():
    got, ref = _gemm_case(O.IQ4_XS, 200, 512, 40, 7200, bias=True)
    check_close(got, ref, "bias")
    got, ref = _gemm_case(O.Q4_K, 200, 512, 40, 7201, residual=True)
    check_close(got, ref, "residual")
    got, ref = _gemm_case(O.Q4_K, 300, 1024, 70, 7202, out_dtype=O.BF16)
    got32, _ = _gemm_case(O.Q4_K, 300, 1024, 70, 7202, out_dtype=O.F32, oracle=False)
    check_bf16_out(got, got32, ref, "bf16 out")


def test_gemm_row_permutation_invariance_full_size():
    """Each output row depends only on its own x row: permuting the 2048 rows
    of configs[2] permutes y bit for bit (size-independent check)."""
    m, n, k = 2048, 14336, 4096
    w = dev(synth.quant_weights(O.Q4_K, 7301, n, k))
    x = synth.normal_bf16(7302, (m, k))
    perm = np.random.default_rng(5).permutation(m)
    y = host(ffi.matmul(w, O.Q4_K, n, k, bf16_dev(x), out_dtype=O.BF16).view(torch.int16))
    yp = host(ffi.matmul(w, O.Q4_K, n, k, bf16_dev(x[perm]), out_dtype=O.BF16).view(torch.int16))
    assert np.array_equal(yp, y[perm])


@pytest.mark.parametrize("m,n,k", [(16, 64, 512), (520, 32768, 256)])
def test_gemm_large_activation_rows_scaled_exactly(m, n, k):
    """Rows with |x| >= 2^15 go through the power-of-two row scale (the
    128-row tile and the 256-row LDS-decoded tile)."""
    w = synth.quant_weights(O.Q4_K, 7401, n, k)
    xf = synth.normal_f32(7402, (m, k))
    xf[3] *= 1e6
    xf[7, 5] = 3e9
    x = synth.to_bf16_bits(xf)
    y = host(ffi.matmul(dev(w), O.Q4_K, n, k, bf16_dev(x)))
    cols = np.arange(0, n, max(1, n // 512))
    ref = O.matmul(O.Q4_K, np.ascontiguousarray(w[cols]), len(cols), k, x, O.BF16)
    check_close(y[:, cols], ref, "large rows")
