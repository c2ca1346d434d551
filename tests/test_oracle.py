"""Pins the CPU oracle (the checker) before anything is compared against it.

Each oracle function is checked against the reference's own golden vectors
(tests/golden, copied from crates/r9v-format/tests/fixtures) or against what
the mathematics fixes: closed forms, brute force in f64, exhaustive
enumeration, and invariants chosen so a dropped term, a wrong index or a
transposed operand fails.
"""
from __future__ import annotations

import pathlib
import re
import struct
import subprocess

import numpy as np
import pytest

import oracle_ffi as O
from golden_io import a23_cases, iq4_cases, q4k_cases
from r9v_amd import synth

ROOT = pathlib.Path(__file__).resolve().parent.parent
KVALUES = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113],
                   dtype=np.int8)


def f16(v: float) -> int:
    return int(np.array(v, dtype=np.float16).view(np.uint16))


# ---------------------------------------------------------------- codecs

def test_f16_to_f32_exhaustive():
    """scales.rs:13-36 equals numpy's exact float16 widening on all 65536 patterns."""
    L = O.lib()
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([L.rxo_f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_bf16_rne_matches_torch_and_ties():
    torch = pytest.importorskip("torch")
    L = O.lib()
    rng = np.random.default_rng(7)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32),
        # exact ties: low half = 0x8000 with even / odd kept LSB
        np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x7F7FFFFF, 0x00008000, 0x80000000],
                 dtype=np.uint32).view(np.float32),
    ])
    want = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([L.rxo_f32_to_bf16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, want)
    assert np.array_equal(synth.to_bf16_bits(vals), want)


# ---------------------------------------------------------------- Q4_K decode

def test_q4k_golden_bit_exact():
    """crates/r9v-format/tests/schemes.rs:482-516: decode matches llama.cpp /
    gguf-py dequantize bit for bit on all six reference blocks."""
    for c in q4k_cases():
        got = O.dequantize(O.Q4_K, c["block"], 1, 256)[0]
        assert np.array_equal(got.view(np.uint32), c["y_bits"]), c["name"]


def test_q4k_scale_unpack_golden():
    L = O.lib()
    for c in q4k_cases():
        sc = np.zeros(8, dtype=np.uint8)
        mn = np.zeros(8, dtype=np.uint8)
        payload = np.ascontiguousarray(c["block"][4:16])
        L.rxo_q4k_unpack_scales(O._p(payload), O._p(sc), O._p(mn))
        assert list(sc) == c["sc"] and list(mn) == c["mn"], c["name"]
        assert int(c["block"][0]) | (int(c["block"][1]) << 8) == c["d_bits"]
        assert int(c["block"][2]) | (int(c["block"][3]) << 8) == c["dmin_bits"]


def test_q4k_nibble_order_against_logical_q():
    """The fixture's logical q (row-major nibbles) pins the wire nibble order:
    with d=1, dmin=0, every sc=1 the decode returns q itself."""
    for c in q4k_cases():
        blk = c["block"].copy()
        blk[0:2] = np.frombuffer(struct.pack("<H", f16(1.0)), np.uint8)
        blk[2:4] = 0
        blk[4:16] = np.array([1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1], dtype=np.uint8)  # sc=1, mn=0
        got = O.dequantize(O.Q4_K, blk, 1, 256)[0]
        assert np.array_equal(got, np.array(c["q"], dtype=np.float32)), c["name"]


def test_q4k_closed_form_formula():
    """w = (d*sc)*q - (dmin*mn) with a distinct value per sub-block."""
    blk = np.zeros(144, dtype=np.uint8)
    blk[0:2] = np.frombuffer(struct.pack("<H", f16(0.5)), np.uint8)
    blk[2:4] = np.frombuffer(struct.pack("<H", f16(0.25)), np.uint8)
    sc = [1, 2, 3, 4, 17, 33, 49, 63]
    mn = [5, 6, 7, 8, 20, 40, 60, 61]
    pay = np.zeros(12, dtype=np.uint8)
    for j in range(4):
        pay[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        pay[j + 4] = mn[j] | ((mn[j + 4] >> 4) << 6)
        pay[j + 8] = (sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4)
    blk[4:16] = pay
    q = np.arange(256) % 16
    for j in range(8):
        for p in range(32):
            byte = blk[16 + (j // 2) * 32 + p]
            byte |= (q[j * 32 + p] << (4 * (j % 2)))
            blk[16 + (j // 2) * 32 + p] = byte
    got = O.dequantize(O.Q4_K, blk, 1, 256)[0]
    want = np.array([np.float32(0.5 * sc[i // 32]) * np.float32(q[i]) - np.float32(0.25 * mn[i // 32])
                     for i in range(256)], dtype=np.float32)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------- IQ4_XS decode

def test_iq4xs_golden_bit_exact():
    """crates/r9v-format/tests/iq.rs:159-172: IQ4_XS 3x512 matches gguf-py 0.19.0."""
    c = iq4_cases()["IQ4_XS"]
    got = O.dequantize(O.IQ4_XS, c["wire"], c["n"], c["k"])
    assert np.array_equal(got.reshape(-1).view(np.uint32), c["y_bits"])


def _iq3s_grid_words():
    text = (ROOT / "r9v_amd" / "csrc" / "r9vx_iq3s_grid.h").read_text()
    body = text.split("#define R9VX_IQ3S_GRID_WORDS")[1].split("#endif")[0]
    return np.array([int(t, 16) for t in re.findall(r"0x([0-9a-f]{8})u", body)], dtype=np.uint32)


def test_iq3s_golden_bit_exact():
    """crates/r9v-format/tests/iq.rs:159-197: the IQ3_S 3x1024 case (seeded
    payloads, all-zero and all-0xFF blocks) matches gguf-py 0.19.0."""
    c = iq4_cases()["IQ3_S"]
    got = O.dequantize(O.IQ3_S, c["wire"], c["n"], c["k"])
    assert np.array_equal(got.reshape(-1).view(np.uint32), c["y_bits"])


def test_iq3s_grid_facts():
    """The codebook's facts from crates/r9v-format/tests/iq.rs:505,514-516
    (2048 values, all odd and <= 15), plus strict ascent of the 512 words."""
    w = _iq3s_grid_words()
    assert w.size == 512 and np.all(np.diff(w.astype(np.int64)) > 0)
    b = w.view(np.uint8)
    assert np.all(b % 2 == 1) and np.all(b <= 15)
    assert (w[0], w[1], w[511]) == (0x01010101, 0x01010103, 0x0F0F0101)


def _iq3s_llama_loop(blocks, grid):
    """llama.cpp's dequantize_row_iq3_s, restated in numpy: two groups of 32
    per step, the grid index's ninth bit taken as (qh << (8 - 2l)) & 256 and
    (qh << (7 - 2l)) & 256, signs through the 0x01..0x80 bit masks."""
    out = []
    g8 = grid.view(np.uint8).reshape(512, 4)
    for blk in blocks:
        d = np.float32(np.frombuffer(blk[0:2].tobytes(), np.float16)[0])
        qs, qh, signs, scales = blk[2:66], blk[66:74], blk[74:106], blk[106:110]
        y = []
        for ib32 in range(0, 8, 2):
            sc = int(scales[ib32 // 2])
            for half, s in ((0, sc & 0xF), (1, sc >> 4)):
                db = np.float32(d * np.float32(1 + 2 * s))
                q = qs[8 * (ib32 + half):8 * (ib32 + half) + 8]
                h = int(qh[ib32 + half])
                sg = signs[4 * (ib32 + half):4 * (ib32 + half) + 4]
                for l in range(4):
                    i1 = int(q[2 * l]) | ((h << (8 - 2 * l)) & 256)
                    i2 = int(q[2 * l + 1]) | ((h << (7 - 2 * l)) & 256)
                    for j in range(4):
                        v = np.float32(db * np.float32(g8[i1, j]))
                        y.append(-v if int(sg[l]) & (1 << j) else v)
                    for j in range(4):
                        v = np.float32(db * np.float32(g8[i2, j]))
                        y.append(-v if int(sg[l]) & (1 << (j + 4)) else v)
        out.append(np.array(y, dtype=np.float32))
    return np.concatenate(out)


def test_iq3s_matches_llama_cpp_loop():
    """Random blocks (finite d): the oracle equals the llama.cpp loop form."""
    rng = np.random.default_rng(321)
    blocks = rng.integers(0, 256, size=(24, 110), dtype=np.uint8)
    blocks[:, 0:2] = np.frombuffer(rng.normal(0, 0.05, 24).astype(np.float16).tobytes(), np.uint8).reshape(24, 2)
    got = O.dequantize(O.IQ3_S, blocks.reshape(-1), 3, 2048)
    want = _iq3s_llama_loop(blocks, _iq3s_grid_words())
    assert np.array_equal(got.reshape(-1).view(np.uint32), want.view(np.uint32))


def test_iq3s_nonfinite_scale_refused():
    blk = np.zeros(110, dtype=np.uint8)
    blk[0:2] = np.frombuffer(np.float16(np.inf).tobytes(), np.uint8)
    with pytest.raises(O.OracleError):
        O.dequantize(O.IQ3_S, blk, 1, 256)


def test_iq4xs_closed_form_codebook():
    """Every codebook slot and every 6-bit scale field: w = (d*(s-32))*kv[q]."""
    blk = np.zeros(136, dtype=np.uint8)
    blk[0:2] = np.frombuffer(struct.pack("<H", f16(0.125)), np.uint8)
    svals = [0, 1, 31, 32, 33, 47, 62, 63]
    sh = 0
    for g, s in enumerate(svals):
        blk[4 + g // 2] |= (s & 0xF) << (4 * (g % 2))
        sh |= ((s >> 4) & 3) << (2 * g)
    blk[2:4] = np.frombuffer(struct.pack("<H", sh), np.uint8)
    qv = np.array([(j * 7 + g) % 16 for g in range(8) for j in range(32)])
    for g in range(8):
        for j in range(32):
            b = 8 + 16 * g + (j % 16)
            blk[b] |= qv[g * 32 + j] << (0 if j < 16 else 4)
    got = O.dequantize(O.IQ4_XS, blk, 1, 256)[0]
    want = np.array([np.float32(np.float32(0.125) * np.float32(svals[i // 32] - 32))
                     * np.float32(KVALUES[qv[i]]) for i in range(256)], dtype=np.float32)
    assert np.array_equal(got, want)


def test_dequantize_refuses_nonfinite_scale():
    w = synth.quant_weights(O.Q4_K, 3, 2, 256).copy()
    w[1, 2:4] = np.frombuffer(struct.pack("<H", 0x7C00), np.uint8)  # dmin = inf
    with pytest.raises(O.OracleError):
        O.dequantize(O.Q4_K, w, 2, 256)
    w = synth.quant_weights(O.IQ4_XS, 3, 2, 256).copy()
    w[0, 0:2] = np.frombuffer(struct.pack("<H", 0x7E00), np.uint8)  # d = nan
    with pytest.raises(O.OracleError):
        O.dequantize(O.IQ4_XS, w, 2, 256)


# ------------------------------------------------------ Q6_K / Q8_0 decode

def test_a23_golden_bit_exact():
    """crates/r9v-format/tests/gguf.rs:172-180: Q8_0 (5x128), Q4_K and Q6_K
    (3x1024) wire decode to gguf-py 0.19.0's dequantize, bit for bit."""
    cases = a23_cases()
    assert set(cases) == {"Q8_0", "Q4_K", "Q6_K"}
    for name, scheme in (("Q8_0", O.Q8_0), ("Q4_K", O.Q4_K), ("Q6_K", O.Q6_K)):
        c = cases[name]
        got = O.dequantize(scheme, c["wire"], c["n"], c["k"])
        assert np.array_equal(got.reshape(-1).view(np.uint32), c["y_bits"]), name


def _q6k_llamacpp_rows(wire, n, k):
    """The textbook Q6_K row loop (llama.cpp dequantize_row_q6_K form): per
    128-weight half, l in 0..32 yields four weights from ql[l], ql[l+32] and
    the four bit pairs of qh[l]; y = d * sc * (q - 32) in f32."""
    blocks = wire.reshape(-1, 210)
    out = np.empty((blocks.shape[0], 256), dtype=np.float32)
    for b, blk in enumerate(blocks):
        d = np.frombuffer(blk[208:210].tobytes(), dtype=np.float16).astype(np.float32)[0]
        sc = blk[192:208].view(np.int8).astype(np.float32)
        for half in range(2):
            ql, qh, s = blk[64 * half:64 * half + 64].astype(np.int32), blk[128 + 32 * half:160 + 32 * half].astype(np.int32), sc[8 * half:8 * half + 8]
            for l in range(32):
                qs = [(ql[l] & 15) | ((qh[l] & 3) << 4), (ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4),
                      (ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4), (ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)]
                for r in range(4):
                    dl = np.float32(d * s[l // 16 + 2 * r])
                    out[b, 128 * half + 32 * r + l] = np.float32(dl * np.float32(qs[r] - 32))
    return out.reshape(n, k)


def test_q6k_matches_the_llamacpp_row_loop():
    """A restatement with a different structure (llama.cpp's loop over l with
    four outputs per step) agrees bit for bit on random blocks, so a wrong
    nibble, bit pair, byte index or scale index in either would show."""
    n, k = 3, 512
    w = synth.random_bytes(4242, n * (k // 256) * 210).reshape(-1, 210)
    w[:, 208:210] = synth.half_normal_f16_bits(4243, w.shape[0], 0.02).view(np.uint8).reshape(-1, 2)
    got = O.dequantize(O.Q6_K, w, n, k)
    assert np.array_equal(got.view(np.uint32), _q6k_llamacpp_rows(w.reshape(-1), n, k).view(np.uint32))


def test_q80_closed_form():
    n, k = 4, 96
    w = synth.random_bytes(77, n * (k // 32) * 34).reshape(-1, 34)
    w[:, 0:2] = synth.half_normal_f16_bits(78, w.shape[0], 0.05).view(np.uint8).reshape(-1, 2)
    d = w[:, 0:2].copy().view(np.float16).astype(np.float32)
    want = (d * w[:, 2:].view(np.int8).astype(np.float32)).astype(np.float32)
    assert np.array_equal(O.dequantize(O.Q8_0, w, n, k).reshape(-1, 32), want)


def test_q6k_q80_refuse_nonfinite_scales():
    w = synth.random_bytes(5, 2 * 210).reshape(2, 210)
    w[:, 208:210] = 0
    w[1, 208:210] = np.frombuffer(struct.pack("<H", 0x7C00), np.uint8)
    with pytest.raises(O.OracleError):
        O.dequantize(O.Q6_K, w, 2, 256)
    w = np.zeros((1, 34), dtype=np.uint8)
    w[0, 0:2] = np.frombuffer(struct.pack("<H", 0xFE00), np.uint8)
    with pytest.raises(O.OracleError):
        O.dequantize(O.Q8_0, w, 1, 32)


# ---------------------------------------------------------------- expf twin

def test_expf_twin_matches_libm_exhaustively(tmp_path):
    """The router's GPU exp equals the host expf on every float in [-104, 0]
    (the whole domain of exp(s - max)); 1.12e9 inputs."""
    exe = tmp_path / "expf_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fopenmp",
                    "-I", str(ROOT / "r9v_amd" / "csrc"), str(ROOT / "tests" / "expf_twin_check.c"),
                    "-o", str(exe), "-lm"], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    n, bad = map(int, out.stdout.split())
    assert n == 1120927745 and bad == 0, out.stdout


def test_expf_table_regenerates_from_definition():
    """Table entry i = bits(2^(i/32) rounded to double) - (i << 47)."""
    from decimal import Decimal, getcontext
    getcontext().prec = 60
    src = (ROOT / "r9v_amd" / "csrc" / "r9vx_expf.h").read_text()
    import re
    block = src[src.index("#define R9VX_EXP2_TAB_INIT"):]
    vals = [int(v, 16) for v in re.findall(r"(0x[0-9a-f]{16})ull", block)[:32]]
    entries = dict(enumerate(vals))
    for i in range(32):
        v = float(Decimal(2) ** (Decimal(i) / Decimal(32)))
        want = (struct.unpack("<Q", struct.pack("<d", v))[0] - (i << 47)) & (2**64 - 1)
        assert entries[i] == want, i


# ---------------------------------------------------------------- Branch-D matmul

def test_matmul_known_answer_1408():
    """crates/r9v-t0/tests/matmul_tests.rs:208-265: d=1, dmin=0.5, sc=2, mn=1,
    q=3 -> every weight 5.5; x = 1 over K = 256 -> y = 1408.0 exactly."""
    blk = np.zeros(144, dtype=np.uint8)
    blk[0:2] = np.frombuffer(struct.pack("<H", f16(1.0)), np.uint8)
    blk[2:4] = np.frombuffer(struct.pack("<H", f16(0.5)), np.uint8)
    blk[4:8] = 2
    blk[8:12] = 1
    blk[12:16] = 0x12  # sc[4..7]=2 (low nibble), mn[4..7]=1 (high nibble)
    blk[16:] = 0x33
    x = np.ones((1, 256), dtype=np.float32)
    y = O.matmul(O.Q4_K, blk, 1, 256, x, O.F32)
    assert y[0, 0] == 1408.0
    xb = synth.to_bf16_bits(x)
    assert O.matmul(O.Q4_K, blk, 1, 256, xb, O.BF16)[0, 0] == 1408.0


@pytest.mark.parametrize("scheme", [O.Q4_K, O.IQ4_XS])
def test_matmul_one_hot_selects_weight(scheme):
    """x = e_k gives y[:, n] = w[n, k] exactly: pins operand order and indexing."""
    n, k = 7, 512
    w = synth.quant_weights(scheme, 11, n, k)
    deq = O.dequantize(scheme, w, n, k)
    ks = [0, 1, 31, 32, 255, 256, 300, 511]
    x = np.zeros((len(ks), k), dtype=np.float32)
    for i, kk in enumerate(ks):
        x[i, kk] = 1.0
    y = O.matmul(scheme, w, n, k, x, O.F32)
    for i, kk in enumerate(ks):
        assert np.array_equal(y[i], deq[:, kk])


@pytest.mark.parametrize("scheme", [O.Q4_K, O.IQ4_XS])
def test_matmul_vs_f64_bruteforce(scheme):
    n, k, m = 24, 1024, 3
    w = synth.quant_weights(scheme, 21, n, k)
    deq = O.dequantize(scheme, w, n, k).astype(np.float64)
    x = synth.normal_f32(22, (m, k))
    y = O.matmul(scheme, w, n, k, x, O.F32)
    ref = x.astype(np.float64) @ deq.T
    assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref))
    # the f32 ascending-K accumulation itself, restated in numpy
    acc = np.zeros((m, n), dtype=np.float32)
    deq32 = deq.astype(np.float32)
    for kk in range(k):
        acc = (acc + (x[:, kk:kk + 1] * deq32[None, :, kk])).astype(np.float32)
    assert np.array_equal(acc, y)


def test_matmul_batch_invariance_and_bf16_out():
    n, k = 16, 512
    w = synth.quant_weights(O.Q4_K, 31, n, k)
    x = synth.normal_bf16(32, (5, k))
    y = O.matmul(O.Q4_K, w, n, k, x, O.BF16)
    for r in range(5):
        yr = O.matmul(O.Q4_K, w, n, k, x[r:r + 1], O.BF16)
        assert np.array_equal(yr[0], y[r])
    yb = O.matmul(O.Q4_K, w, n, k, x, O.BF16, y_dtype=O.BF16)
    assert np.array_equal(yb, synth.to_bf16_bits(y))
    ymt = O.matmul(O.Q4_K, w, n, k, x, O.BF16, threads=4)
    assert np.array_equal(ymt, y)


def test_matmul_epilogues():
    n, k = 8, 256
    w = synth.quant_weights(O.IQ4_XS, 41, n, k)
    x = synth.normal_f32(42, (2, k))
    bias = synth.normal_f32(43, (n,))
    res = synth.normal_f32(44, (2, n))
    y = O.matmul(O.IQ4_XS, w, n, k, x, O.F32)
    assert np.array_equal(O.matmul(O.IQ4_XS, w, n, k, x, O.F32, bias=bias), (y + bias).astype(np.float32))
    assert np.array_equal(O.matmul(O.IQ4_XS, w, n, k, x, O.F32, residual=res), (y + res).astype(np.float32))


# ---------------------------------------------------------------- moe_route

def test_route_equal_logits_select_lowest_ids():
    """crates/r9v-t0/tests/moe_route_tests.rs:107-126."""
    logits = np.ones((2, 6), dtype=np.float32)
    for scoring in (0, 1):
        ids, _ = O.moe_route(logits, 3, scoring=scoring)
        assert ids.reshape(-1).tolist() == [0, 1, 2, 0, 1, 2]


def test_route_matches_f64_softmax_and_invariants():
    t, e, k = 64, 512, 10
    logits = synth.normal_f32(51, (t, e))
    ids, w = O.moe_route(logits, k)
    l64 = logits.astype(np.float64)
    p = np.exp(l64 - l64.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    for r in range(t):
        want = np.lexsort((np.arange(e), -p[r]))[:k]
        assert ids[r].tolist() == want.tolist()
        assert len(set(ids[r].tolist())) == k
        sel = p[r, want] / p[r, want].sum()
        assert np.allclose(w[r], sel, rtol=1e-5, atol=0)
        assert abs(float(w[r].astype(np.float64).sum()) - 1.0) < k * 2 ** -23


def test_route_scale_bias_and_no_renorm():
    t, e, k = 4, 32, 4
    logits = synth.normal_f32(52, (t, e))
    bias = synth.normal_f32(53, (e,))
    ids_b, _ = O.moe_route(logits, k, bias=bias)
    ids_s, _ = O.moe_route((logits + bias).astype(np.float32), k)
    assert np.array_equal(ids_b, ids_s)
    ids, w = O.moe_route(logits, k, scale=2.5, renormalize=False)
    l64 = logits.astype(np.float64)
    p = np.exp(l64 - l64.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    assert np.allclose(w, 2.5 * np.take_along_axis(p, ids.astype(np.int64), 1), rtol=1e-5)


def test_route_refuses_nonfinite():
    logits = np.zeros((2, 8), dtype=np.float32)
    logits[1, 3] = np.inf
    with pytest.raises(O.OracleError):
        O.moe_route(logits, 2)


# ---------------------------------------------------------------- permute

def test_sort_matches_stable_argsort_and_invariants():
    t, e, k = 300, 64, 6
    logits = synth.zipf_logits(61, t, e)
    ids, _ = O.moe_route(logits, k)
    counts, offsets, order = O.moe_sort(ids, e)
    flat = ids.reshape(-1)
    want = np.argsort(flat, kind="stable")
    assert np.array_equal(order, want.astype(np.uint32))
    assert np.array_equal(counts, np.bincount(flat, minlength=e).astype(np.uint32))
    assert offsets[0] == 0 and offsets[-1] == t * k
    assert np.array_equal(np.diff(offsets.astype(np.int64)), counts.astype(np.int64))
    inv = np.empty_like(order)
    inv[order] = np.arange(t * k, dtype=np.uint32)
    assert np.array_equal(order[inv], np.arange(t * k, dtype=np.uint32))


def test_sort_refuses_out_of_range_id():
    ids = np.array([[0, 5]], dtype=np.uint32)
    with pytest.raises(O.OracleError):
        O.moe_sort(ids, 4)


# ---------------------------------------------------------------- moe_ffn

def _tiny_moe(seed, t=5, e=4, k=2, dm=256, dff=256, shared=0, schemes=(O.IQ4_XS, O.Q4_K)):
    gu = synth.quant_weights(schemes[0], seed, (e + shared) * 2 * dff, dm)
    dn = synth.quant_weights(schemes[1], seed + 1, (e + shared) * dm, dff)
    x = synth.normal_bf16(seed + 2, (t, dm))
    logits = synth.normal_f32(seed + 3, (t, e))
    ids, w = O.moe_route(logits, k)
    return x, ids, w, gu, dn


def test_moe_ffn_sliced_equals_full_t0_form():
    """moe_ffn.rs:41-46 claims the per-expert slice is bit-identical to the
    full-matrix GEMM; the oracle's sliced form must agree bit for bit."""
    x, ids, w, gu, dn = _tiny_moe(71)
    y = O.moe_ffn(x, O.BF16, ids, w, 4, 256, gu, dn)
    yf = O.moe_ffn_full(x, O.BF16, ids, w, 4, 256, gu, dn)
    assert np.array_equal(y, yf)


def test_dot_rows_four_at_once_equals_one_at_a_time():
    """The oracle's dots run four rows per pass over k by default and one row
    at a time (T0's loop, the CPU baseline's form) when asked: same bits,
    including the rows left over past a multiple of four."""
    n, k = 24, 768
    w = synth.quant_weights(O.Q4_K, 33, n, k)
    x = synth.normal_bf16(34, (7, k))
    x_, ids, wt, gu, dn = _tiny_moe(97, t=11, e=3, k=2, shared=1)
    y4 = O.matmul(O.Q4_K, w, n, k, x, O.BF16)
    f4 = O.moe_ffn(x_, O.BF16, ids, wt, 3, 256, gu, dn, shared=1)
    O.set_rows_at_once(1)
    try:
        y1 = O.matmul(O.Q4_K, w, n, k, x, O.BF16)
        f1 = O.moe_ffn(x_, O.BF16, ids, wt, 3, 256, gu, dn, shared=1)
    finally:
        O.set_rows_at_once(4)
    assert np.array_equal(y1, y4)
    assert np.array_equal(f1, f4)


def test_moe_ffn_threaded_equals_serial():
    """The OpenMP form (each expert's rows split into 64-row chunks over the
    threads, which the full-output GPU parity tests use) is the serial
    oracle bit for bit: ~100 rows per expert, so every expert spans chunks,
    plus a shared expert over all 200 tokens."""
    x, ids, w, gu, dn = _tiny_moe(95, t=200, e=4, k=2, shared=1)
    y = O.moe_ffn(x, O.BF16, ids, w, 4, 256, gu, dn, shared=1)
    ymt = O.moe_ffn(x, O.BF16, ids, w, 4, 256, gu, dn, shared=1, threads=4)
    assert np.array_equal(ymt, y)


@pytest.mark.parametrize("schemes", [(O.IQ4_XS, O.Q4_K), (O.Q8_0, O.Q8_0), (O.Q6_K, O.Q6_K), (O.IQ3_S, O.IQ3_S),
                                     (O.Q4_K, O.IQ4_XS)])
def test_moe_ffn_vs_f64_bruteforce_and_shared(schemes):
    """moe_ffn over every expert weight type against f64 arithmetic on the
    pinned decodes (the dequantize goldens): gather, SwiGLU, down, the
    weighted sum and a shared expert."""
    t, e, k, dm, dff = 4, 3, 2, 256, 256
    x, ids, w, gu, dn = _tiny_moe(81, t=t, e=e, k=k, shared=1, schemes=schemes)
    y = O.moe_ffn(x, O.BF16, ids, w, e, dff, gu, dn, scheme_gu=schemes[0], scheme_dn=schemes[1], shared=1)
    xf = synth.bf16_bits_to_f32(x).astype(np.float64)
    G = O.dequantize(schemes[0], gu, (e + 1) * 2 * dff, dm).astype(np.float64).reshape(e + 1, 2 * dff, dm)
    D = O.dequantize(schemes[1], dn, (e + 1) * dm, dff).astype(np.float64).reshape(e + 1, dm, dff)

    def ffn(ex, xr):
        g = xr @ G[ex, :dff].T
        u = xr @ G[ex, dff:].T
        h = g / (1 + np.exp(-g)) * u
        return h @ D[ex].T

    ref = np.zeros((t, dm))
    for tok in range(t):
        for s in range(k):
            ref[tok] += w[tok, s] * ffn(int(ids[tok, s]), xf[tok:tok + 1])[0]
        ref[tok] += ffn(e, xf[tok:tok + 1])[0]
    assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref))


def test_moe_ffn_token_permutation_and_duplicates():
    x, ids, w, gu, dn = _tiny_moe(91, t=6)
    y = O.moe_ffn(x, O.BF16, ids, w, 4, 256, gu, dn)
    perm = np.array([3, 0, 5, 1, 4, 2])
    yp = O.moe_ffn(x[perm], O.BF16, ids[perm], w[perm], 4, 256, gu, dn)
    assert np.array_equal(yp, y[perm])  # moe_ffn_tests.rs:278
    # duplicate slots: (e, e) with weights (a, b) == one slot with a then b added
    ids2 = ids.copy()
    ids2[:, 1] = ids2[:, 0]
    y2 = O.moe_ffn(x, O.BF16, ids2, w, 4, 256, gu, dn)
    single = O.moe_ffn(x, O.BF16, ids2[:, :1], np.ones_like(w[:, :1]), 4, 256, gu, dn)
    want = ((w[:, :1] * single).astype(np.float32) + (w[:, 1:2] * single).astype(np.float32))
    assert np.array_equal(y2, want.astype(np.float32))


def test_act_mul_silu_against_f64():
    """silu(g) * u in f32 (act_mul.rs:86-99): within 2 ulp-ish of the f64 value
    over a wide range; exact special points."""
    rng = np.random.default_rng(9)
    g = np.concatenate([rng.normal(0, 4, 5000), [0.0, -0.0, 20.0, -20.0, 88.0, -88.0, 1e-30]]).astype(np.float32)
    u = rng.normal(0, 2, g.size).astype(np.float32)
    got = O.act_mul_silu(g, u)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    want = g64 / (1.0 + np.exp(-g64)) * u64
    assert np.all(np.abs(got - want) <= 4 * np.finfo(np.float32).eps * np.abs(want) + 1e-37)
    assert got[g.size - 7] == 0.0 and got[g.size - 6] == 0.0


def test_router_logits_sequential_order():
    """The router-logit oracle is T0's loop: a numpy restatement that walks k
    in ascending order with f32 mul-then-add agrees bit for bit, and an f64
    dot agrees to rounding."""
    t, e, dm = 3, 70, 256
    x = synth.normal_bf16(11, (t, dm))
    w = synth.normal_f32(12, (e, dm), 0.05)
    got = O.router_logits(x, w)
    xf = synth.bf16_bits_to_f32(x)
    acc = np.zeros((t, e), dtype=np.float32)
    for k in range(dm):
        acc = (acc + (xf[:, k:k + 1] * w[None, :, k]).astype(np.float32)).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), acc.view(np.uint32))
    ref = xf.astype(np.float64) @ w.astype(np.float64).T
    assert np.max(np.abs(got - ref)) <= 1e-4 * np.max(np.abs(ref))
