"""Batch-invariance and determinism gates of matmul and moe_ffn, in the form
of the reference's gate engine (crates/r9v-t0/src/harness.rs:791-948, gates 2
and 3 of specs/spec-04-kernel-generator.md:213-223; the contract is
specs/spec-01-op-ir.md:299): one logical row is launched alone, in a padded
batch and embedded among random rows, at other row indices and batch sizes of
the same variant, and its output bytes must be bit-equal every time; a second
run of the same launch must be bit-equal too.  Every case also checks the
pinned row against the oracle (gate 1).

Across buckets the path has two arithmetics, and the gates check each across
its own buckets: matmul m_bucket 1..8 (the GEMV) and m_bucket >= 16 (the MFMA
GEMM); moe_ffn t_bucket 1..8 (the decode GEMVs, f32 h) and t_bucket >= 16 (the
grouped MFMA GEMMs, fp16 h).  The two forms of one op differ from each other
within the north-star tolerance, not bit for bit."""
from __future__ import annotations

import numpy as np
import pytest

import gpu_synth
import oracle_ffi as O
from r9v_amd import ffi, synth
from tol import check_close

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.cpu().numpy()


def bits(t):
    """The bytes of a device tensor as a host integer array."""
    t = t.contiguous()
    if t.dtype in (torch.float32, torch.int32):
        return host(t.view(torch.int32))
    return host(t.view(torch.int16))


def _batch(row, m, at, seed, pad, dtype):
    """[m, k] activations with `row` at index `at`; the other rows random
    (embedded) or zero (padded)."""
    k = row.shape[-1]
    if pad:
        x = torch.zeros((m, k), dtype=dtype, device="cuda")
    else:
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        x = torch.randn((m, k), generator=g, device="cuda").to(dtype)
    x[at] = row
    return x


# ---------------------------------------------------------------- matmul, decode buckets (GEMV)

@pytest.mark.parametrize("scheme", [O.Q4_K, O.IQ4_XS])
@pytest.mark.parametrize("k", [2048, 4096, 14336])
@pytest.mark.parametrize("x_f32", [False, True])
def test_matmul_decode_buckets(scheme, k, x_f32):
    """m_bucket 1 and 8: the row alone, padded to 8, and embedded at every
    batch size 2..8 (at the last index) gives the same bytes."""
    n = 320
    dtype = torch.float32 if x_f32 else torch.bfloat16
    w_h = synth.quant_weights(scheme, 8100 + k, n, k)
    w = dev(w_h)
    row = torch.randn((k,), generator=torch.Generator(device="cuda").manual_seed(8101 + k), device="cuda").to(dtype)
    want = bits(ffi.matmul(w, scheme, n, k, row[None], m_bucket=1))[0]
    runs = [(1, 0, False, 8), (8, 3, True, 8)] + [(m, m - 1, False, 8) for m in range(2, 9)]
    for m, at, pad, mb in runs:
        x = _batch(row, m, at, 8200 + m, pad, dtype)
        got = bits(ffi.matmul(w, scheme, n, k, x, m_bucket=mb))
        assert np.array_equal(got[at], want), f"m={m} at={at} pad={pad} m_bucket={mb}"
    x = _batch(row, 8, 5, 8300, False, dtype)
    assert np.array_equal(bits(ffi.matmul(w, scheme, n, k, x, m_bucket=8)),
                          bits(ffi.matmul(w, scheme, n, k, x, m_bucket=8)))  # run twice
    xr = host(row.float()) if x_f32 else synth.to_bf16_bits(host(row.float()))
    ref = O.matmul(scheme, w_h, n, k, xr[None], O.F32 if x_f32 else O.BF16)
    check_close(want.view(np.float32)[None], ref, "pinned row vs oracle")


# ---------------------------------------------------------------- matmul, prefill buckets (MFMA)

def _mfma_gate(scheme, n, k, w, runs, cross, out_dtype=O.F32, w_scales=None, seed=0):
    """`runs`: (m, at, pad) launches of one m_bucket = max m; `cross`: other
    buckets (m_bucket, m, at) the row must match too."""
    row = torch.randn((k,), generator=torch.Generator(device="cuda").manual_seed(seed), device="cuda").to(
        torch.bfloat16)
    mb = max(m for m, _, _ in runs)
    want = None
    for m, at, pad in runs:
        x = _batch(row, m, at, seed + m, pad, torch.bfloat16)
        y = ffi.matmul(w, scheme, n, k, x, out_dtype=out_dtype, m_bucket=mb, w_scales=w_scales)
        got = bits(y)[at]
        if want is None:
            want = got
        assert np.array_equal(got, want), f"m={m} at={at} pad={pad} m_bucket={mb}"
    for mbk, m, at in cross:
        x = _batch(row, m, at, seed + 7 * m, False, torch.bfloat16)
        got = bits(ffi.matmul(w, scheme, n, k, x, out_dtype=out_dtype, m_bucket=mbk, w_scales=w_scales))[at]
        assert np.array_equal(got, want), f"m_bucket={mbk} m={m} at={at}"
    m, at = runs[-1][0], runs[-1][1]
    x = _batch(row, m, at, seed + 99, False, torch.bfloat16)
    y1 = bits(ffi.matmul(w, scheme, n, k, x, out_dtype=out_dtype, m_bucket=mb, w_scales=w_scales))
    y2 = bits(ffi.matmul(w, scheme, n, k, x, out_dtype=out_dtype, m_bucket=mb, w_scales=w_scales))
    assert np.array_equal(y1, y2)  # run twice
    return row, want


@pytest.mark.parametrize("scheme", [O.Q4_K, O.IQ4_XS])
def test_matmul_prefill_bucket_2048_configs2_shape(scheme):
    """configs[2]'s weight (14336 x 4096) at m_bucket 2048: m = 1, 9, 1024,
    1025, 2048 embedded, 2048 padded, and the buckets 16 and 1024 beside it
    (bf16 and f32 outputs)."""
    n, k = 14336, 4096
    w = gpu_synth.quant_weights_gpu(torch, scheme, 8400 + scheme, n, k)
    runs = [(1, 0, False), (9, 8, False), (1024, 700, False), (1025, 1024, False), (2048, 1500, True),
            (2048, 2047, False)]
    cross = [(16, 1, 0), (16, 9, 4), (1024, 1024, 513)]
    row, want = _mfma_gate(scheme, n, k, w, runs, cross, seed=8410 + scheme)
    _mfma_gate(scheme, n, k, w, runs[:3] + runs[-1:], cross[:1], out_dtype=O.BF16, seed=8420 + scheme)
    cols = np.arange(0, n, 7)
    w_h = host(w)[cols]
    ref = O.matmul(scheme, w_h, len(cols), k, synth.to_bf16_bits(host(row.float()))[None], O.BF16, threads=8)
    check_close(want.view(np.float32)[cols][None], ref, "pinned row vs oracle")


@pytest.mark.parametrize("scheme", [O.Q4_K, O.IQ4_XS])
def test_matmul_prefill_ragged_n(scheme):
    """N % 256 != 0 (the register-decoded 256 x 256 tile) at m_bucket 512."""
    n, k = 5000, 2048
    w_h = synth.quant_weights(scheme, 8500, n, k)
    runs = [(1, 0, False), (9, 3, False), (300, 299, False), (512, 200, True), (512, 511, False)]
    row, want = _mfma_gate(scheme, n, k, dev(w_h), runs, [(16, 5, 2)], seed=8510 + scheme)
    ref = O.matmul(scheme, w_h, n, k, synth.to_bf16_bits(host(row.float()))[None], O.BF16, threads=8)
    check_close(want.view(np.float32)[None], ref, "pinned row vs oracle")


@pytest.mark.parametrize("scheme,n", [(O.Q8_0, 300), (O.Q8_0, 512), (O.Q6_K, 300), (O.Q6_K, 512), (O.IQ3_S, 300),
                                      (O.IQ3_S, 512)])
def test_matmul_prefill_repacked_schemes(scheme, n):
    """Q8_0 / Q6_K / IQ3_S at m_bucket 64 on the 256 x 256 loop, with a
    ragged last weight block (n = 300) and whole blocks (n = 512)."""
    k = 1024
    wire = synth.quant_weights(scheme, 8600 + scheme + n, n, k)
    w, sc = ffi.repack(dev(wire), scheme, n, k)
    runs = [(1, 0, False), (9, 8, False), (64, 20, True), (64, 63, False)]
    row, want = _mfma_gate(scheme, n, k, w, runs, [(16, 3, 1), (256, 200, 150)], w_scales=sc,
                           seed=8610 + scheme)
    ref = O.matmul(scheme, wire, n, k, synth.to_bf16_bits(host(row.float()))[None], O.BF16)
    check_close(want.view(np.float32)[None], ref, "pinned row vs oracle")


# ---------------------------------------------------------------- moe_ffn

def _moe_inputs(t, at, e, k, dm, pin, seed, pad, zipf):
    """(x, ids, weights) device tensors of t tokens with the pinned token
    (x row, ids, weights) at index `at`; the others routed from random
    (Zipf) logits, or padding tokens (zero x, ids 0..K-1, weight 0)."""
    x_row, ids_row, w_row = pin
    if pad:
        x = torch.zeros((t, dm), dtype=torch.bfloat16, device="cuda")
        ids = torch.arange(k, dtype=torch.int32, device="cuda").repeat(t, 1)
        w = torch.zeros((t, k), dtype=torch.float32, device="cuda")
    else:
        g = torch.Generator(device="cuda").manual_seed(seed)
        x = torch.randn((t, dm), generator=g, device="cuda").to(torch.bfloat16)
        logits = synth.zipf_logits(seed, t, e) if zipf else synth.normal_f32(seed, (t, e))
        ids, w = ffi.moe_route(dev(logits), k)
    x[at], ids[at], w[at] = x_row, ids_row, w_row
    return x, ids, w


def _moe_gate(e, k, dm, dff, shared, gu, dn, gu_s, dn_s, t_bucket, runs, cross, seed, gsc=None, dsc=None):
    """`runs`: (t, at, pad, zipf) launches at `t_bucket`; `cross`: (bucket, t,
    at) launches at other buckets of the same form."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    x_row = torch.randn((dm,), generator=g, device="cuda").to(torch.bfloat16)
    ids_row = torch.randperm(e, generator=g, device="cuda")[:k].to(torch.int32)
    w_row = torch.rand((k,), generator=g, device="cuda") + 0.05
    w_row = w_row / w_row.sum()
    pin = (x_row, ids_row, w_row)
    kw = dict(shared=shared, gate_up_scheme=gu_s, down_scheme=dn_s, w_gate_up_scales=gsc, w_down_scales=dsc)
    want = None
    for t, at, pad, zipf in runs:
        x, ids, w = _moe_inputs(t, at, e, k, dm, pin, seed + t, pad, zipf)
        y, ws, st = ffi.moe_ffn(x, ids, w, gu, dn, e, dff, t_bucket=t_bucket, **kw)
        assert ffi.moe_ffn_status(st, ws) == 0
        got = bits(y)[at]
        if want is None:
            want = got
        assert np.array_equal(got, want), f"t={t} at={at} pad={pad} t_bucket={t_bucket}"
    for tb, t, at in cross:
        x, ids, w = _moe_inputs(t, at, e, k, dm, pin, seed + 3 * t, False, False)
        y, _, _ = ffi.moe_ffn(x, ids, w, gu, dn, e, dff, t_bucket=tb, **kw)
        assert np.array_equal(bits(y)[at], want), f"t_bucket={tb} t={t} at={at}"
    t, at = runs[-1][0], runs[-1][1]
    x, ids, w = _moe_inputs(t, at, e, k, dm, pin, seed + 77, False, True)
    y1, ws, _ = ffi.moe_ffn(x, ids, w, gu, dn, e, dff, t_bucket=t_bucket, **kw)
    b1 = bits(y1)
    y2, _, _ = ffi.moe_ffn(x, ids, w, gu, dn, e, dff, t_bucket=t_bucket, workspace=ws, **kw)
    assert np.array_equal(b1, bits(y2))  # run twice
    return pin, want


def _moe_pinned_oracle(pin, gu, dn, gu_s, dn_s, e, dm, dff, shared):
    """The oracle's output for the pinned token alone, on host copies of its
    experts (re-numbered 0..K-1) and the shared ones."""
    x_row, ids_row, w_row = pin
    experts = [int(v) for v in host(ids_row)]
    uniq = sorted(set(experts))
    remap = {ex: i for i, ex in enumerate(uniq)}
    local = np.array([[remap[ex] for ex in experts]], dtype=np.uint32)
    sel = uniq + list(range(e, e + shared))
    gu_r, dn_r = gu.view(e + shared, 2 * dff, -1), dn.view(e + shared, dm, -1)
    idx = torch.tensor(sel, dtype=torch.long, device="cuda")
    gu_h = host(gu_r.index_select(0, idx).reshape(len(sel) * 2 * dff, -1))
    dn_h = host(dn_r.index_select(0, idx).reshape(len(sel) * dm, -1))
    x = synth.to_bf16_bits(host(x_row.float()))[None]
    return O.moe_ffn(x, O.BF16, local, host(w_row)[None], len(uniq), dff, gu_h, dn_h, scheme_gu=gu_s,
                     scheme_dn=dn_s, shared=shared)


def _experts_gpu(e, shared, dm, dff, gu_s, dn_s, seed):
    gu = gpu_synth.quant_weights_gpu(torch, gu_s, seed, (e + shared) * 2 * dff, dm)
    dn = gpu_synth.quant_weights_gpu(torch, dn_s, seed + 1, (e + shared) * dm, dff)
    return gu, dn


def test_moe_ffn_decode_buckets_configs3_shape():
    """configs[3]'s experts (E = 512 + 1 shared, top-10, Dm 2048, Dff 512) at
    t_bucket 8: t = 1 alone, 5 embedded, 8 padded and embedded; t_bucket 1
    beside it."""
    e, k, dm, dff, s = 512, 10, 2048, 512, 1
    gu, dn = _experts_gpu(e, s, dm, dff, O.IQ4_XS, O.Q4_K, 8700)
    runs = [(1, 0, False, False), (5, 3, False, False), (8, 6, True, False), (8, 7, False, False)]
    pin, want = _moe_gate(e, k, dm, dff, s, gu, dn, O.IQ4_XS, O.Q4_K, 8, runs, [(1, 1, 0), (4, 4, 2)], 8710)
    ref = _moe_pinned_oracle(pin, gu, dn, O.IQ4_XS, O.Q4_K, e, dm, dff, s)
    check_close(want.view(np.float32)[None], ref, "pinned token vs oracle")


def test_moe_ffn_prefill_buckets_configs4_shape():
    """configs[4]'s experts (E = 512, top-10, Dm 2048, Dff 512) at t_bucket
    8192: t = 1, 5, 9, 300 embedded, 8192 padded and embedded among
    Zipf-routed tokens; t_bucket 16 and 512 beside it."""
    e, k, dm, dff, s = 512, 10, 2048, 512, 0
    gu, dn = _experts_gpu(e, s, dm, dff, O.IQ4_XS, O.Q4_K, 8800)
    runs = [(1, 0, False, False), (5, 4, False, True), (9, 2, False, True), (300, 150, False, True),
            (8192, 4000, True, False), (8192, 8191, False, True)]
    cross = [(16, 1, 0), (16, 9, 8), (512, 512, 100)]
    pin, want = _moe_gate(e, k, dm, dff, s, gu, dn, O.IQ4_XS, O.Q4_K, 8192, runs, cross, 8810)
    ref = _moe_pinned_oracle(pin, gu, dn, O.IQ4_XS, O.Q4_K, e, dm, dff, s)
    check_close(want.view(np.float32)[None], ref, "pinned token vs oracle")


def test_moe_ffn_prefill_buckets_shared_and_q4k_gate_up():
    """Q4_K gate/up, IQ4_XS down, one shared expert, t_bucket 1024."""
    e, k, dm, dff, s = 64, 6, 1024, 512, 1
    gu, dn = _experts_gpu(e, s, dm, dff, O.Q4_K, O.IQ4_XS, 8900)
    runs = [(1, 0, False, False), (33, 32, False, True), (1024, 600, True, False), (1024, 1023, False, True)]
    pin, want = _moe_gate(e, k, dm, dff, s, gu, dn, O.Q4_K, O.IQ4_XS, 1024, runs, [(16, 7, 3)], 8910)
    ref = _moe_pinned_oracle(pin, gu, dn, O.Q4_K, O.IQ4_XS, e, dm, dff, s)
    check_close(want.view(np.float32)[None], ref, "pinned token vs oracle")


@pytest.mark.parametrize("gu_s,dn_s", [(O.Q6_K, O.Q8_0), (O.IQ3_S, O.Q4_K), (O.Q8_0, O.Q8_0), (O.Q8_0, O.Q6_K)])
@pytest.mark.parametrize("t_bucket", [8, 64])
def test_moe_ffn_buckets_repacked_schemes(gu_s, dn_s, t_bucket):
    """Experts in the split and IQ3_S layouts, decode (t_bucket 8) and grouped
    (t_bucket 64: the 256-row loop)."""
    e, k, dm, dff, s = 16, 4, 512, 256, 1
    gu_w = synth.quant_weights(gu_s, 9000 + gu_s, (e + s) * 2 * dff, dm)
    dn_w = synth.quant_weights(dn_s, 9001 + dn_s, (e + s) * dm, dff)

    def place(wire, scheme, rows, kk):
        if scheme in (O.Q8_0, O.Q6_K, O.IQ3_S):
            return ffi.repack(dev(wire), scheme, rows, kk)
        return dev(wire), None

    gu, gsc = place(gu_w, gu_s, (e + s) * 2 * dff, dm)
    dn, dsc = place(dn_w, dn_s, (e + s) * dm, dff)
    if t_bucket == 8:
        runs = [(1, 0, False, False), (5, 2, False, False), (8, 4, True, False), (8, 7, False, False)]
        cross = [(2, 2, 1)]
    else:
        runs = [(1, 0, False, False), (9, 8, False, True), (64, 30, True, False), (64, 63, False, True)]
        cross = [(16, 3, 1)]
    pin, want = _moe_gate(e, k, dm, dff, s, gu, dn, gu_s, dn_s, t_bucket, runs, cross, 9010 + t_bucket,
                          gsc=gsc, dsc=dsc)
    x_row, ids_row, w_row = pin
    ref = O.moe_ffn(synth.to_bf16_bits(host(x_row.float()))[None], O.BF16, host(ids_row).view(np.uint32)[None],
                    host(w_row)[None], e, dff, gu_w, dn_w, scheme_gu=gu_s, scheme_dn=dn_s, shared=s)
    check_close(want.view(np.float32)[None], ref, "pinned token vs oracle")
