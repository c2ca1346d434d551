"""GPU parity of moe_route (bit-exact ids and weights), the permute
(bit-exact counts/offsets/order) and moe_ffn against
the CPU oracle, through the C ABI."""
from __future__ import annotations

import numpy as np
import pytest

import oracle_ffi as O
from r9v_amd import ffi, synth
from tol import check_close

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.cpu().numpy()


def bf16_dev(bits):
    return dev(bits.view(np.int16)).view(torch.bfloat16)


# ---------------------------------------------------------------- routing

def _route_both(logits, k, **kw):
    ids_o, w_o = O.moe_route(logits, k, **{kk: v for kk, v in kw.items()})
    bias = kw.get("bias")
    ids_g, w_g = ffi.moe_route(dev(logits), k, bias=None if bias is None else dev(bias),
                               scoring=kw.get("scoring", 0), renormalize=kw.get("renormalize", True),
                               scale=kw.get("scale", 1.0))
    torch.cuda.synchronize()
    return (ids_o, w_o), (host(ids_g).view(np.uint32), host(w_g))


def _assert_bit_exact(o, g):
    assert np.array_equal(o[0], g[0]), "expert ids differ"
    assert np.array_equal(o[1].view(np.uint32), g[1].view(np.uint32)), "weights differ"


def test_route_config3_bit_exact():
    """T=5, E=512, top-10 from N(0,1) logits, renormalised softmax."""
    logits = synth.normal_f32(synth.seed_for("c3", "logits"), (5, 512))
    _assert_bit_exact(*_route_both(logits, 10))


def test_route_config4_zipf_bit_exact():
    """T=8192, E=512, top-10, Zipf(1.1)-skewed logits."""
    logits = synth.zipf_logits(synth.seed_for("c4", "logits"), 8192, 512)
    _assert_bit_exact(*_route_both(logits, 10))


@pytest.mark.parametrize("t,e,k", [(1, 8, 1), (3, 64, 8), (65, 128, 4), (200, 1024, 32), (7, 100, 7)])
def test_route_shapes_bit_exact(t, e, k):
    logits = synth.normal_f32(700 + t + e + k, (t, e), sigma=3.0)
    _assert_bit_exact(*_route_both(logits, k))


def test_route_ties_bias_sigmoid_scale():
    logits = np.ones((2, 6), dtype=np.float32)
    for scoring in (0, 1):
        o, g = _route_both(logits, 3, scoring=scoring)
        assert g[0].reshape(-1).tolist() == [0, 1, 2, 0, 1, 2]
        _assert_bit_exact(o, g)
    logits = synth.normal_f32(801, (100, 256))
    bias = synth.normal_f32(802, (256,))
    _assert_bit_exact(*_route_both(logits, 6, bias=bias))
    _assert_bit_exact(*_route_both(logits, 6, scoring=1))
    _assert_bit_exact(*_route_both(logits, 6, scale=2.5, renormalize=False))
    _assert_bit_exact(*_route_both(logits, 6, scoring=1, renormalize=False, scale=0.75))
    # quantised logits produce many exact score ties: lowest id must win
    tied = (np.round(synth.normal_f32(803, (300, 512)) * 2) / 2).astype(np.float32)
    _assert_bit_exact(*_route_both(tied, 10))


def _quotient_tie_rows(n_rows, e):
    """Softmax rows where two experts' exp values differ by one ulp but their
    quotients by the ordered sum round to the same f32, with the larger value
    at the higher id (5) and the smaller at id 3; expert 0 holds the maximum
    logit 0 and every other expert -200 (exp = 0).  Found by search with the
    host libm expf (the function the oracle and the reference call)."""
    import ctypes

    libm = ctypes.CDLL("libm.so.6")
    libm.expf.restype, libm.expf.argtypes = ctypes.c_float, [ctypes.c_float]
    f32 = np.float32
    rng = np.random.default_rng(2026)
    rows = []
    while len(rows) < n_rows:
        l1 = f32(-0.105 + rng.uniform(-0.01, 0.01))
        v1 = f32(libm.expf(l1))
        l2, v2 = l1, v1
        for _ in range(64):
            l2 = np.nextafter(l2, f32(-1))
            v2 = f32(libm.expf(l2))
            if v2 < v1:
                break
        if v2 != np.nextafter(v1, f32(0)):
            continue
        s = f32(f32(f32(1.0) + v2) + v1)  # ascending id: 0, 3, 5
        if f32(v1 / s) != f32(v2 / s):
            continue
        row = np.full(e, -200.0, np.float32)
        row[0], row[3], row[5] = 0.0, l2, l1
        rows.append(row)
    return np.stack(rows)


@pytest.mark.parametrize("e", [64, 512])
def test_route_quotient_ties_bit_exact(e):
    """The reference ranks the divided scores, where id 3 beats id 5 on the
    tie; ranking the undivided exp values would put id 5 first.  Covers the
    router's tie test at the K-th/(K+1)-th boundary (K=2) and between two
    selected neighbours (K=3), and the exact path it falls back to."""
    logits = _quotient_tie_rows(6, e)
    for k in (2, 3):
        o, g = _route_both(logits, k)
        assert (o[0][:, 1] == 3).all(), "oracle must take id 3 on the quotient tie"
        _assert_bit_exact(o, g)


@pytest.mark.parametrize("t", [4, 300])
def test_route_refuses_nonfinite_before_writing(t):
    logits = synth.normal_f32(901, (t, 64))
    logits[t // 2, 5] = np.nan
    ids = torch.full((t, 4), 77, dtype=torch.int32, device="cuda")
    w = torch.full((t, 4), -1.0, dtype=torch.float32, device="cuda")
    ffi.moe_route(dev(logits), 4, ids=ids, weights=w)
    assert ffi.moe_route_status() & ffi.STATUS_NONFINITE
    assert (host(ids) == 77).all() and (host(w) == -1.0).all()
    # the next valid call clears the status and writes
    ffi.moe_route(dev(np.zeros((t, 64), np.float32)), 4, ids=ids, weights=w)
    assert ffi.moe_route_status() == 0
    assert (host(ids)[:, 0] == 0).all()


def test_route_host_refusals():
    with pytest.raises(ffi.R9vxError) as e:
        ffi.moe_route(dev(np.zeros((2, 4), np.float32)), 5)
    assert "top_k 5 cannot exceed" in str(e.value)
    with pytest.raises(ffi.R9vxError):
        ffi.moe_route(dev(np.zeros((2, 4), np.float32)), 2, scale=0.0)


# ---------------------------------------------------------------- permute

@pytest.mark.parametrize("t,e,k", [(5, 512, 10), (8192, 512, 10), (1, 4, 2), (103, 1024, 32), (3000, 7, 3),
                                   (2, 1024, 32), (7, 100, 9), (64, 3, 1), (13, 5, 5)])
def test_sort_bit_exact(t, e, k):
    if e >= 64:
        logits = synth.zipf_logits(1000 + t + e, t, e)
        ids, _ = O.moe_route(logits, k)
    else:
        ids = (synth.splitmix64(1001 + t, t * k) % np.uint64(e)).astype(np.uint32).reshape(t, k)
    c_o, off_o, srt_o = O.moe_sort(ids, e)
    c_g, off_g, srt_g = ffi.moe_sort(dev(ids.view(np.int32)), e)
    assert np.array_equal(host(c_g).view(np.uint32), c_o)
    assert np.array_equal(host(off_g).view(np.uint32), off_o)
    assert np.array_equal(host(srt_g).view(np.uint32), srt_o)


# ---------------------------------------------------------------- moe_ffn

def _experts(seed, e, s, dm, dff, active):
    """Stacked expert weights with the `active` experts (and the shared ones)
    filled from the seeded generator and the rest zero blocks."""
    bb_gu, bb_dn = synth.BLOCK_BYTES[synth.IQ4_XS], synth.BLOCK_BYTES[synth.Q4_K]
    gu = np.zeros(((e + s) * 2 * dff, dm // 256 * bb_gu), dtype=np.uint8)
    dn = np.zeros(((e + s) * dm, dff // 256 * bb_dn), dtype=np.uint8)
    for ex in sorted(set(int(v) for v in active)) + list(range(e, e + s)):
        gu[ex * 2 * dff:(ex + 1) * 2 * dff] = synth.quant_weights(synth.IQ4_XS, seed + 2 * ex, 2 * dff, dm)
        dn[ex * dm:(ex + 1) * dm] = synth.quant_weights(synth.Q4_K, seed + 2 * ex + 1, dm, dff)
    return gu, dn


def _moe_case(t, e, k, dm, dff, shared, seed, zipf=False):
    logits = synth.zipf_logits(seed, t, e) if zipf else synth.normal_f32(seed, (t, e))
    ids, w = O.moe_route(logits, k)
    gu, dn = _experts(seed + 10, e, shared, dm, dff, ids.reshape(-1))
    x = synth.normal_bf16(seed + 3, (t, dm))
    ref = O.moe_ffn(x, O.BF16, ids, w, e, dff, gu, dn, shared=shared)
    y, ws, st = ffi.moe_ffn(bf16_dev(x), dev(ids.view(np.int32)), dev(w), dev(gu), dev(dn), e, dff,
                            shared=shared)
    torch.cuda.synchronize()
    assert ffi.moe_ffn_status(st, ws) == 0
    return host(y), ref


def test_moe_ffn_config3_decode():
    """T=5 (MTP4 verify), hidden 2048, 512 experts, top-10, IQ4_XS
    gate/up [2048 -> 2x512] + Q4_K down [512 -> 2048], plus one shared expert."""
    got, ref = _moe_case(5, 512, 10, 2048, 512, 1, synth.seed_for("c3", "moe") % (1 << 32))
    check_close(got, ref, "config3")


@pytest.mark.parametrize("t,e,k,dm,dff,shared", [(1, 8, 2, 256, 256, 0), (3, 16, 4, 512, 256, 1),
                                                  (8, 32, 3, 256, 512, 2), (2, 4, 4, 768, 256, 0)])
def test_moe_ffn_decode_shapes(t, e, k, dm, dff, shared):
    got, ref = _moe_case(t, e, k, dm, dff, shared, 1100 + t + e)
    check_close(got, ref, f"t={t} e={e}")


def test_moe_ffn_decode_repeated_calls_one_workspace():
    """Back-to-back decode calls on one workspace, each with new routing and
    activations: every y matches the oracle (the down GEMV's last wave per
    row block sums rows the other waves of the same launch stored, counted
    per launch), and a refused call in between leaves its y untouched and the
    next call's status clean."""
    t, e, k, dm, dff, shared = 5, 32, 4, 512, 256, 1
    gu, dn = _experts(1401, e, shared, dm, dff, range(e))
    gu_d, dn_d = dev(gu), dev(dn)
    ws = st = None
    for i in range(24):
        logits = synth.normal_f32(1410 + i, (t, e))
        ids, w = O.moe_route(logits, k)
        x = synth.normal_bf16(1450 + i, (t, dm))
        if i == 12:  # a refused call: an id >= E
            bad = ids.copy()
            bad[3, 2] = e
            y2 = torch.full((t, dm), 7.0, dtype=torch.float32, device="cuda")
            ffi.moe_ffn(bf16_dev(x), dev(bad.view(np.int32)), dev(w), gu_d, dn_d, e, dff, shared=shared, y=y2,
                        workspace=ws)
            assert ffi.moe_ffn_status(st, ws) & ffi.STATUS_BAD_EXPERT
            assert (host(y2) == 7.0).all()
        ref = O.moe_ffn(x, O.BF16, ids, w, e, dff, gu, dn, shared=shared)
        y, ws, st = ffi.moe_ffn(bf16_dev(x), dev(ids.view(np.int32)), dev(w), gu_d, dn_d, e, dff, shared=shared,
                                workspace=ws)
        torch.cuda.synchronize()
        assert ffi.moe_ffn_status(st, ws) == 0
        check_close(host(y), ref, f"call {i}")


def test_moe_ffn_duplicate_slots_and_refusal():
    t, e, k, dm, dff = 4, 8, 3, 256, 256
    ids = np.array([[1, 1, 5], [0, 7, 7], [2, 3, 4], [6, 6, 6]], dtype=np.uint32)
    w = synth.normal_f32(1201, (t, k))
    gu, dn = _experts(1202, e, 0, dm, dff, range(e))
    x = synth.normal_bf16(1203, (t, dm))
    ref = O.moe_ffn(x, O.BF16, ids, w, e, dff, gu, dn)
    y, ws, st = ffi.moe_ffn(bf16_dev(x), dev(ids.view(np.int32)), dev(w), dev(gu), dev(dn), e, dff)
    check_close(host(y), ref, "duplicates")
    bad = ids.copy()
    bad[2, 1] = e  # out of range
    y2 = torch.full((t, dm), 3.0, dtype=torch.float32, device="cuda")
    ffi.moe_ffn(bf16_dev(x), dev(bad.view(np.int32)), dev(w), dev(gu), dev(dn), e, dff, y=y2, workspace=ws)
    assert ffi.moe_ffn_status(st, ws) & ffi.STATUS_BAD_EXPERT
    assert (host(y2) == 3.0).all()


def test_moe_ffn_token_permutation_invariance():
    """Permuting tokens permutes outputs bit for bit (moe_ffn_tests.rs:278)."""
    t, e, k, dm, dff = 6, 16, 4, 512, 256
    logits = synth.normal_f32(1301, (t, e))
    ids, w = O.moe_route(logits, k)
    gu, dn = _experts(1302, e, 0, dm, dff, range(e))
    x = synth.normal_bf16(1303, (t, dm))
    perm = np.array([4, 2, 0, 5, 1, 3])
    y, _, _ = ffi.moe_ffn(bf16_dev(x), dev(ids.view(np.int32)), dev(w), dev(gu), dev(dn), e, dff)
    yp, _, _ = ffi.moe_ffn(bf16_dev(x[perm]), dev(ids[perm].view(np.int32)), dev(w[perm]), dev(gu), dev(dn), e, dff)
    assert np.array_equal(host(yp), host(y)[perm])


# ---------------------------------------------------------------- prefill (grouped MFMA)

def test_moe_ffn_config4_prefill_full():
    """8192 tokens, hidden 2048, 512 experts, top-10 over
    Zipf(1.1) logits; full GPU run (route -> permute -> grouped GEMMs ->
    combine); every one of the 8192 x 2048 outputs against the oracle (its
    OpenMP form on all host threads, bit-identical to the serial one)."""
    import gpu_synth
    t, e, k, dm, dff = 8192, 512, 10, 2048, 512
    logits = synth.zipf_logits(synth.seed_for("c4", "logits"), t, e)
    ids_d, w_d = ffi.moe_route(dev(logits), k)
    ids, w = host(ids_d).view(np.uint32), host(w_d)
    gu = gpu_synth.quant_weights_gpu(torch, O.IQ4_XS, 41, e * 2 * dff, dm)
    dn = gpu_synth.quant_weights_gpu(torch, O.Q4_K, 42, e * dm, dff)
    x = synth.normal_bf16(synth.seed_for("c4", "x"), (t, dm))
    y, ws, st = ffi.moe_ffn(bf16_dev(x), ids_d, w_d, gu, dn, e, dff)
    torch.cuda.synchronize()
    assert ffi.moe_ffn_status(st, ws) == 0
    ref = O.moe_ffn(x, O.BF16, ids, w, e, dff, host(gu), host(dn), threads=O.host_threads())
    check_close(host(y), ref, "config4 full")


@pytest.mark.parametrize("t,e,k,dm,dff,shared,gu_s,dn_s", [
    (9, 8, 2, 256, 256, 0, O.IQ4_XS, O.Q4_K),
    (130, 16, 4, 512, 256, 1, O.IQ4_XS, O.Q4_K),
    (300, 64, 6, 256, 512, 2, O.Q4_K, O.IQ4_XS),
    (257, 4, 3, 768, 256, 0, O.Q4_K, O.Q4_K),
])
def test_moe_ffn_prefill_shapes(t, e, k, dm, dff, shared, gu_s, dn_s):
    logits = synth.zipf_logits(1400 + t, t, e)
    ids, w = O.moe_route(logits, k)
    gu = synth.quant_weights(gu_s, 1401 + t, (e + shared) * 2 * dff, dm)
    dn = synth.quant_weights(dn_s, 1402 + t, (e + shared) * dm, dff)
    x = synth.normal_bf16(1403 + t, (t, dm))
    ref = O.moe_ffn(x, O.BF16, ids, w, e, dff, gu, dn, scheme_gu=gu_s, scheme_dn=dn_s, shared=shared)
    y, ws, st = ffi.moe_ffn(bf16_dev(x), dev(ids.view(np.int32)), dev(w), dev(gu), dev(dn), e, dff,
                            shared=shared, gate_up_scheme=gu_s, down_scheme=dn_s)
    torch.cuda.synchronize()
    assert ffi.moe_ffn_status(st, ws) == 0
    check_close(host(y), ref, f"prefill t={t} e={e}")


@pytest.mark.parametrize("dn_s", [O.Q4_K, O.IQ4_XS])
def test_moe_ffn_prefill_h_blocks_at_different_scales(dn_s):
    """h rows whose 128-column blocks need different fp16 scales, some none:
    the gate/up d of h columns 128-511 is multiplied by 2^-8, so those
    blocks of h stay below 2^15 (scale 1) while block 0 passes it (checked on
    the shared expert's h).  The gate/up GEMM scales each block by its own
    power of two and the down GEMM undoes them block by block; y must match
    the oracle."""
    t, e, k, dm, dff, shared = 300, 16, 4, 512, 512, 1
    seed = 1700 + dn_s
    logits = synth.zipf_logits(seed, t, e)
    ids, w = O.moe_route(logits, k)
    gu = synth.quant_weights(O.IQ4_XS, seed + 1, (e + shared) * 2 * dff, dm)
    dn = synth.quant_weights(dn_s, seed + 2, (e + shared) * dm, dff)
    bb = synth.BLOCK_BYTES[synth.IQ4_XS]
    blocks = gu.reshape((e + shared) * 2 * dff, dm // 256, bb)
    for ex in range(e + shared):  # d (the first fp16 of an IQ4_XS block) of gate and up rows 128-511
        for base in (ex * 2 * dff + 128, ex * 2 * dff + dff + 128):
            d = blocks[base:base + dff - 128, :, 0:2].copy().view(np.float16)
            blocks[base:base + dff - 128, :, 0:2] = (d.astype(np.float32) / 256.0).astype(np.float16).view(np.uint8)
    x = synth.normal_bf16(seed + 3, (t, dm))
    h = O.matmul_swiglu(O.IQ4_XS, gu[e * 2 * dff:], dff, dm, x, O.BF16)  # the shared expert
    bmax = np.abs(h).reshape(t, dff // 128, 128).max(axis=2)
    assert ((bmax[:, 0] >= 32768) & (bmax[:, 1:].max(axis=1) < 32768)).sum() >= t // 4
    ref = O.moe_ffn(x, O.BF16, ids, w, e, dff, gu, dn, scheme_gu=O.IQ4_XS, scheme_dn=dn_s, shared=shared)
    y, ws, st = ffi.moe_ffn(bf16_dev(x), dev(ids.view(np.int32)), dev(w), dev(gu), dev(dn), e, dff,
                            shared=shared, gate_up_scheme=O.IQ4_XS, down_scheme=dn_s)
    torch.cuda.synchronize()
    assert ffi.moe_ffn_status(st, ws) == 0
    check_close(host(y), ref, f"h block scales down={dn_s}")


def test_moe_ffn_prefill_permutation_invariance_full_size():
    """Permuting the 8192 tokens of configs[4] permutes y bit for bit (rows
    keep their K order wherever they land in the expert tiles)."""
    import gpu_synth
    t, e, k, dm, dff = 8192, 512, 10, 2048, 512
    logits = synth.zipf_logits(1501, t, e)
    ids_d, w_d = ffi.moe_route(dev(logits), k)
    gu = gpu_synth.quant_weights_gpu(torch, O.IQ4_XS, 51, e * 2 * dff, dm)
    dn = gpu_synth.quant_weights_gpu(torch, O.Q4_K, 52, e * dm, dff)
    x = bf16_dev(synth.normal_bf16(1502, (t, dm)))
    y, ws, st = ffi.moe_ffn(x, ids_d, w_d, gu, dn, e, dff)
    perm = torch.from_numpy(np.random.default_rng(9).permutation(t)).cuda()
    yp, _, _ = ffi.moe_ffn(x[perm].contiguous(), ids_d[perm].contiguous(), w_d[perm].contiguous(), gu, dn, e,
                           dff, workspace=ws)
    assert torch.equal(yp, y[perm])


@pytest.mark.gpu
@pytest.mark.parametrize("t", [5, 300])
def test_route_status_words_are_per_launch(t):
    """Two routings on two streams, each with its own status word: the one
    with a NaN row reports NONFINITE and writes nothing, the other reports 0
    and writes its ids -- neither sees the other's status."""
    bad = synth.normal_f32(911, (t, 64))
    bad[t // 3, 7] = np.nan
    good = synth.normal_f32(912, (t, 64))
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    w1 = torch.full((1,), 0x55, dtype=torch.int32, device="cuda")
    w2 = torch.full((1,), 0x55, dtype=torch.int32, device="cuda")
    ids1 = torch.full((t, 4), 77, dtype=torch.int32, device="cuda")
    wt1 = torch.full((t, 4), -1.0, dtype=torch.float32, device="cuda")
    ids2 = torch.full((t, 4), 77, dtype=torch.int32, device="cuda")
    wt2 = torch.full((t, 4), -1.0, dtype=torch.float32, device="cuda")
    lb, lg = dev(bad), dev(good)
    torch.cuda.synchronize()
    for _ in range(3):  # interleaved launches on both streams
        ffi.moe_route(lb, 4, ids=ids1, weights=wt1, stream=s1, status=w1)
        ffi.moe_route(lg, 4, ids=ids2, weights=wt2, stream=s2, status=w2)
    torch.cuda.synchronize()
    assert ffi.status_read(w1) == ffi.STATUS_NONFINITE
    assert ffi.status_read(w2) == 0
    assert (host(ids1) == 77).all() and (host(wt1) == -1.0).all()
    rid, rw = O.moe_route(good, 4)
    assert np.array_equal(host(ids2).view(np.uint32), rid.astype(np.uint32))
    assert np.array_equal(host(wt2).view(np.uint32), rw.view(np.uint32))


@pytest.mark.parametrize("t", [5, 300])
def test_plain_route_status_words_are_per_stream(t):
    """The plain launch on two streams: each stream's word reports its own
    routing (NONFINITE where a row holds a NaN, 0 on the other), reading a
    word clears it, and a stream with no plain launch reads 0."""
    bad = synth.normal_f32(921, (t, 64))
    bad[t // 2, 3] = np.inf
    good = synth.normal_f32(922, (t, 64))
    s1, s2, s3 = torch.cuda.Stream(), torch.cuda.Stream(), torch.cuda.Stream()
    ids1 = torch.full((t, 4), 77, dtype=torch.int32, device="cuda")
    wt1 = torch.full((t, 4), -1.0, dtype=torch.float32, device="cuda")
    ids2 = torch.empty((t, 4), dtype=torch.int32, device="cuda")
    wt2 = torch.empty((t, 4), dtype=torch.float32, device="cuda")
    lb, lg = dev(bad), dev(good)
    torch.cuda.synchronize()
    for _ in range(3):
        ffi.moe_route(lb, 4, ids=ids1, weights=wt1, stream=s1)
        ffi.moe_route(lg, 4, ids=ids2, weights=wt2, stream=s2)
    assert ffi.moe_route_status(stream=s1) == ffi.STATUS_NONFINITE
    assert ffi.moe_route_status(stream=s2) == 0
    assert ffi.moe_route_status(stream=s1) == 0  # read and cleared
    assert ffi.moe_route_status(stream=s3) == 0  # never used
    assert (host(ids1) == 77).all() and (host(wt1) == -1.0).all()
    rid, rw = O.moe_route(good, 4)
    assert np.array_equal(host(ids2).view(np.uint32), rid.astype(np.uint32))
    assert np.array_equal(host(wt2).view(np.uint32), rw.view(np.uint32))
