"""moe_ffn with every expert weight type the GGUF path loads: IQ3_S (112-byte
device blocks) and Q8_0 / Q6_K (split layout: body plus f16 d array, passed
as w_gate_up_scales / w_down_scales) for the gate/up and the down experts,
beside Q4_K / IQ4_XS.  Decode (t <= 8: the dequant-fused GEMVs) and grouped
prefill (t = 300: the LDS-decoded MFMA kernels) against the oracle at the
north-star tolerance, through the C ABI."""
from __future__ import annotations

import numpy as np
import pytest

import oracle_ffi as O
from r9v_amd import ffi, synth
from tol import check_close

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

REPACKED = (ffi.Q8_0, ffi.Q6_K, ffi.IQ3_S)
PAIRS = [(ffi.Q8_0, ffi.Q8_0), (ffi.Q6_K, ffi.Q6_K), (ffi.IQ4_XS, ffi.IQ3_S), (ffi.IQ3_S, ffi.IQ3_S),
         (ffi.Q4_K, ffi.Q6_K), (ffi.Q8_0, ffi.IQ4_XS), (ffi.Q6_K, ffi.Q8_0)]
NAMES = {ffi.Q4_K: "q4k", ffi.IQ4_XS: "iq4xs", ffi.Q8_0: "q80", ffi.Q6_K: "q6k", ffi.IQ3_S: "iq3s"}


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def device_weights(wire, scheme, rows, k):
    """Wire blocks -> (device weights, split d array or None)."""
    w = dev(wire)
    if scheme in REPACKED:
        return ffi.repack(w, scheme, rows, k)
    return w, None


@pytest.mark.parametrize("t", [5, 300])
@pytest.mark.parametrize("gu_s,dn_s", PAIRS, ids=[f"{NAMES[g]}-{NAMES[d]}" for g, d in PAIRS])
def test_moe_ffn_expert_schemes(gu_s, dn_s, t):
    e, k, dm, dff = 16, 4, 512, 256
    shared = 1 if t <= 8 else 0
    seed = 3100 + 7 * gu_s + dn_s + t
    logits = synth.zipf_logits(seed, t, e)
    ids, w = O.moe_route(logits, k)
    gu = synth.quant_weights(gu_s, seed + 1, (e + shared) * 2 * dff, dm)
    dn = synth.quant_weights(dn_s, seed + 2, (e + shared) * dm, dff)
    x = synth.normal_bf16(seed + 3, (t, dm))
    ref = O.moe_ffn(x, O.BF16, ids, w, e, dff, gu, dn, scheme_gu=gu_s, scheme_dn=dn_s, shared=shared)
    gw, gsc = device_weights(gu, gu_s, (e + shared) * 2 * dff, dm)
    dw, dsc = device_weights(dn, dn_s, (e + shared) * dm, dff)
    y, ws, st = ffi.moe_ffn(dev(x.view(np.int16)).view(torch.bfloat16), dev(ids.view(np.int32)), dev(w), gw, dw, e,
                            dff, shared=shared, gate_up_scheme=gu_s, down_scheme=dn_s, w_gate_up_scales=gsc,
                            w_down_scales=dsc)
    torch.cuda.synchronize()
    assert ffi.moe_ffn_status(st, ws) == 0
    check_close(y.cpu().numpy(), ref, f"{NAMES[gu_s]}/{NAMES[dn_s]} t={t}")


BIG_PAIRS = [(ffi.IQ3_S, ffi.Q4_K), (ffi.IQ3_S, ffi.IQ4_XS), (ffi.Q6_K, ffi.Q8_0), (ffi.Q8_0, ffi.Q8_0),
             (ffi.Q8_0, ffi.Q6_K), (ffi.IQ3_S, ffi.Q6_K)]


@pytest.mark.parametrize("t", [4, 200])
@pytest.mark.parametrize("gu_s,dn_s", BIG_PAIRS, ids=[f"{NAMES[g]}-{NAMES[d]}" for g, d in BIG_PAIRS])
def test_moe_ffn_expert_schemes_model_shape(gu_s, dn_s, t):
    """A model-like shape: E = 64, Dm = 2048 (several K segments in the
    decode GEMVs), Dff = 768 (three 256-column blocks), top-8, expert tiles
    past 128 rows at t = 200; tokens are independent, so at t = 200 the
    oracle runs on 16 sampled tokens."""
    e, k, dm, dff = 64, 8, 2048, 768
    seed = 4100 + 7 * gu_s + dn_s + t
    logits = synth.zipf_logits(seed, t, e)
    ids, w = O.moe_route(logits, k)
    gu = synth.quant_weights(gu_s, seed + 1, e * 2 * dff, dm)
    dn = synth.quant_weights(dn_s, seed + 2, e * dm, dff)
    x = synth.normal_bf16(seed + 3, (t, dm))
    gw, gsc = device_weights(gu, gu_s, e * 2 * dff, dm)
    dw, dsc = device_weights(dn, dn_s, e * dm, dff)
    y, ws, st = ffi.moe_ffn(dev(x.view(np.int16)).view(torch.bfloat16), dev(ids.view(np.int32)), dev(w), gw, dw, e,
                            dff, gate_up_scheme=gu_s, down_scheme=dn_s, w_gate_up_scales=gsc, w_down_scales=dsc)
    torch.cuda.synchronize()
    assert ffi.moe_ffn_status(st, ws) == 0
    rows = np.arange(t) if t <= 8 else np.random.default_rng(seed).choice(t, 16, replace=False)
    ref = O.moe_ffn(np.ascontiguousarray(x[rows]), O.BF16, np.ascontiguousarray(ids[rows]),
                    np.ascontiguousarray(w[rows]), e, dff, gu, dn, scheme_gu=gu_s, scheme_dn=dn_s)
    check_close(y.cpu().numpy()[rows], ref, f"{NAMES[gu_s]}/{NAMES[dn_s]} t={t} E={e} Dm={dm} Dff={dff}")


def test_split_scales_are_required_and_inline_scales_refused():
    e, k, dm, dff, t = 4, 2, 256, 256, 3
    x = dev(synth.normal_bf16(1, (t, dm)).view(np.int16)).view(torch.bfloat16)
    ids = dev(np.array([[0, 1], [2, 3], [1, 2]], dtype=np.int32))
    w = dev(np.full((t, k), 0.5, dtype=np.float32))
    gu = synth.quant_weights(ffi.Q8_0, 2, e * 2 * dff, dm)
    dn = synth.quant_weights(ffi.Q4_K, 3, e * dm, dff)
    gw, gsc = device_weights(gu, ffi.Q8_0, e * 2 * dff, dm)
    with pytest.raises(ffi.R9vxError, match="w_gate_up_scales is required"):
        ffi.moe_ffn(x, ids, w, gw, dev(dn), e, dff, gate_up_scheme=ffi.Q8_0, down_scheme=ffi.Q4_K)
    with pytest.raises(ffi.R9vxError, match="w_down_scales must be NULL"):
        ffi.moe_ffn(x, ids, w, gw, dev(dn), e, dff, gate_up_scheme=ffi.Q8_0, down_scheme=ffi.Q4_K,
                    w_gate_up_scales=gsc, w_down_scales=gsc)


def test_gguf_loads_split_and_iq3s_experts():
    """Q8_0 gate and up expert tensors (stacked by r9vx_gguf_upload_gate_up_split),
    a Q6_K down tensor (r9vx_gguf_upload_split) and, in a second checkpoint, a
    fused Q6_K gate_up with IQ3_S down (host repack): the loaded arrays equal
    the device repack of the stacked wire blocks byte for byte, and moe_ffn on
    them meets the oracle."""
    from gguf_build import build
    from r9v_amd import gguf

    e, dm, dff, k, t = 4, 512, 256, 2, 6
    gate = synth.quant_weights(ffi.Q8_0, 81, e * dff, dm)
    up = synth.quant_weights(ffi.Q8_0, 82, e * dff, dm)
    down = synth.quant_weights(ffi.Q6_K, 83, e * dm, dff)
    fused = synth.quant_weights(ffi.Q6_K, 84, e * 2 * dff, dm)
    down3 = synth.quant_weights(ffi.IQ3_S, 85, e * dm, dff)
    b1 = build([("general.architecture", (8, "qwen3moe"))], [
        ("blk.0.ffn_gate_exps.weight", (dm, dff, e), 8, gate.tobytes()),
        ("blk.0.ffn_up_exps.weight", (dm, dff, e), 8, up.tobytes()),
        ("blk.0.ffn_down_exps.weight", (dff, dm, e), 14, down.tobytes())])
    b2 = build([("general.architecture", (8, "qwen3moe"))], [
        ("blk.0.ffn_gate_up_exps.weight", (dm, 2 * dff, e), 14, fused.tobytes()),
        ("blk.0.ffn_down_exps.weight", (dff, dm, e), 21, down3.tobytes())])
    logits = synth.normal_f32(86, (t, e))
    ids, w = O.moe_route(logits, k)
    x = synth.normal_bf16(87, (t, dm))
    xd = dev(x.view(np.int16)).view(torch.bfloat16)
    stacked = np.concatenate([gate.reshape(e, dff, -1), up.reshape(e, dff, -1)], axis=1).reshape(-1)
    cases = [(b1, "blk.0.ffn_gate_exps.weight", "blk.0.ffn_up_exps.weight", stacked, down, ffi.Q8_0, ffi.Q6_K),
             (b2, "blk.0.ffn_gate_up_exps.weight", None, fused, down3, ffi.Q6_K, ffi.IQ3_S)]
    for b, g, u, gu_wire, dn_wire, gu_s, dn_s in cases:
        f = gguf.GgufFile.parse(b)
        ex = gguf.load_moe_experts(f, b, g, u, "blk.0.ffn_down_exps.weight", t_bucket=8, k=k)
        st, w_gu, w_dn = ex
        assert (st.gate_up.scheme, st.down.scheme) == (gu_s, dn_s)
        assert st.gate_up.layout == ffi.weight_layout(gu_s) and st.down.layout == ffi.weight_layout(dn_s)
        rg, rgs = device_weights(gu_wire, gu_s, e * 2 * dff, dm)
        rd, rds = device_weights(dn_wire, dn_s, e * dm, dff)
        assert torch.equal(w_gu, rg) and torch.equal(w_dn, rd)
        for got, want in ((ex.w_gate_up_scales, rgs), (ex.w_down_scales, rds)):
            assert (got is None) == (want is None) and (got is None or torch.equal(got, want))
        y, ws, st2 = ffi.moe_ffn(xd, dev(ids.view(np.int32)), dev(w), w_gu, w_dn, e, dff, gate_up_scheme=gu_s,
                                 down_scheme=dn_s, w_gate_up_scales=ex.w_gate_up_scales,
                                 w_down_scales=ex.w_down_scales)
        ref = O.moe_ffn(x, O.BF16, ids, w, e, dff, gu_wire, dn_wire, scheme_gu=gu_s, scheme_dn=dn_s)
        check_close(y.cpu().numpy(), ref, f"gguf {NAMES[gu_s]}/{NAMES[dn_s]}")
