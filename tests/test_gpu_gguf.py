"""GPU tests of the GGUF load step (include/r9vx_gguf.h): a checkpoint built
in memory by the gguf-py layout rules is parsed by libr9vx, its Q4_K / IQ4_XS
tensors are bound to matmul / moe_ffn variant keys and copied to the device,
and the kernels run on what was loaded.

Device bytes must equal the file's entry bytes (gate and up experts stacked
per expert, crates/r9v-t0/src/moe_ffn.rs:51-55), results on loaded weights
must equal results on the same blocks uploaded directly (bit for bit: same
kernels, same bytes), and both must meet the oracle at the north-star
tolerance."""
from __future__ import annotations

import numpy as np
import pytest

import oracle_ffi as O
from gguf_build import build
from r9v_amd import ffi, gguf, synth
from tol import check_close

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def bf16_dev(bits):
    return dev(bits.view(np.int16)).view(torch.bfloat16)


def host(t):
    return t.cpu().numpy()


E, DFF, DM = 6, 256, 512


def _experts(seed):
    gate = np.stack([synth.quant_weights(synth.IQ4_XS, seed + e, DFF, DM) for e in range(E)])
    up = np.stack([synth.quant_weights(synth.IQ4_XS, seed + 100 + e, DFF, DM) for e in range(E)])
    down = np.stack([synth.quant_weights(synth.Q4_K, seed + 200 + e, DM, DFF) for e in range(E)])
    return gate, up, down


def _split_keys(no, count, total):
    return [("split.no", (2, no)), ("split.count", (2, count)), ("split.tensors.count", (5, total))]


@pytest.fixture(scope="module")
def checkpoint():
    wq = synth.quant_weights(synth.Q4_K, 901, 320, 2048)
    wk = synth.quant_weights(synth.IQ4_XS, 902, 192, 1024)
    gate, up, down = _experts(950)
    shard0 = build([("general.architecture", (8, "qwen3moe")), ("general.alignment", (4, 64))]
                   + _split_keys(0, 2, 5), [
        ("blk.0.attn_q.weight", (2048, 320), 12, wq.tobytes()),
        ("blk.0.attn_k.weight", (1024, 192), 23, wk.tobytes()),
        ("blk.0.ffn_gate_exps.weight", (DM, DFF, E), 23, gate.tobytes()),
    ], alignment=64)
    shard1 = build([("general.architecture", (8, "qwen3moe"))] + _split_keys(1, 2, 5), [
        ("blk.0.ffn_up_exps.weight", (DM, DFF, E), 23, up.tobytes()),
        ("blk.0.ffn_down_exps.weight", (DFF, DM, E), 12, down.tobytes()),
    ])
    return {"wq": wq, "wk": wk, "gate": gate, "up": up, "down": down, "shards": [shard0, shard1]}


@pytest.mark.parametrize("name,key,m", [("blk.0.attn_q.weight", "wq", 1), ("blk.0.attn_q.weight", "wq", 5),
                                        ("blk.0.attn_k.weight", "wk", 3), ("blk.0.attn_q.weight", "wq", 40)])
def test_loaded_matmul_weight_runs_like_a_direct_upload(checkpoint, name, key, m):
    b = checkpoint["shards"][0]
    f = gguf.GgufFile.parse(b)
    st, w, ws = gguf.load_matmul_weight(f, b, name, m_bucket=m)
    assert ws is None
    wire = checkpoint[key]
    assert np.array_equal(host(w), wire.reshape(-1))
    n, k = wire.shape[0], st.k
    assert (st.n, st.k) == (n, wire.shape[1] // ffi.BLOCK_BYTES[st.w_scheme] * 256)
    x = synth.normal_bf16(77 + m, (m, k))
    y = host(ffi.matmul(w, st.w_scheme, st.n, st.k, bf16_dev(x)))
    y_direct = host(ffi.matmul(dev(wire), st.w_scheme, n, k, bf16_dev(x)))
    assert np.array_equal(y.view(np.uint32), y_direct.view(np.uint32))
    check_close(y, O.matmul(st.w_scheme, wire, n, k, x, O.BF16), f"{name} m={m}")


@pytest.mark.parametrize("t", [5, 300])
def test_experts_stacked_from_two_shards_run_moe_ffn(checkpoint, t):
    s0, s1 = checkpoint["shards"]
    f0, f1 = gguf.GgufFile.parse(s0), gguf.GgufFile.parse(s1)
    shards = gguf.ShardSet.open([f0, f1])
    assert shards.tensor("blk.0.ffn_up_exps.weight")[0] == 1
    w_gate_up = gguf.upload_gate_up(f0, s0, "blk.0.ffn_gate_exps.weight", f1, s1, "blk.0.ffn_up_exps.weight")
    w_down = gguf.upload(f1, s1, "blk.0.ffn_down_exps.weight")
    gate, up, down = checkpoint["gate"], checkpoint["up"], checkpoint["down"]
    stacked = np.concatenate([gate, up], axis=1)          # [E, 2*Dff, row bytes]
    assert np.array_equal(host(w_gate_up), stacked.reshape(-1))
    assert np.array_equal(host(w_down), down.reshape(-1))
    assert ffi.validate_weights(w_gate_up, ffi.IQ4_XS, E * 2 * DFF, DM) == 0

    logits = synth.normal_f32(31 + t, (t, E))
    ids, w = O.moe_route(logits, 2)
    x = synth.normal_bf16(32 + t, (t, DM))
    y, ws, st = ffi.moe_ffn(bf16_dev(x), dev(ids.view(np.int32)), dev(w), w_gate_up, w_down, E, DFF)
    torch.cuda.synchronize()
    assert ffi.moe_ffn_status(st, ws) == 0
    y_direct, _, _ = ffi.moe_ffn(bf16_dev(x), dev(ids.view(np.int32)), dev(w), dev(stacked), dev(down), E, DFF)
    assert np.array_equal(host(y).view(np.uint32), host(y_direct).view(np.uint32))
    check_close(host(y), O.moe_ffn(x, O.BF16, ids, w, E, DFF, stacked.reshape(E * 2 * DFF, -1),
                                   down.reshape(E * DM, -1)), f"moe_ffn t={t}")


def test_fused_gate_up_checkpoint_loads_through_moe_ffn_static(checkpoint):
    gate, up, down = checkpoint["gate"], checkpoint["up"], checkpoint["down"]
    stacked = np.concatenate([gate, up], axis=1)
    b = build([], [("blk.0.ffn_gate_up_exps.weight", (DM, 2 * DFF, E), 23, stacked.tobytes()),
                   ("blk.0.ffn_down_exps.weight", (DFF, DM, E), 12, down.tobytes())])
    f = gguf.GgufFile.parse(b)
    st, w_gate_up, w_down = gguf.load_moe_experts(f, b, "blk.0.ffn_gate_up_exps.weight", None,
                                                  "blk.0.ffn_down_exps.weight", t_bucket=8, k=2)
    assert (st.e_local, st.dm, st.dff) == (E, DM, DFF)
    assert np.array_equal(host(w_gate_up), stacked.reshape(-1))
    assert np.array_equal(host(w_down), down.reshape(-1))


def test_load_refuses_nonfinite_scales_and_short_destinations(checkpoint):
    wq = checkpoint["wq"].copy()
    wq[7, 144 * 3:144 * 3 + 2] = np.frombuffer(np.float16(np.inf).tobytes(), np.uint8)  # block 3 of row 7: d = inf
    b = build([], [("w", (2048, 320), 12, wq.tobytes())])
    f = gguf.GgufFile.parse(b)
    with pytest.raises(gguf.GgufError, match="1 block"):
        gguf.load_matmul_weight(f, b, "w")
    short = torch.empty(wq.size - 1, dtype=torch.uint8, device="cuda")
    with pytest.raises(gguf.GgufError, match="dst holds"):
        gguf.upload(f, b, "w", out=short)
    with pytest.raises(gguf.GgufError, match="beyond buffer size"):
        gguf.upload(f, b[:len(b) - 64], "w")
