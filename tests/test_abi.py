"""CPU checks of the C-ABI boundary: the library loads, exports every function
include/r9vx.h declares, the argument structs follow the kgen layout rule, and
host-side refusals happen before any device call."""
from __future__ import annotations

import ctypes
import pathlib
import re
import subprocess

import pytest

from r9v_amd import ffi

ROOT = pathlib.Path(__file__).resolve().parent.parent
HEADERS = sorted((ROOT / "include").glob("*.h"))


def declared_functions():
    names = set()
    for h in HEADERS:
        names |= set(re.findall(r"^[a-z_0-9 *]*?\b(r9vx_[a-z_0-9]+)\s*\(", h.read_text(), flags=re.M))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    lib = ffi.load()
    names = declared_functions()
    assert len(names) >= 16
    for n in names:
        assert hasattr(lib, n), n
    assert sorted(n for n, _, _ in ffi.EXPORTS) == names
    assert lib.r9vx_abi_version() == 3


def kgen_layout(fields):
    """crates/r9v-kgen/src/abi/layout.rs:102-180: stable sort by descending
    alignment, natural padding, total rounded to the max alignment."""
    order = sorted(range(len(fields)), key=lambda i: (-fields[i][1], i))
    off, offs, maxal = 0, {}, 1
    for i in order:
        name, al = fields[i]
        off = (off + al - 1) // al * al
        offs[name] = off
        off += al
        maxal = max(maxal, al)
    return offs, (off + maxal - 1) // maxal * maxal


# Key declaration order of MatmulStatic / MoeRouteStatic / MoeFfnStatic
# (crates/r9v-registry/src/types.rs:727-770, 774-800, 801-860), u32 each;
# MoeRouteStatic.group (Option<MoeGroup {n_group, topk_group}>) sits between
# renormalize and scale_bits.
STATICS = {
    "r9vx_matmul_static": ["m_bucket", "n", "k", "w_dtype", "w_scheme", "w_layout", "in_dtype", "act_scheme",
                           "out_dtype", "epilogue", "residual_dtype", "transpose_w", "interleave", "sparse"],
    "r9vx_moe_ffn_static": ["t_bucket", "e_local", "k_topk", "dm", "dff", "gate_up.dtype", "gate_up.scheme",
                            "gate_up.layout", "down.dtype", "down.scheme", "down.layout", "in_dtype", "act_scheme",
                            "act", "out_dtype", "shared_experts", "placement_kind"],
    "r9vx_moe_route_static": ["t_bucket", "e_total", "top_k", "scoring", "renormalize", "n_group", "topk_group",
                              "scale_bits", "has_bias"],
}


def test_static_structs_follow_the_registry_key_order(tmp_path):
    src = tmp_path / "statics.c"
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "r9vx.h"', "int main(void){"]
    for st, fields in STATICS.items():
        lines.append(f'printf("{st} size %zu\\n", sizeof({st}));')
        for name in fields:
            lines.append(f'printf("{st} {name} %zu\\n", offsetof({st}, {name}));')
    lines.append("return 0;}")
    src.write_text("\n".join(lines))
    exe = tmp_path / "statics"
    subprocess.run(["gcc", "-std=c11", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    got = {}
    for line in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines():
        st, field, val = line.split()
        got[(st, field)] = int(val)
    for st, fields in STATICS.items():
        assert got[(st, "size")] == 4 * len(fields), st
        for i, name in enumerate(fields):
            assert got[(st, name)] == 4 * i, (st, name)
    assert ctypes.sizeof(ffi.MatmulStatic) == got[("r9vx_matmul_static", "size")]
    assert ctypes.sizeof(ffi.MoeFfnStatic) == got[("r9vx_moe_ffn_static", "size")]
    assert ctypes.sizeof(ffi.MoeRouteStatic) == got[("r9vx_moe_route_static", "size")]
    for st, cls in (("r9vx_matmul_static", ffi.MatmulStatic), ("r9vx_moe_route_static", ffi.MoeRouteStatic)):
        for name in STATICS[st]:
            assert getattr(cls, name).offset == got[(st, name)], (st, name)


# SchemeId::code (crates/r9v-format/src/scheme.rs:115-138) of every scheme, and
# the GGUF type ids the reference keeps out of that code space (:78-87).
SCHEME_IDS = {"I4K": 3, "I8B32F": 5, "I6K": 11, "I4Xs": 15, "Iq3S": 17}
GGML_IDS = {"Q4_K": 12, "Q8_0": 8, "Q6_K": 14, "IQ4_XS": 23, "IQ3_S": 21}


def test_statics_carry_scheme_id_codes():
    """w_scheme / proj.scheme are SchemeId codes: the five this path reads
    are accepted, and the codes that are GGUF ids of the same formats -- 8, 12,
    14, 21 -- are refused, being SchemeId codes of other schemes (I5B32F,
    I3K, I4Nl, Iq1S) that a registry would pass for those; so is 23 (no
    scheme).  The GGUF type -> scheme translation is the reference's."""
    assert (ffi.Q4_K, ffi.Q8_0, ffi.Q6_K, ffi.IQ4_XS, ffi.IQ3_S) == tuple(SCHEME_IDS.values())
    lib = ffi.load()
    for name, code in GGML_IDS.items():
        assert lib.r9vx_scheme_from_ggml_type(code) == getattr(ffi, name)
    for code in (0, 1, 2, 4, 6, 7, 9, 10, 13, 16, 18, 19, 20, 22, 24, 30, 1001):
        assert lib.r9vx_scheme_from_ggml_type(code) == 0, code
    args = ffi.MatmulArgs()
    args.m = 1
    fargs = ffi.MoeFfnArgs()
    fargs.t = 1
    for code in (8, 12, 14, 21, 23):
        st = ffi.matmul_static(n=64, k=512, w_scheme=ffi.Q4_K, in_dtype=ffi.BF16, out_dtype=ffi.F32)
        st.w_scheme = code
        assert _call(lib.r9vx_matmul_launch, st, args) == -2, code
        assert f"w_scheme {code} is not the SchemeId code" in lib.r9vx_last_error().decode()
        fst = ffi.ffn_static(t_bucket=4, e=4, k=2, dm=256, dff=256)
        fst.gate_up.scheme = code
        fst.down.scheme = code
        assert _call(lib.r9vx_moe_ffn_launch, fst, fargs) < 0, code
        msg = lib.r9vx_last_error().decode()
        assert f"gate_up scheme {code}:" in msg and f"down scheme {code}:" in msg, msg
        assert lib.r9vx_dequantize_launch(code, None, 0, 256, None, None) == -2
    for code in SCHEME_IDS.values():  # accepted: only the missing operands are refused
        st = ffi.matmul_static(n=64, k=512, w_scheme=code, in_dtype=ffi.BF16, out_dtype=ffi.F32)
        assert _call(lib.r9vx_matmul_launch, st, args) == -3, code
        assert "w_scheme" not in lib.r9vx_last_error().decode()


def test_route_static_group_key_is_refused():
    lib = ffi.load()
    args = ffi.MoeRouteArgs()
    args.t = 1
    for n_group, topk_group in ((4, 2), (0, 1)):
        st = ffi.route_static(e=64, k=4, t_bucket=1)
        st.n_group, st.topk_group = n_group, topk_group
        assert _call(lib.r9vx_moe_route_launch, st, args) == -2
        assert f"grouped expert routing (n_group {n_group}, topk_group {topk_group})" in \
            lib.r9vx_last_error().decode()


def test_reference_layouts_and_keys_are_refused():
    """A weight in the reference's own L0 / L1 / L1S layout, a transposed or
    interleaved or sparse weight, quantized activations, or a dtype that does not
    match the scheme are typed refusals, never reinterpreted bytes."""
    lib = ffi.load()
    args = ffi.MatmulArgs()
    args.m = 1
    for layout, name in ((ffi.LAYOUT_L1, "(L1)"), (ffi.LAYOUT_L0, "(L0)"), (ffi.LAYOUT_L1S, "(L1S)"),
                         (ffi.LAYOUT_SPLIT, "(split)")):
        st = ffi.matmul_static(n=64, k=512, w_scheme=ffi.Q4_K, in_dtype=ffi.BF16, out_dtype=ffi.F32, w_layout=layout)
        assert _call(lib.r9vx_matmul_launch, st, args) == -2
        msg = lib.r9vx_last_error().decode()
        assert name in msg and "gguf_wire layout (code 256) only" in msg, msg
    st = ffi.matmul_static(n=64, k=512, w_scheme=ffi.IQ3_S, in_dtype=ffi.BF16, out_dtype=ffi.F32,
                           w_layout=ffi.LAYOUT_GGUF_WIRE)
    assert _call(lib.r9vx_matmul_launch, st, args) == -2
    assert "iq3s_112 layout (code 258) only" in lib.r9vx_last_error().decode()
    st = ffi.matmul_static(n=64, k=512, w_scheme=ffi.Q8_0, in_dtype=ffi.BF16, out_dtype=ffi.F32)
    st.w_dtype, st.transpose_w, st.interleave, st.sparse, st.act_scheme = ffi.I4, 1, 1, 1, 3
    assert _call(lib.r9vx_matmul_launch, st, args) == -2
    msg = lib.r9vx_last_error().decode()
    for part in ("w dtype 6", "transpose_w", "interleave", "sparse", "act_scheme 3"):
        assert part in msg, msg
    fst = ffi.ffn_static(t_bucket=4, e=4, k=2, dm=256, dff=256)
    fst.gate_up.layout = ffi.LAYOUT_L1
    fst.down.dtype = ffi.I8
    fst.placement_kind = 2
    fargs = ffi.MoeFfnArgs()
    fargs.t = 2
    assert _call(lib.r9vx_moe_ffn_launch, fst, fargs) < 0
    msg = lib.r9vx_last_error().decode()
    for part in ("gate_up layout 2 (L1)", "down dtype 5", "placement_kind 2"):
        assert part in msg, msg


def test_route_ex_needs_its_own_status_word():
    lib = ffi.load()
    st = ffi.route_static(e=64, k=4, t_bucket=8)
    args = ffi.MoeRouteArgs()
    args.t = 2
    assert lib.r9vx_moe_route_launch_ex(ctypes.byref(st), ctypes.byref(args), None, None) == -3
    msg = lib.r9vx_last_error().decode()
    assert "status word is NULL" in msg and "logits" in msg, msg
    assert lib.r9vx_moe_route_launch_ex(ctypes.byref(st), ctypes.byref(args), ctypes.c_void_p(0x1002), None) < 0
    assert "4-byte aligned" in lib.r9vx_last_error().decode()
    assert lib.r9vx_status_read(None, None, None) == -3


# Field declaration order of crates/r9v-kgen/src/abi/per_op.rs:794-968
# (pointer = 8 bytes, u32 = 4 bytes); the workspace slot is appended where
# add_workspace_slot is called.
KGEN = {
    "r9vx_matmul_args": [("w", 8), ("w_scales", 8), ("w_indices", 8), ("x", 8), ("x_scale", 8), ("bias", 8),
                         ("residual", 8), ("y", 8), ("workspace", 8), ("m", 4)],
    "r9vx_moe_route_args": [("logits", 8), ("bias", 8), ("expert_ids", 8), ("weights", 8), ("t", 4)],
    "r9vx_moe_ffn_args": [("x", 8), ("expert_ids", 8), ("weights", 8), ("w_gate_up", 8),
                          ("w_gate_up_scales", 8), ("w_down", 8), ("w_down_scales", 8), ("y", 8),
                          ("sort_workspace", 8), ("t", 4)],
}


def test_arg_structs_match_kgen_layout(tmp_path):
    src = tmp_path / "layout.c"
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "r9vx.h"', "int main(void){"]
    for st, fields in KGEN.items():
        lines.append(f'printf("{st} size %zu\\n", sizeof({st}));')
        for name, _ in fields:
            lines.append(f'printf("{st} {name} %zu\\n", offsetof({st}, {name}));')
    lines.append("return 0;}")
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    got = {}
    for line in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines():
        st, field, val = line.split()
        got[(st, field)] = int(val)
    for st, fields in KGEN.items():
        offs, size = kgen_layout(fields)
        assert got[(st, "size")] == size, st
        for name, _ in fields:
            assert got[(st, name)] == offs[name], (st, name)
    # the ctypes mirror agrees with the C header
    assert ctypes.sizeof(ffi.MatmulArgs) == got[("r9vx_matmul_args", "size")]
    assert ctypes.sizeof(ffi.MoeRouteArgs) == got[("r9vx_moe_route_args", "size")]
    assert ctypes.sizeof(ffi.MoeFfnArgs) == got[("r9vx_moe_ffn_args", "size")]


def _call(fn, st, args):
    return fn(ctypes.byref(st) if st is not None else None, ctypes.byref(args) if args is not None else None, None)


def test_host_refusals_collect_all_problems():
    lib = ffi.load()
    assert _call(lib.r9vx_matmul_launch, None, None) == -3
    st = ffi.matmul_static(n=0, k=300, w_scheme=99, in_dtype=5, out_dtype=ffi.F32)
    args = ffi.MatmulArgs()
    args.m = 1
    rc = _call(lib.r9vx_matmul_launch, st, args)
    msg = lib.r9vx_last_error().decode()
    assert rc < 0
    for part in ("w_scheme 99", "k=300", "n must be positive", "in_dtype 5", "w is NULL"):
        assert part in msg, msg
    rst = ffi.route_static(e=4, k=5, t_bucket=1, scale=-1.0)
    rargs = ffi.MoeRouteArgs()
    rargs.t = 2
    assert _call(lib.r9vx_moe_route_launch, rst, rargs) < 0
    msg = lib.r9vx_last_error().decode()
    for part in ("scale must be finite", "top_k 5 cannot exceed", "t=2 exceeds t_bucket=1", "logits"):
        assert part in msg, msg
    fst = ffi.ffn_static(t_bucket=4, e=4, k=2, dm=300, dff=256)
    fargs = ffi.MoeFfnArgs()
    fargs.t = 2
    assert _call(lib.r9vx_moe_ffn_launch, fst, fargs) < 0
    msg = lib.r9vx_last_error().decode()
    assert "Dm=300" in msg and "sort_workspace is NULL" in msg


def test_workspace_and_static_figures():
    st = ffi.matmul_static(n=5120, k=2048, w_scheme=ffi.IQ4_XS, in_dtype=ffi.BF16, out_dtype=ffi.F32, m_bucket=5)
    assert ffi.matmul_static_bytes(st, 1) == 5_595_136  # BASELINE.md config 1, M=1
    assert ffi.matmul_static_bytes(st, 5) == 5_693_440  # M=5
    st0 = ffi.matmul_static(n=4096, k=4096, w_scheme=ffi.Q4_K, in_dtype=ffi.F32, out_dtype=ffi.F32)
    assert ffi.matmul_static_bytes(st0, 1) == 9_469_952  # config 0
    fst = ffi.ffn_static(t_bucket=8192, e=512, k=10, dm=2048, dff=512)
    lib = ffi.load()
    assert lib.r9vx_moe_ffn_static_flops(ctypes.byref(fst), 8192) == 515_396_075_520  # config 4
    assert ffi.ffn_workspace_bytes(fst) > 81920 * 2048 * 4
    # one expert = IQ4_XS gate/up [1024 x 2048] + Q4_K down [2048 x 512]
    assert lib.r9vx_moe_ffn_expert_bytes(ctypes.byref(fst)) == 1_703_936
    # config 4 upper bound: all 512 experts + x + ids/weights + y
    assert lib.r9vx_moe_ffn_static_bytes(ctypes.byref(fst), 8192) == (512 * 1_703_936 + 8192 * 2048 * 2
                                                                       + 81920 * 8 + 8192 * 2048 * 4)
    # config 3: t=5, K=10 -> at most 50 routed experts, + the shared one
    c3 = ffi.ffn_static(t_bucket=5, e=512, k=10, dm=2048, dff=512, shared=1)
    assert lib.r9vx_moe_ffn_static_bytes(ctypes.byref(c3), 5) == 51 * 1_703_936 + 5 * 2048 * 6 + 50 * 8
    rst = ffi.route_static(e=512, k=10, t_bucket=5)
    assert lib.r9vx_moe_route_static_flops(ctypes.byref(rst), 5) == 5 * (4 * 512 + 3 * 10)
    assert lib.r9vx_moe_route_static_bytes(ctypes.byref(rst), 5) == 5 * 512 * 4 + 5 * 10 * 8


def test_split_scheme_refusals_and_figures():
    """Q8_0 / Q6_K: bf16 activations and a w_scales array required; Q4_K / IQ4_XS take none; the device
    repack refuses schemes that need none and overlapping buffers."""
    lib = ffi.load()
    for scheme in (ffi.Q6_K, ffi.Q8_0):
        st = ffi.matmul_static(n=64, k=512, w_scheme=scheme, in_dtype=ffi.F32, out_dtype=ffi.F32, m_bucket=16)
        args = ffi.MatmulArgs()
        args.m = 1
        assert _call(lib.r9vx_matmul_launch, st, args) < 0
        msg = lib.r9vx_last_error().decode()
        for part in ("bf16 activations only", "w_scales (the f16 d array", "w is NULL"):
            assert part in msg, msg
        good = ffi.matmul_static(n=64, k=512, w_scheme=scheme, in_dtype=ffi.BF16, out_dtype=ffi.F32)
        bb, bl = ffi.BLOCK_BYTES[scheme], ffi.BLOCK_LEN[scheme]
        assert ffi.matmul_static_bytes(good, 1) == 64 * 512 // bl * bb + 512 * 2 + 64 * 4
    st = ffi.matmul_static(n=64, k=512, w_scheme=ffi.Q4_K, in_dtype=ffi.BF16, out_dtype=ffi.F32)
    args = ffi.MatmulArgs()
    args.m = 1
    args.w_scales = 16
    assert _call(lib.r9vx_matmul_launch, st, args) < 0
    assert "inline scales" in lib.r9vx_last_error().decode()
    buf = ctypes.create_string_buffer(4096)
    base = ctypes.addressof(buf) + (-ctypes.addressof(buf) % 16)
    rc = lib.r9vx_repack_launch(ffi.Q4_K, base, 1, 256, base + 1024, base + 2048, None)
    assert rc == -2 and "device layout" in lib.r9vx_last_error().decode()
    rc = lib.r9vx_repack_launch(ffi.Q6_K, base, 4, 256, base + 16, base + 2048, None)
    assert rc == -1 and "overlap" in lib.r9vx_last_error().decode()


def test_iq3s_refusals_and_figures():
    """IQ3_S: bf16 activations, no w_scales (d is inline in the 112-byte block), and a repack that takes
    no scales array and refuses an overlapping body."""
    lib = ffi.load()
    st = ffi.matmul_static(n=64, k=512, w_scheme=ffi.IQ3_S, in_dtype=ffi.F32, out_dtype=ffi.F32)
    args = ffi.MatmulArgs()
    args.m = 1
    args.w_scales = 16
    assert _call(lib.r9vx_matmul_launch, st, args) < 0
    msg = lib.r9vx_last_error().decode()
    assert "bf16 activations only" in msg and "inline scales" in msg, msg
    good = ffi.matmul_static(n=64, k=512, w_scheme=ffi.IQ3_S, in_dtype=ffi.BF16, out_dtype=ffi.F32)
    assert ffi.matmul_static_bytes(good, 1) == 64 * 2 * 112 + 512 * 2 + 64 * 4  # the 112-byte device blocks
    buf = ctypes.create_string_buffer(8192)
    base = ctypes.addressof(buf) + (-ctypes.addressof(buf) % 16)
    rc = lib.r9vx_repack_launch(ffi.IQ3_S, base, 1, 256, base + 1024, base + 2048, None)
    assert rc == -1 and "scales must be NULL for IQ3_S" in lib.r9vx_last_error().decode()
    rc = lib.r9vx_repack_launch(ffi.IQ3_S, base, 4, 256, base + 16, None, None)
    assert rc == -1 and "must not overlap" in lib.r9vx_last_error().decode()
    rc = lib.r9vx_repack_launch(ffi.IQ3_S, base, 1, 300, base + 1024, None, None)
    assert rc == -1 and "multiple of 256" in lib.r9vx_last_error().decode()


def test_swiglu_epilogue_refusals_and_figures():
    lib = ffi.load()
    st = ffi.matmul_static(n=64, k=512, w_scheme=ffi.Q4_K, in_dtype=ffi.F32, out_dtype=ffi.F32, m_bucket=16,
                           epilogue=ffi.EPILOGUE_SWIGLU)
    args = ffi.MatmulArgs()
    args.m = 1
    args.bias = 64
    assert _call(lib.r9vx_matmul_launch, st, args) < 0
    msg = lib.r9vx_last_error().decode()
    assert "decode GEMV only" in msg and "bias given without bias epilogue" in msg
    good = ffi.matmul_static(n=64, k=512, w_scheme=ffi.Q4_K, in_dtype=ffi.BF16, out_dtype=ffi.F32,
                             epilogue=ffi.EPILOGUE_SWIGLU)
    assert ffi.matmul_static_bytes(good, 1) == 128 * 2 * 144 + 512 * 2 + 64 * 4  # 2n weight rows
    assert lib.r9vx_matmul_static_flops(ctypes.byref(good), 3) == 4 * 3 * 64 * 512


def test_route_hidden_refusals():
    lib = ffi.load()
    st = ffi.route_static(e=512, k=10, t_bucket=16)
    args = ffi.MoeRouteHiddenArgs()
    args.t = 12
    args.dm = 100
    assert _call(lib.r9vx_moe_route_hidden_launch, st, args) < 0
    msg = lib.r9vx_last_error().decode()
    for part in ("decode form (t_bucket <= 8)", "dm=100", "x, w_router", "workspace of"):
        assert part in msg, msg
    assert lib.r9vx_moe_route_hidden_workspace_bytes(ctypes.byref(st)) == 16 * 512 * 4 + 256


def test_moe_ffn_noalloc_host_refusals():
    """The no-alloc moe_ffn launch refuses a caller workspace and statics whose
    workspace exceeds its scratch before touching the device."""
    lib = ffi.load()
    fake = ctypes.c_void_p(1 << 20)  # 256-byte aligned, never dereferenced: the call is refused first
    st = ffi.ffn_static(t_bucket=4, e=8, k=2, dm=256, dff=256)
    args = ffi.MoeFfnArgs(fake, fake, fake, fake, None, fake, None, fake, fake, 4, 0)
    assert lib.r9vx_moe_ffn_launch_noalloc(ctypes.byref(st), ctypes.byref(args), None, None) == -1
    assert "sort_workspace must be NULL" in lib.r9vx_last_error().decode()
    big = ffi.ffn_static(t_bucket=8192, e=512, k=10, dm=2048, dff=512)
    assert ffi.ffn_workspace_bytes(big) > ffi.NOALLOC_SCRATCH_BYTES
    args.sort_workspace = None
    assert lib.r9vx_moe_ffn_launch_noalloc(ctypes.byref(big), ctypes.byref(args), None, None) == -2
    assert "exceeds the no-alloc scratch (16777216 bytes)" in lib.r9vx_last_error().decode()
    # configs[3] (T=5, E=512 + 1 shared, top-10, 2048 / 512) fits
    c3 = ffi.ffn_static(t_bucket=5, e=512, k=10, dm=2048, dff=512, shared=1)
    assert ffi.ffn_workspace_bytes(c3) <= ffi.NOALLOC_SCRATCH_BYTES
    assert lib.r9vx_moe_ffn_launch_noalloc(None, ctypes.byref(args), None, None) == -3
