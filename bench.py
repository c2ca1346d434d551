#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-weight matrix path (one GPU).

Headline (the largest single-GPU configuration):
MoE prefill, T = 8192 tokens, E = 512 experts, top-10 Zipf(1.1) routing,
hidden 2048, expert width 512, IQ4_XS gate/up and Q4_K down experts.  A step
is one moe_ffn launch over the whole batch -- the on-GPU permute, the grouped
gate/up GEMM with SwiGLU, the grouped down GEMM and the weighted unpermute-
sum -- with two weight copies alternating (1.7 GB, well past the 256 MB
Infinity Cache) so every step reads its experts from HBM.  `value` =
515,396,075,520 algorithmic FLOP per step / the measured time per step
(TFLOP/s; K steps bracketed by device synchronisations, each step also
timed by its own HIP events for the median).  `roofline` is the dominant
kernel, the gate/up grouped GEMM (343.6 GFLOP per launch), relaunched on its
own through the stage probe and timed with HIP events on its stream.

`extras` carries configs[0..3] with their own roofline figures (GB/s for the
HBM-bound GEMVs and MoE decode, TFLOP/s for the dense prefill GEMM), the
measured ceilings, and CPU figures for every config: the oracle (a scalar C
restatement of R9V's T0 path) on a bounded sample on this host, 1 thread,
plus an all-threads OpenMP variant for the grouped MoE GEMM.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only c0,c1,c2,c3,gemv_n,schemes,ceilings]
    python bench.py --pmc-case c4|c3|c2|c1m5|c0|gemvn|ceil  # short fixed run for rocprofv3 --pmc
    python bench.py --pmc-summary DIR ... [--pmc-kernels a,b]  # FETCH_SIZE/WRITE_SIZE dirs -> traffic text
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0  # dense fp16 / bf16 MFMA, MI355X
IC_BYTES = 256 << 20
METRIC = "quant GEMV/MoE HBM GB/s (% of peak); prefill grouped-GEMM TFLOP/s (% MFMA)"

# configs[4]
C4_T, C4_E, C4_K, C4_DM, C4_DFF = 8192, 512, 10, 2048, 512
C4_FLOPS = C4_T * C4_K * (2 * 2 * C4_DFF * C4_DM + 2 * C4_DM * C4_DFF)  # 515,396,075,520
C4_GU_FLOPS = C4_T * C4_K * 2 * 2 * C4_DFF * C4_DM                     # 343,597,383,680
HEAD_KERNEL = "moe_gu_m3_kernel<15>"  # gate/up grouped GEMM, IQ4_XS (scheme code 15)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "moe_gu_m3_c4_traffic.txt")
PMC_COPY_BYTES = 64 << 20


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of CPU work per baseline sample")
    ap.add_argument("--only", default="", help="comma list of extras: c0,c1,c2,c3,gemv_n,schemes,ceilings ('none' for the "
                                               "headline only)")
    ap.add_argument("--pmc-case", default="", help="run a short fixed workload for counter collection: c4, c3, c2, c1m5, "
                                                   "c0, gemvn, ceil")
    ap.add_argument("--pmc-summary", nargs="*", default=None,
                    help="rocprofv3 --pmc output dirs (FETCH_SIZE, WRITE_SIZE) to summarise as traffic")
    ap.add_argument("--clock-summary", nargs=2, default=None, metavar=("KT_DIR", "PMC_DIR"),
                    help="rocprofv3 --kernel-trace and --pmc GRBM_GUI_ACTIVE output dirs of one workload: each "
                         "kernel's mean shader clock")
    ap.add_argument("--pmc-kernels", default="", help="comma list of kernel-name substrings for --pmc-summary "
                                                      "(default: the headline kernel)")
    return ap.parse_args()


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def copies_for(nbytes):
    return max(2, -(-2 * IC_BYTES // max(nbytes, 1)))


def hbm(bytes_, ms):
    gbs = bytes_ / (ms * 1e-3) / 1e9
    return {"GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}


def mfma(flops, ms):
    tf = flops / (ms * 1e-3) / 1e12
    return {"TFLOP/s": round(tf, 1), "frac_mfma": round(tf / MFMA_PEAK_TFLOPS, 4)}


def timed_steps(torch, fn, steps, warmup):
    """Runs `warmup` untimed calls fn(i), then `steps` calls each bracketed by
    HIP events on the launch stream, the whole run bracketed by device
    synchronisations.  Returns (total ms / steps, median per-call ms)."""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for i in range(steps):
        ev[i][0].record(s)
        fn(warmup + i)
        ev[i][1].record(s)
    torch.cuda.synchronize()
    total = ev[0][0].elapsed_time(ev[-1][1])
    return total / steps, statistics.median(a.elapsed_time(b) for a, b in ev)


def graph_time(torch, fn, copies, reps=10):
    """ms per launch of back-to-back calls fn(i, stream) captured in a HIP
    graph: max(copies, 64) launches (so every weight copy is touched whatever
    the caller's step count), one untimed replay, then `reps` (>= 2) replays
    each between events on the replay stream; the median replay is used."""
    launches = max(copies, 64)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(launches):
            fn(i, s)
        s.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for i in range(launches):
                fn(i, s)
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    cur = torch.cuda.current_stream()
    times = []
    for _ in range(max(reps, 2)):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(cur)
        g.replay()
        e1.record(cur)
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) / launches)
    return statistics.median(times)


def cpu_threads():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def host_cpu():
    model = "unknown host CPU"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return f"{model}, {cpu_threads()} threads available to this process"


def oracle():
    """The CPU oracle in T0's own loop structure (one row at a time through
    each dot), which is what the CPU baseline times."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_ffi as O

    O.set_rows_at_once(1)
    return O


def loop_for(budget_s, fn):
    """Calls fn() until budget_s seconds have passed; returns (calls, seconds)."""
    calls, t0 = 0, time.perf_counter()
    while True:
        fn()
        calls += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            return calls, el


# ---------------------------------------------------------------- configs[4]

class MoePrefill:
    """configs[4] on the device: seeded Zipf(1.1) logits routed once (the
    routing is not part of moe_ffn's step), IQ4_XS gate/up and Q4_K down
    experts in two alternating copies."""

    def __init__(self, torch, ffi, synth, gsynth):
        self.torch, self.ffi = torch, ffi
        t, e, k, dm, dff = C4_T, C4_E, C4_K, C4_DM, C4_DFF
        self.logits_host = synth.zipf_logits(synth.seed_for("c4", "logits"), t, e)
        self.x_host = synth.normal_bf16(synth.seed_for("c4", "x"), (t, dm))
        gu = gsynth.quant_weights_gpu(torch, ffi.IQ4_XS, 401, e * 2 * dff, dm)
        dn = gsynth.quant_weights_gpu(torch, ffi.Q4_K, 402, e * dm, dff)
        self.wsets = [(gu, dn), (gu.clone(), dn.clone())]
        self.x = torch.from_numpy(self.x_host.view(np.int16)).cuda().view(torch.bfloat16)
        self.ids = torch.empty((t, k), dtype=torch.int32, device="cuda")
        self.w = torch.empty((t, k), dtype=torch.float32, device="cuda")
        self.y = torch.empty((t, dm), dtype=torch.float32, device="cuda")
        self.st = ffi.ffn_static(t, e, k, dm, dff)
        self.wsp = torch.empty(ffi.ffn_workspace_bytes(self.st), dtype=torch.uint8, device="cuda")
        ffi.moe_route(torch.from_numpy(self.logits_host).cuda(), k, ids=self.ids, weights=self.w)
        torch.cuda.synchronize()

    def step(self, i):
        gu, dn = self.wsets[i % 2]
        self.ffi.moe_ffn(self.x, self.ids, self.w, gu, dn, C4_E, C4_DFF, y=self.y, workspace=self.wsp)

    def stage_ms(self, stage, launches=20):
        """Median ms of one relaunched stage (1 gate/up GEMM, 2 down GEMM, 3
        combine) over `launches` launches, alternating weight copies."""
        torch = self.torch

        def fn(i):
            gu, dn = self.wsets[i % 2]
            self.ffi.probe_moe_stage(self.x, self.ids, self.w, gu, dn, C4_E, C4_DFF, stage, self.y, self.wsp)

        _, med = timed_steps(torch, fn, launches, 2)
        return med

    def cpu_sample(self, budget_s, threads):
        """The per-expert sliced T0 algorithm (the oracle's moe_ffn body) on the
        experts in ascending id order until budget_s has passed; returns
        (TFLOP/s, pairs, experts, seconds)."""
        O = oracle()
        ids = self.ids.cpu().numpy().astype(np.uint32)
        gu, dn = self.wsets[0]
        gu_rows = gu.view(C4_E, -1)
        dn_rows = dn.view(C4_E, -1)
        pairs = experts = 0
        t0 = time.perf_counter()
        for ex in range(C4_E):
            toks = np.nonzero((ids == ex).any(axis=1))[0].astype(np.uint32)
            if len(toks) == 0:
                continue
            O.moe_expert(self.x_host, O.BF16, toks, C4_DFF, gu_rows[ex].cpu().numpy(), dn_rows[ex].cpu().numpy(),
                         threads=threads)
            pairs += len(toks)
            experts += 1
            if time.perf_counter() - t0 >= budget_s:
                break
        el = time.perf_counter() - t0
        return pairs * (C4_FLOPS // (C4_T * C4_K)) / el / 1e12, pairs, experts, el


# ---------------------------------------------------------------- configs[0..3]

class Gemv:
    def __init__(self, torch, ffi, synth, scheme, n, k, m, x_dtype, tag):
        self.torch, self.ffi = torch, ffi
        self.scheme, self.n, self.k, self.m, self.x_dtype = scheme, n, k, m, x_dtype
        self.w_host = synth.quant_weights(scheme, synth.seed_for(tag, "w"), n, k)
        wd = torch.from_numpy(self.w_host).cuda()
        self.ws = [wd] + [wd.clone() for _ in range(copies_for(self.w_host.nbytes) - 1)]
        if x_dtype == ffi.BF16:
            self.x_host = synth.normal_bf16(synth.seed_for(tag, "x"), (m, k))
            self.x = torch.from_numpy(self.x_host.view(np.int16)).cuda().view(torch.bfloat16)
        else:
            self.x_host = synth.normal_f32(synth.seed_for(tag, "x"), (m, k))
            self.x = torch.from_numpy(self.x_host).cuda()
        self.y = torch.empty((m, n), dtype=torch.float32, device="cuda")
        self.bytes = ffi.matmul_static_bytes(ffi.matmul_static(n, k, scheme, x_dtype, ffi.F32, m_bucket=m), m)

    def launch(self, i, stream=None):
        self.ffi.matmul(self.ws[i % len(self.ws)], self.scheme, self.n, self.k, self.x, y=self.y, stream=stream)

    def graph_ms(self):
        return graph_time(self.torch, self.launch, len(self.ws))

    def cpu(self, budget_s):
        O = oracle()
        calls, el = loop_for(budget_s, lambda: O.matmul(self.scheme, self.w_host, self.n, self.k, self.x_host,
                                                          self.x_dtype))
        return {"GB/s": round(self.bytes * calls / el / 1e9, 4), "cores": 1, "kind": "port",
                "sample": f"{calls} whole GEMVs in {el:.1f} s"}


def gemv_extra(torch, ffi, synth, scheme, n, k, m, x_dtype, tag, cpu_s, workload):
    b = Gemv(torch, ffi, synth, scheme, n, k, m, x_dtype, tag)
    ms = b.graph_ms()
    out = {"workload": workload, "us_per_launch": round(ms * 1e3, 3), "bytes": b.bytes, "weight_copies": len(b.ws),
           **hbm(b.bytes, ms)}
    if cpu_s:
        out["cpu"] = b.cpu(cpu_s)
    del b
    torch.cuda.empty_cache()
    return out


def c2_extra(torch, ffi, synth, gsynth, steps, cpu_s, steps_only=False):
    m, n, k = 2048, 14336, 4096
    w0 = gsynth.quant_weights_gpu(torch, ffi.Q4_K, 201, n, k)
    ws = [w0] + [w0.clone() for _ in range(copies_for(w0.numel()) - 1)]
    x_host = synth.normal_bf16(synth.seed_for("c2", "x"), (m, k))
    x = torch.from_numpy(x_host.view(np.int16)).cuda().view(torch.bfloat16)
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    st = ffi.matmul_static(n, k, ffi.Q4_K, ffi.BF16, ffi.BF16, m_bucket=m)
    wsp = torch.empty(ffi.matmul_workspace_bytes(st), dtype=torch.uint8, device="cuda")

    def step(i):
        ffi.matmul(ws[i % len(ws)], ffi.Q4_K, n, k, x, out_dtype=ffi.BF16, y=y, workspace=wsp)

    if steps_only:  # a fixed run for counter collection
        for i in range(steps):
            step(i)
        return None
    ms, med = timed_steps(torch, step, max(steps, len(ws)), 3)
    flops = 2 * m * n * k
    out = {"workload": "configs[2]: x bf16 [2048x4096] . Q4_K [14336x4096]^T -> bf16, fp16 MFMA",
           "ms_per_step": round(ms, 4), "median_ms_per_step": round(med, 4), "tokens/s": round(m / (ms * 1e-3), 1),
           "flops": flops, "weight_copies": len(ws), **mfma(flops, ms)}
    if cpu_s:
        # whole-row sample: all 2048 tokens against the first c output columns
        O = oracle()
        c = 32
        w_host = w0[:c].cpu().numpy()
        calls, el = loop_for(cpu_s, lambda: O.matmul(ffi.Q4_K, w_host, c, k, x_host, O.BF16))
        out["cpu"] = {"TFLOP/s": round(2 * m * c * k * calls / el / 1e12, 6), "cores": 1, "kind": "port",
                      "sample": f"{calls} x (2048 tokens x {c} of 14336 output columns) in {el:.1f} s, extrapolated "
                                f"per FLOP"}
    del ws, w0
    torch.cuda.empty_cache()
    return out


def schemes_extra(torch, ffi, synth, gsynth, steps):
    """The other weight types at the headline shapes (measurement only; all
    three run the headline kernels' 256-row loop): the configs[2] dense GEMM
    and the configs[4] moe_ffn step with Q8_0, Q6_K and IQ3_S weights in
    their device layouts (split body + f16 d array; 112-byte IQ3_S blocks)."""
    out = {"gemm_c2_shape": {}, "moe_ffn_c4_shape": {}}
    m, n, k = 2048, 14336, 4096
    x_host = synth.normal_bf16(synth.seed_for("c2", "x"), (m, k))
    x = torch.from_numpy(x_host.view(np.int16)).cuda().view(torch.bfloat16)
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    names = {ffi.Q8_0: "Q8_0", ffi.Q6_K: "Q6_K", ffi.IQ3_S: "IQ3_S"}
    for scheme, name in names.items():
        body, sc = ffi.repack(gsynth.quant_weights_gpu(torch, scheme, 501 + scheme, n, k), scheme, n, k)
        st = ffi.matmul_static(n, k, scheme, ffi.BF16, ffi.BF16, m_bucket=m)
        wsp = torch.empty(ffi.matmul_workspace_bytes(st), dtype=torch.uint8, device="cuda")
        ms, _ = timed_steps(torch, lambda i: ffi.matmul(body, scheme, n, k, x, out_dtype=ffi.BF16, y=y, workspace=wsp,
                                                        w_scales=sc), steps, 2)
        out["gemm_c2_shape"][name] = {"ms_per_step": round(ms, 4), **mfma(2 * m * n * k, ms)}
        del body, sc, wsp
        torch.cuda.empty_cache()
    del x, y
    t, e, kk, dm, dff = C4_T, C4_E, C4_K, C4_DM, C4_DFF
    xm = torch.from_numpy(synth.normal_bf16(synth.seed_for("c4", "x"), (t, dm)).view(np.int16)).cuda().view(
        torch.bfloat16)
    ids = torch.empty((t, kk), dtype=torch.int32, device="cuda")
    wts = torch.empty((t, kk), dtype=torch.float32, device="cuda")
    ffi.moe_route(torch.from_numpy(synth.zipf_logits(synth.seed_for("c4", "logits"), t, e)).cuda(), kk, ids=ids,
                  weights=wts)
    ym = torch.empty((t, dm), dtype=torch.float32, device="cuda")
    for scheme, name in names.items():
        gu, gus = ffi.repack(gsynth.quant_weights_gpu(torch, scheme, 511 + scheme, e * 2 * dff, dm), scheme,
                             e * 2 * dff, dm)
        dn, dns = ffi.repack(gsynth.quant_weights_gpu(torch, scheme, 521 + scheme, e * dm, dff), scheme, e * dm, dff)
        st = ffi.ffn_static(t, e, kk, dm, dff, 0, scheme, scheme)
        wsp = torch.empty(ffi.ffn_workspace_bytes(st), dtype=torch.uint8, device="cuda")
        ms, _ = timed_steps(torch, lambda i: ffi.moe_ffn(xm, ids, wts, gu, dn, e, dff, gate_up_scheme=scheme,
                                                         down_scheme=scheme, y=ym, workspace=wsp,
                                                         w_gate_up_scales=gus, w_down_scales=dns), steps, 2)
        out["moe_ffn_c4_shape"][name] = {"ms_per_step": round(ms, 4), **mfma(C4_FLOPS, ms)}
        del gu, gus, dn, dns, wsp
        torch.cuda.empty_cache()
    return out


def c3_extra(torch, ffi, synth, gsynth, steps, cpu_s, steps_only=False):
    """MoE decode: T=5, E=512 routed + 1 shared, top-10; per step the router
    and the FFN over freshly routed tokens (8 routing patterns rotate)."""
    t, e, k, dm, dff, shared = 5, 512, 10, 2048, 512, 1
    pats_host = [synth.normal_f32(synth.seed_for("c3", f"logits{i}"), (t, e)) for i in range(8)]
    pats = [torch.from_numpy(p).cuda() for p in pats_host]
    gu0 = gsynth.quant_weights_gpu(torch, ffi.IQ4_XS, 301, (e + shared) * 2 * dff, dm)
    dn0 = gsynth.quant_weights_gpu(torch, ffi.Q4_K, 302, (e + shared) * dm, dff)
    wsets = [(gu0, dn0)] + [(gu0.clone(), dn0.clone()) for _ in range(6)]
    x_host = synth.normal_bf16(synth.seed_for("c3", "x"), (t, dm))
    x = torch.from_numpy(x_host.view(np.int16)).cuda().view(torch.bfloat16)
    ids = torch.empty((t, k), dtype=torch.int32, device="cuda")
    w = torch.empty((t, k), dtype=torch.float32, device="cuda")
    y = torch.empty((t, dm), dtype=torch.float32, device="cuda")
    st = ffi.ffn_static(t, e, k, dm, dff, shared)
    wsp = torch.empty(ffi.ffn_workspace_bytes(st), dtype=torch.uint8, device="cuda")
    uniq = []
    for p in pats:
        ffi.moe_route(p, k, ids=ids, weights=w)
        uniq.append(len(set(ids.cpu().numpy().reshape(-1).tolist())))

    def step(i, stream=None):
        ffi.moe_route(pats[i % len(pats)], k, ids=ids, weights=w, stream=stream)
        gu, dn = wsets[i % len(wsets)]
        ffi.moe_ffn(x, ids, w, gu, dn, e, dff, shared=shared, y=y, workspace=wsp, t_bucket=t, stream=stream)

    if steps_only:  # a fixed run for counter collection
        for i in range(steps):
            step(i)
        return None
    ms, med = timed_steps(torch, step, max(200, steps), 10)
    # the same steps captured in a HIP graph (56 steps: every routing pattern
    # and weight copy), as a decode loop would replay them
    gms = graph_time(torch, step, len(pats) * len(wsets))
    u = float(np.mean(uniq))
    per_expert = int(ffi.load().r9vx_moe_ffn_expert_bytes(__import__("ctypes").byref(st)))
    bytes_ = (u + shared) * per_expert + t * dm * 2 + t * dm * 4 + t * e * 4
    flops = (t * k + t * shared) * (2 * 2 * dff * dm + 2 * dm * dff)
    out = {"workload": "configs[3]: MoE decode T=5, E=512+1 shared, top-10, IQ4_XS gate/up + Q4_K down "
                       "(route + permute + expert GEMVs + combine per step)",
           "ms_per_step": round(ms, 4), "median_ms_per_step": round(med, 4),
           "graph_ms_per_step": round(gms, 4), "graph_tokens/s": round(t / (gms * 1e-3), 1),
           "graph_hbm_frac": round(bytes_ / (gms * 1e-3) / 8e12, 4), "distinct_experts_mean": u,
           "bytes_per_step": int(bytes_), "tokens/s": round(t / (ms * 1e-3), 1), "flops": flops,
           "weight_copies": len(wsets), **hbm(bytes_, ms)}
    if cpu_s:
        O = oracle()
        gu_h, dn_h = gu0.cpu().numpy(), dn0.cpu().numpy()

        def one():
            rid, rw = O.moe_route(pats_host[0], k)
            O.moe_ffn(x_host, O.BF16, rid, rw, e, dff, gu_h, dn_h, shared=shared)

        calls, el = loop_for(cpu_s, one)
        out["cpu"] = {"GB/s": round(bytes_ * calls / el / 1e9, 4), "tokens/s": round(t * calls / el, 2), "cores": 1,
                      "kind": "port", "sample": f"{calls} whole steps (route + moe_ffn) in {el:.1f} s"}
    del wsets, gu0, dn0
    torch.cuda.empty_cache()
    return out


def ceilings(torch, ffi):
    """Measured ceilings of this device: 128-bit streaming reads at the
    configs' working-set sizes (rotated copies, graph-replayed launches) and
    an MFMA-only loop (fp16 32x32x16)."""
    out = {}
    for label, nbytes in (("5.6MB", 5_693_440), ("9.5MB", 9_469_952), ("84MB", 84 << 20), ("1GB", 1 << 30)):
        nbytes -= nbytes % 16
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1) for _ in range(copies_for(nbytes))]
        ms = graph_time(torch, lambda i, s: ffi.probe_stream(bufs[i % len(bufs)], stream=s), len(bufs), reps=5)
        out[f"stream_{label}"] = {"us": round(ms * 1e3, 2), **hbm(nbytes, ms)}
        del bufs
        torch.cuda.empty_cache()
    blocks, iters = 256 * 8, 256
    sink = torch.empty(blocks * 256, dtype=torch.float32, device="cuda")
    _, ms = timed_steps(torch, lambda i: ffi.probe_mfma(blocks, iters, sink=sink), 5, 2)
    out["mfma_f16_32x32x16"] = {"us": round(ms * 1e3, 1), **mfma(blocks * 4 * iters * 16 * 32768, ms)}
    return out


# ---------------------------------------------------------------- counters

def pmc_case(torch, ffi, synth, gsynth, name):
    """A short fixed run for `rocprofv3 --pmc`: 6 steps of configs[4]
    (moe_ffn), configs[3] (route + moe_ffn) or configs[2] (the dense GEMM),
    200 launches of the configs[1] M=5 / configs[0] GEMV, or (ceil) the
    measured ceilings' MFMA-only loop and 1 GB streaming read --
    the summaries take medians over a kernel's launches, so the first
    launch's cold caches do not count -- then 5 launches of a plain copy
    kernel of known size (torch.neg, f32 -> f32, 64 MiB read + 64 MiB
    written) that calibrate what FETCH_SIZE / WRITE_SIZE report per byte."""
    if name == "c4":
        p = MoePrefill(torch, ffi, synth, gsynth)
        for i in range(6):
            p.step(i)
    elif name == "c3":
        c3_extra(torch, ffi, synth, gsynth, 6, 0, steps_only=True)
    elif name == "c2":
        c2_extra(torch, ffi, synth, gsynth, 6, 0, steps_only=True)
    elif name == "ceil":
        # the measured ceilings' two probes: 5 launches each of the MFMA-only
        # loop and of the 1 GB streaming read
        blocks, iters = 256 * 8, 256
        sink = torch.empty(blocks * 256, dtype=torch.float32, device="cuda")
        for _ in range(5):
            ffi.probe_mfma(blocks, iters, sink=sink)
        buf = torch.empty(1 << 30, dtype=torch.uint8, device="cuda").fill_(1)
        for _ in range(5):
            ffi.probe_stream(buf)
    elif name in ("c1m5", "c0", "gemvn"):
        # 200 GEMV launches over the rotated weight copies (each launch reads
        # its copy from HBM, not the Infinity Cache)
        shape = {"c1m5": (ffi.IQ4_XS, 5120, 2048, 5, ffi.BF16), "c0": (ffi.Q4_K, 4096, 4096, 1, ffi.F32),
                 "gemvn": (ffi.Q4_K, 32768, 4096, 1, ffi.BF16)}[name]
        b = Gemv(torch, ffi, synth, *shape, name)
        for i in range(200):
            b.launch(i)
    else:
        raise SystemExit(f"unknown --pmc-case {name!r} (known: c0, c1m5, gemvn, c2, c3, c4, ceil)")
    torch.cuda.synchronize()
    src = torch.ones(PMC_COPY_BYTES // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(5):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    print(json.dumps({"pmc_case": name, "steps": 6, "copy_bytes_read": PMC_COPY_BYTES,
                      "copy_bytes_written": PMC_COPY_BYTES}))


def pmc_summary(dirs, kernels=None):
    """Medians of FETCH_SIZE / WRITE_SIZE (KiB per dispatch) from rocprofv3
    counter-collection output of `--pmc-case` runs, each scaled by the copy
    kernel's reading of its known byte count: the headline kernel, or each
    kernel whose name contains one of `kernels`."""
    import csv
    import glob
    import sqlite3

    per = {}
    for d in dirs:
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                per.setdefault((r["Counter_Name"], r["Kernel_Name"]), []).append(float(r["Counter_Value"]))
        for f in glob.glob(os.path.join(d, "**", "*_results.db"), recursive=True):
            c = sqlite3.connect(f)
            for cn, kn, v in c.execute("select counter_name, kernel_name, value from counters_collection"):
                per.setdefault((cn, kn), []).append(float(v))

    def find(counter, pred):
        return [x for (c, k), v in per.items() if c == counter and pred(k) for x in v]

    head = HEAD_KERNEL.split("<")[0]
    targets = [(k, lambda name, k=k: k in name) for k in kernels] if kernels else \
        [(HEAD_KERNEL, lambda name: head in name and "<15>" in name)]
    lines = ["counter      kernel                                      dispatches   median KiB/dispatch"]
    for label, pred in targets:
        out = {}
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            g = find(counter, pred)
            c = find(counter, lambda k: "neg_kernel" in k or ("elementwise" in k and "neg" in k.lower()))
            if not g or not c:
                lines.append(f"{counter:12s} (missing: {label} {len(g)} / copy {len(c)} dispatches)")
                continue
            gm, cm = statistics.median(g), statistics.median(c)
            factor = PMC_COPY_BYTES / (cm * 1024.0)
            out[counter] = gm * 1024.0 * factor
            lines.append(f"{counter:12s} {label[:43]:43s} {len(g):10d}   {gm:12.1f}")
            lines.append(f"{counter:12s} {'copy (torch.neg 64 MiB f32)':43s} {len(c):10d}   {cm:12.1f}")
            lines.append(f"{counter:12s} calibration factor = {PMC_COPY_BYTES} B / ({cm:.1f} KiB * 1024) = {factor:.4f}")
        if len(out) == 2:
            tag = "" if not kernels else f"{label} "
            lines.append(f"{tag}fetch_bytes_per_launch: {out['FETCH_SIZE']:.0f}")
            lines.append(f"{tag}write_bytes_per_launch: {out['WRITE_SIZE']:.0f}")
            lines.append(f"{tag}traffic_bytes_per_launch: {out['FETCH_SIZE'] + out['WRITE_SIZE']:.0f}")
    print("\n".join(lines))


def clock_summary(kt_dir, pmc_dir, kernels):
    """Each kernel's median duration (a `rocprofv3 --kernel-trace` run) and
    median GRBM_GUI_ACTIVE (a `--pmc GRBM_GUI_ACTIVE` run of the same
    workload), and from them the mean shader clock while it ran: the counter
    adds up the busy GPU clocks of the 8 XCDs, so clock = counter / 8 /
    duration.  The counter's window also covers the dispatch's start and
    drain, so for launches of a few microseconds the figure overstates the
    clock; for the long GEMM launches it is the clock."""
    import glob
    import re
    import sqlite3

    def short(name):
        name = name.replace("(anonymous namespace)::", "")
        m = re.search(r"(\w+(<[^>]*>)?)\(", name)
        return m.group(1) if m else name[:48]

    dur, grbm = {}, {}
    for f in glob.glob(os.path.join(kt_dir, "**", "*_results.db"), recursive=True):
        for n, d in sqlite3.connect(f).execute("select name, duration from kernels"):
            dur.setdefault(short(n), []).append(float(d))
    for f in glob.glob(os.path.join(pmc_dir, "**", "*_results.db"), recursive=True):
        q = "select counter_name, kernel_name, value from counters_collection"
        for cn, kn, v in sqlite3.connect(f).execute(q):
            if cn == "GRBM_GUI_ACTIVE":
                grbm.setdefault(short(kn), []).append(float(v))
    lines = ["kernel                                    dispatches  median_us  GRBM_GUI_ACTIVE  clock_GHz"]
    for k in sorted(dur, key=lambda k: -statistics.median(dur[k]) * len(dur[k])):
        if kernels and not any(s in k for s in kernels):
            continue
        if k not in grbm:
            continue
        d_us = statistics.median(dur[k]) / 1e3
        g = statistics.median(grbm[k])
        lines.append(f"{k[:41]:41s} {len(dur[k]):10d} {d_us:10.2f} {g:16.0f} {g / 8 / (d_us * 1e3):10.3f}")
    print("\n".join(lines))


def read_traffic():
    try:
        for line in open(TRAFFIC_FILE):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


# ---------------------------------------------------------------- main

def main():
    args = parse()
    if args.pmc_summary is not None:
        pmc_summary(args.pmc_summary, [k for k in args.pmc_kernels.split(",") if k] or None)
        return 0
    if args.clock_summary:
        clock_summary(args.clock_summary[0], args.clock_summary[1], [k for k in args.pmc_kernels.split(",") if k])
        return 0
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: multi-GPU figures are out of scope, "
                                   "run with --gpus 1"}))
        return 2
    import torch

    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import gpu_synth as gsynth

    from r9v_amd import ffi, synth

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU"}))
        return 1
    ffi.load()
    if args.pmc_case:
        pmc_case(torch, ffi, synth, gsynth, args.pmc_case)
        return 0
    only = set(filter(None, args.only.split(",")))
    cpu_s = 0.0 if args.no_cpu else args.cpu_budget

    def want(name):
        return not only or name in only

    log("c4: MoE prefill T=8192 E=512 top-10")
    head = MoePrefill(torch, ffi, synth, gsynth)
    ms, med = timed_steps(torch, head.step, args.steps, args.warmup)
    value = C4_FLOPS / (ms * 1e-3) / 1e12
    stages = {name: head.stage_ms(st) for name, st in (("gate_up_gemm", 1), ("down_gemm", 2), ("combine", 3))}
    gu_ms = stages["gate_up_gemm"]
    gu_tf = C4_GU_FLOPS / (gu_ms * 1e-3) / 1e12
    log(f"  {ms:.4f} ms/step ({value:.1f} TFLOP/s), median {med:.4f}; stages {stages}")

    cpu = None
    extras = {"c4_stage_ms": {k: round(v, 4) for k, v in stages.items()}}
    if cpu_s:
        tf1, pairs, nexp, el = head.cpu_sample(cpu_s, 1)
        cpu = {"value": round(tf1, 6), "unit": "TFLOP/s", "cores": 1, "kind": "port",
               "sample": f"the oracle's per-expert sliced T0 moe_ffn body (gather, gate/up, SiLU*up, down; 1 thread) "
                         f"on experts 0.. in id order of the configs[4] routing: {nexp} experts, {pairs} (token, "
                         f"expert) pairs in {el:.1f} s, extrapolated per FLOP to the whole step; {host_cpu()}"}
        nt = cpu_threads()
        tfn, pairs_n, nexp_n, el_n = head.cpu_sample(cpu_s, nt)
        extras["c4_cpu_all_threads"] = {"TFLOP/s": round(tfn, 6), "cores": nt, "kind": "port",
                                        "sample": f"the same body with each expert's rows split over {nt} OpenMP "
                                                  f"threads: {nexp_n} experts, {pairs_n} pairs in {el_n:.1f} s"}
        log(f"  cpu 1 thread {tf1:.6f} TFLOP/s, {nt} threads {tfn:.6f} TFLOP/s")
    del head
    torch.cuda.empty_cache()

    if want("c1"):
        log("c1 ...")
        extras["c1_iq4xs_gemv_m5"] = gemv_extra(torch, ffi, synth, ffi.IQ4_XS, 5120, 2048, 5, ffi.BF16, "c1m5", cpu_s,
                                                "configs[1]: IQ4_XS GEMV K=2048 N=5120 M=5, x bf16, y f32")
        extras["c1_iq4xs_gemv_m1"] = gemv_extra(torch, ffi, synth, ffi.IQ4_XS, 5120, 2048, 1, ffi.BF16, "c1m1", 0,
                                                "configs[1]: IQ4_XS GEMV K=2048 N=5120 M=1, x bf16, y f32")
        log(f"  {extras['c1_iq4xs_gemv_m5']}")
    if want("c0"):
        log("c0 ...")
        extras["c0_q4k_gemv_f32"] = gemv_extra(torch, ffi, synth, ffi.Q4_K, 4096, 4096, 1, ffi.F32, "c0", cpu_s,
                                               "configs[0]: Q4_K GEMV 4096x4096, x f32, y f32")
        log(f"  {extras['c0_q4k_gemv_f32']}")
    if want("gemv_n"):
        log("gemv large N ...")
        extras["gemv_q4k_32768x4096_m1"] = gemv_extra(torch, ffi, synth, ffi.Q4_K, 32768, 4096, 1, ffi.BF16, "gemvN", 0,
                                                      "Q4_K GEMV N=32768 K=4096 M=1, x bf16, y f32 (75.5 MB of weights: "
                                                      "the GEMV's steady streaming rate)")
        log(f"  {extras['gemv_q4k_32768x4096_m1']}")
    if want("c2"):
        log("c2 ...")
        extras["c2"] = c2_extra(torch, ffi, synth, gsynth, args.steps, cpu_s)
        log(f"  {extras['c2']}")
    if want("c3"):
        log("c3 ...")
        extras["c3"] = c3_extra(torch, ffi, synth, gsynth, args.steps, cpu_s)
        log(f"  {extras['c3']}")
    if want("schemes"):
        log("Q8_0 / Q6_K / IQ3_S at the configs[2] and configs[4] shapes ...")
        extras["other_schemes"] = schemes_extra(torch, ffi, synth, gsynth, 5)
        log(f"  {extras['other_schemes']}")
    if want("ceilings"):
        extras["measured_ceilings"] = ceilings(torch, ffi)
        log(f"  ceilings {extras['measured_ceilings']}")

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic: seeded Zipf(1.1) router logits (routed once, not timed), x ~ N(0,1) bf16, GGUF IQ4_XS "
                "gate/up and Q4_K down experts (uniform quants and 6-bit scales, d = f16|N(0,0.02)|, dmin = "
                "f16|N(0,0.01)|)",
        "config": {"workload": "configs[4]: MoE prefill grouped GEMM, T=8192 tokens, E=512 experts, top-10, hidden "
                               "2048, expert width 512; one moe_ffn launch per step (permute, gate/up GEMM + SwiGLU, "
                               "down GEMM, weighted unpermute-sum to f32)",
                   "tokens": C4_T, "experts": C4_E, "top_k": C4_K, "dm": C4_DM, "dff": C4_DFF,
                   "flops_per_step": C4_FLOPS, "median_ms_per_step": round(med, 6),
                   "tokens_per_s": round(C4_T / (ms * 1e-3), 1), "weight_copies": 2,
                   "arithmetic": "fp16 MFMA operands (bf16 activations and SwiGLU rows scaled per row by a power "
                                 "of two, weights decoded by the f32 formula rounded once to fp16; Q4_K up to the f32 rounding of a "
                                 "precomputed addend), f32 accumulate; "
                                 "expert output rows kept as fp16 scaled by a power of two per (row, 64 columns) "
                                 "until the f32 weighted sum",
                   "parallelism": "single GPU",
                   "timing": "K steps between device synchronisations; HIP events per step for the median"},
        "roofline": {"bound": "mfma", "achieved": round(gu_tf, 1), "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(gu_tf / MFMA_PEAK_TFLOPS, 4), "traffic": read_traffic(), "kernel": HEAD_KERNEL,
                     "flops_per_launch": C4_GU_FLOPS, "ms_per_launch": round(gu_ms, 5),
                     "timing": "median of 20 relaunches of the gate/up stage (r9vx_probe_moe_stage_launch), HIP "
                               "events on its stream"},
        "cpu_baseline": cpu,
        "extras": extras,
    }
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
