#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-weight matrix path (one GPU).

Headline: the IQ4_XS dequant-fused GEMV at
K=2048, N=5120, M=5 (1 + 4 MTP draft tokens), bf16 x, f32 y.  A step is one
GEMV launch over one batch; the weights rotate through enough distinct copies
(>= 2x the 256 MB Infinity Cache) that every step reads them from HBM.  The K
timed steps are captured in one HIP graph and replayed once between two
device synchronisations; `value` = algorithmic bytes per step / time per
step, every input resident in HBM.  `roofline` is the same kernel's
per-launch figure; `roofline.traffic` is the HBM bytes per launch that the
FETCH_SIZE / WRITE_SIZE counters report (calibrated on a copy kernel of known
size), read from the committed counter summary when it is present.

`extras` carries the other configs with their own roofline figures:
configs[0] Q4_K GEMV (HBM), configs[2] dense dequant-GEMM (MFMA),
configs[3] MoE decode (HBM), configs[4] MoE prefill grouped GEMM (MFMA),
plus the router on its own.  `cpu_baseline` times the oracle (a scalar C
restatement of R9V's T0 Branch-D path) on a bounded sample of the headline
workload on this host.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only c0,c2,...]
    python bench.py --pmc-case c1m5          # short fixed run for rocprofv3 --pmc
    python bench.py --pmc-summary DIR ...    # FETCH_SIZE/WRITE_SIZE dirs -> traffic text
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0  # dense bf16/fp16 MFMA, MI355X
IC_BYTES = 256 << 20
METRIC = "quant GEMV/MoE HBM GB/s (% of peak); prefill grouped-GEMM TFLOP/s (% MFMA)"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default="",
                    help="comma list of extras: c0,c1m1,c2,c3,c4,ceilings; 'paths' (not run by default) times "
                         "the Q6_K / Q8_0, SwiGLU and fused-router paths")
    ap.add_argument("--pmc-case", default="", help="run a short fixed workload for counter collection: c1m5")
    ap.add_argument("--pmc-summary", nargs="*", default=None,
                    help="rocprofv3 --pmc output dirs (FETCH_SIZE, WRITE_SIZE) to summarise as traffic")
    return ap.parse_args()


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def copies_for(nbytes):
    return max(2, -(-2 * IC_BYTES // max(nbytes, 1)))


def event_time(torch, fn, steps, warmup):
    """ms per call over `steps` calls, events on the launch stream."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(steps):
        fn()
    e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def graph_time(torch, fn, launches, reps=20):
    """ms per launch of `launches` back-to-back calls captured in a HIP graph."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
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
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(cur)
    for _ in range(reps):
        g.replay()
    e1.record(cur)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (reps * launches)


def graph_steps(torch, fn, steps, warmup):
    """ms per step of `steps` calls fn(i, stream) captured in one HIP graph:
    `warmup` eager calls and one untimed replay first, then one replay timed
    between two device synchronisations (events on the replay stream)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(max(warmup, 1)):
            fn(i, s)
        s.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for i in range(steps):
                fn(i, s)
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    cur = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(cur)
    g.replay()
    e1.record(cur)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def hbm(bytes_, ms):
    gbs = bytes_ / (ms * 1e-3) / 1e9
    return {"GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}


def mfma(flops, ms):
    tf = flops / (ms * 1e-3) / 1e12
    return {"TFLOP/s": round(tf, 1), "frac_mfma": round(tf / MFMA_PEAK_TFLOPS, 4)}


class Gemv:
    def __init__(self, torch, ffi, synth, gsynth, scheme, n, k, m, x_dtype, tag):
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
        self.i = 0

    def launch(self, i=None, stream=None):
        if i is None:
            i, self.i = self.i, self.i + 1
        self.ffi.matmul(self.ws[i % len(self.ws)], self.scheme, self.n, self.k, self.x, y=self.y, stream=stream)

    def graph_ms(self):
        return graph_time(self.torch, lambda i, s: self.launch(i, s), len(self.ws))

    def cpu_baseline(self, budget_s=12.0):
        sys.path.insert(0, os.path.join(ROOT, "tests"))
        import oracle_ffi as O

        calls, t0 = 0, time.perf_counter()
        while True:
            O.matmul(self.scheme, self.w_host, self.n, self.k, self.x_host, self.x_dtype)
            calls += 1
            el = time.perf_counter() - t0
            if el >= budget_s:
                break
        return self.bytes * calls / el / 1e9, calls, el


def bench_c2(torch, ffi, synth, gsynth, steps):
    m, n, k = 2048, 14336, 4096
    w0 = gsynth.quant_weights_gpu(torch, ffi.Q4_K, 201, n, k)
    ws = [w0] + [w0.clone() for _ in range(copies_for(w0.numel()) - 1)]
    x = torch.from_numpy(synth.normal_bf16(synth.seed_for("c2", "x"), (m, k)).view(np.int16)).cuda().view(torch.bfloat16)
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    st = ffi.matmul_static(n, k, ffi.Q4_K, ffi.BF16, ffi.BF16, m_bucket=m)
    wsp = torch.empty(ffi.matmul_workspace_bytes(st), dtype=torch.uint8, device="cuda")
    it = [0]

    def step():
        ffi.matmul(ws[it[0] % len(ws)], ffi.Q4_K, n, k, x, out_dtype=ffi.BF16, y=y, workspace=wsp)
        it[0] += 1

    ms = event_time(torch, step, steps, 3)
    flops = 2 * m * n * k
    out = {"workload": "configs[2]: x bf16 [2048x4096] . Q4_K [14336x4096]^T -> bf16, fp16 MFMA",
           "ms_per_step": round(ms, 4), "tokens/s": round(m / (ms * 1e-3), 1), "flops": flops,
           "weight_copies": len(ws)}
    out.update(mfma(flops, ms))
    return out


def moe_weights(torch, gsynth, ffi, e, dm, dff, seed, copies):
    gu = gsynth.quant_weights_gpu(torch, ffi.IQ4_XS, seed, e * 2 * dff, dm)
    dn = gsynth.quant_weights_gpu(torch, ffi.Q4_K, seed + 1, e * dm, dff)
    return [(gu, dn)] + [(gu.clone(), dn.clone()) for _ in range(copies - 1)]


def bench_c3(torch, ffi, synth, gsynth, steps):
    """MoE decode: T=5, E=512 routed + 1 shared, top-10; per step the router
    and the FFN over freshly routed tokens (8 routing patterns rotate)."""
    t, e, k, dm, dff, shared = 5, 512, 10, 2048, 512, 1
    per_expert = 2 * dff * dm // 256 * 136 + dm * dff // 256 * 144
    pats = [torch.from_numpy(synth.normal_f32(synth.seed_for("c3", f"logits{i}"), (t, e))).cuda() for i in range(8)]
    # working set per step ~ (U+1) experts; rotate copies so it misses the Infinity Cache
    wsets = moe_weights(torch, gsynth, ffi, e + shared, dm, dff, 301, 7)
    x = torch.from_numpy(synth.normal_bf16(synth.seed_for("c3", "x"), (t, dm)).view(np.int16)).cuda().view(torch.bfloat16)
    ids = torch.empty((t, k), dtype=torch.int32, device="cuda")
    w = torch.empty((t, k), dtype=torch.float32, device="cuda")
    y = torch.empty((t, dm), dtype=torch.float32, device="cuda")
    st = ffi.ffn_static(t, e, k, dm, dff, shared)
    wsp = torch.empty(ffi.ffn_workspace_bytes(st), dtype=torch.uint8, device="cuda")
    uniq = []
    for p in pats:
        ffi.moe_route(p, k, ids=ids, weights=w)
        uniq.append(len(set(ids.cpu().numpy().reshape(-1).tolist())))
    it = [0]

    def ffn_step():
        i = it[0]
        it[0] += 1
        ffi.moe_route(pats[i % len(pats)], k, ids=ids, weights=w)
        gu, dn = wsets[i % len(wsets)]
        ffi.moe_ffn(x, ids, w, gu, dn, e, dff, shared=shared, y=y, workspace=wsp, t_bucket=t)

    ms = event_time(torch, ffn_step, steps, 10)
    u = float(np.mean(uniq))
    bytes_ = (u + shared) * per_expert + t * dm * 2 + t * dm * 4 + t * e * 4
    flops = (t * k + t * shared) * (2 * 2 * dff * dm + 2 * dm * dff)
    out = {"workload": "configs[3]: MoE decode T=5, E=512+1 shared, top-10, IQ4_XS gate/up + Q4_K down "
                       "(route + permute + expert GEMVs + combine per step)",
           "ms_per_step": round(ms, 4), "distinct_experts_mean": u, "bytes_per_step": int(bytes_),
           "tokens/s": round(t / (ms * 1e-3), 1), "flops": flops, "weight_copies": len(wsets)}
    out.update(hbm(bytes_, ms))
    return out


def bench_c4(torch, ffi, synth, gsynth, steps):
    """MoE prefill: T=8192, E=512, top-10, Zipf(1.1) routing."""
    t, e, k, dm, dff = 8192, 512, 10, 2048, 512
    logits = torch.from_numpy(synth.zipf_logits(synth.seed_for("c4", "logits"), t, e)).cuda()
    wsets = moe_weights(torch, gsynth, ffi, e, dm, dff, 401, 2)
    x = torch.from_numpy(synth.normal_bf16(synth.seed_for("c4", "x"), (t, dm)).view(np.int16)).cuda().view(torch.bfloat16)
    ids = torch.empty((t, k), dtype=torch.int32, device="cuda")
    w = torch.empty((t, k), dtype=torch.float32, device="cuda")
    y = torch.empty((t, dm), dtype=torch.float32, device="cuda")
    st = ffi.ffn_static(t, e, k, dm, dff)
    wsp = torch.empty(ffi.ffn_workspace_bytes(st), dtype=torch.uint8, device="cuda")
    ffi.moe_route(logits, k, ids=ids, weights=w)
    it = [0]

    def ffn_step():
        gu, dn = wsets[it[0] % len(wsets)]
        it[0] += 1
        ffi.moe_ffn(x, ids, w, gu, dn, e, dff, y=y, workspace=wsp)

    def route_step():
        ffi.moe_route(logits, k, ids=ids, weights=w)

    ms = event_time(torch, ffn_step, steps, 2)
    rms = event_time(torch, route_step, steps, 2)
    flops = t * k * (2 * 2 * dff * dm + 2 * dm * dff)
    out = {"workload": "configs[4]: MoE prefill T=8192, E=512, top-10 Zipf(1.1); permute + grouped fp16-MFMA "
                       "gate/up+SwiGLU and down + weighted unpermute-sum to f32",
           "ms_per_step": round(ms, 4), "tokens/s": round(t / (ms * 1e-3), 1), "flops": flops,
           "route_ms": round(rms, 4), "route_GB/s": round(t * e * 4 / (rms * 1e-3) / 1e9, 1)}
    out.update(mfma(flops, ms))
    return out


def bench_paths(torch, ffi, synth):
    """The paths beyond configs[0..4], timed at their documented shapes (run
    with --only paths; not part of the default run): Q6_K / Q8_0 decode GEMVs
    and prefill GEMMs on the split layout, IQ3_S ones on its 112-byte blocks, the gated (SwiGLU) GEMV over
    stacked gate/up rows, and routing from hidden states."""
    out = {}

    def weights(scheme, rows, k, seed, copies):
        wire = torch.from_numpy(synth.quant_weights(scheme, seed, rows, k)).cuda()
        if scheme in ffi.SPLIT_SCHEMES:
            body, scales = ffi.repack(wire, scheme, rows, k)
            return [(body, scales)] + [(body.clone(), scales.clone()) for _ in range(copies - 1)]
        if scheme == ffi.IQ3_S:  # the 112-byte device blocks
            body, _ = ffi.repack(wire, scheme, rows, k)
            return [(body, None)] + [(body.clone(), None) for _ in range(copies - 1)]
        return [(wire, None)] + [(wire.clone(), None) for _ in range(copies - 1)]

    def wbytes(scheme, rows, k):
        bb = ffi.IQ3S_DEV_BYTES if scheme == ffi.IQ3_S else ffi.BLOCK_BYTES[scheme]
        return rows * (k // ffi.BLOCK_LEN[scheme]) * bb

    for name, scheme, n, k, m in (("q6k_head_gemv", ffi.Q6_K, 32768, 4096, 1),
                                  ("q8_0_proj_gemv", ffi.Q8_0, 14336, 4096, 1),
                                  ("q6k_gemv_c1shape", ffi.Q6_K, 5120, 2048, 1),
                                  ("iq3s_proj_gemv", ffi.IQ3_S, 14336, 4096, 1),
                                  ("iq3s_gemv_c1shape", ffi.IQ3_S, 5120, 2048, 1)):
        nb = wbytes(scheme, n, k)
        ws = weights(scheme, n, k, 11, copies_for(nb))
        x = torch.from_numpy(synth.normal_bf16(3, (m, k)).view(np.int16)).cuda().view(torch.bfloat16)
        y = torch.empty((m, n), dtype=torch.float32, device="cuda")
        ms = graph_time(torch, lambda i, s: ffi.matmul(ws[i % len(ws)][0], scheme, n, k, x, y=y, stream=s,
                                                       w_scales=ws[i % len(ws)][1]), len(ws))
        out[name] = {"n": n, "k": k, "m": m, "us_per_launch": round(ms * 1e3, 2), **hbm(nb, ms)}
        log(f"  {name} {out[name]}")
        del ws
        torch.cuda.empty_cache()
    for mm in (1, 4):
        n, k = 14336, 4096
        nb = wbytes(ffi.Q4_K, 2 * n, k)
        ws = weights(ffi.Q4_K, 2 * n, k, 12, copies_for(nb))
        x = torch.from_numpy(synth.normal_bf16(4, (mm, k)).view(np.int16)).cuda().view(torch.bfloat16)
        y = torch.empty((mm, n), dtype=torch.float32, device="cuda")
        ms = graph_time(torch, lambda i, s: ffi.matmul(ws[i % len(ws)][0], ffi.Q4_K, n, k, x, y=y, stream=s,
                                                       swiglu=True), len(ws))
        out[f"swiglu_gemv_m{mm}"] = {"dff": n, "k": k, "m": mm, "us_per_launch": round(ms * 1e3, 2), **hbm(nb, ms)}
        log(f"  swiglu m{mm} {out[f'swiglu_gemv_m{mm}']}")
        del ws
        torch.cuda.empty_cache()
    for name, scheme in (("q6k_prefill_gemm", ffi.Q6_K), ("q8_0_prefill_gemm", ffi.Q8_0),
                         ("iq3s_prefill_gemm", ffi.IQ3_S)):
        m, n, k = 2048, 14336, 4096
        (w, sc), = weights(scheme, n, k, 13, 1)
        x = torch.from_numpy(synth.normal_bf16(5, (m, k)).view(np.int16)).cuda().view(torch.bfloat16)
        y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
        st = ffi.matmul_static(n, k, scheme, ffi.BF16, ffi.BF16, m_bucket=m)
        wsp = torch.empty(ffi.matmul_workspace_bytes(st), dtype=torch.uint8, device="cuda")
        ms = event_time(torch, lambda: ffi.matmul(w, scheme, n, k, x, out_dtype=ffi.BF16, y=y, workspace=wsp,
                                                  w_scales=sc), 10, 3)
        out[name] = {"m": m, "n": n, "k": k, "ms": round(ms, 4), **mfma(2 * m * n * k, ms)}
        log(f"  {name} {out[name]}")
        del w, sc
        torch.cuda.empty_cache()
    t, e, dm, kk = 5, 512, 2048, 10
    x = torch.from_numpy(synth.normal_bf16(6, (t, dm)).view(np.int16)).cuda().view(torch.bfloat16)
    wr = ffi.router_repack(torch.from_numpy(synth.normal_f32(7, (e, dm), 0.05)).cuda())
    ids = torch.empty((t, kk), dtype=torch.int32, device="cuda")
    wt = torch.empty((t, kk), dtype=torch.float32, device="cuda")
    _, _, rws = ffi.moe_route_hidden(x, wr, kk, ids=ids, weights=wt, e=e)
    ms = graph_time(torch, lambda i, s: ffi.moe_route_hidden(x, wr, kk, ids=ids, weights=wt, workspace=rws, e=e,
                                                            stream=s), 50)
    out["route_hidden_t5"] = {"t": t, "e": e, "dm": dm, "k": kk, "us_per_launch": round(ms * 1e3, 2)}
    log(f"  route_hidden {out['route_hidden_t5']}")
    return out


def bench_ceilings(torch, ffi):
    """Measured ceilings of this device: 128-bit streaming reads at the
    configs' working-set sizes (rotated copies, graph-replayed launches) and
    an MFMA-only loop (fp16 32x32x16)."""
    out = {}
    for label, nbytes in (("5.6MB", 5_693_440), ("9.5MB", 9_469_952), ("84MB", 84 << 20), ("1GB", 1 << 30)):
        nbytes -= nbytes % 16
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1) for _ in range(copies_for(nbytes))]
        ms = graph_time(torch, lambda i, s: ffi.probe_stream(bufs[i % len(bufs)], stream=s), len(bufs), reps=10)
        out[f"stream_{label}"] = {"us": round(ms * 1e3, 2), **hbm(nbytes, ms)}
        del bufs
    blocks, iters = 256 * 8, 256
    sink = torch.empty(blocks * 256, dtype=torch.float32, device="cuda")
    ms = event_time(torch, lambda: ffi.probe_mfma(blocks, iters, sink=sink), 5, 2)
    flops = blocks * 4 * iters * 16 * 32768
    out["mfma_f16_32x32x16"] = {"us": round(ms * 1e3, 1), **mfma(flops, ms)}
    return out


HEAD_KERNEL = "gemv_kernel<23, 5, false, 1, 6, 5, 1>"  # IQ4_XS (type 23), M = 5, bf16 x, 1 chunk per lane, 64 lanes per row, 5 rows per lane group, one K segment
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemv_iq4xs_k2048_n5120_m5_traffic.txt")
PMC_COPY_BYTES = 64 << 20


def pmc_case(torch, ffi, synth, gsynth, name):
    """A short fixed run for `rocprofv3 --pmc`: 200 headline GEMV launches over
    rotated weight copies (the summary takes the median, so the first
    launches' write-back of the copies' dirty cache lines does not count),
    then 5 launches of a plain copy kernel of known size (torch.neg, f32 ->
    f32, 64 MiB read + 64 MiB written) that calibrate what FETCH_SIZE /
    WRITE_SIZE report per byte."""
    if name != "c1m5":
        raise SystemExit(f"unknown --pmc-case {name!r} (known: c1m5)")
    head = Gemv(torch, ffi, synth, gsynth, ffi.IQ4_XS, 5120, 2048, 5, ffi.BF16, "c1m5")
    for i in range(200):
        head.launch(i)
    src = torch.ones(PMC_COPY_BYTES // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(5):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    print(json.dumps({"pmc_case": name, "gemv_launches": 200, "bytes_per_launch": head.bytes,
                      "copy_bytes_read": PMC_COPY_BYTES, "copy_bytes_written": PMC_COPY_BYTES}))


def pmc_summary(dirs):
    """Medians of FETCH_SIZE / WRITE_SIZE (KiB per dispatch) from rocprofv3
    counter-collection CSVs of `--pmc-case c1m5` runs, each scaled by the
    copy kernel's reading of its known byte count."""
    import csv
    import glob
    import statistics

    per = {}
    for d in dirs:
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                key = (r["Counter_Name"], r["Kernel_Name"])
                per.setdefault(key, []).append(float(r["Counter_Value"]))
    def find(counter, pred):
        vals = [v for (c, k), v in per.items() if c == counter and pred(k)]
        return [x for v in vals for x in v]
    lines = ["counter      kernel                                      dispatches   median KiB/dispatch"]
    out = {}
    for counter, copy_bytes in (("FETCH_SIZE", PMC_COPY_BYTES), ("WRITE_SIZE", PMC_COPY_BYTES)):
        g = find(counter, lambda k: HEAD_KERNEL.split("<")[0] in k and HEAD_KERNEL.split("<")[1][:6] in k)
        c = find(counter, lambda k: "neg_kernel" in k or ("vectorized_elementwise_kernel" in k and "neg" in k.lower()))
        if not g or not c:
            lines.append(f"{counter:12s} (missing: headline {len(g)} / copy {len(c)} dispatches)")
            continue
        gm, cm = statistics.median(g), statistics.median(c)
        factor = copy_bytes / (cm * 1024.0)
        out[counter] = gm * 1024.0 * factor
        lines.append(f"{counter:12s} {HEAD_KERNEL:43s} {len(g):10d}   {gm:12.1f}")
        lines.append(f"{counter:12s} {'copy (torch.neg 64 MiB f32)':43s} {len(c):10d}   {cm:12.1f}")
        lines.append(f"{counter:12s} calibration factor = {copy_bytes} B / ({cm:.1f} KiB * 1024) = {factor:.4f}")
    if len(out) == 2:
        lines.append(f"fetch_bytes_per_launch: {out['FETCH_SIZE']:.0f}")
        lines.append(f"write_bytes_per_launch: {out['WRITE_SIZE']:.0f}")
        lines.append(f"traffic_bytes_per_launch: {out['FETCH_SIZE'] + out['WRITE_SIZE']:.0f}")
    print("\n".join(lines))


def host_cpu():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return f"{line.split(':', 1)[1].strip()} ({os.cpu_count()} logical CPUs visible)"
    except OSError:
        pass
    return "unknown host CPU"


def read_traffic():
    try:
        for line in open(TRAFFIC_FILE):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def main():
    args = parse()
    if args.pmc_summary is not None:
        pmc_summary(args.pmc_summary)
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

    def want(name):
        if name == "paths":  # only when asked for
            return name in only
        return not only or name in only

    log("c1 m5: IQ4_XS GEMV K=2048 N=5120 M=5")
    head = Gemv(torch, ffi, synth, gsynth, ffi.IQ4_XS, 5120, 2048, 5, ffi.BF16, "c1m5")
    ms = graph_steps(torch, lambda i, s: head.launch(i, s), args.steps, args.warmup)
    value = head.bytes / (ms * 1e-3) / 1e9
    eager_ms = event_time(torch, head.launch, min(args.steps, 500), 20)
    log(f"  {ms * 1e3:.2f} us/step graph-replayed ({value:.0f} GB/s), {eager_ms * 1e3:.2f} us/step eager")

    extras = {}
    if want("c1m1"):
        b = Gemv(torch, ffi, synth, gsynth, ffi.IQ4_XS, 5120, 2048, 1, ffi.BF16, "c1m1")
        gm = b.graph_ms()
        extras["c1_iq4xs_gemv_m1"] = {"us_per_launch": round(gm * 1e3, 3), "bytes": b.bytes, **hbm(b.bytes, gm)}
        del b
    if want("c0"):
        b = Gemv(torch, ffi, synth, gsynth, ffi.Q4_K, 4096, 4096, 1, ffi.F32, "c0")
        gm = b.graph_ms()
        extras["c0_q4k_gemv_f32"] = {"us_per_launch": round(gm * 1e3, 3), "bytes": b.bytes, **hbm(b.bytes, gm)}
        del b
    if want("ceilings"):
        extras["measured_ceilings"] = bench_ceilings(torch, ffi)
        log(f"  ceilings {extras['measured_ceilings']}")
    if want("paths"):
        log("other paths ...")
        extras["paths"] = bench_paths(torch, ffi, synth)
    for name, fn, st in (("c2", bench_c2, 20), ("c3", bench_c3, 200), ("c4", bench_c4, 10)):
        if want(name):
            log(f"{name} ...")
            extras[name] = fn(torch, ffi, synth, gsynth, st)
            log(f"  {extras[name]}")
            torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu:
        v, calls, el = head.cpu_baseline()
        cpu = {"value": round(v, 4), "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": f"{calls} full configs[1] M=5 GEMVs by the oracle (scalar C restatement of T0 "
                         f"Branch D, 1 thread) in {el:.1f} s on {host_cpu()}"}

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded GGUF IQ4_XS blocks (uniform 4-bit indices / 6-bit scales, "
                "d = f16|N(0,0.02)|), x ~ N(0,1) bf16",
        "config": {"workload": "configs[1]: IQ4_XS dequant GEMV K=2048 N=5120 M=5, x bf16, y f32",
                   "weight_copies": len(head.ws), "parallelism": "single GPU",
                   "timing": "K steps in one HIP graph, one replay between device synchronisations",
                   "eager_us_per_step": round(eager_ms * 1e3, 3)},
        "roofline": {"bound": "hbm", "achieved": round(value, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / HBM_PEAK_GBS, 4), "traffic": read_traffic(),
                     "kernel": HEAD_KERNEL, "bytes_per_launch": head.bytes,
                     "us_per_launch": round(ms * 1e3, 3),
                     "measured_ceiling": extras.get("measured_ceilings", {}).get("stream_5.6MB")},
        "cpu_baseline": cpu,
        "extras": extras,
    }
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
