#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-weight matrix path (one GPU).

Headline: IQ4_XS dequant-fused GEMV, K=2048,
N=5120, M=5 (1 + 4 MTP draft tokens), bf16 x, f32 y.  A step is one GEMV over
one batch; weights rotate through enough distinct copies (>= 2x the 256 MB
Infinity Cache) that every step reads them from HBM.  value = algorithmic
bytes / wall time of the K timed steps, inputs resident in HBM.

The other configs are reported in `extras` with their own roofline figures.
The CPU baseline times the oracle (a scalar restatement of R9V's T0 path) on
a bounded sample of the same workload on this host.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
IC_BYTES = 256 << 20
METRIC = "quant GEMV/MoE HBM GB/s (% of peak); prefill grouped-GEMM TFLOP/s (% MFMA)"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default="", help="comma list of extras to run (c0,c1m1)")
    return ap.parse_args()


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class GemvBench:
    """One dense GEMV workload with rotated weight copies."""

    def __init__(self, torch, ffi, synth, scheme, n, k, m, x_dtype, seed):
        self.torch, self.ffi = torch, ffi
        self.scheme, self.n, self.k, self.m, self.x_dtype = scheme, n, k, m, x_dtype
        w = synth.quant_weights(scheme, synth.seed_for(seed, "w"), n, k)
        self.w_host = w
        self.w_bytes = w.nbytes
        copies = max(2, -(-2 * IC_BYTES // w.nbytes))
        wd = torch.from_numpy(w).cuda()
        self.ws = [wd] + [wd.clone() for _ in range(copies - 1)]
        if x_dtype == ffi.BF16:
            self.x_host = synth.normal_bf16(synth.seed_for(seed, "x"), (m, k))
            self.x = torch.from_numpy(self.x_host.view(np.int16)).cuda().view(torch.bfloat16)
        else:
            self.x_host = synth.normal_f32(synth.seed_for(seed, "x"), (m, k))
            self.x = torch.from_numpy(self.x_host).cuda()
        self.y = torch.empty((m, n), dtype=torch.float32, device="cuda")
        self.st = ffi.matmul_static(n, k, scheme, x_dtype, ffi.F32, m_bucket=m)
        self.bytes = ffi.matmul_static_bytes(self.st, m)
        self.flops = 2 * m * n * k
        self.i = 0

    def step(self):
        w = self.ws[self.i % len(self.ws)]
        self.i += 1
        self.ffi.matmul(w, self.scheme, self.n, self.k, self.x, y=self.y)

    def timed(self, steps, warmup):
        torch = self.torch
        for _ in range(warmup):
            self.step()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for _ in range(steps):
            self.step()
        e1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ms = e0.elapsed_time(e1)
        return ms / steps, wall

    def graph_timed(self, reps):
        """Per-launch time of back-to-back launches replayed from a HIP graph
        (one launch per rotated weight copy), measured with events on the
        launch stream."""
        torch = self.torch
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            for _ in range(3):
                for w in self.ws:
                    self.ffi.matmul(w, self.scheme, self.n, self.k, self.x, y=self.y, stream=s)
            s.synchronize()
            with torch.cuda.graph(g, stream=s):
                for w in self.ws:
                    self.ffi.matmul(w, self.scheme, self.n, self.k, self.x, y=self.y, stream=s)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        cur = torch.cuda.current_stream()
        e0.record(cur)
        for _ in range(reps):
            g.replay()
        e1.record(cur)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / (reps * len(self.ws))

    def cpu_baseline(self, budget_s=12.0):
        """Scalar oracle (1 thread) on whole GEMVs until ~budget_s of CPU time."""
        sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "tests"))
        import oracle_ffi as O

        n_calls, t0 = 0, time.perf_counter()
        while True:
            O.matmul(self.scheme, self.w_host, self.n, self.k, self.x_host, self.x_dtype)
            n_calls += 1
            el = time.perf_counter() - t0
            if el >= budget_s:
                break
        return self.bytes * n_calls / el / 1e9, n_calls, el


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; multi-GPU figures are out of scope "
                                   "(--gpus must be 1)"}))
        return 2
    import torch

    from r9v_amd import ffi, synth

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU"}))
        return 1
    ffi.load()

    # headline: configs[1], IQ4_XS GEMV, M = 5
    log("setup c1 (IQ4_XS GEMV K=2048 N=5120 M=5)")
    head = GemvBench(torch, ffi, synth, ffi.IQ4_XS, 5120, 2048, 5, ffi.BF16, "c1m5")
    ms, wall = head.timed(args.steps, args.warmup)
    value = head.bytes / (ms * 1e-3) / 1e9
    g_ms = head.graph_timed(20)
    achieved = head.bytes / (g_ms * 1e-3) / 1e9
    log(f"c1 m5: {ms*1e3:.2f} us/step stream, {g_ms*1e3:.2f} us/launch graph -> {achieved:.0f} GB/s")

    extras = {}
    only = set(filter(None, args.only.split(",")))

    def want(name):
        return not only or name in only

    if want("c1m1"):
        b = GemvBench(torch, ffi, synth, ffi.IQ4_XS, 5120, 2048, 1, ffi.BF16, "c1m1")
        gm = b.graph_timed(20)
        extras["c1_iq4xs_gemv_m1"] = {"us_per_launch": round(gm * 1e3, 3),
                                      "GB/s": round(b.bytes / (gm * 1e-3) / 1e9, 1),
                                      "frac_hbm": round(b.bytes / (gm * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                      "bytes": b.bytes}
        del b
    if want("c0"):
        b = GemvBench(torch, ffi, synth, ffi.Q4_K, 4096, 4096, 1, ffi.F32, "c0")
        gm = b.graph_timed(20)
        extras["c0_q4k_gemv_f32"] = {"us_per_launch": round(gm * 1e3, 3),
                                     "GB/s": round(b.bytes / (gm * 1e-3) / 1e9, 1),
                                     "frac_hbm": round(b.bytes / (gm * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                     "bytes": b.bytes}
        del b

    cpu = None
    if not args.no_cpu:
        v, calls, el = head.cpu_baseline()
        cpu = {"value": round(v, 4), "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": f"{calls} full c1 M=5 GEMVs (oracle, scalar T0 Branch-D restatement) in {el:.1f} s"}

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
        "data": "synthetic (seeded SplitMix64; GGUF IQ4_XS blocks, x ~ N(0,1) bf16)",
        "config": {"workload": "configs[1]: IQ4_XS dequant GEMV K=2048 N=5120 M=5, x bf16, y f32",
                   "weight_copies": len(head.ws), "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "gemv_kernel<IQ4_XS, M=5, bf16>",
                     "bytes_per_launch": head.bytes, "us_per_launch": round(g_ms * 1e3, 3)},
        "cpu_baseline": cpu,
        "extras": extras,
    }
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
