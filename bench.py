#!/usr/bin/env python3
"""Headline benchmark: Q4_K decode GEMV at Llama-3-8B layer shapes on one MI355X.

Workload: one step is one pass over a Llama-3-8B layer's
seven Q4_K matrix-vector products at batch 1 -- q and o 4096x4096, k and v
1024x4096, gate and up 14336x4096, down 4096x14336 -- in the f32-activation
mode (the mode that matches the CPU oracle to 1e-5). Weights are synthetic
with the BASELINE distribution and rotate over >= 1 GiB of distinct device
copies so the 256 MB Infinity Cache cannot serve them. Each step is one
replay of a captured HIP graph; the timed region is bracketed by stream
synchronisation and HIP events recorded on the library's own stream.

value = algorithmic bytes (weights + x + y, each once) per step * steps / time.

Also reported: the int8-activation mode, per-shape GEMV rates, the roofline
of the dominant kernel (the 14336x4096 gate/up GEMV) and the CPU baseline
(the C restatement of CpuBackend::qmatmul, timed on this host's cores on a
bounded sample of the same step).
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MALL_DEFEAT_BYTES = 1 << 30
SHAPES = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
          ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]
Q4K = 12
SEED = 20261201


def alg_bytes(rows, cols, tokens=1, mode="f32"):
    w = rows * (cols // 256) * 144
    x = tokens * cols * 4 if mode == "f32" else tokens * (cols + 4 * cols // 256)
    return w + x + tokens * rows * 4


class HipEvents:
    """hipEvent timing on a given stream (libamdhip64, same runtime instance as the backend)."""

    def __init__(self):
        self.h = C.CDLL("libamdhip64.so")
        for n in ("hipEventCreate", "hipEventRecord", "hipEventSynchronize", "hipEventElapsedTime",
                  "hipEventDestroy", "hipStreamSynchronize"):
            getattr(self.h, n).restype = C.c_int

    def event(self):
        e = C.c_void_p()
        assert self.h.hipEventCreate(C.byref(e)) == 0
        return e

    def record(self, e, stream):
        assert self.h.hipEventRecord(e, C.c_void_p(stream)) == 0

    def elapsed_ms(self, a, b):
        assert self.h.hipEventSynchronize(b) == 0
        ms = C.c_float()
        assert self.h.hipEventElapsedTime(C.byref(ms), a, b) == 0
        return ms.value


def build_workload(be, mode):
    from mdma_amd import synth

    layer_bytes = sum(r * (c // 256) * 144 for _, r, c in SHAPES)
    copies = -(-MALL_DEFEAT_BYTES // layer_bytes)
    raws = {name: synth.weight(Q4K, r, c, SEED + i) for i, (name, r, c) in enumerate(SHAPES)}
    layers = []
    for _ in range(copies):
        layers.append({name: be.upload_weight(raws[name], Q4K, (r, c)) for name, r, c in SHAPES})
    x = {4096: be.f32_buf(synth.normal_f32(4096, SEED + 100)), 14336: be.f32_buf(synth.normal_f32(14336, SEED + 101))}
    y = {name: be.alloc(r * 4) for name, r, _ in SHAPES}
    return raws, layers, x, y, copies, layer_bytes


def run_step(be, layer, x, y, mode):
    fn = be.qmatmul_f32 if mode == "f32" else be.qmatmul_i8
    for name, r, c in SHAPES:
        fn(layer[name], x[c], y[name])


def time_graphs(be, ev, graphs, steps, warmup):
    for i in range(warmup):
        graphs[i % len(graphs)].launch()
    be.join_execution()
    a, b = ev.event(), ev.event()
    ev.record(a, be.stream())
    for i in range(steps):
        graphs[i % len(graphs)].launch()
    ev.record(b, be.stream())
    ms = ev.elapsed_ms(a, b)
    be.join_execution()
    return ms


def per_shape(be, ev, layers, x, y, mode, reps):
    """Average launch duration of each shape's GEMV: a graph of back-to-back
    launches over every distinct copy, replayed `reps` times."""
    fn = be.qmatmul_f32 if mode == "f32" else be.qmatmul_i8
    out = {}
    for name, r, c in SHAPES:
        if name in ("k", "v", "up", "o"):
            continue  # same kernel and shape as q/gate already measured
        mats = [L[n] for L in layers for n, rr, cc in SHAPES if (rr, cc) == (r, c)]
        g = be.capture(lambda: [fn(m, x[c], y[name]) for m in mats])
        ms = time_graphs(be, ev, [g], reps, 2)
        launches = reps * len(mats)
        us = ms * 1e3 / launches
        out[f"{r}x{c}"] = {"us_per_launch": round(us, 3), "GBps": round(alg_bytes(r, c, 1, mode) / us / 1e3, 1),
                           "distinct_copies": len(mats), "launches": launches}
        g.close()
    return out


def cpu_baseline(raws, budget_s):
    from oracle import ffi

    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    cores = max(1, min(cores, 16))
    xs = {4096: np.random.default_rng(1).standard_normal(4096).astype(np.float32),
          14336: np.random.default_rng(2).standard_normal(14336).astype(np.float32)}
    step_bytes = sum(alg_bytes(r, c) for _, r, c in SHAPES)
    n, t0 = 0, time.perf_counter()
    ffi.qmatmul(Q4K, raws["q"], 4096, 4096, xs[4096], threads=cores)  # warm
    t0 = time.perf_counter()
    while True:
        for name, r, c in SHAPES:
            ffi.qmatmul(Q4K, raws[name], r, c, xs[c], threads=cores)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return {"value": round(step_bytes * n / el / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"{n} full Q4_K layer steps (7 GEMVs, f32 activations) of the same shapes, "
                      f"{el:.1f} s; oracle/oracle.c restating CpuBackend::qmatmul",
            "ms_per_step": round(el * 1e3 / n, 2)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--reps", type=int, default=200, help="graph replays per shape in the roofline probe")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU's share of the workload; --gpus {args.gpus} is not supported "
              "(this build runs on a single MI355X).", file=sys.stderr)
        sys.exit(2)

    from mdma_amd.backend import Gfx950Backend

    be = Gfx950Backend(0)
    ev = HipEvents()
    raws, layers, x, y, copies, layer_bytes = build_workload(be, "f32")
    be.reserve_scratch(64 << 20)
    step_bytes = {m: sum(alg_bytes(r, c, 1, m) for _, r, c in SHAPES) for m in ("f32", "i8")}

    results = {}
    for mode in ("f32", "i8"):
        graphs = [be.capture(lambda L=L: run_step(be, L, x, y, mode)) for L in layers]
        ms = time_graphs(be, ev, graphs, args.steps, args.warmup)
        results[mode] = {"ms_per_step": ms / args.steps, "GBps": step_bytes[mode] * args.steps / (ms * 1e-3) / 1e9}
        results[mode]["per_shape"] = per_shape(be, ev, layers, x, y, mode, max(10, args.reps // 10))
        for g in graphs:
            g.close()

    dom = results["f32"]["per_shape"]["14336x4096"]
    roof = {"bound": "hbm", "achieved": dom["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(dom["GBps"] / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": "gemv_q4k_f32<1,false> at 14336x4096 (ffn gate/up shape)",
            "bytes_per_launch": alg_bytes(14336, 4096), "us_per_launch": dom["us_per_launch"]}
    cpu = None if args.no_cpu else cpu_baseline(raws, args.cpu_seconds)
    f = results["f32"]
    line = {
        "metric": "Q4_K GEMV HBM GB/s (% of peak) @8B shapes; decode tok/s, 1 MI355X",
        "value": round(f["GBps"], 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(f["ms_per_step"], 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "Q4_K GEMV, Llama-3-8B layer shapes (q,k,v,o,gate,up,down), batch 1, "
                               "f32 activations", "global_batch": 1, "seq_len": 1, "parallelism": "none",
                   "weight_copies": copies, "rotated_bytes": copies * layer_bytes, "seed": SEED},
        "pct_of_hbm_peak": round(100 * f["GBps"] / HBM_PEAK_GBS, 2),
        "roofline": roof,
        "cpu_baseline": cpu,
        "i8_mode": {"GBps": round(results["i8"]["GBps"], 1), "ms_per_step": round(results["i8"]["ms_per_step"], 5),
                    "pct_of_hbm_peak": round(100 * results["i8"]["GBps"] / HBM_PEAK_GBS, 2),
                    "per_shape": results["i8"]["per_shape"]},
        "per_shape_f32": f["per_shape"],
        "device": be.device_label(),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
