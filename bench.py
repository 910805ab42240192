#!/usr/bin/env python3
"""Headline benchmark: Q4_K decode GEMV at Llama-3-8B layer shapes on one MI355X.

Workload (the Q4_K decode-GEMV benchmark configuration): one step is one pass over a Llama-3-8B layer's
seven Q4_K matrix-vector products at batch 1 (q and o 4096x4096, k and v
1024x4096, gate and up 14336x4096, down 4096x14336), issued the way the decode
path issues them: fused QKV, o, fused gate/up + SiLU, down -- four launches,
after the rmsnorm that writes their 4096-wide input. The three 4096-wide
launches read that input's int8 form, which the rmsnorm writes beside it (the
decode path fuses the quantization into the producers of these inputs:
rmsnorm and attention); the down projection reads an f32 input and quantizes
it in its own prologue, as in the decode path. The rmsnorm is part of every
step (and of its bytes), so each graph replay rewrites what the GEMVs read. Weights are synthetic (f16 d, dmin = |N(0,1)|*1e-3,
six-bit scales and mins uniform in [0,63], nibbles uniform in [0,15]) and rotate over >= 1 GiB of distinct device copies so the 256 MB
Infinity Cache cannot serve them. Each step is one replay of a captured HIP
graph; the timed region is bracketed by stream synchronisation and HIP events
recorded on the library's own stream.

value = algorithmic bytes per step * steps / time, in the int8-activation mode
(activations quantized per 256 with an f32 scale: the reference's production
decode mode). The f32-activation mode (exact parity with the CPU oracle) is
reported beside it. Algorithmic bytes count each weight byte, each launch's
input and each output once (int8 inputs: values, per-256 scales and per-16
sums).

Also reported: per-launch rates (kernel-only from the dispatch's own
timestamps, and back to back in a graph), the roofline of the dominant
kernel (the fused gate/up GEMV, 66 MB per launch), the prefill GEMMs
(512x4096->14336 and 2048x14336->4096: Q4_K on the f16-path GEMM and on the
int8 MFMA GEMM, Q8_0 and Q6_K on the int8 MFMA GEMM; TOPS against the 5.0
POPS int8 and 2.5 PFLOP/s f16 dense peaks), the Q6_K GEMVs of
the Q6_K configuration (output head 128256x4096 and down 4096x14336 at batch 1, 4
and 8), a device copy-bandwidth probe, and the CPU baseline (the C
restatement of CpuBackend::qmatmul on this host's cores, on a bounded sample
of the same step).
"""
import argparse
import ctypes as C
import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MALL_DEFEAT_BYTES = 1 << 30
SHAPES = {"q": (4096, 4096), "k": (1024, 4096), "v": (1024, 4096), "o": (4096, 4096),
          "gate": (14336, 4096), "up": (14336, 4096), "down": (4096, 14336)}
# The four launches of a decode layer: (name, weights, n_in, output rows).
LAUNCHES = [("qkv", ("q", "k", "v"), 4096, 6144), ("o", ("o",), 4096, 4096),
            ("gate_up", ("gate", "up"), 4096, 14336), ("down", ("down",), 14336, 4096)]
Q4K = 12
SEED = 20261201
# HBM bytes per launch of the dominant kernel (the fused gate/up reading x's
# int8 form, staged in LDS) from rocprofv3 --pmc FETCH_SIZE (32,306.2 KiB per
# dispatch) and WRITE_SIZE (112.0 KiB) over 50 dispatches, FETCH_SIZE scaled
# by 2.0 and WRITE_SIZE by 1.0: a 1 GiB device copy reads 524,301 KiB on
# FETCH_SIZE and 1,048,576 KiB on WRITE_SIZE on this device. Algorithmic
# bytes per launch: 66,122,816 (0.23% below).
TRAFFIC_GATE_UP = 66_277_875


def w_bytes(name):
    r, c = SHAPES[name]
    return r * (c // 256) * 144


def x_bytes(n_in, mode):
    return n_in * 4 if mode == "f32" else n_in + 4 * (n_in // 256) + 4 * (n_in // 16)


def launch_bytes(launch, mode):
    """Weight bytes + input bytes as the launch reads them + f32 outputs. In
    the int8 mode the down projection reads its f32 input (quantized in the
    kernel); the others read an int8 form."""
    name, names, n_in, rows = launch
    return sum(w_bytes(n) for n in names) + x_bytes(n_in, "f32" if name == "down" else mode) + rows * 4


class HipEvents:
    """hipEvent timing on a given stream (libamdhip64, same runtime instance as the backend)."""

    def __init__(self):
        self.h = C.CDLL("libamdhip64.so")

    def event(self):
        e = C.c_void_p()
        assert self.h.hipEventCreate(C.byref(e)) == 0
        return e

    def record(self, e, stream):
        assert self.h.hipEventRecord(e, C.c_void_p(stream)) == 0

    def destroy(self, e):
        self.h.hipEventDestroy(e)

    def elapsed_ms(self, a, b):
        assert self.h.hipEventSynchronize(b) == 0
        ms = C.c_float()
        assert self.h.hipEventElapsedTime(C.byref(ms), a, b) == 0
        return ms.value


class Workload:
    def __init__(self, be):
        from mdma_amd import synth

        layer_bytes = sum(w_bytes(n) for n in SHAPES)
        self.copies = -(-MALL_DEFEAT_BYTES // layer_bytes)
        self.layer_bytes = layer_bytes
        self.raws = {n: synth.weight(Q4K, r, c, SEED + i) for i, (n, (r, c)) in enumerate(SHAPES.items())}
        self.layers = [{n: be.upload_weight(self.raws[n], Q4K, SHAPES[n]) for n in SHAPES}
                       for _ in range(self.copies)]
        # The 4096-wide input is an rmsnorm output (prepare() writes it and,
        # in the int8 mode, its int8 form); x_raw is the rmsnorm's input.
        self.x_raw = be.f32_buf(synth.normal_f32(4096, SEED + 100))
        self.ones = be.f32_buf(np.ones(4096, np.float32))
        self.x = {"x4k": be.alloc(4096 * 4), "down": be.f32_buf(synth.normal_f32(14336, SEED + 103))}
        self.y = {n: be.alloc(SHAPES[n][0] * 4) for n in SHAPES}
        self.act = be.alloc(14336 * 4)

    def prepare(self, be):
        """Write the 4096-wide input (and its int8 form, in the int8 mode)
        the way the decode path does: by a fused rmsnorm. Every graph replay
        drops the library's record of it, so this precedes each capture and
        each run of eager launches."""
        be.rmsnorm(self.ones, self.x_raw, self.x["x4k"], 1e-5)

    def launch(self, be, L, which):
        x = self.x["x4k"]
        if which == "qkv":
            be.qmatmul_qkv(L["q"], L["k"], L["v"], x, self.y["q"], self.y["k"], self.y["v"])
        elif which == "o":
            be.qmatmul(L["o"], x, self.y["o"])
        elif which == "gate_up":
            be.ffn_gate_up(L["gate"], L["up"], x, self.y["gate"], self.y["up"], self.act)
        else:
            be.qmatmul(L["down"], self.x["down"], self.y["down"])

    def step(self, be, L):
        """One layer step: the rmsnorm that writes the 4096-wide input and, in
        the int8 mode, its int8 form (captured with the GEMVs, so every
        replay rewrites what they read), then the four GEMV launches."""
        self.prepare(be)
        for name, _, _, _ in LAUNCHES:
            self.launch(be, L, name)


def norm_bytes(mode):
    """The step's rmsnorm: x and the norm weight read, y written, and in the
    int8 mode y's int8 form (values, per-256 scales, per-16 sums)."""
    return 3 * 4096 * 4 + (x_bytes(4096, "i8") if mode == "i8" else 0)


def step_bytes(mode):
    return sum(launch_bytes(l, mode) for l in LAUNCHES) + norm_bytes(mode)


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


def per_launch(be, ev, wl, mode, reps, graph=True, only=None, durations=None):
    """Per launch kind, over every distinct weight copy, each launch as the
    step issues it (in the int8 mode the down projection quantizes its f32 x
    in its own prologue, so its time includes that quantization):
      - us_kernel: kernel duration from the dispatch's own start/end
        timestamps (hipExtLaunchKernel events, the figure a profiler's
        kernel trace reports), averaged over reps * copies eager launches;
      - us_graph: time per launch of a graph replaying that launch over every
        copy back to back (includes the gap between graph nodes)."""
    out = {}
    n = reps * len(wl.layers)
    starts, stops = [ev.event() for _ in range(n)], [ev.event() for _ in range(n)]
    all_durs = {}
    for launch in LAUNCHES:
        name = launch[0]
        if only and name != only:
            continue
        us_graph = float("nan")
        if graph:
            # The graph starts with the rmsnorm writing the launches' input (and
            # its int8 form): us_graph includes a ninth of that kernel.
            g = be.capture(lambda: [wl.prepare(be)] + [wl.launch(be, L, name) for L in wl.layers])
            ms = time_graphs(be, ev, [g], reps, 2)
            g.close()
            us_graph = ms * 1e3 / n
        wl.prepare(be)
        for L in wl.layers:  # warm: code loaded
            wl.launch(be, L, name)
        be.join_execution()
        i = 0
        for _ in range(reps):
            for L in wl.layers:
                be.time_next_gemv(starts[i].value, stops[i].value)
                wl.launch(be, L, name)
                i += 1
        be.join_execution()
        durs = [ev.elapsed_ms(starts[k], stops[k]) * 1e3 for k in range(n)]
        all_durs[name] = durs
        us = sum(durs) / n
        b = launch_bytes(launch, mode)
        pct = np.percentile(durs, [10, 50, 90])
        out[name] = {"us_kernel": round(us, 3), "us_kernel_median": round(float(np.median(durs)), 3),
                     "us_kernel_p10_p50_p90_max": [round(float(v), 3) for v in pct] + [round(max(durs), 3)],
                     "GBps_kernel": round(b / us / 1e3, 1),
                     "us_graph": round(us_graph, 3), "GBps_graph": round(b / us_graph / 1e3, 1),
                     "bytes_per_launch": b, "launches_timed": n}
    for e in starts + stops:
        ev.destroy(e)
    if durations is not None:
        durations.update(all_durs)
    return out


def gate_up_x_in_kernel(be, ev, wl, reps):
    """The fused gate/up GEMV given an f32 x with no int8 form (a caller
    outside the decode path): the kernel quantizes x in its own prologue.
    Kernel-only us per launch."""
    x = wl.x_raw
    n = reps * len(wl.layers)
    starts, stops = [ev.event() for _ in range(n)], [ev.event() for _ in range(n)]
    for L in wl.layers:
        be.ffn_gate_up(L["gate"], L["up"], x, wl.y["gate"], wl.y["up"], wl.act)
    i = 0
    for _ in range(reps):
        for L in wl.layers:
            be.time_next_gemv(starts[i].value, stops[i].value)
            be.ffn_gate_up(L["gate"], L["up"], x, wl.y["gate"], wl.y["up"], wl.act)
            i += 1
    be.join_execution()
    us = sum(ev.elapsed_ms(starts[j], stops[j]) for j in range(n)) * 1e3 / n
    for e in starts + stops:
        ev.destroy(e)
    return us


Q6K = 14
# Q6_K GEMVs of the Q4_K_M mix: the output head and the down projection
# of the Q4_K_M mix, at batch 1, 4 and 8.
Q6_SHAPES = {"q6k_head": (128256, 4096), "q6k_down": (4096, 14336)}


def q6k_gemvs(be, ev, reps):
    """Kernel-only rates (dispatch timestamps) of the Q6_K GEMVs, weights
    rotated over >= 1 GiB of copies; int8 mode at T = 1, 4, 8 and the f32
    mode at T = 1. Bytes: weights + activations + outputs, each once. The
    batched calls run twice: reading the weights' row planes (`_rows`), then
    their tile images, as batched decode sessions do (made at each copy's
    first batched call with the batch layout on, before the timed ones)."""
    from mdma_amd import synth
    from mdma_amd.backend import ACT_F32, ACT_I8

    out = {}
    for name, (rows, k) in Q6_SHAPES.items():
        raw = synth.weight(Q6K, rows, k, SEED + 7)
        copies = max(2, -(-MALL_DEFEAT_BYTES // len(raw)))
        ws = [be.upload_weight(raw, Q6K, (rows, k)) for _ in range(copies)]
        for T, mode, tiles in ((1, "i8", False), (4, "i8", False), (8, "i8", False), (4, "i8", True),
                               (8, "i8", True), (1, "f32", False)):
            be.set_batch_layout(tiles)
            be.set_act_mode(ACT_I8 if mode == "i8" else ACT_F32)
            x = be.f32_buf(synth.normal_f32(T * k, SEED + 8))
            y = be.alloc(T * rows * 4)
            for w in ws:
                be.qmatmul(w, x, y)
            be.join_execution()
            n = reps * copies
            st, sp = [ev.event() for _ in range(n)], [ev.event() for _ in range(n)]
            for i in range(n):
                be.time_next_gemv(st[i].value, sp[i].value)
                be.qmatmul(ws[i % copies], x, y)
            be.join_execution()
            us = sum(ev.elapsed_ms(st[i], sp[i]) for i in range(n)) * 1e3 / n
            for e in st + sp:
                ev.destroy(e)
            b = len(raw) + T * (x_bytes(k, mode)) + T * rows * 4
            out[f"{name}_T{T}_{mode}" + ("_rows" if T > 1 and not tiles else "")] = {"us_kernel": round(us, 3), "GBps_kernel": round(b / us / 1e3, 1),
                                          "pct_of_hbm_peak": round(100 * b / us / 1e3 / HBM_PEAK_GBS, 1),
                                          "bytes_per_launch": b, "launches_timed": n}
            x.close()
            y.close()
        for w in ws:
            w.buf.close()
    be.set_act_mode(ACT_I8)
    be.set_batch_layout(False)
    return out


INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA, 5.0 POPS
F16_PEAK_TOPS = 2500.0   # MI355X dense f16 MFMA, 2.5 PFLOP/s
GEMM_SHAPES = [(512, 4096, 14336), (2048, 14336, 4096)]  # (M tokens, K, N)


def prefill_gemms(be, ev, reps):
    """Prefill GEMMs at the two prefill shapes: Q4_K and Q6_K (the Q4_K_M
    mix's attention and down type) weights on the f16-path GEMM (their
    default) and on the int8 MFMA GEMM, Q8_0 on the int8 MFMA GEMM.
    Kernel-only GEMM duration (dispatch timestamps) and the whole qmatmul
    call (per-32 activation quantization + GEMM) timed by events on the
    stream. TOPS = 2*M*N*K / time, against the int8 and the f16 dense peaks."""
    from mdma_amd import synth
    from mdma_amd.backend import ACT_I8, PREFILL_AUTO, PREFILL_I8

    be.set_act_mode(ACT_I8)
    out = {}
    for M, K, N in GEMM_SHAPES:
        x = be.f32_buf(synth.normal_f32(M * K, SEED + 20))
        y = be.alloc(M * N * 4)
        for dt, name, kind in ((12, "q4k_f16path", PREFILL_AUTO), (12, "q4k_i8", PREFILL_I8), (8, "q8_0", PREFILL_I8),
                               (14, "q6k_f16path", PREFILL_AUTO), (14, "q6k_i8", PREFILL_I8)):
            be.set_prefill_kernel(kind)
            raw = synth.weight(dt, N, K, SEED + 21)
            w = be.upload_weight(raw, dt, (N, K))
            be.qmatmul(w, x, y)
            be.join_execution()
            st, sp = [ev.event() for _ in range(reps)], [ev.event() for _ in range(reps)]
            for i in range(reps):
                be.time_next_gemv(st[i].value, sp[i].value)
                be.qmatmul(w, x, y)
            be.join_execution()
            us = sum(ev.elapsed_ms(st[i], sp[i]) for i in range(reps)) * 1e3 / reps
            a, b = ev.event(), ev.event()
            ev.record(a, be.stream())
            for i in range(reps):
                be.qmatmul(w, x, y)
            ev.record(b, be.stream())
            us_call = ev.elapsed_ms(a, b) * 1e3 / reps
            for e in st + sp + [a, b]:
                ev.destroy(e)
            ops = 2.0 * M * N * K
            out[f"{name}_M{M}_K{K}_N{N}"] = {
                "us_kernel": round(us, 2), "TOPS_kernel": round(ops / us / 1e6, 1),
                "pct_of_int8_peak": round(100 * ops / us / 1e6 / INT8_PEAK_TOPS, 2),
                "pct_of_f16_peak": round(100 * ops / us / 1e6 / F16_PEAK_TOPS, 2),
                "us_call": round(us_call, 2), "TOPS_call": round(ops / us_call / 1e6, 1), "launches_timed": reps}
            w.buf.close()
        x.close()
        y.close()
    be.set_prefill_kernel(PREFILL_AUTO)
    return out


E2E_PATH = "/tmp/mdma_bench_llama3_8b_q4km.gguf"


def e2e_decode(be, n_prompt=512, n_gen=256, batches=(1, 8), path=E2E_PATH, capacity=4096):
    """Llama-3-8B geometry, Q4_K_M mix (attention and down Q6_K, gate/up and
    token_embd Q4_K, head Q6_K), random init written as GGUF; a 512-token
    random prompt prefill, then greedy decode at batch 1 and 8, int8
    activations, f16 KV caches of config 5's context (4096 positions per
    sequence). Step times come from HIP events recorded on the stream between
    steps (the whole generation is queued on the device; tokens feed back
    through device memory)."""
    from mdma_amd import llama_synth
    from mdma_amd.backend import ACT_I8
    from mdma_amd.model import Model

    t0 = time.perf_counter()
    if not os.path.exists(path):
        llama_synth.write(path, llama_synth.LLAMA3_8B, llama_synth.Q4_K_M, SEED, fast=True)
    print(f"[bench] e2e: model written in {time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)
    be.set_act_mode(ACT_I8)
    t0 = time.perf_counter()
    m = Model(be, path)
    load_s = time.perf_counter() - t0
    out = {"model": "Llama-3-8B geometry, Q4_K_M mix, random init", "weight_bytes": int(m.plan(1).weight_bytes),
           "load_seconds": round(load_s, 2), "prompt_tokens": n_prompt, "decode_tokens": n_gen,
           "kv_capacity": capacity}
    from mdma_amd import synth
    for B in batches:
        s = m.session(capacity, B, n_prompt)
        prompts = np.stack([synth.tokens(n_prompt, 128256, SEED + 50 + b) for b in range(B)])
        s.generate(prompts, 4)  # warm: code paths, activation buffers, RoPE table
        s.reset()
        toks, secs = s.generate(prompts, n_gen)
        dec = secs[1:]
        out[f"batch{B}"] = {"prefill_and_first_token_ms": round(secs[0] * 1e3, 2),
                            "prefill_tok_s": round(B * n_prompt / secs[0], 1),
                            "decode_tok_s": round(B * len(dec) / dec.sum(), 1),
                            "decode_ms_per_step_p50": round(float(np.median(dec)) * 1e3, 3),
                            "decode_ms_per_step_p90": round(float(np.percentile(dec, 90)) * 1e3, 3),
                            "weight_stream_GBps": round(out["weight_bytes"] / float(np.median(dec)) / 1e9, 1),
                            "tokens_sha1": hashlib.sha1(np.ascontiguousarray(toks).tobytes()).hexdigest()[:16]}
        print(f"[bench] e2e batch {B}: {out[f'batch{B}']}", file=sys.stderr, flush=True)
        s.close()
    m.close()
    return out


def e2e_cpu_order(be, n_prompt=512, n_gen=32, path=E2E_PATH, capacity=4096):
    """The CPU-order mode (MDMA_ACT_F32_CPU: every output in the CPU
    backend's rounding order, logits bit-identical to it) on the config-5
    model: a 512-token prompt, then n_gen greedy steps at batch 1, decode
    replaying the captured step. A parity mode, not a throughput one: each
    output row is one lane's sequential chain of n_in additions."""
    from mdma_amd import llama_synth, synth
    from mdma_amd.backend import ACT_F32, ACT_F32_CPU
    from mdma_amd.model import Model

    if not os.path.exists(path):
        llama_synth.write(path, llama_synth.LLAMA3_8B, llama_synth.Q4_K_M, SEED, fast=True)
    be.set_act_mode(ACT_F32_CPU)
    try:
        m = Model(be, path)
        s = m.session(capacity, 1, n_prompt)
        prompt = synth.tokens(n_prompt, 128256, SEED + 50)[None, :]
        s.generate(prompt, 2)  # warm
        s.reset()
        toks, secs = s.generate(prompt, n_gen)
        s.close()
        m.close()
    finally:
        be.set_act_mode(ACT_F32)
    dec = secs[1:]
    return {"prompt_tokens": n_prompt, "decode_tokens": n_gen, "kv_capacity": capacity,
            "prefill_and_first_token_ms": round(secs[0] * 1e3, 1), "decode_tok_s": round(len(dec) / dec.sum(), 2),
            "decode_ms_per_step_p50": round(float(np.median(dec)) * 1e3, 2),
            "tokens_sha1": hashlib.sha1(np.ascontiguousarray(toks).tobytes()).hexdigest()[:16]}


CONFIG1_SEED, CONFIG1_PROMPT_SEED = 1, 1001


def config1_model(path):
    """Config 1: TinyStories-15M geometry, every linear Q8_0, random init
    (seed CONFIG1_SEED) written as GGUF; the CPU leg writes the same file."""
    from mdma_amd import llama_synth

    llama_synth.write(path, llama_synth.TINYSTORIES, llama_synth.Q8_ALL, CONFIG1_SEED)


def e2e_config1(be, n_gen=64):
    """Config 1 on the GPU: the seeded 8-token prompt, 64 greedy tokens, in
    the f32-activation mode (whose tokens must be the CPU backend's) and the
    int8 mode; decode replays the captured step. Tokens are returned for the
    comparison with the CPU leg."""
    import tempfile

    from mdma_amd import synth
    from mdma_amd.backend import ACT_F32, ACT_I8
    from mdma_amd.model import Model

    out, toks = {}, {}
    prompt = synth.tokens(8, 32000, CONFIG1_PROMPT_SEED)
    with tempfile.TemporaryDirectory() as d:
        p = os.path.join(d, "tiny.gguf")
        config1_model(p)
        for mode, name in ((ACT_F32, "f32"), (ACT_I8, "i8")):
            be.set_act_mode(mode)
            m = Model(be, p)
            s = m.session(8 + n_gen, 1, 8)
            s.generate(prompt[None, :], 4)  # warm
            s.reset()
            t, secs = s.generate(prompt[None, :], n_gen)
            dec = secs[1:]
            out[name] = {"prompt_tokens": 8, "decode_tokens": len(dec), "prefill_ms": round(secs[0] * 1e3, 3),
                         "decode_tok_s": round(len(dec) / dec.sum(), 1),
                         "decode_ms_per_step_p50": round(float(np.median(dec)) * 1e3, 4),
                         "tokens_sha1": hashlib.sha1(np.ascontiguousarray(t[0]).tobytes()).hexdigest()[:16]}
            toks[name] = t[0].astype(np.uint32)
            s.close()
            m.close()
    be.set_act_mode(ACT_I8)
    print(f"[bench] config 1 on the GPU: {out}", file=sys.stderr, flush=True)
    return out, toks


def copy_probe(be, ev, nbytes=1 << 30, reps=10):
    """Device-to-device copy rate (bytes read + bytes written per second) of
    hipMemcpyAsync on the library's stream: the achievable-bandwidth
    reference beside the 8 TB/s spec peak, and the plain copy of known size
    that calibrates rocprof's FETCH_SIZE / WRITE_SIZE counters."""
    from mdma_amd.backend import POOL_SCRATCH

    a, b = be.alloc(nbytes, POOL_SCRATCH), be.alloc(nbytes, POOL_SCRATCH)
    be.copy(a, 0, b, 0, nbytes)
    be.join_execution()
    e0, e1 = ev.event(), ev.event()
    ev.record(e0, be.stream())
    for _ in range(reps):
        be.copy(a, 0, b, 0, nbytes)
    ev.record(e1, be.stream())
    ms = ev.elapsed_ms(e0, e1)
    a.close()
    b.close()
    return {"bytes_per_copy": nbytes, "us_per_copy": round(ms * 1e3 / reps, 2),
            "GBps_read_plus_write": round(2 * nbytes * reps / (ms * 1e-3) / 1e9, 1)}


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(raws, budget_s):
    """The CPU oracle (oracle/oracle.c, restating CpuBackend::qmatmul:
    rows over threads, each row dequantized to f32, a sequential f32 dot)
    on every core this process may run on (sched_getaffinity), for about
    budget_s seconds of the same layer step (f32 activations)."""
    from oracle import ffi

    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    rng = np.random.default_rng(1)
    xs = {4096: rng.standard_normal(4096).astype(np.float32), 14336: rng.standard_normal(14336).astype(np.float32)}
    gemv_bytes = sum(launch_bytes(l, "f32") for l in LAUNCHES)
    ffi.qmatmul(Q4K, raws["q"], 4096, 4096, xs[4096], threads=cores)  # warm
    n, t0 = 0, time.perf_counter()
    while True:
        for name, (r, c) in SHAPES.items():
            ffi.qmatmul(Q4K, raws[name], r, c, xs[c], threads=cores)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    # Prefill on the CPU (CpuBackend::qmatmul over 64 token rows, each weight
    # row dequantized once and dotted with every token): a bounded sample of
    # the first prefill GEMM shape, 64 of its 512 tokens, f32 activations.
    pm, pk, pn = 64, 4096, 14336
    xp = rng.standard_normal(pm * pk).astype(np.float32)
    t0 = time.perf_counter()
    reps = 0
    while reps < 2 or time.perf_counter() - t0 < 2.0:
        ffi.qmatmul(Q4K, raws["gate"], pn, pk, xp, threads=cores)
        reps += 1
    pel = (time.perf_counter() - t0) / reps
    return {"value": round(gemv_bytes * n / el / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "cpu": cpu_model(),
            "sample": f"{n} full Q4_K layer steps (the same 7 GEMV shapes, f32 activations), {el:.1f} s, "
                      "oracle/oracle.c restating CpuBackend::qmatmul (row-parallel, sequential f32 dot)",
            "ms_per_step": round(el * 1e3 / n, 2),
            "prefill": {"GOPS": round(2.0 * pm * pk * pn / pel / 1e9, 2), "ms": round(pel * 1e3, 2),
                        "sample": f"Q4_K {pn}x{pk} over {pm} token rows (f32 activations), {reps} calls"}}


def cpu_e2e(path_8b, cores):
    """End-to-end greedy decode on the host cores, the oracle restating
    Model::forward / Llama::run_layers (f32 activations, f16-rounded KV):
      - config 1 (TinyStories-15M geometry, Q8_0): 8-token prompt, 64 tokens;
      - config 5 (Llama-3-8B geometry, Q4_K_M), a bounded sample: a
        16-token prompt and 3 decode steps (each step streams all 5.2 GB of
        weights through the row-parallel dequantize-and-dot)."""
    import tempfile

    from mdma_amd import gguf, llama_synth, synth
    from oracle import ffi

    out = {"cores": cores, "cpu": cpu_model(), "kind": "port"}
    with tempfile.TemporaryDirectory() as d:
        p1 = os.path.join(d, "tiny.gguf")
        config1_model(p1)
        r = gguf.Reader(p1)
        ffi.llama_timed(r, synth.tokens(8, 32000, CONFIG1_PROMPT_SEED), 4, threads=cores)  # warm
        toks, secs = ffi.llama_timed(r, synth.tokens(8, 32000, CONFIG1_PROMPT_SEED), 64, threads=cores)
        dec = secs[1:]
        out["config1"] = {"prompt_tokens": 8, "decode_tokens": 63, "prefill_ms": round(secs[0] * 1e3, 2),
                          "decode_tok_s": round(len(dec) / dec.sum(), 1),
                          "decode_ms_per_step_p50": round(float(np.median(dec)) * 1e3, 2),
                          "tokens": np.asarray(toks, dtype=np.uint32)}
    r = gguf.Reader(path_8b)
    _, secs = ffi.llama_timed(r, synth.tokens(16, 128256, SEED + 60), 4, threads=cores)
    dec = secs[1:]
    out["config5_sample"] = {"prompt_tokens": 16, "decode_tokens": len(dec), "prefill_s": round(secs[0], 2),
                             "decode_tok_s": round(len(dec) / dec.sum(), 3),
                             "decode_s_per_step_p50": round(float(np.median(dec)), 3)}
    print(f"[bench] cpu e2e: {out}", file=sys.stderr, flush=True)
    return out


def mdma_bench(be, path, init_seconds, prompt_len=512, steps=256, repetitions=2, execution="eager"):
    """The reference's mdma-bench protocol (src/bin/mdma-bench.rs:19-116) on
    the same model: load with a memory budget, then one untimed warmup trial
    and `repetitions` timed trials, each on a fresh KV cache: a prefill of
    prompt_len tokens, then `steps` decode steps, each downloading the
    logits and taking the host's greedy argmax, in the int8 mode. Its
    MDMA_BENCH_DECODER choices (:23-25, :72-90): "eager" steps
    Model::forward; "executor" steps the backend's decoder (here the graph
    decode executor), made outside the timer. Its JSON fields; the prompt is
    seeded token ids (no tokenizer)."""
    from mdma_amd import synth
    from mdma_amd.backend import ACT_I8
    from mdma_amd.model import Model

    be.set_act_mode(ACT_I8)
    t0 = time.perf_counter()
    m = Model(be, path)
    load_s = time.perf_counter() - t0
    cap = prompt_len + steps
    tokens = synth.tokens(prompt_len, 128256, SEED + 70)
    plan_p, plan_d = m.plan(cap, 1, prompt_len), m.plan(cap, 1, 1)
    trials = []
    for trial in range(repetitions + 1):
        s = m.session(cap, 1, prompt_len)
        be.join_execution()
        a = time.perf_counter()
        logits = s.prefill(tokens, 0)
        pre = time.perf_counter() - a
        if execution == "executor":
            d = s.decoder()
            a = time.perf_counter()
            for i in range(steps):
                logits = d.forward(int(np.argmax(logits)), prompt_len + i)
            dec = time.perf_counter() - a
            d.close()
        else:
            a = time.perf_counter()
            for i in range(steps):
                logits = s.forward(int(np.argmax(logits)), prompt_len + i)
            dec = time.perf_counter() - a
        assert np.all(np.isfinite(logits))
        s.close()
        if trial > 0:
            trials.append({"prefill_seconds": round(pre, 5), "decode_seconds": round(dec, 5),
                           "prefill_tokens_per_second": round(prompt_len / pre, 1),
                           "decode_tokens_per_second": round(steps / dec, 1)})
    out = {"backend": "gfx950", "architecture": "llama", "model": os.path.basename(path), "execution": execution,
           "artifact_bytes": os.path.getsize(path), "backend_init_seconds": round(init_seconds, 4),
           "load_seconds": round(load_s, 3), "prompt_tokens": prompt_len, "decode_steps": steps,
           "context_capacity": cap, "kv_element_bytes": be.kv_elem_bytes(),
           "native_weight_bytes": int(plan_p.weight_bytes), "native_kv_bytes": int(plan_p.kv_bytes),
           "native_prefill_workspace_bytes": int(plan_p.workspace_bytes),
           "native_decode_workspace_bytes": int(plan_d.workspace_bytes),
           "native_peak_tensor_bytes": int(plan_p.weight_bytes + plan_p.kv_bytes +
                                           max(plan_p.workspace_bytes, plan_d.workspace_bytes)),
           "warmup_trials": 1, "trials": trials}
    m.close()
    print(f"[bench] mdma-bench ({execution}): {trials}", file=sys.stderr, flush=True)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--reps", type=int, default=40, help="graph replays per launch kind in the roofline probe")
    ap.add_argument("--no-e2e", action="store_true", help="skip the Llama-3-8B end-to-end decode")
    ap.add_argument("--e2e-only", action="store_true",
                    help="only the Llama-3-8B end-to-end leg (for a profiler's kernel trace of decode steps)")
    ap.add_argument("--roofline-only", action="store_true",
                    help="only the int8 per-launch leg and the roofline object computed from it (for a profiler's "
                         "kernel trace whose dispatches are exactly the ones the roofline averages)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the prefill GEMM leg (for profiler traces and counters of the GEMMs)")
    ap.add_argument("--q6-only", action="store_true",
                    help="only the Q6_K GEMV leg (head and down at 1, 4 and 8 tokens; for profiler traces)")
    ap.add_argument("--cpu-order-only", action="store_true",
                    help="only the CPU-order mode's end-to-end decode (parity mode: the CPU backend's rounding order)")
    ap.add_argument("--eager-decode", action="store_true",
                    help="end-to-end decode steps launched eagerly instead of replayed from a captured HIP graph "
                         "(the same kernels; for profilers that do not follow graph replays)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU's share of the workload; --gpus {args.gpus} is not supported "
              "(this build runs on a single MI355X).", file=sys.stderr)
        sys.exit(2)

    from mdma_amd.backend import ACT_F32, ACT_I8, Gfx950Backend

    t0 = time.perf_counter()
    be = Gfx950Backend(0)
    init_s = time.perf_counter() - t0
    if args.eager_decode:
        be.set_graph_decode(False)
    if args.cpu_order_only:
        print(json.dumps({"e2e_cpu_order": e2e_cpu_order(be), "device": be.device_label()}), flush=True)
        return
    if args.e2e_only:
        print(json.dumps({"e2e_llama3_8b": e2e_decode(be), "device": be.device_label()}), flush=True)
        return
    ev = HipEvents()
    if args.q6_only:
        print(json.dumps({"q6k_gemv": q6k_gemvs(be, ev, max(2, args.reps // 4)), "device": be.device_label()}),
              flush=True)
        return
    if args.prefill_only:
        print(json.dumps({"prefill_gemm_i8": prefill_gemms(be, ev, max(2, args.reps // 4)),
                          "device": be.device_label()}), flush=True)
        return
    if args.roofline_only:
        wl = Workload(be)
        be.reserve_scratch(64 << 20)
        be.set_act_mode(ACT_I8)
        # Only the gate/up, no graph replays: the kernel's dispatches are one
        # untimed warm pass over the weight copies, then the timed launches.
        durs = {}
        dom = per_launch(be, ev, wl, "i8", args.reps, graph=False, only="gate_up", durations=durs)["gate_up"]
        print(json.dumps({"roofline": {"kernel": "gemv_team<Q4G, int8, gated, x staged in LDS>",
                                       "bytes_per_launch": dom["bytes_per_launch"], "us_per_launch": dom["us_kernel"],
                                       "us_per_launch_median": dom["us_kernel_median"],
                                       "us_p10_p50_p90_max": dom["us_kernel_p10_p50_p90_max"],
                                       "launches_timed": dom["launches_timed"],
                                       "us_each": [round(v, 3) for v in durs["gate_up"]],
                                       "frac": round(dom["GBps_kernel"] / HBM_PEAK_GBS, 4)},
                          "device": be.device_label()}), flush=True)
        return
    probe = copy_probe(be, ev)
    wl = Workload(be)
    be.reserve_scratch(64 << 20)
    results = {}
    for mode, code in (("i8", ACT_I8), ("f32", ACT_F32)):
        be.set_act_mode(code)
        graphs = [be.capture(lambda L=L: wl.step(be, L)) for L in wl.layers]
        ms = time_graphs(be, ev, graphs, args.steps, args.warmup)
        for g in graphs:
            g.close()
        sb = step_bytes(mode)
        results[mode] = {"ms_per_step": ms / args.steps, "GBps": sb * args.steps / (ms * 1e-3) / 1e9,
                         "step_bytes": sb, "per_launch": per_launch(be, ev, wl, mode, args.reps)}
    be.set_act_mode(ACT_I8)
    q6 = q6k_gemvs(be, ev, max(2, args.reps // 4))
    gemm = prefill_gemms(be, ev, max(2, args.reps // 4))
    print("[bench] GEMV, GEMM legs done", file=sys.stderr, flush=True)

    main_mode = results["i8"]
    dom = main_mode["per_launch"]["gate_up"]
    be.set_act_mode(ACT_I8)
    us_xk = gate_up_x_in_kernel(be, ev, wl, args.reps)
    b_xk = dom["bytes_per_launch"] + 3 * 4096  # x read as f32, not int8
    roof = {"bound": "hbm", "achieved": dom["GBps_kernel"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(dom["GBps_kernel"] / HBM_PEAK_GBS, 4), "traffic": TRAFFIC_GATE_UP,
            "kernel": "gemv_team<Q4G, int8, gated, x staged in LDS> (fused ffn gate/up + SiLU, 2 x 14336x4096 Q4_K, "
                      "x's int8 form from the fused rmsnorm)",
            "bytes_per_launch": dom["bytes_per_launch"], "us_per_launch": dom["us_kernel"],
            "us_per_launch_median": dom["us_kernel_median"],
            "us_p10_p50_p90_max": dom["us_kernel_p10_p50_p90_max"],
            "timing": (f"achieved = bytes_per_launch / us_per_launch, us_per_launch the mean of "
                       f"{dom['launches_timed']} kernel-only durations from the dispatches' own start/end "
                       "timestamps (the statistic rocprofv3 --stats reports as its average)"),
            "x_quantized_in_kernel": {"kernel": "gemv_team<Q4G, int8, gated, x-quant> (f32 x quantized in the prologue)",
                                      "us_per_launch": round(us_xk, 3),
                                      "achieved": round(b_xk / us_xk / 1e3, 1),
                                      "frac": round(b_xk / us_xk / 1e3 / HBM_PEAK_GBS, 4)}}
    for L in wl.layers:  # free the rotated layer copies before the 8B model loads
        for w in L.values():
            w.buf.close()
    e2e = None if args.no_e2e else e2e_decode(be)
    c1, c1_toks = (None, None) if args.no_e2e else e2e_config1(be)
    protocol = None if args.no_e2e else mdma_bench(be, E2E_PATH, init_s)
    protocol_x = None if args.no_e2e else mdma_bench(be, E2E_PATH, init_s, execution="executor")
    cpu = None if args.no_cpu else cpu_baseline(wl.raws, args.cpu_seconds)
    if cpu is not None and not args.no_e2e:
        cpu["e2e"] = cpu_e2e(E2E_PATH, cpu["cores"])
        # Greedy tokens of the same model and prompt: the GPU's f32 mode
        # against the CPU backend's (BASELINE's exact-match requirement).
        cpu_toks = cpu["e2e"]["config1"].pop("tokens")
        c1["f32_tokens_equal_cpu"] = bool(np.array_equal(c1_toks["f32"], cpu_toks))
    f = results["f32"]
    line = {
        "metric": "Q4_K GEMV HBM GB/s (% of peak) @8B shapes; decode tok/s, 1 MI355X",
        "value": round(main_mode["GBps"], 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(main_mode["ms_per_step"], 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "i8", "data": "synthetic",
        "config": {"workload": "Q4_K decode GEMV, one Llama-3-8B layer (rmsnorm writing x and its int8 form, "
                               "then fused qkv, o, fused gate/up+SiLU reading that int8 form, and the down "
                               "projection quantizing its f32 input in the kernel), batch 1, int8 activations",
                   "global_batch": 1, "seq_len": 1, "parallelism": "none",
                   "weight_copies": wl.copies, "rotated_bytes": wl.copies * wl.layer_bytes, "seed": SEED},
        "pct_of_hbm_peak": round(100 * main_mode["GBps"] / HBM_PEAK_GBS, 2),
        "roofline": roof,
        "cpu_baseline": cpu,
        "per_launch_i8": main_mode["per_launch"],
        "f32_mode": {"GBps": round(f["GBps"], 1), "ms_per_step": round(f["ms_per_step"], 5),
                     "pct_of_hbm_peak": round(100 * f["GBps"] / HBM_PEAK_GBS, 2), "per_launch": f["per_launch"]},
        "q6k_gemv": q6,
        "prefill_gemm_i8": gemm,
        "e2e_llama3_8b": e2e,
        "e2e_config1": c1,
        "mdma_bench": protocol,
        "mdma_bench_executor": protocol_x,
        "copy_probe": probe,
        "device": be.device_label(),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
