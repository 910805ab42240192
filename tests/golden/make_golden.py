#!/usr/bin/env python3
"""Writes the committed golden fixtures under tests/golden/ from the CPU oracle.

- config1_tokens.json: 64 greedy tokens of the TinyStories-15M-geometry model
  (TinyStories-15M geometry, Q8_0 linears, seeds 1 and 2, f16-rounded KV).
- qmatmul_small.npz: raw blocks, x and oracle outputs for Q8_0 / Q4_K / Q6_K
  at the reference's test shapes (rows 1/7/9/20 x K 256/512/768 as in
  /root/reference/src/backend/rocm/decode/tests.rs:81-96), each output checked
  here against an f64 dot product of the dequantized rows before it is written.
- int8_small.npz: activations, their int8 quantization and block dots.
- config5_greedy.json (`config5_greedy [seq ...]` argument): the configured
  config-5 workload, free-running (see config5_greedy).
- config5_steps.json (`config5` argument; about a minute of CPU): the
  Llama-3-8B geometry with the Q4_K_M mix (random init, written by
  mdma_amd.llama_synth with fast=True and CONFIG5_SEED), f32 activations,
  f16-rounded KV. A 64-token prompt (the prefill GEMM route in the int8
  mode), then 15 teacher-forced random tokens: every step's greedy token,
  top-2 margin, largest |logit| and top-8 (token, logit) pairs, in the f32
  mode and in the int8 mode (x requantized before every GEMV).

Run from the repository root: python tests/golden/make_golden.py [config5]
"""
import json
import os
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from mdma_amd import gguf, llama_synth, synth  # noqa: E402
from oracle import ffi  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


CONFIG5_SEED = 20261202
CONFIG5_PROMPT, CONFIG5_STEPS = 64, 16
# The configured workload: a 512-token prompt, then 256 greedy tokens; the
# batch-8 prompts are sequences 0..7 of config5_prompts (sequence 0 is the
# batch-1 prompt).
GREEDY_PROMPT, GREEDY_GEN, GREEDY_BATCH = 512, 256, 8


def config5_prompts(seed=CONFIG5_SEED, n=GREEDY_PROMPT, batch=GREEDY_BATCH):
    V = llama_synth.LLAMA3_8B["vocab"]
    return np.stack([synth.tokens(n, V, seed + 100 + b) for b in range(batch)])


def logits_sha1(v):
    import hashlib
    return hashlib.sha1(np.ascontiguousarray(v, dtype="<f4").tobytes()).hexdigest()


def step_record(lg, tok):
    order = np.argsort(lg)[::-1][:4]
    assert int(order[0]) == int(tok) or lg[order[0]] == lg[tok]
    return {"greedy": int(tok), "margin": float(lg[order[0]] - lg[order[1]]), "max_abs": float(np.max(np.abs(lg))),
            "top4": [[int(t), float(lg[t])] for t in order], "sha1": logits_sha1(lg)}


def config5_greedy(path="/tmp/mdma_config5.gguf", seqs=(0,)):
    """config5_greedy.json: the oracle's free-running greedy decode of the
    configured workload (512-token prompt, 256 tokens, f16-rounded KV) in
    the f32 mode and the int8 mode, for the prompts `seqs` of
    config5_prompts; per step the greedy token, top-2 margin, largest
    |logit|, top-4 (token, logit) and the sha1 of the logits' f32 bytes."""
    import time
    if not os.path.exists(path):
        llama_synth.write(path, llama_synth.LLAMA3_8B, llama_synth.Q4_K_M, CONFIG5_SEED, fast=True)
    r = gguf.Reader(path)
    prompts = config5_prompts()
    out = {"seed": CONFIG5_SEED, "n_prompt": GREEDY_PROMPT, "n_gen": GREEDY_GEN,
           "prompts_sha1": hashlib_sha1(prompts), "seqs": {}}
    for b in seqs:
        rec = {}
        for mode, act_i8 in (("f32", False), ("i8", True)):
            t0 = time.time()
            toks, logits = ffi.llama_run(r, prompts[b], GREEDY_GEN, kv_f16=True, act_i8=act_i8)
            rec[mode] = [step_record(logits[i], toks[i]) for i in range(GREEDY_GEN)]
            rec[mode + "_cpu_seconds"] = round(time.time() - t0, 1)
            print(f"config5 greedy seq {b} {mode}: {time.time() - t0:.0f} s; tokens {toks[:16].tolist()}...", flush=True)
        out["seqs"][str(b)] = rec
        with open(os.path.join(HERE, "config5_greedy.json"), "w") as f:
            json.dump(out, f)


def hashlib_sha1(a):
    import hashlib
    return hashlib.sha1(np.ascontiguousarray(a, dtype="<u4").tobytes()).hexdigest()


def config5(path="/tmp/mdma_config5.gguf"):
    if not os.path.exists(path):
        llama_synth.write(path, llama_synth.LLAMA3_8B, llama_synth.Q4_K_M, CONFIG5_SEED, fast=True)
    r = gguf.Reader(path)
    V = llama_synth.LLAMA3_8B["vocab"]
    prompt = synth.tokens(CONFIG5_PROMPT, V, CONFIG5_SEED + 1)
    forced = synth.tokens(CONFIG5_STEPS - 1, V, CONFIG5_SEED + 2)
    out = {"seed": CONFIG5_SEED, "prompt": prompt.tolist(), "forced": forced.tolist()}
    for mode, act_i8 in (("f32", False), ("i8", True)):
        toks, logits = ffi.llama_run(r, prompt, CONFIG5_STEPS, forced=forced, kv_f16=True, act_i8=act_i8)
        steps = []
        for i in range(CONFIG5_STEPS):
            lg = logits[i]
            order = np.argsort(lg)[::-1][:8]
            steps.append({"greedy": int(toks[i]), "margin": float(lg[order[0]] - lg[order[1]]),
                          "max_abs": float(np.max(np.abs(lg))),
                          "top8": [[int(t), float(lg[t])] for t in order]})
            assert steps[-1]["greedy"] == int(order[0])
        out[mode] = steps
        print(f"config5 {mode} margins / max|logit|:", [round(s["margin"] / s["max_abs"], 5) for s in steps])
    with open(os.path.join(HERE, "config5_steps.json"), "w") as f:
        json.dump(out, f)


def main():
    toks = {}
    for seed in (1, 2):
        with tempfile.TemporaryDirectory() as d:
            p = os.path.join(d, "m.gguf")
            llama_synth.write(p, llama_synth.TINYSTORIES, llama_synth.Q8_ALL, seed)
            prompt = synth.tokens(8, 32000, 1000 + seed)
            out, _ = ffi.llama_generate(gguf.Reader(p), prompt, 64, kv_f16=True)
            toks[str(seed)] = {"prompt": prompt.tolist(), "tokens": out.tolist()}
    with open(os.path.join(HERE, "config1_tokens.json"), "w") as f:
        json.dump(toks, f)

    arrays = {}
    for dt in (8, 12, 14):
        for rows in (1, 7, 9, 20):
            for k in (256, 512, 768):
                raw = synth.weight(dt, rows, k, 7 * rows + k + dt)
                x = synth.normal_f32(2 * k, rows + k)
                y = ffi.qmatmul(dt, raw, rows, k, x)
                W = ffi.dequantize_row(dt, raw, rows * k).reshape(rows, k).astype(np.float64)
                exact = x.reshape(2, k).astype(np.float64) @ W.T
                gamma = k * 2 ** -24 / (1 - k * 2 ** -24)
                bound = gamma * (np.abs(x.reshape(2, k)).astype(np.float64) @ np.abs(W).T)
                assert np.all(np.abs(y - exact) <= bound), (dt, rows, k)
                key = f"{dt}_{rows}_{k}"
                arrays[key + "_w"], arrays[key + "_x"], arrays[key + "_y"] = raw, x, y
    np.savez_compressed(os.path.join(HERE, "qmatmul_small.npz"), **arrays)

    x = synth.normal_f32(2 * 512, 99) * 3
    x[:256] = 0
    q, d, s16 = ffi.quantize_act(x, 256)
    dots = {}
    for dt in (8, 12, 14):
        raw = synth.weight(dt, 5, 512, 100 + dt)
        dots[f"w{dt}"] = raw
        dots[f"dot{dt}"] = ffi.block_dot_i32(dt, raw, 5, 512, q, 2)
        sub = 16 if dt == 14 else 32
        Wi = ffi.dequantize_row(dt, raw, 5 * 512)  # values are d*sc*q: integers need unit scales, checked in tests
        assert Wi.shape == (5 * 512,) and dots[f"dot{dt}"].shape == (2, 5, 512 // sub)
    np.savez_compressed(os.path.join(HERE, "int8_small.npz"), x=x, q=q, d=d, s16=s16, **dots)
    print("golden fixtures written")


if __name__ == "__main__":
    if len(sys.argv) > 1 and sys.argv[1] == "config5":
        config5()
    elif len(sys.argv) > 1 and sys.argv[1] == "config5_greedy":
        config5_greedy(seqs=tuple(int(b) for b in sys.argv[2:]) or (0,))
    else:
        main()
