#!/usr/bin/env python3
"""Writes the committed golden fixtures under tests/golden/ from the CPU oracle.

- config1_tokens.json: 64 greedy tokens of the TinyStories-15M-geometry model
  (TinyStories-15M geometry, Q8_0 linears, seeds 1 and 2, f16-rounded KV).
- qmatmul_small.npz: raw blocks, x and oracle outputs for Q8_0 / Q4_K / Q6_K
  at the reference's test shapes (rows 1/7/9/20 x K 256/512/768 as in
  /root/reference/src/backend/rocm/decode/tests.rs:81-96), each output checked
  here against an f64 dot product of the dequantized rows before it is written.
- int8_small.npz: activations, their int8 quantization and block dots.

Run from the repository root: python tests/golden/make_golden.py
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
    main()
