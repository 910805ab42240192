"""Synthetic Llama GGUF models with the benchmark geometries and distributions.

config 1: TinyStories-15M geometry, every linear Q8_0 (d = f16(|N|*0.02),
          quants uniform in [-127, 127]), embeddings and norms f32 N(0, 0.02).
config 5: Llama-3-8B geometry, Q4_K_M mix: attention (q/k/v/o) and
          ffn_down Q6_K, gate/up and token_embd Q4_K, output Q6_K.

Tensor names and metadata keys follow the GGUF llama convention the
reference loads (/root/reference/src/model/arch/llama.rs:16-38,96-132).
"""
from __future__ import annotations

import numpy as np

from . import gguf, synth
from .synth import GGML_F32, GGML_Q4_K, GGML_Q6_K, GGML_Q8_0

TINYSTORIES = dict(n_layers=6, n_embd=288, n_heads=6, n_kv_heads=6, n_ff=768, vocab=32000, n_ctx=256,
                   rms_eps=1e-5, rope_theta=10000.0)
LLAMA3_8B = dict(n_layers=32, n_embd=4096, n_heads=32, n_kv_heads=8, n_ff=14336, vocab=128256, n_ctx=4096,
                 rms_eps=1e-5, rope_theta=500000.0)

Q8_ALL = {"attn_q": GGML_Q8_0, "attn_k": GGML_Q8_0, "attn_v": GGML_Q8_0, "attn_output": GGML_Q8_0,
          "ffn_gate": GGML_Q8_0, "ffn_up": GGML_Q8_0, "ffn_down": GGML_Q8_0, "output": GGML_Q8_0,
          "token_embd": GGML_F32}
Q4_K_M = {"attn_q": GGML_Q6_K, "attn_k": GGML_Q6_K, "attn_v": GGML_Q6_K, "attn_output": GGML_Q6_K,
          "ffn_gate": GGML_Q4_K, "ffn_up": GGML_Q4_K, "ffn_down": GGML_Q6_K, "output": GGML_Q6_K,
          "token_embd": GGML_Q4_K}


def _weight(dtype, rows, cols, seed, fast=False):
    if dtype == GGML_F32:
        return synth.normal_f32(rows * cols, seed, 0.02).view(np.uint8)
    return synth.weight(dtype, rows, cols, seed, fast)


def tensors(geom: dict, dtypes: dict, seed: int, fast: bool = False):
    """Yields (name, dtype, [rows, cols] or [n], make_payload) in load order; the
    payload is generated only when make_payload() is called."""
    E, F, V = geom["n_embd"], geom["n_ff"], geom["vocab"]
    hd = E // geom["n_heads"]
    qd, kd = geom["n_heads"] * hd, geom["n_kv_heads"] * hd
    k = [seed * 1000]

    def nxt():
        k[0] += 1
        return k[0]

    def norm():
        s = nxt()
        return lambda: synth.normal_f32(E, s, 0.02)

    def mat(dtype, rows, cols):
        s = nxt()
        return lambda: _weight(dtype, rows, cols, s, fast)

    yield "token_embd.weight", dtypes["token_embd"], (V, E), mat(dtypes["token_embd"], V, E)
    for i in range(geom["n_layers"]):
        p = f"blk.{i}."
        yield p + "attn_norm.weight", GGML_F32, (E,), norm()
        for name, rows, cols in (("attn_q", qd, E), ("attn_k", kd, E), ("attn_v", kd, E), ("attn_output", E, qd)):
            yield p + name + ".weight", dtypes[name], (rows, cols), mat(dtypes[name], rows, cols)
        yield p + "ffn_norm.weight", GGML_F32, (E,), norm()
        for name, rows, cols in (("ffn_gate", F, E), ("ffn_up", F, E), ("ffn_down", E, F)):
            yield p + name + ".weight", dtypes[name], (rows, cols), mat(dtypes[name], rows, cols)
    yield "output_norm.weight", GGML_F32, (E,), norm()
    yield "output.weight", dtypes["output"], (V, E), mat(dtypes["output"], V, E)


def metadata(geom: dict) -> dict:
    return {"general.architecture": "llama", "general.name": "mdma-synthetic",
            "llama.embedding_length": geom["n_embd"], "llama.block_count": geom["n_layers"],
            "llama.feed_forward_length": geom["n_ff"], "llama.attention.head_count": geom["n_heads"],
            "llama.attention.head_count_kv": geom["n_kv_heads"], "llama.context_length": geom["n_ctx"],
            "llama.attention.layer_norm_rms_epsilon": float(geom["rms_eps"]),
            "llama.rope.freq_base": float(geom["rope_theta"])}


def write(path: str, geom: dict, dtypes: dict, seed: int, fast: bool = False) -> None:
    gguf.write_stream(path, metadata(geom), list(tensors(geom, dtypes, seed, fast)))
