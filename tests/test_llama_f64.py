"""Pins the oracle's Llama composition (orc_llama_run) against an independent
float64 statement of the reference's layer loop (tests/llama_f64.py).

Both run the same synthetic GGUF models: the TinyStories-15M geometry with
Q8_0 linears (config 1) and a grouped-query geometry with the Q4_K_M type mix
(4 query heads per KV head, the Llama-3-8B arrangement). The oracle computes
in f32 with the reference CPU backend's operation order; the statement in
f64 with exact weights. Teacher-forced on the oracle's own greedy tokens,
every step's logits must agree within LOGIT_RTOL of the step's largest
|logit|, and the greedy token must agree wherever the f64 top-2 margin
exceeds twice that bound.

The bound is discriminating: the same comparison fails by orders of
magnitude when the oracle is given swapped attention/FFN norms, and when the
f64 statement drops the attention residual (the mistakes a composition
check must catch).
"""
import numpy as np
import pytest

from llama_f64 import LlamaF64
from mdma_amd import gguf, llama_synth, synth
from oracle import ffi

# f32 rounding through a few layers: measured at 6e-7..1.6e-6 of max|logit|
# on these models; 1e-5 leaves headroom and stays over two decades below
# what a composition mistake produces.
LOGIT_RTOL = 1e-5
N_PROMPT, N_GEN = 8, 6
GQA_SMALL = dict(n_layers=2, n_embd=512, n_heads=8, n_kv_heads=2, n_ff=1024, vocab=2048, n_ctx=128,
                 rms_eps=1e-5, rope_theta=500000.0)


@pytest.fixture(scope="module")
def models(tmp_path_factory):
    d = tmp_path_factory.mktemp("f64")
    out = {}
    for name, geom, mix, seed in (("tiny", llama_synth.TINYSTORIES, llama_synth.Q8_ALL, 1),
                                  ("gqa", GQA_SMALL, llama_synth.Q4_K_M, 3)):
        p = str(d / f"{name}.gguf")
        llama_synth.write(p, geom, mix, seed)
        out[name] = (p, geom["vocab"])
    return out


class SwappedNorms:
    """A reader whose attention and FFN norm tensors trade places."""

    def __init__(self, r):
        self.r, self.metadata, self.tensors = r, r.metadata, r.tensors

    def bytes_of(self, name):
        if "attn_norm" in name:
            name = name.replace("attn_norm", "ffn_norm")
        elif "ffn_norm" in name:
            name = name.replace("ffn_norm", "attn_norm")
        return self.r.bytes_of(name)


def rel_err(a, b):
    return np.max(np.abs(a - b), axis=1) / np.max(np.abs(b), axis=1)


def compare(oracle_logits, ref_logits, oracle_tokens):
    err = rel_err(oracle_logits.astype(np.float64), ref_logits)
    top2 = np.sort(ref_logits, axis=1)[:, -2:]
    margin = (top2[:, 1] - top2[:, 0]) / np.max(np.abs(ref_logits), axis=1)
    clear = margin > 2 * LOGIT_RTOL
    agree = ref_logits.argmax(axis=1) == oracle_tokens
    return err, clear, agree


@pytest.mark.parametrize("name", ["tiny", "gqa"])
def test_oracle_llama_matches_f64_statement(models, name):
    path, vocab = models[name]
    r = gguf.Reader(path)
    prompt = synth.tokens(N_PROMPT, vocab, 5000 + vocab)
    toks, logits = ffi.llama_run(r, prompt, N_GEN, kv_f16=False)
    ref = LlamaF64(r).forward_all(np.concatenate([prompt, toks[:-1]]), N_PROMPT)
    assert ref.shape == logits.shape
    err, clear, agree = compare(logits, ref, toks)
    print(f"{name}: per-step max|dlogit|/max|logit| = {np.array2string(err, precision=2)}")
    assert np.all(err <= LOGIT_RTOL), err
    assert clear.sum() >= N_GEN - 1, "test case too close to ties to pin the tokens"
    assert np.all(agree[clear]), (agree, clear)


def test_composition_mistakes_exceed_the_bound(models):
    path, vocab = models["gqa"]
    r = gguf.Reader(path)
    prompt = synth.tokens(N_PROMPT, vocab, 5000 + vocab)
    toks, logits = ffi.llama_run(r, prompt, N_GEN, kv_f16=False)
    seq = np.concatenate([prompt, toks[:-1]])
    # A planted mistake in the oracle's inputs: the two norms swapped.
    _, swapped = ffi.llama_run(SwappedNorms(r), prompt, N_GEN, forced=toks, kv_f16=False)
    ref = LlamaF64(r).forward_all(seq, N_PROMPT)
    assert np.min(rel_err(swapped.astype(np.float64), ref)) > 100 * LOGIT_RTOL
    # A planted mistake in the statement: no residual around attention.
    dropped = NoResidualF64(r).forward_all(seq, N_PROMPT)
    assert np.min(rel_err(logits.astype(np.float64), dropped)) > 100 * LOGIT_RTOL


class NoResidualF64(LlamaF64):
    """forward_all with x = attn_out @ Wo^T instead of x + attn_out @ Wo^T."""

    def forward_all(self, tokens, n_prompt):
        E, L, hd = self.E, self.L, self.hd
        kvw = self.KVH * hd
        n = len(tokens)
        kc = [np.zeros((n, kvw)) for _ in range(L)]
        vc = [np.zeros((n, kvw)) for _ in range(L)]
        emb = self.w("token_embd.weight")
        out = []
        for p0, p1 in [(0, n_prompt)] + [(p, p + 1) for p in range(n_prompt, n)]:
            x = emb[np.asarray(tokens[p0:p1])]
            proj = None
            for i in range(L):
                pre = f"blk.{i}."
                if proj is not None:
                    x = x + proj
                h = self.rmsnorm(x, self.w(pre + "attn_norm.weight"))
                q, k = h @ self.w(pre + "attn_q.weight").T, h @ self.w(pre + "attn_k.weight").T
                v = h @ self.w(pre + "attn_v.weight").T
                pos = np.arange(p0, p1)
                q, k = self.rope(q, pos, self.H), self.rope(k, pos, self.KVH)
                kc[i][p0:p1], vc[i][p0:p1] = k, v
                x = self.attention(q, kc[i], vc[i], p1) @ self.w(pre + "attn_output.weight").T
                h = self.rmsnorm(x, self.w(pre + "ffn_norm.weight"))
                g, u = h @ self.w(pre + "ffn_gate.weight").T, h @ self.w(pre + "ffn_up.weight").T
                proj = (g / (1.0 + np.exp(-g)) * u) @ self.w(pre + "ffn_down.weight").T
            x = x + proj
            out.append((self.rmsnorm(x[-1:], self.w("output_norm.weight")) @ self.w("output.weight").T)[0])
            if p1 == n:
                break
        return np.stack(out)


def test_int8_mode_oracle_routing_and_quantization_error(models):
    """The oracle's int8 activation mode requantizes x before each GEMV the
    device quantizes for: per 32 where the prefill GEMM runs, per 256 for a
    decode GEMV, not at all for float weights or widths that are not whole
    256-column groups. Its logits differ from the f32 mode's by the
    quantization error only (the reference bounds rel-RMS by 0.03,
    src/backend/rocm/tests.rs:306-376)."""
    assert ffi.GEMM_MIN_TOKENS == 64
    assert ffi.i8_group(12, 4096, 4096, 1) == 256
    assert ffi.i8_group(14, 128256, 4096, 8) == 256
    assert ffi.i8_group(12, 14336, 4096, 16) == 256  # batch GEMV
    assert ffi.i8_group(12, 14336, 4096, 63) == 256
    assert ffi.i8_group(12, 14336, 4096, 64) == 32   # prefill GEMM
    assert ffi.i8_group(8, 768, 288, 1) == 0       # 288 is not whole 256-groups
    assert ffi.i8_group(8, 288, 768, 63) == 256
    assert ffi.i8_group(8, 288, 768, 64) == 32     # Q8_0 GEMM: whole 128-column tiles
    assert ffi.i8_group(8, 768, 384, 64) == 32
    assert ffi.i8_group(8, 768, 384, 63) == 0
    assert ffi.i8_group(0, 64, 256, 1) == 0
    path, vocab = models["gqa"]
    r = gguf.Reader(path)
    prompt = synth.tokens(70, vocab, 77)  # 70 rows: the prefill GEMVs take the per-32 route
    t32, l32 = ffi.llama_run(r, prompt, 4, kv_f16=True)
    t8, l8 = ffi.llama_run(r, prompt, 4, forced=t32, kv_f16=True, act_i8=True)
    rel_rms = np.sqrt(np.mean((l8 - l32) ** 2, axis=1) / np.mean(l32 ** 2, axis=1))
    assert np.all(rel_rms < 0.03) and np.all(rel_rms > 0), rel_rms
