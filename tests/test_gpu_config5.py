"""Config 5 end to end: the full Llama-3-8B geometry with the Q4_K_M mix
(32 layers, dim 4096, 32 query / 8 KV heads, FFN 14336, vocab 128256; random
init written as GGUF with the fixture's seed), against the CPU oracle's run
of the same model committed in tests/golden/config5_steps.json.

A 64-token prompt, then 15 teacher-forced random tokens (a random model left
to itself repeats one token; forcing makes every step a new context). In
both modes every step's logits at the oracle's top-8 tokens must agree, and
the greedy token must be the oracle's where its top-2 margin is clear:
  - f32 activations: within F32_LOGIT_RTOL of max|logit| (both sides round
    K/V to f16 through 32 layers; a value an ulp apart may round to the
    neighbouring half, a 2^-11 step);
  - int8 activations (the production path; the 64-token prompt takes the
    prefill GEMM): within I8_LOGIT_RTOL, the activation-flip scale measured
    on the small models (tests/test_gpu_model.py).
Batched decode of 8 sequences must give each sequence's single-sequence
tokens (f32 mode: every GEMV is the correctly rounded dot product, whatever
the batch).

Then the configured workload itself, free running (tests/golden/
config5_greedy.json, written by make_golden.py config5_greedy): a 512-token
prompt, 256 greedy tokens, a session of 4096 positions, against the
oracle's own free-running decode (f16-rounded KV) in the f32 and int8 modes:
  - the CPU-order mode's logits equal the oracle's bytes at all 256 steps;
  - the f32 and int8 modes keep the top-4 logits within the bars above and
    give the oracle's 256 greedy tokens;
  - int8 batch-8 decode gives the oracle's tokens for sequence 0 and every
    sequence's single-sequence tokens.
"""
import json
import os

import numpy as np
import pytest

from mdma_amd import llama_synth, synth
from mdma_amd.backend import ACT_F32, ACT_F32_CPU, ACT_I8
from mdma_amd.model import Model

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "config5_steps.json")
F32_LOGIT_RTOL = 1e-3
I8_LOGIT_RTOL = 3e-2
I8_TOKEN_MARGIN = 2e-2


@pytest.fixture(scope="module")
def config5(tmp_path_factory):
    fx = json.load(open(GOLDEN))
    p = str(tmp_path_factory.mktemp("c5") / "llama3_8b_q4km.gguf")
    llama_synth.write(p, llama_synth.LLAMA3_8B, llama_synth.Q4_K_M, fx["seed"], fast=True)
    yield p, fx
    os.remove(p)


def forced_logits(backend, path, prompt, forced):
    m = Model(backend, path)
    s = m.session(len(prompt) + len(forced) + 1, 1, len(prompt))
    out = [s.prefill(prompt, 0)]
    for i, t in enumerate(forced):
        out.append(s.forward(int(t), len(prompt) + i))
    s.close()
    m.close()
    return np.stack(out)


@pytest.mark.parametrize("mode", ["f32", "i8"])
def test_config5_teacher_forced_steps_match_oracle(backend, config5, mode):
    path, fx = config5
    backend.set_act_mode(ACT_F32 if mode == "f32" else ACT_I8)
    try:
        got = forced_logits(backend, path, np.array(fx["prompt"], np.uint32), np.array(fx["forced"], np.uint32))
    finally:
        backend.set_act_mode(ACT_F32)
    steps = fx[mode]
    assert got.shape == (len(steps), 128256) and np.all(np.isfinite(got))
    rtol = F32_LOGIT_RTOL if mode == "f32" else I8_LOGIT_RTOL
    margin = 2 * F32_LOGIT_RTOL if mode == "f32" else I8_TOKEN_MARGIN
    worst, compared = 0.0, 0
    for i, st in enumerate(steps):
        toks = np.array([t for t, _ in st["top8"]])
        want = np.array([v for _, v in st["top8"]])
        err = float(np.max(np.abs(got[i, toks] - want)) / st["max_abs"])
        worst = max(worst, err)
        assert err <= rtol, (mode, i, err)
        if st["margin"] / st["max_abs"] > margin:
            assert int(np.argmax(got[i])) == st["greedy"], (mode, i)
            compared += 1
    print(f"config5 {mode}: worst top-8 |dlogit|/max|logit| {worst:.2e}; greedy compared at {compared} steps")
    assert compared >= len(steps) // 2, "test case too close to ties"


def test_config5_batched_decode_equals_single_sequences(backend, config5):
    path, fx = config5
    backend.set_act_mode(ACT_F32)
    prompts = np.stack([synth.tokens(16, 128256, fx["seed"] + 10 + b) for b in range(8)])
    m = Model(backend, path)
    s = m.session(16 + 8, 8, 16)
    batched, _ = s.generate(prompts, 8)
    s.close()
    s = m.session(16 + 8, 1, 16)
    for b in range(8):
        s.reset()
        one, _ = s.generate(prompts[b:b + 1], 8)
        assert np.array_equal(one[0], batched[b]), b
    s.close()
    m.close()


# ---- the configured workload, free-running: 512-token prompt, 256 greedy tokens, ctx 4096 ----
GREEDY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "config5_greedy.json")
N_PROMPT, N_GEN, CAPACITY = 512, 256, 4096


def config5_prompts(seed, batch=8):
    # tests/golden/make_golden.py config5_prompts: sequence b from seed + 100 + b.
    return np.stack([synth.tokens(N_PROMPT, 128256, seed + 100 + b) for b in range(batch)])


def greedy_last(v):
    return int(v.size - 1 - np.argmax(v[::-1]))  # sampler::greedy: ties to the last index


def free_run(backend, path, prompt):
    """Prefill, then greedy decode through Model::forward steps on a cache of
    config 5's context: (tokens [N_GEN], logits [N_GEN, vocab])."""
    m = Model(backend, path)
    s = m.session(CAPACITY, 1, N_PROMPT)
    lg = s.prefill(prompt, 0)
    toks, logits = [], []
    for i in range(N_GEN):
        logits.append(lg)
        toks.append(greedy_last(lg))
        if i + 1 < N_GEN:
            lg = s.forward(toks[-1], N_PROMPT + i)
    s.reset()
    gen, _ = s.generate(prompt[None, :], N_GEN)  # the captured, replayed decode loop
    s.close()
    m.close()
    return np.array(toks), np.stack(logits), gen[0]


def sha1(v):
    import hashlib
    return hashlib.sha1(np.ascontiguousarray(v, dtype="<f4").tobytes()).hexdigest()


@pytest.fixture(scope="module")
def greedy_fx(config5):
    fx = json.load(open(GREEDY))
    assert fx["seed"] == config5[1]["seed"] and fx["n_prompt"] == N_PROMPT and fx["n_gen"] == N_GEN
    prompts = config5_prompts(fx["seed"])
    import hashlib
    assert hashlib.sha1(np.ascontiguousarray(prompts, dtype="<u4").tobytes()).hexdigest() == fx["prompts_sha1"]
    return fx, prompts


def top4_error(logits, steps):
    """Per step: max over the oracle's top-4 tokens of |gpu - oracle| / max|logit|."""
    err = np.zeros(len(steps))
    for i, st in enumerate(steps):
        t = np.array([t for t, _ in st["top4"]])
        want = np.array([v for _, v in st["top4"]])
        err[i] = np.max(np.abs(logits[i, t] - want)) / st["max_abs"]
    return err


def first_token_mismatch(toks, steps):
    bad = [i for i, st in enumerate(steps) if int(toks[i]) != st["greedy"]]
    if not bad:
        return None
    i = bad[0]
    return f"step {i}: gpu {int(toks[i])}, oracle {steps[i]['greedy']} (oracle top-2 margin / max|logit| " \
           f"{steps[i]['margin'] / steps[i]['max_abs']:.2e}); {len(bad)} steps differ"


def test_config5_cpu_order_greedy_bit_identical(backend, config5, greedy_fx):
    """The CPU-order mode: every one of the 256 steps' logits has the oracle's
    bytes (sha1 of the f32 logits), so all 256 greedy tokens are the CPU
    backend's, near-ties included; generate's replayed loop gives the same
    tokens."""
    path = config5[0]
    fx, prompts = greedy_fx
    steps = fx["seqs"]["0"]["f32"]
    backend.set_act_mode(ACT_F32_CPU)
    try:
        toks, logits, gen = free_run(backend, path, prompts[0])
    finally:
        backend.set_act_mode(ACT_F32)
    bad = [i for i in range(N_GEN) if sha1(logits[i]) != steps[i]["sha1"]]
    assert not bad, f"logits differ from the oracle's at steps {bad[:8]}"
    assert toks.tolist() == [st["greedy"] for st in steps]
    assert np.array_equal(gen, toks)
    print(f"config5 cpu-order: 256 steps bit-identical; smallest top-2 margin / max|logit| "
          f"{min(st['margin'] / st['max_abs'] for st in steps):.2e}")


@pytest.mark.parametrize("mode", ["f32", "i8"])
def test_config5_greedy_tokens_match_oracle(backend, config5, greedy_fx, mode):
    """The fast f32 mode and the int8 mode (the benchmarked path), free
    running at the configured workload: every step's top-4 logits agree with
    the oracle's within the teacher-forced test's bars, and all 256 greedy
    tokens are the oracle's. Their sums round differently from the CPU's, so
    a step whose top-2 margin falls within that error could flip; none of
    the fixture's does today, and a change that flips one fails here with
    the step and its margin. (The random-init model keeps choosing one
    token, whatever the context; the logits differ at every step, which is
    what the top-4 check and the CPU-order test's sha1s follow.)
    generate's replayed loop gives the eager tokens."""
    path = config5[0]
    fx, prompts = greedy_fx
    steps = fx["seqs"]["0"][mode]
    backend.set_act_mode(ACT_F32 if mode == "f32" else ACT_I8)
    try:
        toks, logits, gen = free_run(backend, path, prompts[0])
    finally:
        backend.set_act_mode(ACT_F32)
    rtol = F32_LOGIT_RTOL if mode == "f32" else I8_LOGIT_RTOL
    err = top4_error(logits, steps)
    assert np.all(err <= rtol), (mode, int(np.argmax(err)), float(err.max()))
    mism = first_token_mismatch(toks, steps)
    assert mism is None, f"{mode}: {mism}"
    assert np.array_equal(gen, toks)
    print(f"config5 {mode}: 256 greedy tokens equal the oracle's; worst top-4 |dlogit|/max|logit| {err.max():.2e}, "
          f"smallest oracle margin {min(st['margin'] / st['max_abs'] for st in steps):.2e}")


def test_config5_int8_batch8_decode(backend, config5, greedy_fx):
    """int8 batch-8 decode at Llama-3-8B geometry on a 4096-position cache
    (the ring GEMVs over the Q6_K tile images, the benchmarked batch path):
    sequence 0's 256 tokens are the oracle's int8 tokens, and every
    sequence's tokens are its single-sequence decode's until a step where
    they part. Batched and single GEMVs sum blocks in different orders, so
    an activation can quantize to the neighbouring int8 value and the logits
    differ by up to the int8 bar (I8_LOGIT_RTOL of max|logit|, the error
    measured against the oracle); a parting step must therefore be a
    near-tie of the single run (top-2 margin within twice that bar), never a
    clear choice."""
    path = config5[0]
    fx, prompts = greedy_fx
    backend.set_act_mode(ACT_I8)
    try:
        m = Model(backend, path)
        s = m.session(CAPACITY, 8, N_PROMPT)
        batched, _ = s.generate(prompts, N_GEN)
        s.close()
        m.close()
        singles = [free_run(backend, path, prompts[b]) for b in range(8)]
    finally:
        backend.set_act_mode(ACT_F32)
    steps = fx["seqs"]["0"]["i8"]
    mism = first_token_mismatch(batched[0], steps)
    assert mism is None, f"batch 8, sequence 0 against the oracle: {mism}"
    report = []
    for b in range(8):
        toks, logits, _ = singles[b]
        diff = np.nonzero(batched[b] != toks)[0]
        if not diff.size:
            report.append("all 256")
            continue
        i = int(diff[0])
        srt = np.sort(logits[i])
        rel = float((srt[-1] - srt[-2]) / np.max(np.abs(logits[i])))
        assert rel <= 2 * I8_LOGIT_RTOL, (b, i, rel)
        report.append(f"{i} (near-tie, margin {rel:.1e})")
    print(f"config5 int8 batch 8: sequence 0 equals the oracle for 256 steps; each sequence equals its "
          f"single-sequence decode up to step: {report}")
