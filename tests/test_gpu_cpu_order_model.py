"""End-to-end decoding in the CPU-order mode: logits bit-identical to the CPU
oracle at every step, so greedy tokens are the CPU backend's whatever the
margins (the north star's "greedy tokens bit-identical to the CPU backend").

Prefill (Model::prefill, /root/reference/src/model.rs:398-468), eager decode
steps (Model::forward, :326-393), the graph decoder (HipDecoder's
Decoder::forward, src/backend/rocm/graph.rs:105-262), generate's
graph-replayed loop and batched decode all run the same CPU-order kernels;
the oracle (oracle/oracle.c) restates the CPU backend's Llama forward with
the K/V cache rounded through f16 as the device stores it.
"""
import json
import os

import numpy as np
import pytest

from mdma_amd import gguf, llama_synth, synth
from mdma_amd.backend import ACT_F32, ACT_F32_CPU
from mdma_amd.model import Model
from oracle import ffi

pytestmark = pytest.mark.gpu
GOLDEN1 = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "config1_tokens.json")
GQA_SMALL = dict(n_layers=2, n_embd=512, n_heads=8, n_kv_heads=2, n_ff=1024, vocab=2048, n_ctx=256,
                 rms_eps=1e-5, rope_theta=500000.0)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def models(tmp_path_factory):
    d = tmp_path_factory.mktemp("cpu_order")
    paths = {"tiny": str(d / "tiny.gguf"), "gqa": str(d / "gqa.gguf")}
    llama_synth.write(paths["tiny"], llama_synth.TINYSTORIES, llama_synth.Q8_ALL, 1)
    llama_synth.write(paths["gqa"], GQA_SMALL, llama_synth.Q4_K_M, 12)
    return paths


@pytest.fixture
def cpu_mode(backend):
    backend.set_act_mode(ACT_F32_CPU)
    yield backend
    backend.set_act_mode(ACT_F32)


def step_logits(s, prompt, tokens):
    """Prefill's logits, then one forward per token of `tokens[:-1]`."""
    out = [s.prefill(prompt, 0)]
    for i, t in enumerate(tokens[:-1]):
        out.append(s.forward(int(t), len(prompt) + i))
    return np.stack(out)


@pytest.mark.parametrize("name,n_prompt,n_gen", [("tiny", 8, 64), ("gqa", 12, 40)])
def test_every_step_bit_identical_to_oracle(cpu_mode, models, name, n_prompt, n_gen):
    path = models[name]
    V = gguf.Reader(path).tensors["output.weight"].shape[0]
    prompt = synth.tokens(n_prompt, V, 1001)
    want_tok, want = ffi.llama_run(gguf.Reader(path), prompt, n_gen, kv_f16=True)
    m = Model(cpu_mode, path)
    s = m.session(n_prompt + n_gen, 1, n_prompt)
    got = step_logits(s, prompt, want_tok)
    diff = [i for i in range(n_gen) if not np.array_equal(bits(got[i]), bits(want[i]))]
    assert not diff, f"logits differ from the oracle's at steps {diff[:8]}"
    # generate: prefill, then the captured self-advancing step replayed.
    s.reset()
    toks, _ = s.generate(prompt[None, :], n_gen)
    assert np.array_equal(toks[0], want_tok)
    s.close()
    m.close()


def test_config1_fixture_tokens(cpu_mode, models):
    fx = json.load(open(GOLDEN1))["1"]
    m = Model(cpu_mode, models["tiny"])
    s = m.session(8 + 64, 1, 8)
    toks, _ = s.generate(np.array(fx["prompt"], np.uint32)[None, :], 64)
    assert toks[0].tolist() == fx["tokens"]
    s.close()
    m.close()


def test_graph_decoder_and_batched_decode(cpu_mode, models):
    path = models["gqa"]
    prompts = np.stack([synth.tokens(6, 2048, 50 + b) for b in range(3)])
    n_gen = 24
    want = [ffi.llama_run(gguf.Reader(path), prompts[b], n_gen, kv_f16=True) for b in range(3)]
    m = Model(cpu_mode, path)
    # Batched decode: one GEMV per matrix for the three sequences.
    s = m.session(6 + n_gen, 3, 6)
    toks, _ = s.generate(prompts, n_gen)
    for b in range(3):
        assert np.array_equal(toks[b], want[b][0]), b
    s.close()
    # The graph decoder: replayed steps give the oracle's logits.
    s = m.session(6 + n_gen, 1, 6)
    d = s.decoder(0)
    lg = s.prefill(prompts[0], 0)
    assert np.array_equal(bits(lg), bits(want[0][1][0]))
    replays = 0
    for i in range(n_gen - 1):
        lg = d.forward(int(want[0][0][i]), 6 + i)
        replays += d.replayed
        assert np.array_equal(bits(lg), bits(want[0][1][i + 1])), i
    assert replays >= n_gen // 2
    d.close()
    s.close()
    m.close()
