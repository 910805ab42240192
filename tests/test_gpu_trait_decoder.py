"""The graph decode executor through the trait: a decode step made only of
trait-level C-ABI calls (embed, rmsnorm, qmatmul_qkv, rope_kv_write, attn,
qmatmul, add_rmsnorm, ffn_gate_up; tests/trait_llama.py), captured once with
the replay parameters set (mdma_gfx950_set_replay_params: token and position
read from device memory) and replayed, against the same calls run eagerly
on a second cache: the pattern of the reference's graph decoder tests
(src/backend/test_support/graph.rs:16-75, src/backend/rocm/graph/tests.rs:
35-46), which compare HipDecoder with EagerDecoder bit for bit.
"""
import numpy as np
import pytest

from trait_llama import TraitDecoder, TraitLlama
from mdma_amd import llama_synth
from mdma_amd.backend import ACT_F32, ACT_F32_CPU, ACT_I8, ShapeMismatch

pytestmark = pytest.mark.gpu

GQA = dict(n_layers=2, n_embd=512, n_heads=8, n_kv_heads=2, n_ff=1024, vocab=2048, n_ctx=512,
           rms_eps=1e-5, rope_theta=500000.0)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def path(tmp_path_factory):
    p = str(tmp_path_factory.mktemp("trait") / "gqa.gguf")
    llama_synth.write(p, GQA, llama_synth.Q4_K_M, 31)
    return p


@pytest.mark.parametrize("mode", [ACT_F32, ACT_I8, ACT_F32_CPU])
def test_trait_level_captured_step_replays_eager_bits(backend, path, mode):
    backend.set_act_mode(mode)
    cap, prompt = 256, [5, 900, 77, 1203, 64, 2000]
    eager, graph = TraitLlama(backend, path, cap, len(prompt)), TraitLlama(backend, path, cap, len(prompt))
    dec = TraitDecoder(graph)
    try:
        eager.run(prompt, 0)
        graph.run(prompt, 0)
        logits = backend.download_f32(eager.logits)
        replays = 0
        for pos in range(len(prompt), len(prompt) + 70):
            token = logits.size - 1 - int(np.argmax(logits[::-1]))  # greedy, ties to the last index
            logits = eager.forward(token, pos)
            got = dec.forward(token, pos)
            replays += dec.replayed
            assert np.array_equal(bits(got), bits(logits)), f"replayed logits at position {pos}"
        assert replays == 69, replays  # captured at the first step, replayed after
        # Replay reads only one token: a multi-token embed is refused while set.
        backend.set_replay_params(dec.params, cap)
        try:
            with pytest.raises(ShapeMismatch):
                graph.run([1, 2], 0)
        finally:
            backend.set_replay_params(None)
    finally:
        dec.close()
        backend.set_act_mode(ACT_F32)


def test_trait_level_graph_refuses_after_buffer_epoch_change(backend, path):
    backend.set_act_mode(ACT_F32)
    cap = 128
    eager, graph = TraitLlama(backend, path, cap, 4), TraitLlama(backend, path, cap, 4)
    dec = TraitDecoder(graph)
    try:
        eager.run([1, 2, 3, 4], 0)
        graph.run([1, 2, 3, 4], 0)
        assert np.array_equal(bits(dec.forward(9, 4)), bits(eager.forward(9, 4)))
        assert not dec.replayed
        assert np.array_equal(bits(dec.forward(10, 5)), bits(eager.forward(10, 5)))
        assert dec.replayed
        # A setting that selects kernels changed and changed back: the graph
        # (captured under an older buffer epoch) refuses to replay, the
        # decoder captures again, the bits still match.
        backend.set_norm_fusion(False)
        backend.set_norm_fusion(True)
        assert np.array_equal(bits(dec.forward(11, 6)), bits(eager.forward(11, 6)))
        assert not dec.replayed
        assert np.array_equal(bits(dec.forward(12, 7)), bits(eager.forward(12, 7)))
        assert dec.replayed
    finally:
        dec.close()
