"""The graph decode executor against eager decode.

The reference's pattern (src/backend/test_support/graph.rs:16-75, run by
src/backend/rocm/graph/tests.rs:35-46): a captured decoder and the eager
Model::forward step through the same tokens and positions and must give the
same logits bit for bit at every position; a second captured decoder fed
other tokens on its own KV cache is interleaved with the first (isolation);
invalid tokens and positions are refused; after a prefill moves the KV
position, the decoder (recapturing as needed) still equals eager. And
generate's graph-replayed decode gives the eager loop's tokens.
"""
import numpy as np
import pytest

from mdma_amd import llama_synth
from mdma_amd.backend import ACT_F32, ACT_I8, ShapeMismatch
from mdma_amd.model import Model

pytestmark = pytest.mark.gpu

GQA_SMALL = dict(n_layers=2, n_embd=512, n_heads=8, n_kv_heads=2, n_ff=1024, vocab=2048, n_ctx=256,
                 rms_eps=1e-5, rope_theta=500000.0)
PROMPT = [1, 918, 672, 446, 976, 505]


@pytest.fixture(scope="module", params=["tinystories-q8", "gqa-q4km"])
def model_path(request, tmp_path_factory):
    p = str(tmp_path_factory.mktemp("graph") / "m.gguf")
    if request.param == "tinystories-q8":
        llama_synth.write(p, llama_synth.TINYSTORIES, llama_synth.Q8_ALL, 11)
    else:
        llama_synth.write(p, GQA_SMALL, llama_synth.Q4_K_M, 12)
    return p


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("mode", [ACT_F32, ACT_I8])
def test_graph_decoder_matches_eager(backend, model_path, mode):
    steps, capacity = 70, 128
    backend.set_act_mode(mode)
    m = Model(backend, model_path)
    s = m.session(capacity, batch=3, max_tokens=8)  # seq 0: decoder a, 1: decoder b, 2: eager
    da, db = s.decoder(0), s.decoder(1)
    try:
        logits = None
        replays = 0
        for pos in range(steps):
            token = PROMPT[pos] if pos < len(PROMPT) else logits.size - 1 - int(np.argmax(logits[::-1]))  # ties to last
            want = s.forward(token, pos, seq=2)
            logits = da.forward(token, pos)
            assert np.array_equal(bits(logits), bits(want)), f"graph logits at position {pos}"
            replays += da.replayed
            db.forward((pos + 17) % m.config.vocab, pos)
        # Captured on the first step and replayed after (a step after the
        # context replaced a captured buffer runs eagerly and recaptures).
        assert replays >= steps // 2, replays
        with pytest.raises(ShapeMismatch):
            da.forward(m.config.vocab, steps)  # no such token
        with pytest.raises(ShapeMismatch):
            da.forward(1, steps + 1)  # past the KV prefix
        with pytest.raises(ShapeMismatch):
            da.forward(1, capacity)  # past the capacity
        # A prefill moves the position (and may grow the context's buffers):
        # the decoder still equals eager there.
        s.prefill([31, 47, 59], pos=steps, seq=0)
        s.prefill([31, 47, 59], pos=steps, seq=2)
        pos = steps + 3
        want = s.forward(99, pos, seq=2)
        assert np.array_equal(bits(da.forward(99, pos)), bits(want))
    finally:
        da.close(), db.close()
        s.close(), m.close()
        backend.set_act_mode(ACT_F32)


@pytest.mark.parametrize("batch", [1, 3])
@pytest.mark.parametrize("mode", [ACT_F32, ACT_I8])
def test_generate_graph_equals_eager(backend, model_path, mode, batch):
    backend.set_act_mode(mode)
    m = Model(backend, model_path)
    rng = np.random.default_rng(batch)
    prompts = rng.integers(0, m.config.vocab, size=(batch, 7)).astype(np.uint32)
    try:
        out = {}
        for graph in (False, True):
            backend.set_graph_decode(graph)
            s = m.session(96, batch=batch, max_tokens=8)
            out[graph], _ = s.generate(prompts, 40)
            s.close()
        assert np.array_equal(out[True], out[False])
    finally:
        backend.set_graph_decode(True)
        m.close()
        backend.set_act_mode(ACT_F32)


GQA_LONG = dict(GQA_SMALL, n_ctx=2048)


@pytest.mark.parametrize("mode", [ACT_F32, ACT_I8])
def test_graph_decoder_split_runs_match_eager_at_long_capacity(backend, tmp_path, mode):
    # A captured step sizes its attention grid for the whole cache and splits
    # the live keys into runs on the device. At capacity 1280 (20 tiles of 64
    # keys) the runs for the whole cache (10 of 2 tiles) are fewer than the
    # run limit for live lengths of 10 to 16 tiles, where the eager launch
    # takes one tile per run: positions 640-1023 are where a device rule that
    # started from the grid's run count instead of the host's would merge
    # different partials.
    p = str(tmp_path / "gqa_long.gguf")
    llama_synth.write(p, GQA_LONG, llama_synth.Q4_K_M, 21)
    backend.set_act_mode(mode)
    m = Model(backend, p)
    s = m.session(1280, batch=2, max_tokens=640)
    d = s.decoder(0)
    try:
        rng = np.random.default_rng(3)
        prompt = rng.integers(0, m.config.vocab, size=640).astype(np.uint32)
        s.prefill(prompt, 0, seq=0)
        s.prefill(prompt, 0, seq=1)
        replays = 0
        for pos in range(640, 1024):
            token = (pos * 37) % m.config.vocab
            want = s.forward(token, pos, seq=1)
            got = d.forward(token, pos)
            replays += d.replayed
            assert np.array_equal(bits(got), bits(want)), f"graph logits at position {pos}"
        assert replays >= 380, replays
    finally:
        d.close()
        s.close(), m.close()
        backend.set_act_mode(ACT_F32)


def test_decoder_recaptures_after_a_mode_change(backend, model_path):
    # A kernel-selecting setting changes what a capture would record: the
    # graph captured before it refuses to replay and the decoder captures
    # again, so its logits stay equal to forward's in the new mode.
    backend.set_act_mode(ACT_F32)
    m = Model(backend, model_path)
    s = m.session(64, batch=2, max_tokens=8)
    d = s.decoder(0)
    try:
        for pos in range(12):
            mode = ACT_I8 if pos >= 6 else ACT_F32
            backend.set_act_mode(mode)
            want = s.forward(pos + 5, pos, seq=1)
            got = d.forward(pos + 5, pos)
            assert np.array_equal(bits(got), bits(want)), pos
            if pos == 6:
                assert not d.replayed  # recaptured under the new mode
    finally:
        d.close()
        s.close(), m.close()
        backend.set_act_mode(ACT_F32)
