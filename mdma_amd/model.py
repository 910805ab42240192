"""Python host mirror of mdma's Model / KvCache / generate over the C ABI.

`Model.load` is Model::load_with_budget (/root/reference/src/model.rs:141-149),
`Session` holds a KvCache and workspace (src/kv_cache.rs:16, src/model.rs:41-74),
and `Session.generate` is prefill + the greedy loop of inference::sample
(src/inference.rs:102-124). All compute runs in libmdma_gfx950.so.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from .backend import Gfx950Backend, _check, lib

_P, _U64 = C.c_void_p, C.c_uint64


class ModelConfig(C.Structure):
    _fields_ = [(n, _U64) for n in ("n_layers", "n_embd", "n_ff", "n_heads", "n_kv_heads", "head_dim", "n_ctx",
                                    "vocab")] + [("rope_theta", C.c_float), ("rms_eps", C.c_float)]


class MemoryPlan(C.Structure):
    _fields_ = [(n, _U64) for n in ("weight_bytes", "kv_bytes", "workspace_bytes", "headroom_bytes", "total_bytes",
                                    "device_bytes", "available_bytes", "max_context")]


_SIGS = {
    "model_load": ([_P, C.c_char_p, _U64, _P], C.c_int), "model_free": ([_P], None),
    "model_config": ([_P, _P], C.c_int), "model_plan": ([_P, _U64, _U64, _U64, _P], C.c_int),
    "session_new": ([_P, _U64, _U64, _U64, _P], C.c_int), "session_free": ([_P], None),
    "session_reset": ([_P], C.c_int), "prefill": ([_P, _U64, _P, _U64, C.c_uint32, _P], C.c_int),
    "forward": ([_P, _U64, C.c_uint32, C.c_uint32, _P], C.c_int),
    "generate": ([_P, _P, _U64, _U64, _P, _P], C.c_int),
    "decoder_new": ([_P, _U64, _P], C.c_int), "decoder_forward": ([_P, C.c_uint32, C.c_uint32, _P], C.c_int),
    "decoder_replayed": ([_P], C.c_int), "decoder_free": ([_P], None),
}
_bound = False


def _lib():
    global _bound
    L = lib()
    if not _bound:
        for n, (args, res) in _SIGS.items():
            f = getattr(L, "mdma_gfx950_" + n)
            f.argtypes = args
            f.restype = res
        _bound = True
    return L


def exported_symbols() -> list[str]:
    return ["mdma_gfx950_" + n for n in _SIGS]


class Model:
    def __init__(self, backend: Gfx950Backend, path: str, budget_bytes: int = 0):
        self.backend = backend
        h = C.c_void_p()
        _check(_lib().mdma_gfx950_model_load(backend.ctx, path.encode(), budget_bytes, C.byref(h)))
        self.handle = h.value

    @property
    def config(self) -> ModelConfig:
        c = ModelConfig()
        _check(_lib().mdma_gfx950_model_config(self.handle, C.byref(c)))
        return c

    def plan(self, capacity: int, batch: int = 1, tokens: int = 1) -> MemoryPlan:
        p = MemoryPlan()
        _check(_lib().mdma_gfx950_model_plan(self.handle, capacity, batch, tokens, C.byref(p)))
        return p

    def session(self, capacity: int, batch: int = 1, max_tokens: int = 1) -> "Session":
        return Session(self, capacity, batch, max_tokens)

    def close(self):
        if self.handle and self.backend.ctx is not None:
            _lib().mdma_gfx950_model_free(self.handle)
        self.handle = None


class Session:
    def __init__(self, model: Model, capacity: int, batch: int, max_tokens: int):
        self.model = model
        self.batch = batch
        h = C.c_void_p()
        _check(_lib().mdma_gfx950_session_new(model.handle, capacity, batch, max_tokens, C.byref(h)))
        self.handle = h.value

    def reset(self):
        _check(_lib().mdma_gfx950_session_reset(self.handle))

    def prefill(self, tokens, pos: int = 0, seq: int = 0) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        logits = np.empty(self.model.config.vocab, np.float32)
        _check(_lib().mdma_gfx950_prefill(self.handle, seq, t.ctypes.data, t.size, pos, logits.ctypes.data))
        return logits

    def forward(self, token: int, pos: int, seq: int = 0) -> np.ndarray:
        logits = np.empty(self.model.config.vocab, np.float32)
        _check(_lib().mdma_gfx950_forward(self.handle, seq, token, pos, logits.ctypes.data))
        return logits

    def generate(self, prompts, n_gen: int):
        """prompts: [batch, n_prompt] token ids. Returns (tokens [batch, n_gen],
        step_seconds [n_gen]: prefill + first token, then each decode step)."""
        p = np.ascontiguousarray(np.atleast_2d(prompts), dtype=np.uint32)
        assert p.shape[0] == self.batch
        out = np.zeros((self.batch, n_gen), np.uint32)
        secs = np.zeros(n_gen, np.float64)
        _check(_lib().mdma_gfx950_generate(self.handle, p.ctypes.data, p.shape[1], n_gen, out.ctypes.data,
                                           secs.ctypes.data))
        return out, secs

    def decoder(self, seq: int = 0) -> "Decoder":
        return Decoder(self, seq)

    def close(self):
        if self.handle and self.model.backend.ctx is not None:
            _lib().mdma_gfx950_session_free(self.handle)
        self.handle = None


class Decoder:
    """The graph decode executor (HipDecoder, src/backend/rocm/graph.rs:
    105-262): forward(token, pos) replays one captured decode step of the
    session's sequence `seq`; close it before the session."""

    def __init__(self, session: Session, seq: int = 0):
        self.session = session
        h = C.c_void_p()
        _check(_lib().mdma_gfx950_decoder_new(session.handle, seq, C.byref(h)))
        self.handle = h.value

    def forward(self, token: int, pos: int) -> np.ndarray:
        logits = np.empty(self.session.model.config.vocab, np.float32)
        _check(_lib().mdma_gfx950_decoder_forward(self.handle, token, pos, logits.ctypes.data))
        return logits

    @property
    def replayed(self) -> bool:
        return bool(_lib().mdma_gfx950_decoder_replayed(self.handle))

    def close(self):
        if self.handle:
            _lib().mdma_gfx950_decoder_free(self.handle)
        self.handle = None
