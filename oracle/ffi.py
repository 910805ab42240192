"""ctypes binding of the CPU oracle (oracle/liboracle.so): TEST INFRASTRUCTURE ONLY.

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg,
never by the product package. Arrays are numpy; every call checks status.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_P = C.c_void_p
_Z = C.c_size_t


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle not built: {LIB_PATH} (run `make -C oracle`)")
        L = C.CDLL(LIB_PATH)
        sig = {
            "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
            "orc_f32_to_f16": (C.c_uint16, [C.c_float]),
            "orc_dequantize_row": (C.c_int, [C.c_int, _P, _Z, _P, _Z]),
            "orc_qmatmul": (C.c_int, [C.c_int, _P, _Z, _Z, _Z, _P, _Z, _P, _Z, C.c_int]),
            "orc_embed": (C.c_int, [C.c_int, _P, _Z, _Z, _Z, _P, _Z, _P, _Z]),
            "orc_rmsnorm": (C.c_int, [_P, _Z, _P, _Z, _P, _Z, C.c_float]),
            "orc_add": (C.c_int, [_P, _P, _Z, _P]),
            "orc_add_rmsnorm": (C.c_int, [_P, _Z, _P, _P, _Z, _P, _P, C.c_float]),
            "orc_silu_mul": (C.c_int, [_P, _P, _Z, _P]),
            "orc_rope": (C.c_int, [_P, _Z, _P, _Z, C.c_uint32, _Z, _Z, C.c_float]),
            "orc_rope_cos_sin": (None, [C.c_uint32, _Z, C.c_float, _P, _P]),
            "orc_attention": (C.c_int, [_P, _Z, _P, _P, _Z, _Z, _Z, _Z, _Z, _P, _Z]),
            "orc_greedy": (C.c_uint32, [_P, _Z]),
            "orc_quantize_act": (C.c_int, [_P, _Z, _Z, _P, _P, _P]),
            "orc_block_dot_i32": (C.c_int, [C.c_int, _P, _Z, _Z, _Z, _P, _Z, _P]),
            "orc_llama_generate": (C.c_int, [_P, _P, _Z, _Z, _P, _P]),
            "orc_llama_run": (C.c_int, [_P, _P, _Z, _Z, _P, _P, _P]),
            "orc_llama_run_timed": (C.c_int, [_P, _P, _Z, _Z, _P, _P, _P, _P]),
            "orc_i8_group": (_Z, [C.c_int, _Z, _Z, _Z]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


class OracleError(RuntimeError):
    def __init__(self, fn, status):
        super().__init__(f"{fn} returned status {status}")
        self.status = status


def _chk(fn, st):
    if st:
        raise OracleError(fn, st)


def f16_to_f32(h: int) -> float:
    return lib().orc_f16_to_f32(h)


def f32_to_f16(f: float) -> int:
    return lib().orc_f32_to_f16(f)


def dequantize_row(dtype: int, raw: np.ndarray, n: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    _chk("dequantize_row", lib().orc_dequantize_row(dtype, _p(raw), raw.nbytes, _p(out), n))
    return out


def dequantize(dtype: int, raw: np.ndarray, n_out: int, n_in: int) -> np.ndarray:
    """[n_out, n_in] f32 matrix, each row as CpuBackend dequantizes it."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(n_out, -1)
    return np.stack([dequantize_row(dtype, raw[r], n_in) for r in range(n_out)]) if n_out else \
        np.zeros((0, n_in), np.float32)


def qmatmul(dtype: int, w: np.ndarray, n_out: int, n_in: int, x: np.ndarray, threads: int = 0,
            y_elems: int | None = None) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    T = x.size // n_in if n_in else 0
    y = np.zeros(y_elems if y_elems is not None else max(T * n_out, 1), dtype=np.float32)
    threads = threads or os.cpu_count() or 1
    _chk("qmatmul", lib().orc_qmatmul(dtype, _p(w), w.nbytes, n_out, n_in, _p(x), x.size, _p(y),
                                      y.size, threads))
    return y[:T * n_out].reshape(T, n_out) if y_elems is None else y


def embed(dtype: int, table: np.ndarray, vocab: int, n_embd: int, ids) -> np.ndarray:
    table = np.ascontiguousarray(table, dtype=np.uint8)
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    out = np.zeros((ids.size, n_embd), dtype=np.float32)
    _chk("embed", lib().orc_embed(dtype, _p(table), table.nbytes, vocab, n_embd, _p(ids), ids.size,
                                  _p(out), out.size))
    return out


def rmsnorm(w, x, eps: float) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    _chk("rmsnorm", lib().orc_rmsnorm(_p(w), w.size, _p(x), x.size, _p(y), y.size, eps))
    return y


def add(a, b) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    y = np.empty_like(a)
    lib().orc_add(_p(a), _p(b), a.size, _p(y))
    return y


def add_rmsnorm(w, a, b, eps: float):
    w = np.ascontiguousarray(w, dtype=np.float32)
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    s, y = np.empty_like(a), np.empty_like(a)
    _chk("add_rmsnorm", lib().orc_add_rmsnorm(_p(w), w.size, _p(a), _p(b), a.size, _p(s), _p(y), eps))
    return s, y


def silu_mul(g, u) -> np.ndarray:
    g = np.ascontiguousarray(g, dtype=np.float32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    y = np.empty_like(g)
    lib().orc_silu_mul(_p(g), _p(u), g.size, _p(y))
    return y


def rope(q, k, pos: int, n_tokens: int, head_dim: int, theta: float):
    q = np.array(q, dtype=np.float32).reshape(-1)
    k = np.array(k, dtype=np.float32).reshape(-1)
    _chk("rope", lib().orc_rope(_p(q), q.size, _p(k), k.size, pos, n_tokens, head_dim, theta))
    return q, k


def rope_cos_sin(pos: int, head_dim: int, theta: float):
    c = np.empty(head_dim // 2, dtype=np.float32)
    s = np.empty(head_dim // 2, dtype=np.float32)
    lib().orc_rope_cos_sin(pos, head_dim, theta, _p(c), _p(s))
    return c, s


def attention(q, k, v, kv_len: int, head_dim: int, n_q_heads: int, n_kv_heads: int) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.float32).reshape(-1)
    k = np.ascontiguousarray(k, dtype=np.float32).reshape(-1)
    v = np.ascontiguousarray(v, dtype=np.float32).reshape(-1)
    o = np.empty_like(q)
    _chk("attention", lib().orc_attention(_p(q), q.size, _p(k), _p(v), min(k.size, v.size), kv_len,
                                          head_dim, n_q_heads, n_kv_heads, _p(o), o.size))
    return o


def greedy(logits) -> int:
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    return int(lib().orc_greedy(_p(logits), logits.size))


def quantize_act(x, group: int):
    """(q int8[n], d f32[n/group], sum16 i32[n/16])."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    q = np.empty(x.size, dtype=np.int8)
    d = np.empty(x.size // group, dtype=np.float32)
    s = np.empty(x.size // 16, dtype=np.int32)
    _chk("quantize_act", lib().orc_quantize_act(_p(x), x.size, group, _p(q), _p(d), _p(s)))
    return q, d, s


def dequantize_act(q, d, group: int) -> np.ndarray:
    """x_hat = q * d, the input the int8 mode is compared on (one f32 rounding)."""
    q = np.asarray(q, dtype=np.int8).reshape(-1, group).astype(np.float32)
    return (q * np.asarray(d, dtype=np.float32).reshape(-1, 1)).astype(np.float32).reshape(-1)


def block_dot_i32(dtype: int, w, n_out: int, n_in: int, qx, n_tokens: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    qx = np.ascontiguousarray(qx, dtype=np.int8)
    sub = 16 if dtype == 14 else 32
    out = np.empty((n_tokens, n_out, n_in // sub), dtype=np.int32)
    _chk("block_dot_i32", lib().orc_block_dot_i32(dtype, _p(w), w.nbytes, n_out, n_in, _p(qx),
                                                  n_tokens, _p(out)))
    return out


class _W(C.Structure):
    _fields_ = [("dtype", C.c_int), ("n_out", _Z), ("n_in", _Z), ("data", _P)]


class _L(C.Structure):
    _fields_ = [(n, _W) for n in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")] + \
               [("attn_norm", _P), ("ffn_norm", _P)]


class _M(C.Structure):
    _fields_ = [(n, _Z) for n in ("n_layers", "n_embd", "n_ff", "n_heads", "n_kv_heads", "head_dim",
                                  "n_ctx", "vocab")] + \
               [("rope_theta", C.c_float), ("rms_eps", C.c_float), ("token_embd", _W), ("output", _W),
                ("output_norm", _P), ("layers", _P), ("kv_f16", C.c_int), ("n_threads", C.c_int),
                ("act_i8", C.c_int)]


# Token count from which the device's int8 mode runs its prefill GEMM
# (activations per 32); fewer tokens take a GEMV (per 256). Mirrors
# ORC_GEMM_MIN_TOKENS in oracle.h.
GEMM_MIN_TOKENS = 64


def i8_group(dtype: int, n_out: int, n_in: int, T: int) -> int:
    """Activation group (32, 256, or 0 for f32) of the int8 mode's GEMV."""
    return int(lib().orc_i8_group(dtype, n_out, n_in, T))


def _model(gguf_reader, kv_f16: bool, threads: int, act_i8: bool):
    g = gguf_reader
    md = g.metadata
    arch = md["general.architecture"]
    keep = []

    def arr(name):
        a = np.ascontiguousarray(g.bytes_of(name))
        keep.append(a)
        return a

    def W(name):
        d = g.tensors[name]
        a = arr(name)
        return _W(d.dtype, d.shape[0], d.shape[1], a.ctypes.data)

    n_layers = md[f"{arch}.block_count"]
    layers = (_L * n_layers)()
    for i in range(n_layers):
        p = f"blk.{i}."
        layers[i] = _L(W(p + "attn_q.weight"), W(p + "attn_k.weight"), W(p + "attn_v.weight"),
                       W(p + "attn_output.weight"), W(p + "ffn_gate.weight"), W(p + "ffn_up.weight"),
                       W(p + "ffn_down.weight"), arr(p + "attn_norm.weight").ctypes.data,
                       arr(p + "ffn_norm.weight").ctypes.data)
    keep.append(layers)
    n_embd, n_heads = md[f"{arch}.embedding_length"], md[f"{arch}.attention.head_count"]
    te = g.tensors["token_embd.weight"]
    m = _M(n_layers, n_embd, md[f"{arch}.feed_forward_length"], n_heads,
           md.get(f"{arch}.attention.head_count_kv", n_heads), n_embd // n_heads,
           md[f"{arch}.context_length"], te.shape[0], float(md.get(f"{arch}.rope.freq_base", 10000.0)),
           float(md[f"{arch}.attention.layer_norm_rms_epsilon"]), W("token_embd.weight"), W("output.weight"),
           arr("output_norm.weight").ctypes.data, C.cast(layers, C.c_void_p), int(kv_f16),
           threads or os.cpu_count() or 1, 31 if act_i8 is True else int(act_i8))
    return m, keep, te.shape[0]


def llama_generate(gguf_reader, prompt, n_gen: int, kv_f16: bool = True, threads: int = 0, act_i8: bool = False):
    """Greedy tokens (and final logits) of the oracle Llama on a GGUF model."""
    toks, logits = llama_run(gguf_reader, prompt, n_gen, kv_f16=kv_f16, threads=threads, act_i8=act_i8)
    return toks, logits[-1]


def llama_run(gguf_reader, prompt, n_gen: int, forced=None, kv_f16: bool = True, threads: int = 0,
              act_i8: bool = False):
    """(greedy token of every step [n_gen], logits of every step [n_gen, vocab]).
    forced: tokens fed to steps 1..n_gen-1 instead of the greedy ones
    (teacher forcing). act_i8: the int8 activation mode, x requantized
    before every GEMV the device quantizes for (i8_group); an int selects
    the GEMVs by bit (1 qkv, 2 o, 4 gate/up, 8 down, 16 head)."""
    m, keep, vocab = _model(gguf_reader, kv_f16, threads, act_i8)
    prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
    out = np.zeros(n_gen, dtype=np.uint32)
    logits = np.zeros((n_gen, vocab), dtype=np.float32)
    fp = None
    if forced is not None:
        forced = np.ascontiguousarray(forced, dtype=np.uint32)
        assert forced.size >= n_gen - 1
        fp = _p(forced)
    _chk("llama_run", lib().orc_llama_run(C.byref(m), _p(prompt), prompt.size, n_gen, fp, _p(out), _p(logits)))
    del keep
    return out, logits


def llama_timed(gguf_reader, prompt, n_gen: int, threads: int = 0, act_i8: bool = False):
    """(greedy tokens [n_gen], wall seconds per step [n_gen]: [0] prefill
    and head, [i] decode step i), f16-rounded KV; the CPU baseline's run."""
    m, keep, vocab = _model(gguf_reader, True, threads, act_i8)
    prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
    out = np.zeros(n_gen, dtype=np.uint32)
    secs = np.zeros(n_gen, dtype=np.float64)
    _chk("llama_run_timed", lib().orc_llama_run_timed(C.byref(m), _p(prompt), prompt.size, n_gen, None, _p(out),
                                                      None, _p(secs)))
    del keep
    return out, secs
