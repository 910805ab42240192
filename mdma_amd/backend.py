"""Python host mirror of mdma's `Backend` trait over the gfx950 C ABI.

`Gfx950Backend` carries the trait's method set (/root/reference/src/backend.rs:190-601)
one-to-one onto `include/mdma_gfx950.h`: the same names, the same argument
meaning (buffers sized in bytes, token counts inferred from x's length,
outputs only large enough) and the same error variants, raised as
`BackendError` subclasses named after `backend::Error` (src/backend.rs:52-93).

There is no CPU fallback: if libmdma_gfx950.so is missing, importing a
backend raises; every op runs the HIP kernels.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

from .synth import BLOCK_SIZE, TYPE_SIZE, GGML_F32, GGML_F16, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K  # noqa: F401

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmdma_gfx950.so")

POOL_WEIGHTS, POOL_KV, POOL_SCRATCH = 0, 1, 2
LAYOUT_GGUF, LAYOUT_GFX950, LAYOUT_ROCM_Q4K_V3 = 0, 1, 2
DOMAIN_DEVICE, DOMAIN_HOST = 0, 1
ACT_F32, ACT_I8, ACT_F32_CPU = 0, 1, 2  # mdma_act_mode
PREFILL_AUTO, PREFILL_I8 = 0, 1  # mdma_prefill_kernel
BATCH_AUTO, BATCH_STAGED = 0, 1  # mdma_batch_kernel

ERROR_NAMES = {1: "ContextLimit", 2: "ShapeMismatch", 3: "NotImplemented", 4: "UnsupportedModel",
               5: "MemoryBudget", 6: "BufferBudget", 7: "InsufficientMemory", 8: "OutOfMemory",
               9: "SizeOverflow", 10: "Backend", 11: "Io"}


class BackendError(RuntimeError):
    code = 0

    def __init__(self, code: int, msg: str):
        super().__init__(f"{ERROR_NAMES.get(code, code)}: {msg}")
        self.code = code
        self.msg = msg

    def is_memory_exhausted(self) -> bool:
        """Error::is_memory_exhausted (src/backend.rs:95-105)."""
        return self.code in (5, 6, 7, 8)


_ERR_TYPES = {code: type(name, (BackendError,), {"code": code}) for code, name in ERROR_NAMES.items()}
globals().update({t.__name__: t for t in _ERR_TYPES.values()})

_P, _U64, _I32, _F = C.c_void_p, C.c_uint64, C.c_int32, C.c_float


class QWeightC(C.Structure):
    _fields_ = [("dtype", _I32), ("rows", _U64), ("cols", _U64), ("buf", _P)]


class RopeSpecC(C.Structure):
    _fields_ = [("head_dim", _U64), ("theta", _F)]


class AttnSpecC(C.Structure):
    _fields_ = [("head_dim", _U64), ("n_q_heads", _U64), ("n_kv_heads", _U64)]


class KvViewC(C.Structure):
    _fields_ = [("k", _P), ("v", _P), ("len", _U64)]


_SIGS = {
    "create": [C.c_int, _P], "destroy": [_P], "last_error": [],
    "device_label": [_P, C.c_char_p, C.c_size_t], "total_device_bytes": [_P],
    "available_device_bytes": [_P, _P], "supports_weight_dtype": [_P, _I32], "max_head_dim": [_P],
    "kv_elem_bytes": [_P], "join_execution": [_P], "set_buffer_budget": [_P, _U64, _U64],
    "buffer_usage": [_P, C.c_int, _P, _P], "set_act_mode": [_P, C.c_int],
    "set_norm_fusion": [_P, C.c_int], "set_prefill_kernel": [_P, C.c_int], "set_batch_kernel": [_P, C.c_int], "set_batch_layout": [_P, C.c_int], "capture_block_dots": [_P, _P], "set_graph_decode": [_P, C.c_int], "stream": [_P],
    "alloc": [_P, _U64, C.c_int, _P], "free": [_P], "buf_len": [_P], "buf_view": [_P, _U64, _U64, _P],
    "upload": [_P, _P, _U64, _P, _U64], "download": [_P, _P, _U64, _P, _U64],
    "copy": [_P, _P, _U64, _P, _U64, _U64], "upload_weight": [_P, _P, _U64, C.c_int, _P],
    "upload_weight_typed": [_P, _P, _U64, C.c_int, _I32, _U64, _U64, _P], "buf_layout": [_P],
    "qmatmul": [_P, _P, _P, _P], "qmatmul_f32": [_P, _P, _P, _P], "qmatmul_i8": [_P, _P, _P, _P],
    "qmatmul_i8_noalloc": [_P, _P, _P, _P],
    "qmatmul_qkv": [_P, _P, _P, _P, _P, _P, _P, _P], "ffn_gate_up": [_P, _P, _P, _P, _P, _P, _P],
    "embed": [_P, _P, _P, _U64, _P], "rmsnorm": [_P, _P, _P, _P, _F],
    "add_rmsnorm": [_P, _P, _P, _P, _P, _P, _F], "add": [_P, _P, _P, _P], "silu_mul": [_P, _P, _P, _P],
    "rope": [_P, _P, _P, C.c_uint32, _U64, _P], "kv_write": [_P, _P, _P, _P, _P, _U64, _U64],
    "rope_kv_write": [_P, _P, _P, _P, _P, _P, _U64, C.c_uint32, _U64, _P, _U64],
    "attn": [_P, _P, _P, _P, _P], "greedy": [_P, _P, _U64, _U64, _P],
    "quantize_act": [_P, _P, _U64, _P, _P, _P], "block_dot_i32": [_P, _P, _P, _P],
    "graph_begin": [_P], "graph_end": [_P, _P], "graph_launch": [_P, _P], "graph_destroy": [_P],
    "reserve_scratch": [_P, _U64], "set_replay_params": [_P, _P, _U64],
    "time_next_gemv": [_P, _P, _P],
    "prepared_bytes": [_I32, _U64, _U64],
    "pack_weight": [_I32, _U64, _U64, _P, _U64, _P, _U64],
    "unpack_weight": [_I32, _U64, _U64, _P, _U64, _P, _U64],
}
_RESTYPES = {"prepared_bytes": _U64, "destroy": None, "graph_destroy": None, "last_error": C.c_char_p, "total_device_bytes": _U64, "max_head_dim": _U64,
             "kv_elem_bytes": _U64, "stream": _P, "buf_len": _U64, "supports_weight_dtype": C.c_int}

_lib = None


def lib():
    """The loaded C ABI; raises if the HIP library has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"gfx950 backend library missing: {LIB_PATH} (run __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        for name, args in _SIGS.items():
            f = getattr(L, "mdma_gfx950_" + name)
            f.argtypes = args
            f.restype = _RESTYPES.get(name, C.c_int)
        _lib = L
    return _lib


def prepared_bytes(dtype: int, rows: int, cols: int) -> int:
    """Bytes of a [rows, cols] weight in the gfx950 prepared layout (0: none)."""
    return int(lib().mdma_gfx950_prepared_bytes(dtype, rows, cols))


def pack_weight(raw, dtype: int, shape) -> np.ndarray:
    """GGUF blocks -> the gfx950 prepared layout (host side, lossless)."""
    a = np.ascontiguousarray(np.frombuffer(bytes(raw) if not isinstance(raw, np.ndarray) else raw, np.uint8))
    out = np.zeros(prepared_bytes(dtype, shape[0], shape[1]), np.uint8)
    _check(lib().mdma_gfx950_pack_weight(dtype, shape[0], shape[1], a.ctypes.data, a.nbytes, out.ctypes.data,
                                         out.nbytes))
    return out


def unpack_weight(prepared, dtype: int, shape) -> np.ndarray:
    """The gfx950 prepared layout -> GGUF blocks (host side, lossless)."""
    a = np.ascontiguousarray(np.frombuffer(prepared, np.uint8))
    out = np.zeros(shape[0] * (shape[1] // BLOCK_SIZE[dtype]) * TYPE_SIZE[dtype], np.uint8)
    _check(lib().mdma_gfx950_unpack_weight(dtype, shape[0], shape[1], a.ctypes.data, a.nbytes, out.ctypes.data,
                                           out.nbytes))
    return out


def exported_symbols() -> list[str]:
    return ["mdma_gfx950_" + n for n in _SIGS]


def _check(st: int):
    if st:
        msg = lib().mdma_gfx950_last_error().decode(errors="replace")
        raise _ERR_TYPES.get(st, BackendError)(st, msg)


class Buf:
    """An owned (or view) device buffer; freed on close()/GC."""

    def __init__(self, handle: int, backend: "Gfx950Backend", owner=True):
        self.handle = handle
        self.backend = backend
        self._owner = owner

    @property
    def len(self) -> int:
        return int(lib().mdma_gfx950_buf_len(self.handle))

    def close(self):
        if self.handle:
            h, self.handle = self.handle, None
            if self.backend.ctx is None:
                return  # the context (and its device) is gone; the process reclaims it
            _check(lib().mdma_gfx950_free(h))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


@dataclass
class QWeight:
    """QWeight (src/backend.rs:114-118): dtype, [n_out, n_in], device buffer."""
    dtype: int
    shape: tuple
    buf: Buf

    def c(self) -> QWeightC:
        return QWeightC(self.dtype, self.shape[0], self.shape[1], self.buf.handle)


@dataclass
class RopeSpec:
    head_dim: int
    theta: float


@dataclass
class AttnSpec:
    head_dim: int
    n_q_heads: int
    n_kv_heads: int


@dataclass
class KvView:
    k: Buf
    v: Buf
    len: int


class Gfx950Backend:
    """The gfx950 implementation of the Backend trait (one device, one stream)."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        _check(lib().mdma_gfx950_create(device, C.byref(h)))
        self.ctx = h.value

    def close(self):
        if self.ctx:
            lib().mdma_gfx950_destroy(self.ctx)
            self.ctx = None

    # -- capability queries --
    def device_label(self) -> str:
        b = C.create_string_buffer(256)
        _check(lib().mdma_gfx950_device_label(self.ctx, b, 256))
        return b.value.decode()

    def total_device_bytes(self) -> int:
        return int(lib().mdma_gfx950_total_device_bytes(self.ctx))

    def available_device_bytes(self) -> int:
        v = C.c_uint64()
        _check(lib().mdma_gfx950_available_device_bytes(self.ctx, C.byref(v)))
        return v.value

    def supports_weight_dtype(self, dtype: int) -> bool:
        return bool(lib().mdma_gfx950_supports_weight_dtype(self.ctx, dtype))

    def max_head_dim(self) -> int:
        return int(lib().mdma_gfx950_max_head_dim(self.ctx))

    def kv_elem_bytes(self) -> int:
        return int(lib().mdma_gfx950_kv_elem_bytes(self.ctx))

    def join_execution(self):
        _check(lib().mdma_gfx950_join_execution(self.ctx))

    def set_buffer_budget(self, device=None, host=None):
        """Backend::set_buffer_budget with BufferBudget::new(device, host):
        None tracks without a quota, 0 forbids the domain."""
        unl = 2**64 - 1
        _check(lib().mdma_gfx950_set_buffer_budget(self.ctx, unl if device is None else device,
                                                   unl if host is None else host))

    def buffer_usage(self, domain: int):
        u, l = C.c_uint64(), C.c_uint64()
        _check(lib().mdma_gfx950_buffer_usage(self.ctx, domain, C.byref(u), C.byref(l)))
        return u.value, l.value

    def set_act_mode(self, mode: int):
        _check(lib().mdma_gfx950_set_act_mode(self.ctx, mode))

    def set_norm_fusion(self, on: bool):
        _check(lib().mdma_gfx950_set_norm_fusion(self.ctx, int(bool(on))))

    def set_graph_decode(self, on: bool):
        """generate's decode steps replayed from one captured HIP graph (default) or run eagerly."""
        _check(lib().mdma_gfx950_set_graph_decode(self.ctx, int(bool(on))))

    def capture_block_dots(self, out):
        """Block-dot capture into the int32 buffer out (None: off); see
        mdma_gfx950_capture_block_dots."""
        _check(lib().mdma_gfx950_capture_block_dots(self.ctx, out.handle if out is not None else None))

    def set_prefill_kernel(self, kind: int):
        """PREFILL_AUTO: the f16-path GEMM for Q4_K prefill calls, the int8
        MFMA GEMM elsewhere; PREFILL_I8: the int8 MFMA GEMM for all."""
        _check(lib().mdma_gfx950_set_prefill_kernel(self.ctx, int(kind)))

    def set_batch_kernel(self, kind: int):
        """BATCH_AUTO: batched int8 GEMVs (3 to 63 tokens) stream through the
        DMA ring kernel; BATCH_STAGED: the register-staged kernel (same bits)."""
        _check(lib().mdma_gfx950_set_batch_kernel(self.ctx, int(kind)))

    def set_batch_layout(self, on: bool):
        """On: the ring kernel reads a tile-major copy of each Q6_K weight,
        made at its first batched call (device memory of the weight's size
        again; same bits)."""
        _check(lib().mdma_gfx950_set_batch_layout(self.ctx, int(bool(on))))

    def stream(self) -> int:
        return int(lib().mdma_gfx950_stream(self.ctx) or 0)

    # -- buffers --
    def alloc(self, nbytes: int, pool: int = POOL_SCRATCH) -> Buf:
        h = C.c_void_p()
        _check(lib().mdma_gfx950_alloc(self.ctx, nbytes, pool, C.byref(h)))
        return Buf(h.value, self)

    def view(self, buf: Buf, offset: int, length: int) -> Buf:
        h = C.c_void_p()
        _check(lib().mdma_gfx950_buf_view(buf.handle, offset, length, C.byref(h)))
        return Buf(h.value, self, owner=False)

    def upload(self, dst: Buf, offset: int, src) -> None:
        a = np.ascontiguousarray(src).view(np.uint8).reshape(-1)
        _check(lib().mdma_gfx950_upload(self.ctx, dst.handle, offset, a.ctypes.data, a.nbytes))

    def download(self, src: Buf, offset: int, nbytes: int) -> np.ndarray:
        out = np.empty(nbytes, dtype=np.uint8)
        _check(lib().mdma_gfx950_download(self.ctx, src.handle, offset, out.ctypes.data, nbytes))
        return out

    def download_f32(self, src: Buf, n: int | None = None, offset: int = 0) -> np.ndarray:
        n = (src.len - offset) // 4 if n is None else n
        return self.download(src, offset, 4 * n).view(np.float32)

    def copy(self, src: Buf, src_off: int, dst: Buf, dst_off: int, length: int):
        _check(lib().mdma_gfx950_copy(self.ctx, src.handle, src_off, dst.handle, dst_off, length))

    def upload_weight(self, raw, dtype: int, shape, layout: int = LAYOUT_GGUF) -> QWeight:
        """upload_weight with the tensor's dtype and [rows, cols] given
        (mdma_gfx950_upload_weight_typed): GGUF K-quant / Q8_0 bytes are
        packed into the prepared layout on the host."""
        a = np.ascontiguousarray(raw).view(np.uint8).reshape(-1)
        h = C.c_void_p()
        _check(lib().mdma_gfx950_upload_weight_typed(self.ctx, a.ctypes.data, a.nbytes, layout, dtype, shape[0],
                                                     shape[1], C.byref(h)))
        return QWeight(dtype, tuple(shape), Buf(h.value, self))

    def upload_weight_bytes(self, raw, layout: int = LAYOUT_GGUF) -> Buf:
        """Backend::upload_weight(bytes, layout) as the trait declares it
        (src/backend.rs:228-237): no dtype or shape; GGUF bytes are repacked
        on the device by the first op that reads them as a QWeight."""
        a = np.ascontiguousarray(raw).view(np.uint8).reshape(-1)
        h = C.c_void_p()
        _check(lib().mdma_gfx950_upload_weight(self.ctx, a.ctypes.data, a.nbytes, layout, C.byref(h)))
        return Buf(h.value, self)

    def buf_layout(self, buf: Buf) -> int:
        return int(lib().mdma_gfx950_buf_layout(buf.handle))

    def f32_buf(self, values, pool: int = POOL_SCRATCH) -> Buf:
        a = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
        b = self.alloc(a.nbytes, pool)
        if a.nbytes:
            self.upload(b, 0, a)
        return b

    # -- quantized-weight hot path --
    def qmatmul(self, w: QWeight, x: Buf, y: Buf):
        _check(lib().mdma_gfx950_qmatmul(self.ctx, C.byref(w.c()), x.handle, y.handle))

    def qmatmul_f32(self, w: QWeight, x: Buf, y: Buf):
        _check(lib().mdma_gfx950_qmatmul_f32(self.ctx, C.byref(w.c()), x.handle, y.handle))

    def qmatmul_i8(self, w: QWeight, x: Buf, y: Buf):
        _check(lib().mdma_gfx950_qmatmul_i8(self.ctx, C.byref(w.c()), x.handle, y.handle))

    def qmatmul_i8_noalloc(self, w: QWeight, x: Buf, y: Buf):
        """qmatmul_i8 with its scratch in the library's static device array:
        no device allocation (callers that cannot allocate)."""
        _check(lib().mdma_gfx950_qmatmul_i8_noalloc(self.ctx, C.byref(w.c()), x.handle, y.handle))

    def qmatmul_qkv(self, wq: QWeight, wk: QWeight, wv: QWeight, x: Buf, q: Buf, k: Buf, v: Buf):
        _check(lib().mdma_gfx950_qmatmul_qkv(self.ctx, C.byref(wq.c()), C.byref(wk.c()), C.byref(wv.c()),
                                             x.handle, q.handle, k.handle, v.handle))

    def ffn_gate_up(self, gate: QWeight, up: QWeight, x: Buf, gate_scratch: Buf, up_scratch: Buf, y: Buf):
        _check(lib().mdma_gfx950_ffn_gate_up(self.ctx, C.byref(gate.c()), C.byref(up.c()), x.handle,
                                             gate_scratch.handle, up_scratch.handle, y.handle))

    # -- per-token ops --
    def embed(self, table: QWeight, token_ids, out: Buf):
        ids = np.ascontiguousarray(token_ids, dtype=np.uint32)
        _check(lib().mdma_gfx950_embed(self.ctx, C.byref(table.c()), ids.ctypes.data, ids.size, out.handle))

    def rmsnorm(self, w: Buf, x: Buf, y: Buf, eps: float):
        _check(lib().mdma_gfx950_rmsnorm(self.ctx, w.handle, x.handle, y.handle, eps))

    def add_rmsnorm(self, w: Buf, a: Buf, b: Buf, sum_: Buf, y: Buf, eps: float):
        _check(lib().mdma_gfx950_add_rmsnorm(self.ctx, w.handle, a.handle, b.handle, sum_.handle, y.handle, eps))

    def add(self, a: Buf, b: Buf, y: Buf):
        _check(lib().mdma_gfx950_add(self.ctx, a.handle, b.handle, y.handle))

    def silu_mul(self, gate: Buf, up: Buf, y: Buf):
        _check(lib().mdma_gfx950_silu_mul(self.ctx, gate.handle, up.handle, y.handle))

    def rope(self, q: Buf, k: Buf, pos: int, n_tokens: int, spec: RopeSpec):
        s = RopeSpecC(spec.head_dim, spec.theta)
        _check(lib().mdma_gfx950_rope(self.ctx, q.handle, k.handle, pos, n_tokens, C.byref(s)))

    def kv_write(self, k: Buf, v: Buf, dst_k: Buf, dst_v: Buf, elem_offset: int, n_elems: int):
        _check(lib().mdma_gfx950_kv_write(self.ctx, k.handle, v.handle, dst_k.handle, dst_v.handle, elem_offset,
                                          n_elems))

    def rope_kv_write(self, q: Buf, k: Buf, v: Buf, dst_k: Buf, dst_v: Buf, elem_offset: int, pos: int,
                      n_tokens: int, spec: RopeSpec, n_elems: int):
        s = RopeSpecC(spec.head_dim, spec.theta)
        _check(lib().mdma_gfx950_rope_kv_write(self.ctx, q.handle, k.handle, v.handle, dst_k.handle,
                                               dst_v.handle, elem_offset, pos, n_tokens, C.byref(s), n_elems))

    def attn(self, q: Buf, kv: KvView, spec: AttnSpec, o: Buf):
        view = KvViewC(kv.k.handle, kv.v.handle, kv.len)
        s = AttnSpecC(spec.head_dim, spec.n_q_heads, spec.n_kv_heads)
        _check(lib().mdma_gfx950_attn(self.ctx, q.handle, C.byref(view), C.byref(s), o.handle))

    # -- extras --
    def greedy(self, logits: Buf, offset: int = 0, n: int | None = None) -> int:
        n = logits.len // 4 - offset if n is None else n
        out = C.c_uint32()
        _check(lib().mdma_gfx950_greedy(self.ctx, logits.handle, offset, n, C.byref(out)))
        return out.value

    def quantize_act(self, x: Buf, group: int, q: Buf, d: Buf, sum16: Buf):
        _check(lib().mdma_gfx950_quantize_act(self.ctx, x.handle, group, q.handle, d.handle, sum16.handle))

    def block_dot_i32(self, w: QWeight, qx: Buf, out: Buf):
        _check(lib().mdma_gfx950_block_dot_i32(self.ctx, C.byref(w.c()), qx.handle, out.handle))

    def time_next_gemv(self, start_event: int, stop_event: int):
        """Have the next GEMV kernel's dispatch timestamp these hipEvent_t handles."""
        _check(lib().mdma_gfx950_time_next_gemv(self.ctx, start_event, stop_event))

    def reserve_scratch(self, nbytes: int):
        _check(lib().mdma_gfx950_reserve_scratch(self.ctx, nbytes))

    def set_replay_params(self, params: "Buf | None", capacity: int = 0):
        """ReplayParams (src/backend/rocm/graph.rs:12-15): with params (a
        device buffer of two uint32, token and position) set, embed, rope,
        rope_kv_write, kv_write and attn read them from device memory when
        they run; None clears it."""
        _check(lib().mdma_gfx950_set_replay_params(self.ctx, params.handle if params is not None else None,
                                                   capacity))

    def capture(self, fn) -> "Graph":
        """Record the launches fn() makes into a replayable HIP graph."""
        _check(lib().mdma_gfx950_graph_begin(self.ctx))
        try:
            fn()
        finally:
            h = C.c_void_p()
            st = lib().mdma_gfx950_graph_end(self.ctx, C.byref(h))
        _check(st)
        return Graph(h.value, self)


class Graph:
    def __init__(self, handle, backend: Gfx950Backend):
        self.handle = handle
        self.backend = backend

    def launch(self):
        _check(lib().mdma_gfx950_graph_launch(self.backend.ctx, self.handle))

    def close(self):
        if self.handle:
            h, self.handle = self.handle, None
            if self.backend.ctx is not None:
                lib().mdma_gfx950_graph_destroy(h)

    def __del__(self):
        self.close()
