"""GGUF v3 writer and reader for synthetic Llama models.

The writer plays the role of the reference's in-memory test writer
(/root/reference/src/gguf/tests.rs:10-128): it lays out a header, typed
metadata, tensor descriptors (ggml dims order: ne0 = columns first) and
32-byte-aligned tensor data. The reader returns descriptors with dims
reversed to mdma's `[rows, cols]` convention (src/gguf.rs:23, :198-231)
and memory-maps payloads, so multi-GB models are never copied whole.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass

import numpy as np

from .synth import BLOCK_SIZE, TYPE_SIZE

MAGIC = b"GGUF"
ALIGN = 32
T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 = range(13)


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(v) -> tuple[int, bytes]:
    if isinstance(v, bool):
        return T_BOOL, struct.pack("<?", v)
    if isinstance(v, int):
        return T_U32, struct.pack("<I", v)
    if isinstance(v, float):
        return T_F32, struct.pack("<f", v)
    if isinstance(v, str):
        return T_STR, _str(v)
    raise TypeError(type(v))


@dataclass
class TensorDesc:
    name: str
    dtype: int
    shape: tuple  # mdma order: [rows, cols]
    offset: int  # absolute file offset
    n_bytes: int


def tensor_bytes(dtype: int, shape) -> int:
    cols = shape[-1]
    rows = int(np.prod(shape[:-1])) if len(shape) > 1 else 1
    if cols % BLOCK_SIZE[dtype]:
        raise ValueError(f"tensor width {cols} is not whole blocks of {BLOCK_SIZE[dtype]}")
    return rows * cols // BLOCK_SIZE[dtype] * TYPE_SIZE[dtype]


def write(path: str, metadata: dict, tensors: list) -> None:
    """tensors: [(name, dtype, shape_rows_cols, payload ndarray-of-bytes)]."""
    kv = b"".join(_str(k) + struct.pack("<I", _value(v)[0]) + _value(v)[1] for k, v in metadata.items())
    infos, offset = [], 0
    for name, dtype, shape, payload in tensors:
        n = tensor_bytes(dtype, shape)
        if payload.nbytes != n:
            raise ValueError(f"{name}: payload {payload.nbytes} bytes, expected {n}")
        dims = list(reversed(shape))
        infos.append(_str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
                     + struct.pack("<IQ", dtype, offset))
        offset += (n + ALIGN - 1) // ALIGN * ALIGN
    head = MAGIC + struct.pack("<IQQ", 3, len(tensors), len(metadata)) + kv + b"".join(infos)
    pad = (-len(head)) % ALIGN
    with open(path, "wb") as f:
        f.write(head + b"\0" * pad)
        for _, dtype, shape, payload in tensors:
            b = np.ascontiguousarray(payload).view(np.uint8).reshape(-1)
            f.write(b.tobytes())
            f.write(b"\0" * ((-b.nbytes) % ALIGN))


def write_stream(path: str, metadata: dict, tensors: list) -> None:
    """Like write(), with each payload given as a zero-argument function that is
    called only when its bytes are written, so multi-GB models never sit in
    memory whole. tensors: [(name, dtype, shape_rows_cols, make_payload)]."""
    kv = b"".join(_str(k) + struct.pack("<I", _value(v)[0]) + _value(v)[1] for k, v in metadata.items())
    infos, offset = [], 0
    for name, dtype, shape, _ in tensors:
        n = tensor_bytes(dtype, shape)
        dims = list(reversed(shape))
        infos.append(_str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
                     + struct.pack("<IQ", dtype, offset))
        offset += (n + ALIGN - 1) // ALIGN * ALIGN
    head = MAGIC + struct.pack("<IQQ", 3, len(tensors), len(metadata)) + kv + b"".join(infos)
    with open(path, "wb") as f:
        f.write(head + b"\0" * ((-len(head)) % ALIGN))
        for name, dtype, shape, make in tensors:
            b = np.ascontiguousarray(make()).view(np.uint8).reshape(-1)
            if b.nbytes != tensor_bytes(dtype, shape):
                raise ValueError(f"{name}: payload {b.nbytes} bytes, expected {tensor_bytes(dtype, shape)}")
            f.write(b.tobytes())
            f.write(b"\0" * ((-b.nbytes) % ALIGN))


class Reader:
    def __init__(self, path: str):
        self.path = path
        self.mm = np.memmap(path, dtype=np.uint8, mode="r")
        self.pos = 0
        if bytes(self.mm[:4]) != MAGIC:
            raise ValueError("not a GGUF file")
        self.pos = 4
        version, n_t, n_kv = self._u32(), self._u64(), self._u64()
        if version not in (2, 3):
            raise ValueError(f"GGUF version {version}")
        self.metadata = {}
        for _ in range(n_kv):
            k = self._s()
            self.metadata[k] = self._val(self._u32())
        align = int(self.metadata.get("general.alignment", ALIGN))
        raw = []
        for _ in range(n_t):
            name = self._s()
            nd = self._u32()
            dims = [self._u64() for _ in range(nd)]
            dtype, off = self._u32(), self._u64()
            raw.append((name, dtype, tuple(reversed(dims)), off))
        data = (self.pos + align - 1) // align * align
        self.tensors = {n: TensorDesc(n, t, s, data + o, tensor_bytes(t, s)) for n, t, s, o in raw}

    def _take(self, n):
        b = bytes(self.mm[self.pos:self.pos + n])
        self.pos += n
        return b

    def _u32(self):
        return struct.unpack("<I", self._take(4))[0]

    def _u64(self):
        return struct.unpack("<Q", self._take(8))[0]

    def _s(self):
        return self._take(self._u64()).decode()

    def _val(self, t):
        fmt = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i", T_F32: "<f",
               T_BOOL: "<?", T_U64: "<Q", T_I64: "<q", T_F64: "<d"}
        if t == T_STR:
            return self._s()
        if t == T_ARR:
            et, n = self._u32(), self._u64()
            return [self._val(et) for _ in range(n)]
        f = fmt[t]
        return struct.unpack(f, self._take(struct.calcsize(f)))[0]

    def bytes_of(self, name: str) -> np.ndarray:
        d = self.tensors[name]
        return self.mm[d.offset:d.offset + d.n_bytes]
