"""Independent numpy statement of the GGUF block formats, in float64.

Test infrastructure. Written from the block layouts the reference restates in
/root/reference/src/backend/rocm/kernels/kernels.hip:13-27,44-68,82-122 and
src/backend/vulkan/kernels/kquant.glsl:30-102, not from oracle/oracle.c, so
that the oracle's decoders and this module check each other.

Each value is the block formula evaluated exactly: for these formats every
product the CPU backend forms in f32 (d*sc, dmin*m, (d*sc)*q) is exact in
f32, so f64 holds the same numbers; the one rounding the CPU adds is the
final f32 subtraction of Q4_K's (d*sc)*q - dmin*m, which f64 keeps exact.
"""
from __future__ import annotations

import numpy as np

F32, F16, Q8_0, Q4_K, Q6_K = 0, 1, 8, 12, 14
BLOCK = {F32: 1, F16: 1, Q8_0: 32, Q4_K: 256, Q6_K: 256}
TYPE_BYTES = {F32: 4, F16: 2, Q8_0: 34, Q4_K: 144, Q6_K: 210}


def _f16(b2: np.ndarray) -> np.ndarray:
    """Little-endian f16 in the last axis (2 bytes) -> f64."""
    return np.ascontiguousarray(b2).view(np.float16)[..., 0].astype(np.float64)


def q8_0(blocks: np.ndarray) -> np.ndarray:
    """[nb, 34] -> [nb, 32]: y = d * q."""
    d = _f16(blocks[:, 0:2])
    q = blocks[:, 2:34].view(np.int8).astype(np.float64)
    return d[:, None] * q


def q4_k_scales(s: np.ndarray):
    """The eight 6-bit (scale, min) pairs of a Q4_K header's 12 scale bytes
    [nb, 12] -> two [nb, 8] int arrays (get_scale_min_k4)."""
    s = s.astype(np.int64)
    sc = np.empty((s.shape[0], 8), np.int64)
    mn = np.empty_like(sc)
    for j in range(4):
        sc[:, j] = s[:, j] & 63
        mn[:, j] = s[:, j + 4] & 63
    for j in range(4, 8):
        sc[:, j] = (s[:, j + 4] & 15) | ((s[:, j - 4] >> 6) << 4)
        mn[:, j] = (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)
    return sc, mn


def q4_k(blocks: np.ndarray) -> np.ndarray:
    """[nb, 144] -> [nb, 256]: sub-block j (32 values) of element e = 32j + l
    takes nibble j%2 of quant byte 32*(j//2) + l; y = d*sc_j*q - dmin*m_j."""
    d, dmin = _f16(blocks[:, 0:2]), _f16(blocks[:, 2:4])
    sc, mn = q4_k_scales(blocks[:, 4:16])
    qs = blocks[:, 16:144].reshape(-1, 4, 32)
    out = np.empty((blocks.shape[0], 8, 32), np.float64)
    for j in range(8):
        q = ((qs[:, j // 2, :] >> (4 * (j % 2))) & 15).astype(np.float64)
        out[:, j, :] = (d * sc[:, j])[:, None] * q - (dmin * mn[:, j])[:, None]
    return out.reshape(-1, 256)


def q6_k(blocks: np.ndarray) -> np.ndarray:
    """[nb, 210] -> [nb, 256]: element e in half n = e//128, quarter r =
    (e%128)//32, lane l = e%32 has low nibble (shift 4 for r >= 2) of ql byte
    64n + l + 32*(r&1), high two bits (shift 2r) of qh byte 128 + 32n + l,
    sub-scale int8 byte 192 + e//16; y = d * sc * (u - 32)."""
    nb = blocks.shape[0]
    d = _f16(blocks[:, 208:210])
    sc = blocks[:, 192:208].view(np.int8).astype(np.float64)
    e = np.arange(256)
    n, r, l = e // 128, (e % 128) // 32, e % 32
    ql = blocks[:, 64 * n + l + 32 * (r & 1)].astype(np.int64)
    low = np.where(r >= 2, ql >> 4, ql) & 15
    high = (blocks[:, 128 + 32 * n + l].astype(np.int64) >> (2 * r)) & 3
    u = (low | (high << 4)) - 32
    return d[:, None] * sc[:, e // 16] * u.astype(np.float64) if nb else np.zeros((0, 256))


def dequantize(dtype: int, raw, rows: int, cols: int) -> np.ndarray:
    """[rows, cols] float64 values of a GGUF tensor's bytes."""
    raw = np.ascontiguousarray(raw).view(np.uint8).reshape(-1)
    if dtype == F32:
        return raw.view(np.float32).astype(np.float64).reshape(rows, cols)
    if dtype == F16:
        return raw.view(np.float16).astype(np.float64).reshape(rows, cols)
    blocks = raw.reshape(-1, TYPE_BYTES[dtype])
    fn = {Q8_0: q8_0, Q4_K: q4_k, Q6_K: q6_k}[dtype]
    return fn(blocks).reshape(rows, cols)
