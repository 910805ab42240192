"""Seeded synthetic GGUF blocks and activations with the benchmark distributions.

One counter-based splitmix64 stream per (seed, purpose) feeds everything, so a
JSON report that names the seed names the exact bytes. Normals come from
Box-Muller over two 53-bit uniforms.

Block layouts are GGUF's (the reference reads them through candle's
`GgmlType`, /root/reference/src/backend/cpu/dequant.rs:40-56):
  Q8_0  34 B:  f16 d | i8 qs[32]
  Q4_K 144 B:  f16 d | f16 dmin | u8 scales[12] | u8 qs[128]
  Q6_K 210 B:  u8 ql[128] | u8 qh[64] | i8 scales[16] | f16 d
"""
from __future__ import annotations

import numpy as np

GGML_F32, GGML_F16, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K = 0, 1, 8, 12, 14
BLOCK_SIZE = {GGML_F32: 1, GGML_F16: 1, GGML_Q8_0: 32, GGML_Q4_K: 256, GGML_Q6_K: 256}
TYPE_SIZE = {GGML_F32: 4, GGML_F16: 2, GGML_Q8_0: 34, GGML_Q4_K: 144, GGML_Q6_K: 210}
NAMES = {GGML_F32: "F32", GGML_F16: "F16", GGML_Q8_0: "Q8_0", GGML_Q4_K: "Q4_K", GGML_Q6_K: "Q6_K"}

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 24


def row_bytes(dtype: int, n_in: int) -> int:
    bs = BLOCK_SIZE[dtype]
    if n_in % bs:
        raise ValueError(f"{NAMES[dtype]} row width {n_in} is not a multiple of {bs}")
    return n_in // bs * TYPE_SIZE[dtype]


class Stream:
    """splitmix64 as a counter-based generator: word i = mix(seed + (i+1)*gamma)."""

    def __init__(self, seed: int):
        self.state = np.uint64(seed & 0xFFFFFFFFFFFFFFFF)
        self.pos = 0

    def u64(self, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.uint64)
        with np.errstate(over="ignore"):
            for s in range(0, n, _CHUNK):
                m = min(_CHUNK, n - s)
                i = np.arange(self.pos + s + 1, self.pos + s + 1 + m, dtype=np.uint64)
                z = self.state + i * _GAMMA
                z = (z ^ (z >> np.uint64(30))) * _M1
                z = (z ^ (z >> np.uint64(27))) * _M2
                out[s:s + m] = z ^ (z >> np.uint64(31))
        self.pos += n
        return out

    def uniform(self, n: int) -> np.ndarray:
        """Uniform doubles in (0, 1)."""
        return ((self.u64(n) >> np.uint64(11)).astype(np.float64) + 0.5) * (1.0 / (1 << 53))

    def ints(self, n: int, lo: int, hi: int) -> np.ndarray:
        """Integers uniform in [lo, hi] (inclusive)."""
        span = np.uint64(hi - lo + 1)
        return (self.u64(n) % span).astype(np.int64) + lo

    def bytes(self, n: int) -> np.ndarray:
        """Uniform bytes: the little-endian bytes of ceil(n/8) words."""
        return self.u64((n + 7) // 8).view(np.uint8)[:n].copy()

    def normal(self, n: int) -> np.ndarray:
        m = (n + 1) // 2
        u1, u2 = self.uniform(m), self.uniform(m)
        r = np.sqrt(-2.0 * np.log(u1))
        z = np.concatenate([r * np.cos(2 * np.pi * u2), r * np.sin(2 * np.pi * u2)])
        return z[:n]


class FastStream:
    """Same interface and distributions as Stream, from numpy's PCG64: for
    large synthetic models whose bytes no test recomputes (about 30x faster)."""

    def __init__(self, seed: int):
        self.rng = np.random.Generator(np.random.PCG64(seed & 0xFFFFFFFFFFFFFFFF))

    def uniform(self, n: int) -> np.ndarray:
        return self.rng.random(n)

    def ints(self, n: int, lo: int, hi: int) -> np.ndarray:
        return self.rng.integers(lo, hi + 1, n, dtype=np.int64)

    def bytes(self, n: int) -> np.ndarray:
        return np.frombuffer(self.rng.bytes(n), dtype=np.uint8).copy()

    def normal(self, n: int) -> np.ndarray:
        return self.rng.standard_normal(n)


def f16_bytes(v: np.ndarray) -> np.ndarray:
    return np.asarray(v, dtype=np.float32).astype(np.float16).view(np.uint8).reshape(-1, 2)


def pack_q4k_scales(sc: np.ndarray, m: np.ndarray) -> np.ndarray:
    """Inverse of get_scale_min_k4 (reference kernels.hip:19-27): 8 six-bit
    scales and mins per block into the 12-byte GGUF field. sc, m: [n, 8]."""
    sc = sc.astype(np.uint8)
    m = m.astype(np.uint8)
    out = np.zeros((sc.shape[0], 12), dtype=np.uint8)
    out[:, 0:4] = (sc[:, 0:4] & 63) | ((sc[:, 4:8] >> 4) << 6)
    out[:, 4:8] = (m[:, 0:4] & 63) | ((m[:, 4:8] >> 4) << 6)
    out[:, 8:12] = (sc[:, 4:8] & 15) | ((m[:, 4:8] & 15) << 4)
    return out


def q4k_blocks(n_blocks: int, seed: int, fast: bool = False, d_scale: float = 1e-3) -> np.ndarray:
    """Q4_K: d, dmin = f16(|N(0,1)|*1e-3), six-bit scales and
    mins uniform in [0,63], 4-bit quants uniform in [0,15]."""
    s = (FastStream if fast else Stream)(seed)
    d = np.abs(s.normal(n_blocks)) * d_scale
    dmin = np.abs(s.normal(n_blocks)) * d_scale
    sc = s.ints(n_blocks * 8, 0, 63).reshape(n_blocks, 8)
    m = s.ints(n_blocks * 8, 0, 63).reshape(n_blocks, 8)
    blk = np.empty((n_blocks, 144), dtype=np.uint8)
    blk[:, 0:2] = f16_bytes(d)
    blk[:, 2:4] = f16_bytes(dmin)
    blk[:, 4:16] = pack_q4k_scales(sc, m)
    blk[:, 16:144] = s.bytes(n_blocks * 128).reshape(n_blocks, 128)
    return blk.reshape(-1)


def q6k_blocks(n_blocks: int, seed: int, fast: bool = False, d_scale: float = 1e-3) -> np.ndarray:
    """Q6_K: uniform ql/qh bytes, int8 sub-scales uniform in
    [-64,63], d = f16(|N(0,1)|*1e-3)."""
    s = (FastStream if fast else Stream)(seed)
    blk = np.empty((n_blocks, 210), dtype=np.uint8)
    blk[:, 0:192] = s.bytes(n_blocks * 192).reshape(n_blocks, 192)
    blk[:, 192:208] = s.ints(n_blocks * 16, -64, 63).astype(np.int8).view(np.uint8).reshape(n_blocks, 16)
    blk[:, 208:210] = f16_bytes(np.abs(s.normal(n_blocks)) * d_scale)
    return blk.reshape(-1)


def q8_0_blocks(n_blocks: int, seed: int, fast: bool = False, d_scale: float = 0.02) -> np.ndarray:
    """Q8_0: fp16 d = |N(0,1)|*0.02, int8 quants uniform in [-127,127]."""
    s = (FastStream if fast else Stream)(seed)
    blk = np.empty((n_blocks, 34), dtype=np.uint8)
    blk[:, 0:2] = f16_bytes(np.abs(s.normal(n_blocks)) * d_scale)
    blk[:, 2:34] = s.ints(n_blocks * 32, -127, 127).astype(np.int8).view(np.uint8).reshape(n_blocks, 32)
    return blk.reshape(-1)


def weight(dtype: int, n_out: int, n_in: int, seed: int, fast: bool = False) -> np.ndarray:
    """Raw GGUF bytes of an [n_out, n_in] weight with the benchmark distribution
    of its dtype (fast: PCG64 stream, see FastStream)."""
    nb = n_out * (n_in // BLOCK_SIZE[dtype])
    if dtype == GGML_Q4_K:
        return q4k_blocks(nb, seed, fast)
    if dtype == GGML_Q6_K:
        return q6k_blocks(nb, seed, fast)
    if dtype == GGML_Q8_0:
        return q8_0_blocks(nb, seed, fast)
    if dtype == GGML_F32:
        return normal_f32(n_out * n_in, seed).view(np.uint8)
    if dtype == GGML_F16:
        return normal_f32(n_out * n_in, seed).astype(np.float16).view(np.uint8)
    raise ValueError(dtype)


def normal_f32(n: int, seed: int, sigma: float = 1.0) -> np.ndarray:
    return (Stream(seed).normal(n) * sigma).astype(np.float32)


def tokens(n: int, vocab: int, seed: int) -> np.ndarray:
    return Stream(seed).ints(n, 0, vocab - 1).astype(np.uint32)
