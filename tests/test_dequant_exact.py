"""Why the rounding order inside the block decoders cannot matter.

The reference's CPU backend dequantizes through candle-core's GgmlType::to_float
(/root/reference/src/backend/cpu/dequant.rs:36; candle is not vendored), the
oracle restates the formulas (oracle/oracle.c deq_*), and the GPU kernels
evaluate them in their own orders. They agree bit for bit because every
product in these formats is exact in f32:
  - Q8_0: q * d, an int8 (8 bits) times an f16 (11 significant bits);
  - Q6_K: d * sc * q, f16 d, int8 sc, 6-bit q: at most 11 + 7 + 5 = 23
    significant bits, so any two of the three multiply exactly and the
    triple product is exact in every order;
  - Q4_K: d * sc and dmin * m (6-bit sc, m: 17 bits) and (d * sc) * q (4-bit
    q: 21 bits) are exact; only the final subtraction d*sc*q - dmin*m rounds,
    once, so a fused multiply-subtract gives the same f32.
The checks run over every finite f16 scale against the integer ranges'
extremes and random interiors, and a format one bit wider fails them (so the
checks can see an inexact product).
"""
import numpy as np

F16 = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
D = F16[np.isfinite(F16)].astype(np.float32)  # every finite f16 value, widened exactly


def exact_in_f32(a32, b32):
    """a * b in f32 equals the exact (f64) product for every pair."""
    prod32 = (a32 * b32).astype(np.float64)
    return np.array_equal(prod32, a32.astype(np.float64) * b32.astype(np.float64))


def test_q8_0_products_exact():
    q = np.arange(-128, 128, dtype=np.float32)
    for chunk in np.array_split(D, 16):
        assert exact_in_f32(chunk[:, None], q[None, :])


def test_q6_k_triple_products_exact_in_every_order():
    rng = np.random.default_rng(1)
    sc = np.concatenate([[-128, -127, -65, -1, 1, 63, 127], rng.integers(-128, 128, 9)]).astype(np.float32)
    q = np.concatenate([[-32, -31, -17, -1, 1, 15, 31], rng.integers(-32, 32, 9)]).astype(np.float32)
    d = D[:, None, None]
    s, qq = sc[None, :, None], q[None, None, :]
    a = (d * s) * qq                     # candle / the oracle: (d * sc) * q
    b = d * (s * qq)                     # the int8 kernels: d * (sc * isum)
    c = (d * qq) * s
    exact = d.astype(np.float64) * s.astype(np.float64) * qq.astype(np.float64)
    assert np.array_equal(a, b) and np.array_equal(a, c)
    assert np.array_equal(a.astype(np.float64), exact)


def test_q4_k_products_exact_and_one_rounding():
    sc = np.arange(64, dtype=np.float32)
    q = np.arange(16, dtype=np.float32)
    for chunk in np.array_split(D, 64):
        d1 = chunk[:, None] * sc[None, :]
        assert np.array_equal(d1.astype(np.float64), chunk[:, None].astype(np.float64) * sc[None, :].astype(np.float64))
        prod = d1[:, :, None] * q[None, None, :]
        assert np.array_equal(prod.astype(np.float64), d1[:, :, None].astype(np.float64) * q.astype(np.float64))


def test_a_wider_format_would_not_be_exact():
    # Negative control: 10-bit scales and 7-bit quants (11 + 10 + 7 > 24
    # bits) give products that f32 rounds, and the checks above would fail.
    d = D[(D > 1) & (D < 2)]
    s = np.float32(1021.0)
    qq = np.float32(127.0)
    assert not exact_in_f32((d * s)[:, None], np.array([qq], np.float32)[None, :])
