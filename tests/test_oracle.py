"""Pins of the CPU oracle (oracle/oracle.c) before any GPU result is trusted.

Each check is independent of the oracle's own code: the reference's own
known-answer tests and hand-computed values (restated with their
file:line), a second restatement of the block layouts from a different
reference file, closed forms, encode->decode round trips, f64 brute force,
and numpy's independent float16 conversion.
"""
import math

import numpy as np
import pytest

from mdma_amd import synth
from oracle import ffi

Q8, Q4K, Q6K, F32 = 8, 12, 14, 0


# ---------------------------------------------------------------- f16 -----

def test_f16_matches_reference_rounding_cases():
    # src/backend/test_support.rs:265-273: adjacent halves around one, a
    # negative value and signed zero.
    got = [ffi.f16_to_f32(ffi.f32_to_f16(v)) for v in (1.0004, 1.0008, -2.0008)]
    assert got == [1.0, np.float32(1.0009766), -2.0]
    assert ffi.f32_to_f16(-0.0) == 0x8000
    # src/backend/test_support.rs:276-281: exact little-endian halves.
    assert [ffi.f32_to_f16(v) for v in (1.0, -2.0, -0.0, 1.0008)] == [0x3C00, 0xC000, 0x8000, 0x3C01]


def test_f16_conversions_match_numpy_everywhere():
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([ffi.f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.all(np.isnan(got[~fin & np.isnan(ref)]))
    xs = np.concatenate([synth.normal_f32(20000, 5) * 10.0 ** np.repeat(np.arange(-8, 6), 20000 // 14 + 1)[:20000],
                         np.array([65504, 65520, 65519.99, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8, 1e-9, 1e6],
                                  np.float32)]).astype(np.float32)
    want = xs.astype(np.float16).view(np.uint16)
    got = np.array([ffi.f32_to_f16(float(v)) for v in xs], dtype=np.uint16)
    assert np.array_equal(got, want)


# ------------------------------------------------------------- Q4_K -------

def q4k_packed_reference(raw: np.ndarray) -> np.ndarray:
    """The reference's known-answer formula (src/cache/layout/tests.rs:8-55):
    blocks repacked as pack_q4k does (src/cache/layout.rs:40-79, restated
    here from its published steps) and decoded through the three bit planes
    with value = 0.125*scale*q - 0.0625*min. A different derivation of the
    six-bit scales than get_scale_min_k4."""
    out = []
    for blk in raw.reshape(-1, 144):
        s = blk[4:16]
        planes = [0, 0, 0]
        for j in range(8):
            if j < 4:
                sc, mn = s[j] & 63, s[j + 4] & 63
            else:
                sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4)
                mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4)
            shift, par = (j // 2) * 8, j % 2
            planes[0] |= int(sc & 15) << (shift + par * 4)
            planes[1] |= int(mn & 15) << (shift + par * 4)
            planes[2] |= (int(sc >> 4) << (shift + par * 2)) | (int(mn >> 4) << (shift + 4 + par * 2))
        for i in range(256):
            j = i // 32
            shift, par = (j // 2) * 8, j % 2
            scale = ((planes[0] >> (shift + par * 4)) & 15) | (((planes[2] >> (shift + par * 2)) & 3) << 4)
            mn = ((planes[1] >> (shift + par * 4)) & 15) | (((planes[2] >> (shift + 4 + par * 2)) & 3) << 4)
            q = (blk[16 + (i // 64) * 32 + i % 32] >> ((j % 2) * 4)) & 15
            out.append(np.float32(0.125) * np.float32(scale) * np.float32(q) - np.float32(0.0625) * np.float32(mn))
    return np.array(out, dtype=np.float32)


@pytest.mark.parametrize("seed", range(0, 256, 5))
def test_q4k_known_answer_every_header_byte(seed):
    raw = (((np.arange(144 * 3, dtype=np.uint32) * 73 + seed * 31) & 255)).astype(np.uint8).reshape(3, 144)
    raw[:, 0:2] = np.frombuffer(np.float16(0.125).tobytes(), np.uint8)
    raw[:, 2:4] = np.frombuffer(np.float16(0.0625).tobytes(), np.uint8)
    got = ffi.embed(Q4K, raw.reshape(-1), 3, 256, [0, 1, 2]).reshape(-1)
    assert np.array_equal(got, q4k_packed_reference(raw.reshape(-1)))


def test_q4k_scale_encoder_roundtrip_and_rounding_order():
    # Every (scale, min) pair in [0,63]^2 appears; d/dmin are not powers of two,
    # so the rounding order (d*sc)*q - dmin*m of kernels.hip:62-67 is checked
    # against an f32 evaluation in that order.
    s = synth.Stream(11)
    n = 512
    sc = s.ints(n * 8, 0, 63).reshape(n, 8)
    m = s.ints(n * 8, 0, 63).reshape(n, 8)
    sc[:64, :] = np.arange(64).reshape(64, 1)
    m[:64, :] = np.arange(64).reshape(64, 1)[::-1]
    d = (np.abs(s.normal(n)) * 1e-3).astype(np.float16)
    dmin = (np.abs(s.normal(n)) * 1e-3).astype(np.float16)
    qs = s.bytes(n * 128).reshape(n, 128)
    blk = np.zeros((n, 144), np.uint8)
    blk[:, 0:2] = d.view(np.uint8).reshape(n, 2)
    blk[:, 2:4] = dmin.view(np.uint8).reshape(n, 2)
    blk[:, 4:16] = synth.pack_q4k_scales(sc, m)
    blk[:, 16:] = qs
    got = ffi.dequantize_row(Q4K, blk.reshape(-1), n * 256).reshape(n, 8, 32)
    for j in range(8):
        q = (qs[:, 32 * (j // 2):32 * (j // 2) + 32] >> (4 * (j % 2))) & 15
        d1 = d.astype(np.float32) * sc[:, j].astype(np.float32)
        m1 = dmin.astype(np.float32) * m[:, j].astype(np.float32)
        want = (d1[:, None] * q.astype(np.float32)).astype(np.float32) - m1[:, None]
        assert np.array_equal(got[:, j, :], want.astype(np.float32)), j


# ------------------------------------------------------------- Q6_K -------

def q6k_glsl_reference(raw: np.ndarray) -> np.ndarray:
    """Element-index formulation of Q6_K from the reference's Vulkan
    restatement (src/backend/vulkan/kernels/kquant.glsl:69-102): for element
    e: jb = e/128, quad = (e%128)/32, l = e%32; ql byte jb*64+l(+32 for odd
    quads), shifted by 4 for quads >= 2; qh byte 128+jb*32+l shifted 2*quad;
    scale byte 192+e/16; value = (d*s) * (u - 32)."""
    blocks = raw.reshape(-1, 210)
    e = np.arange(256)
    jb, within = e // 128, e % 128
    quad, l = within // 32, within % 32
    ql_off = jb * 64 + l + np.where(quad & 1, 32, 0)
    qh_off = 128 + jb * 32 + l
    sc_off = 192 + (jb * 128 + quad * 32 + l) // 16
    ql_shift = np.where(quad >= 2, 4, 0)
    out = []
    for blk in blocks:
        d = np.frombuffer(blk[208:210].tobytes(), np.float16)[0].astype(np.float32)
        u = ((blk[ql_off] >> ql_shift) & 15) | (((blk[qh_off] >> (2 * quad)) & 3) << 4)
        s = blk[sc_off].view(np.int8).astype(np.float32)
        ds = (d * s).astype(np.float32)
        out.append((ds * (u.astype(np.float32) - 32.0)).astype(np.float32))
    return np.concatenate(out)


def test_q6k_matches_second_reference_restatement():
    raw = synth.q6k_blocks(300, seed=3)
    # Extremes of the signed sub-scales with nonzero high bits
    # (src/backend/rocm/decode/tests.rs:60-62).
    raw.reshape(300, 210)[:8, 192] = 128
    raw.reshape(300, 210)[:8, 193] = 127
    got = ffi.dequantize_row(Q6K, raw, 300 * 256)
    assert np.array_equal(got, q6k_glsl_reference(raw))


def test_q6k_encode_decode_roundtrip():
    # Encode known six-bit quants from the element->byte map, decode with the
    # oracle; d = 1 and scale = 1 make the value the integer quant itself.
    s = synth.Stream(9)
    n = 64
    q = s.ints(n * 256, -32, 31).reshape(n, 256)
    blk = np.zeros((n, 210), np.uint8)
    u = (q + 32).astype(np.uint8)
    for e in range(256):
        jb, quad, l = e // 128, (e % 128) // 32, e % 32
        qlb = jb * 64 + l + (32 if quad & 1 else 0)
        blk[:, qlb] |= (u[:, e] & 15) << (4 if quad >= 2 else 0)
        blk[:, 128 + jb * 32 + l] |= (u[:, e] >> 4) << (2 * quad)
    blk[:, 192:208] = 1
    blk[:, 208:210] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    got = ffi.dequantize_row(Q6K, blk.reshape(-1), n * 256)
    assert np.array_equal(got, q.reshape(-1).astype(np.float32))


# ------------------------------------------------------------- Q8_0 -------

def test_q8_0_closed_form():
    raw = synth.q8_0_blocks(1000, seed=4).reshape(1000, 34)
    d = raw[:, :2].copy().view(np.float16).astype(np.float32).reshape(-1, 1)
    q = raw[:, 2:].view(np.int8).astype(np.float32)
    assert np.array_equal(ffi.dequantize_row(Q8, raw.reshape(-1), 32000), (q * d).astype(np.float32).reshape(-1))


# ----------------------------------------------------- qmatmul order ------

def f32w(vals):
    return np.asarray(vals, np.float32).view(np.uint8)


def test_qmatmul_hand_computed():
    # src/backend/test_support.rs:254-268 and src/backend/cpu/tests.rs:75-89.
    w = f32w([1.0, -2.0, 3.0, 4.0, 5.0, -6.0])
    x = np.array([2.0, -1.0, 0.5, -1.0, 2.0, 1.0], np.float32)
    expected = [5.5, 0.0, -2.0, 0.0]
    for tokens in (1, 2):
        got = ffi.qmatmul(F32, w, 2, 3, x[:3 * tokens]).reshape(-1)
        assert list(got) == expected[:2 * tokens]
    got = ffi.qmatmul(F32, f32w([1, 2, 3, 4, 5, 6]), 2, 3, np.ones(3, np.float32)).reshape(-1)
    assert list(got) == [6.0, 15.0]


def test_qmatmul_is_sequential_f32_without_fma():
    # A cancellation case where the sequential f32 sum, the FMA form and the
    # exact sum all differ: the oracle must give the sequential value.
    w = f32w([1e8, 1.0, -1e8, 1.0])
    x = np.ones(4, np.float32)
    got = ffi.qmatmul(F32, w, 1, 4, x)[0, 0]
    seq = np.float32(0)
    for v in (1e8, 1.0, -1e8, 1.0):
        seq = np.float32(seq + np.float32(v))
    assert got == seq == np.float32(1.0)


def test_qmatmul_batched_equals_sequential_and_threads_do_not_matter():
    # 19 tokens: two groups of eight run side by side, then three alone.
    w = synth.weight(Q4K, 33, 512, 5)
    x = synth.normal_f32(19 * 512, 6)
    full = ffi.qmatmul(Q4K, w, 33, 512, x, threads=7)
    for t in range(19):
        one = ffi.qmatmul(Q4K, w, 33, 512, x[t * 512:(t + 1) * 512], threads=1)
        assert np.array_equal(full[t], one[0])


def test_qmatmul_token_groups_keep_each_tokens_sequential_sum():
    # The cancellation case of the test above in every lane of an eight-token
    # group, with the tokens scaled apart: each lane keeps its own order.
    w = f32w([1e8, 1.0, -1e8, 1.0])
    x = np.concatenate([np.float32(2.0 ** k) * np.ones(4, np.float32) for k in range(9)])
    got = ffi.qmatmul(F32, w, 1, 4, x)[:, 0]
    assert list(got) == [np.float32(2.0 ** k) for k in range(9)]


@pytest.mark.parametrize("dtype", [Q8, Q4K, Q6K])
def test_qmatmul_within_rigorous_bound_of_f64(dtype):
    n_out, n_in = 64, 2048
    w = synth.weight(dtype, n_out, n_in, 7)
    x = synth.normal_f32(n_in, 8)
    W = ffi.dequantize(dtype, w, n_out, n_in)
    got = ffi.qmatmul(dtype, w, n_out, n_in, x)[0].astype(np.float64)
    exact = W.astype(np.float64) @ x.astype(np.float64)
    gamma = n_in * 2 ** -24 / (1 - n_in * 2 ** -24)
    bound = gamma * (np.abs(W).astype(np.float64) @ np.abs(x).astype(np.float64))
    assert np.all(np.abs(got - exact) <= bound)


def test_qmatmul_shape_rules():
    w = synth.weight(Q4K, 2, 256, 1)
    with pytest.raises(ffi.OracleError):
        ffi.qmatmul(Q4K, w, 2, 256, np.zeros(300, np.float32))  # not whole rows
    with pytest.raises(ffi.OracleError):
        ffi.qmatmul(Q4K, w, 2, 256, np.zeros(256, np.float32), y_elems=1)  # y too small
    with pytest.raises(ffi.OracleError):
        ffi.qmatmul(Q4K, w, 2, 128, np.zeros(128, np.float32))  # K-quant width


# ----------------------------------------------------- per-token ops ------

def test_rmsnorm_hand_computed():
    # src/backend/cpu/tests.rs:128-140.
    got = ffi.rmsnorm([1.0, 1.0], [3.0, 4.0], 0.0)
    scale = np.float32(1.0) / np.sqrt(np.float32(12.5))
    assert abs(got[0] - 3.0 * scale) < 1e-6 and abs(got[1] - 4.0 * scale) < 1e-6


def test_rmsnorm_rows_are_independent():
    w = np.array([1.0, 0.5, 2.0], np.float32)
    x = np.array([3.0, -1.0, 2.0, 0.5, 4.0, -2.0, 1.0, 1.0, 1.0], np.float32)
    full = ffi.rmsnorm(w, x, 1e-5)
    for t in range(3):
        assert np.array_equal(full[3 * t:3 * t + 3], ffi.rmsnorm(w, x[3 * t:3 * t + 3], 1e-5))


def test_rope_identity_and_angle():
    # src/backend/cpu/tests.rs:142-171.
    q, k = ffi.rope([1.0, 2.0, 3.0, 4.0], [5.0, 6.0], 0, 1, 2, 10000.0)
    assert list(q) == [1, 2, 3, 4] and list(k) == [5, 6]
    q, k = ffi.rope([1.0, 0.0], [1.0, 0.0], 1, 1, 2, 10000.0)
    assert abs(q[0] - math.cos(1.0)) < 1e-6 and abs(q[1] - math.sin(1.0)) < 1e-6


def test_rope_batched_positions_and_theta_formula():
    q = synth.normal_f32(3 * 2 * 8, 1)
    k = synth.normal_f32(3 * 1 * 8, 2)
    qb, kb = ffi.rope(q, k, 5, 3, 8, 500000.0)
    for t in range(3):
        qs, ks = ffi.rope(q[16 * t:16 * t + 16], k[8 * t:8 * t + 8], 5 + t, 1, 8, 500000.0)
        assert np.array_equal(qb[16 * t:16 * t + 16], qs) and np.array_equal(kb[8 * t:8 * t + 8], ks)
    c, s = ffi.rope_cos_sin(7, 8, 500000.0)
    for i in range(4):
        ang = 7 * 500000.0 ** (-2 * i / 8)
        assert abs(c[i] - math.cos(ang)) < 1e-6 and abs(s[i] - math.sin(ang)) < 1e-6


def test_silu_mul_hand_computed():
    got = ffi.silu_mul([0.0, 2.0], [1.0, 1.0])
    assert got[0] == 0.0 and abs(got[1] - 2.0 / (1.0 + math.exp(-2.0))) < 1e-6


def test_attention_hand_computed():
    # src/backend/cpu/tests.rs:186-214.
    o = ffi.attention([1.0, 0.0], [1.0, 0.0, 0.0, 1.0], [10.0, 20.0, 30.0, 40.0], 2, 2, 1, 1)
    scale = 1 / math.sqrt(2)
    e0, e1 = 1.0, math.exp(-scale)
    w0, w1 = e0 / (e0 + e1), e1 / (e0 + e1)
    assert abs(o[0] - (w0 * 10 + w1 * 30)) < 1e-5 and abs(o[1] - (w0 * 20 + w1 * 40)) < 1e-5


def test_attention_batched_causal_equals_decode_steps():
    # src/backend/cpu/tests.rs:306-357, with GQA (4 q heads on 2 kv heads).
    hd, nq, nkv, T = 4, 4, 2, 5
    q = synth.normal_f32(T * nq * hd, 1)
    k = synth.normal_f32(T * nkv * hd, 2)
    v = synth.normal_f32(T * nkv * hd, 3)
    full = ffi.attention(q, k, v, T, hd, nq, nkv)
    for t in range(T):
        kv = (t + 1) * nkv * hd
        one = ffi.attention(q[t * nq * hd:(t + 1) * nq * hd], k[:kv], v[:kv], t + 1, hd, nq, nkv)
        assert np.allclose(full[t * nq * hd:(t + 1) * nq * hd], one, atol=1e-6)


def test_greedy_ties_go_to_last_index_and_total_order():
    # src/sampler.rs:64-74: max_by(total_cmp) keeps the last maximum.
    assert ffi.greedy(np.array([1.0, 3.0, 2.0, 3.0, -1.0], np.float32)) == 3
    assert ffi.greedy(np.array([-0.0, 0.0, -0.0], np.float32)) == 1  # +0 > -0 in total order
    assert ffi.greedy(np.array([5.0], np.float32)) == 0
    assert ffi.greedy(np.zeros(0, np.float32)) == 0
    x = synth.normal_f32(32000, 4)
    assert ffi.greedy(x) == int(np.argmax(x))


# --------------------------------------------------- int8 activations -----

def brute_quantize(x, group):
    q, d = [], []
    for g in x.reshape(-1, group):
        amax = np.float32(0)
        for v in g:
            amax = max(amax, np.float32(abs(v)))
        d.append(np.float32(amax) / np.float32(127))
        inv = np.float32(0) if amax == 0 else np.float32(127) / np.float32(amax)
        for v in g:
            r = np.float32(v) * inv
            q.append(int(math.copysign(math.floor(abs(r) + 0.5), r)))
    return np.array(q, np.int8), np.array(d, np.float32)


@pytest.mark.parametrize("group", [32, 256])
def test_quantize_act_brute_force(group):
    x = synth.normal_f32(4 * 256, 3)
    x[:group] = 0.0  # zero group: d = 0, q = 0
    x[group + 5] = 1e-30
    q, d, s16 = ffi.quantize_act(x, group)
    bq, bd = brute_quantize(x, group)
    assert np.array_equal(q, bq) and np.array_equal(d.view(np.uint32), bd.view(np.uint32))
    assert np.array_equal(s16, q.astype(np.int32).reshape(-1, 16).sum(1))
    assert q.min() >= -127 and np.all(d[0] == 0) and np.all(q[:group] == 0)
    # Half-away rounding at exact .5: amax 127 makes inv = 1.
    x2 = np.zeros(group, np.float32)
    x2[0], x2[1], x2[2] = 127.0, 2.5, -2.5
    q2, _, _ = ffi.quantize_act(x2, group)
    assert list(q2[:3]) == [127, 3, -3]


@pytest.mark.parametrize("dtype", [Q8, Q4K, Q6K])
def test_block_dot_equals_dequantized_integer_weights(dtype):
    """With unit scales (d = 1, sc = 1, dmin = 0) the dequantized weight IS the
    integer quant, so the oracle's block dots must equal f64 sums of the
    dequantizer's output times qx: two independent code paths."""
    n_out, n_in, T = 5, 512, 2
    raw = synth.weight(dtype, n_out, n_in, 21).copy()
    one = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    if dtype == Q4K:
        b = raw.reshape(-1, 144)
        b[:, 0:2] = one
        b[:, 2:4] = 0
        b[:, 4:16] = synth.pack_q4k_scales(np.ones((len(b), 8), np.int64), np.zeros((len(b), 8), np.int64))
    elif dtype == Q6K:
        b = raw.reshape(-1, 210)
        b[:, 192:208] = 1
        b[:, 208:210] = one
    else:
        b = raw.reshape(-1, 34)
        b[:, 0:2] = one
    q, _, _ = ffi.quantize_act(synth.normal_f32(T * n_in, 22), 256)
    W = ffi.dequantize(dtype, raw, n_out, n_in).astype(np.int64)
    sub = 16 if dtype == Q6K else 32
    want = np.einsum("rsk,tsk->trs", W.reshape(n_out, -1, sub), q.astype(np.int64).reshape(T, -1, sub))
    assert np.array_equal(ffi.block_dot_i32(dtype, raw, n_out, n_in, q, T), want)


def test_block_dot_extremes_fit_int32():
    # Q8_0 worst case |isum| = 127*128*32 stays exact.
    raw = np.zeros((1, 34), np.uint8)
    raw[0, 2:] = np.int8(-127).view(np.uint8)
    qx = np.full(32, -128, np.int8)
    assert ffi.block_dot_i32(Q8, raw.reshape(-1), 1, 32, qx, 1)[0, 0, 0] == 127 * 128 * 32


# ------------------------------------------------- independent decoders ----

@pytest.mark.parametrize("dtype", [Q8, Q4K, Q6K])
def test_oracle_decoders_equal_independent_numpy_statement(dtype):
    """tests/npq.py states the block formats independently, in exact f64.
    The oracle's f32 values must be those exact values rounded once to f32
    (Q6_K and Q8_0 values are exact in f32; Q4_K's (d*sc)*q - dmin*m rounds
    once, in the subtraction)."""
    import npq
    rows, k = 64, 512 if dtype != Q8 else 288
    raw = synth.weight(dtype, rows, k, 123)
    got = ffi.dequantize_row(dtype, raw, rows * k)
    want = npq.dequantize(dtype, raw, rows, k).astype(np.float32).reshape(-1)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # All-byte-value blocks (every scale/min/high-bit pattern).
    nb = 300
    tsz = {Q8: 34, Q4K: 144, Q6K: 210}[dtype]
    rb = ((np.arange(nb * tsz, dtype=np.uint32) * 73 + 19) & 255).astype(np.uint8).reshape(nb, tsz)
    off = {Q8: 0, Q4K: 0, Q6K: 208}[dtype]
    rb[:, off:off + 2] = np.frombuffer(np.float16(0.0123).tobytes(), np.uint8)
    if dtype == Q4K:
        rb[:, 2:4] = np.frombuffer(np.float16(0.0071).tobytes(), np.uint8)
    bs = {Q8: 32, Q4K: 256, Q6K: 256}[dtype]
    got = ffi.dequantize_row(dtype, rb.reshape(-1), nb * bs)
    want = npq.dequantize(dtype, rb.reshape(-1), 1, nb * bs).astype(np.float32).reshape(-1)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
