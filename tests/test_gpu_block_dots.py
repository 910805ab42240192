"""The int32 sub-block dots of the production int8 kernels, bit for bit.

The block-dot capture (mdma_gfx950_capture_block_dots) makes the kernels a
call routes to store every int32 sub-block dot they form; each must equal
the oracle's orc_block_dot_i32 on the int8 activations the route quantizes
(per 256 for the GEMVs, per 32 for the prefill GEMMs). This pins the int32
accumulators of the row-team kernels (every activation path: x quantized in
the prologue, x's cached int8 form staged in LDS, quantized x buffers), of
the MFMA batch GEMV and of both prefill GEMMs, as the reference pins its
int8 matrix-core fragments (src/backend/rocm/tests.rs:1861-1925), including
the extremes: activations at +-127 and weights at the ends of their ranges
(Q4_K 0 and 15, Q6_K -32 and 31, Q8_0 -128 and 127).
"""
import numpy as np
import pytest

import npq
from mdma_amd import backend as bm
from mdma_amd import synth
from oracle import ffi
from ties import near_tie_x

pytestmark = pytest.mark.gpu
Q8, Q4K, Q6K = 8, 12, 14
BLOCK = {Q8: (32, 34), Q4K: (256, 144), Q6K: (256, 210)}


def extreme_weight(dtype, rows, k, seed):
    """Raw blocks of the benchmark distribution with the quant range's ends
    planted: row 0's first block all at the maximum, row 1's at the minimum,
    row 2's alternating (rows and blocks past them stay random)."""
    raw = synth.weight(dtype, rows, k, seed).copy()
    bs, ts = BLOCK[dtype]
    blk = raw.reshape(rows, k // bs, ts)
    if dtype == Q8:
        q = blk[:, 0, 2:34].view(np.int8)
        q[0], q[1], q[2, ::2], q[2, 1::2] = 127, -128, 127, -128
    elif dtype == Q4K:
        blk[0, 0, 16:], blk[1, 0, 16:], blk[2, 0, 16:] = 0xFF, 0x00, 0xF0
    else:  # ql (128) and qh (64): 63 everywhere, 0 everywhere, alternating
        blk[0, 0, :192], blk[1, 0, :192] = 0xFF, 0x00
        blk[2, 0, :128], blk[2, 0, 128:192] = 0x0F, 0x33
    return raw


def extreme_x(T, k, seed):
    """Token 0: near-tie activations for the route's quantization group (the
    product's rounding decides them, see tests/ties.py); token 1 at +1
    everywhere (every int8 value 127); token 2 alternating +-1 (+-127); the
    rest normal."""
    group = 32 if T >= ffi.GEMM_MIN_TOKENS else 256
    x = synth.normal_f32(T * k, seed).reshape(T, k)
    x[0] = near_tie_x(k // group, group, seed)
    if T > 1:
        x[1] = 1.0
    if T > 2:
        x[2, ::2], x[2, 1::2] = 1.0, -1.0
    return x.reshape(-1)


def q_of(x, T, k, group):
    return np.concatenate([ffi.quantize_act(x[t * k:(t + 1) * k], group)[0] for t in range(T)])


def subs(dtype, k):
    return k // 16 if dtype == Q6K else k // 32


def capture(be, calls, slots):
    cap = be.alloc(slots * 4)
    be.upload(cap, 0, np.full(slots, -(2 ** 31), np.int32))
    be.capture_block_dots(cap)
    try:
        calls()
        be.join_execution()
    finally:
        be.capture_block_dots(None)
    return be.download(cap, 0, slots * 4).view(np.int32).copy()


def q4k_sub_scales(raw, rows, k):
    """[rows, k/32] six-bit Q4_K sub-block scales (the f16-path GEMM folds
    them into its weight operand: its dots are sc * dot)."""
    hd = raw.reshape(rows, k // 256, 144)[:, :, 4:16].reshape(-1, 12)
    sc, _ = npq.q4_k_scales(hd)
    return sc.reshape(rows, k // 32)


def expected(dtype, raw, rows, k, q, T, folded=False):
    want = ffi.block_dot_i32(dtype, raw, rows, k, q, T)
    if folded:
        want = want * q4k_sub_scales(raw, rows, k)[None].astype(np.int64)
    return want.astype(np.int64)


# Routes by token count: 1 (prologue-quantized x; Q8_0 a quantized buffer),
# 2 (row teams of 2 tokens), 3, 5, 8, 13 and 16 (MFMA batch GEMV), 40 (batch
# GEMV launches of 16, 16 and 8 tokens), 64 and 80 (prefill GEMM,
# activations per 32).
ROUTES = [1, 2, 3, 5, 8, 13, 16, 40, 64, 80]


@pytest.mark.parametrize("k", [1024, 14336])
@pytest.mark.parametrize("dtype", [Q4K, Q6K, Q8])
def test_qmatmul_block_dots_every_route(backend, dtype, k):
    rows = 80
    raw = extreme_weight(dtype, rows, k, 900 + dtype)
    w = backend.upload_weight(raw, dtype, (rows, k))
    backend.set_act_mode(bm.ACT_I8)
    try:
        for T in ROUTES:
            x = extreme_x(T, k, 901 + T)
            xb, yb = backend.f32_buf(x), backend.alloc(T * rows * 4)
            kinds = [bm.PREFILL_AUTO] if T < ffi.GEMM_MIN_TOKENS or dtype != Q4K else [bm.PREFILL_AUTO, bm.PREFILL_I8]
            for kind in kinds:
                backend.set_prefill_kernel(kind)
                got = capture(backend, lambda: backend.qmatmul(w, xb, yb), T * rows * subs(dtype, k))
                group = 32 if T >= ffi.GEMM_MIN_TOKENS else 256
                folded = dtype == Q4K and T >= ffi.GEMM_MIN_TOKENS and kind == bm.PREFILL_AUTO
                want = expected(dtype, raw, rows, k, q_of(x, T, k, group), T, folded)
                g = got.reshape(want.shape)
                bad = np.argwhere(g != want)
                assert bad.size == 0, (f"dtype {dtype} k {k} T {T} kind {kind}: {len(bad)} of {want.size} differ; "
                                       f"first (t, row, sub) {bad[:6].tolist()} got {g[tuple(bad[:6].T)]} "
                                       f"want {want[tuple(bad[:6].T)]}")
            xb.close(), yb.close()
    finally:
        backend.set_prefill_kernel(bm.PREFILL_AUTO)
        backend.set_act_mode(bm.ACT_F32)


@pytest.mark.parametrize("dtype", [Q4K, Q6K])
def test_gate_up_block_dots(backend, dtype):
    """The fused gate/up: one token with x quantized in the prologue, one
    token with x's int8 form cached by the producing rmsnorm (staged through
    LDS), the batch GEMV and the prefill GEMM; gate's dots then up's."""
    rows, k = 96, 4096
    raws = [extreme_weight(dtype, rows, k, 910 + i) for i in range(2)]
    ws = [backend.upload_weight(r, dtype, (rows, k)) for r in raws]
    backend.set_act_mode(bm.ACT_I8)
    try:
        for T, cached in ((1, False), (1, True), (5, False), (16, False), (64, False)):
            x = extreme_x(T, k, 920 + T)
            if cached:
                xr = backend.f32_buf(x)
                xb = backend.alloc(T * k * 4)
                backend.rmsnorm(backend.f32_buf(np.full(k, 0.75, np.float32)), xr, xb, 1e-5)
                x = backend.download_f32(xb).copy()
            else:
                xb = backend.f32_buf(x)
            g, u, y = (backend.alloc(T * rows * 4) for _ in range(3))
            n = T * rows * subs(dtype, k)
            got = capture(backend, lambda: backend.ffn_gate_up(ws[0], ws[1], xb, g, u, y), 2 * n)
            group = 32 if T >= ffi.GEMM_MIN_TOKENS else 256
            q = q_of(x, T, k, group)
            folded = dtype == Q4K and T >= ffi.GEMM_MIN_TOKENS
            for i in range(2):
                want = expected(dtype, raws[i], rows, k, q, T, folded)
                assert np.array_equal(got[i * n:(i + 1) * n].reshape(want.shape), want), (dtype, T, cached, i)
    finally:
        backend.set_act_mode(bm.ACT_F32)


@pytest.mark.parametrize("T", [1, 3])
def test_qkv_block_dots(backend, T):
    """The fused QKV launch (three weights, one activation): each weight's
    dots in its own region."""
    k = 2048
    shapes = [(128, k), (32, k), (48, k)]
    raws = [extreme_weight(Q4K, r, k, 930 + i) for i, (r, _) in enumerate(shapes)]
    ws = [backend.upload_weight(raw, Q4K, s) for raw, s in zip(raws, shapes)]
    x = extreme_x(T, k, 931)
    xb = backend.f32_buf(x)
    outs = [backend.alloc(T * r * 4) for r, _ in shapes]
    backend.set_act_mode(bm.ACT_I8)
    try:
        ns = [T * r * subs(Q4K, k) for r, _ in shapes]
        got = capture(backend, lambda: backend.qmatmul_qkv(ws[0], ws[1], ws[2], xb, *outs), sum(ns))
    finally:
        backend.set_act_mode(bm.ACT_F32)
    q = q_of(x, T, k, 256)
    off = 0
    for i, (r, _) in enumerate(shapes):
        want = expected(Q4K, raws[i], r, k, q, T)
        assert np.array_equal(got[off:off + ns[i]].reshape(want.shape), want), i
        off += ns[i]


def test_capture_rejects_a_short_buffer(backend):
    rows, k = 16, 512
    w = backend.upload_weight(synth.weight(Q4K, rows, k, 940), Q4K, (rows, k))
    xb, yb = backend.f32_buf(synth.normal_f32(k, 941)), backend.alloc(rows * 4)
    small = backend.alloc(rows * subs(Q4K, k) * 4 - 4)
    backend.capture_block_dots(small)
    try:
        with pytest.raises(bm.ShapeMismatch):
            backend.qmatmul_i8(w, xb, yb)
    finally:
        backend.capture_block_dots(None)
    backend.qmatmul_i8(w, xb, yb)  # capture off: runs
