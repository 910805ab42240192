"""The allocation-free int8 qmatmul (mdma_gfx950_qmatmul_i8_noalloc) against
the allocating entry point it varies (mdma_gfx950_qmatmul_i8), through the
C ABI on the GPU: two calls in a row, the second with a smaller input, and
the other int8 routes (row teams, the matrix-core batch GEMV, the prefill
GEMM, which runs unsplit here), plus the size limit.
"""
import numpy as np
import pytest

import npq
from conftest import abs_dot, assert_parity, f32_exact
from mdma_amd import backend as backend_mod
from mdma_amd import synth
from oracle import ffi

pytestmark = pytest.mark.gpu
Q8, Q4K, Q6K = 8, 12, 14
CANARY = np.float32(123456.25)


def both(be, w, x_h, rows):
    """(noalloc output, qmatmul_i8 output), each into a canary-tailed y."""
    T = x_h.size // w.shape[1]
    outs = []
    for fn in (be.qmatmul_i8_noalloc, be.qmatmul_i8):
        xb = be.f32_buf(x_h)  # a fresh buffer: no cached int8 form
        yb = be.f32_buf(np.full(T * rows + 8, CANARY, np.float32))
        fn(w, xb, yb)
        y = be.download_f32(yb)
        assert np.all(y[T * rows:] == CANARY), "wrote past the output"
        outs.append(y[:T * rows])
        xb.close()
        yb.close()
    return outs


def test_noalloc_equals_allocating_entry_two_calls(backend):
    # Call 1: Q4_K 4096x4096, 3 tokens (the matrix-core batch GEMV over int8 x
    # in the array).
    w1 = backend.upload_weight(synth.weight(Q4K, 4096, 4096, 1), Q4K, (4096, 4096))
    a, b = both(backend, w1, synth.normal_f32(3 * 4096, 2), 4096)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # Call 2, smaller: Q6_K 1024x4096, 2 tokens (row teams).
    w2 = backend.upload_weight(synth.weight(Q6K, 1024, 4096, 3), Q6K, (1024, 4096))
    a, b = both(backend, w2, synth.normal_f32(2 * 4096, 4), 1024)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("dtype,rows,k,T", [(Q8, 300, 1024, 1), (Q4K, 640, 4096, 8), (Q6K, 4096, 14336, 5)])
def test_noalloc_routes_bit_exact(backend, dtype, rows, k, T):
    """One token (Q8_0: x quantized separately; K-quants quantize in the
    kernel's prologue) and the batch GEMV (3..16 tokens, matrix cores) give
    the allocating entry point's bits."""
    raw = synth.weight(dtype, rows, k, 10 + T)
    w = backend.upload_weight(raw, dtype, (rows, k))
    a, b = both(backend, w, synth.normal_f32(T * k, 11 + T), rows)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("dtype", [Q8, Q4K, Q6K])
def test_noalloc_prefill_gemm_matches_oracle(backend, dtype):
    """64 tokens: the prefill GEMM route, unsplit here (its split-K partials
    would need scratch), against the oracle's per-32 requantized qmatmul at
    the int8 bar, and against the allocating entry point's result."""
    T, k, rows = 64, 1024, 384
    raw = synth.weight(dtype, rows, k, 20)
    x = synth.normal_f32(T * k, 21)
    w = backend.upload_weight(raw, dtype, (rows, k))
    a, b = both(backend, w, x, rows)
    q, d, _ = ffi.quantize_act(x, 32)
    xq = ffi.dequantize_act(q, d, 32)
    cpu = ffi.qmatmul(dtype, raw, rows, k, xq)
    W = npq.dequantize(dtype, raw, rows, k)
    exact, absum = f32_exact(W, xq), abs_dot(W, xq)
    assert_parity(a, cpu, exact, 1e-3, abs_sum=absum, what=f"noalloc gemm {dtype}")
    assert_parity(b, cpu, exact, 1e-3, abs_sum=absum, what=f"alloc gemm {dtype}")


def test_noalloc_rejects_oversize_and_keeps_cached_activations(backend):
    k, rows = 4096, 64
    w = backend.upload_weight(synth.weight(Q4K, rows, k, 30), Q4K, (rows, k))
    big = backend.alloc(2048 * k * 4)  # 8.4 M values: past the 8 MiB array
    y = backend.alloc(2048 * rows * 4)
    with pytest.raises(backend_mod.BufferBudget):
        backend.qmatmul_i8_noalloc(w, big, y)
    # An rmsnorm in the int8 mode caches its output's int8 form; a noalloc
    # call on another x in between must leave that cache usable.
    backend.set_act_mode(backend_mod.ACT_I8)
    try:
        xn = backend.alloc(k * 4)
        backend.rmsnorm(backend.f32_buf(np.ones(k, np.float32)), backend.f32_buf(synth.normal_f32(k, 31)), xn, 1e-5)
        other, yo = backend.f32_buf(synth.normal_f32(2 * k, 32)), backend.alloc(2 * rows * 4)
        backend.qmatmul_i8_noalloc(w, other, yo)
        y1, y2 = backend.alloc(rows * 4), backend.alloc(rows * 4)
        backend.qmatmul(w, xn, y1)  # reads the cached int8 form of xn
        backend.qmatmul(w, backend.f32_buf(backend.download_f32(xn)), y2)  # quantizes afresh
        assert np.array_equal(backend.download_f32(y1), backend.download_f32(y2))
    finally:
        backend.set_act_mode(backend_mod.ACT_F32)


def test_noalloc_calls_from_two_contexts_on_one_gpu(backend):
    """Two contexts share the GPU's static array: their calls, issued back to
    back without waiting for each other, are ordered by the per-GPU event,
    so each output equals its allocating counterpart's."""
    other = backend_mod.Gfx950Backend(0)
    try:
        k, rows = 4096, 2048
        raw = synth.weight(Q4K, rows, k, 41)
        wa, wb = backend.upload_weight(raw, Q4K, (rows, k)), other.upload_weight(raw, Q4K, (rows, k))
        xs = [synth.normal_f32(5 * k, 50 + i) for i in range(6)]
        outs = []
        for i, x in enumerate(xs):
            be, w = (backend, wa) if i % 2 == 0 else (other, wb)
            xb, yb = be.f32_buf(x), be.alloc(5 * rows * 4)
            be.qmatmul_i8_noalloc(w, xb, yb)
            outs.append((be, w, x, xb, yb))
        for be, w, x, xb, yb in outs:
            want = be.alloc(5 * rows * 4)
            be.qmatmul_i8(w, be.f32_buf(x), want)
            assert np.array_equal(be.download_f32(yb).view(np.uint32), be.download_f32(want).view(np.uint32))
    finally:
        other.close()
