"""GPU parity of the quantized-weight hot path against the CPU oracle.

f32-activation mode: per element within 1e-5 relative / 1e-6 absolute of the
oracle, after allowing for the oracle's own sequential-f32 rounding error
(see conftest.assert_parity). int8-activation mode: the reference's
"requantize then CPU qmatmul" pattern (src/backend/rocm/decode/tests.rs:68-130)
at 1e-3 relative, and the int32 block dots bit-exact. Outputs are allocated
oversize with a canary tail that must survive (decode/tests.rs:98,123-126).
"""
import numpy as np
import pytest

import npq
from conftest import abs_dot, assert_parity, f32_exact
from ties import near_tie_x
from mdma_amd import synth
from mdma_amd import backend as backend_mod
from mdma_amd.backend import DOMAIN_DEVICE
from mdma_amd.backend import LAYOUT_GFX950, POOL_WEIGHTS, QWeight, ShapeMismatch, pack_weight
from oracle import ffi

pytestmark = pytest.mark.gpu
Q8, Q4K, Q6K, F32, F16 = 8, 12, 14, 0, 1
CANARY = np.float32(123456.25)


def ref_weights(dtype, rows, k):
    """The reference's synthetic blocks (src/backend/rocm/decode/tests.rs:47-66):
    every byte varies, d in {1,2,3}/1024, dmin 1/512, Q6_K sub-scales -128/+127."""
    tsz = synth.TYPE_SIZE[dtype]
    nb = rows * (k // synth.BLOCK_SIZE[dtype])
    raw = np.zeros((nb, tsz), np.uint8)
    i = np.arange(tsz)
    for b in range(nb):
        raw[b] = (i * 73 + b * 31 + 19) & 255
        d = np.frombuffer(np.float16((1 + b % 3) / 1024).tobytes(), np.uint8)
        if dtype == Q4K:
            raw[b, 0:2] = d
            raw[b, 2:4] = np.frombuffer(np.float16(1 / 512).tobytes(), np.uint8)
        elif dtype == Q6K:
            raw[b, 208:210] = d
            raw[b, 192], raw[b, 193] = 128, 127
        else:
            raw[b, 0:2] = d
    return raw.reshape(-1)


def x_kind(kind, n):
    i = np.arange(n)
    if kind == 0:
        return (((i * 17) % 255).astype(np.float32) - 127.0) / 32.0
    if kind == 1:
        return -(((i * 7) % 31 + 1).astype(np.float32)) / 16.0
    return np.zeros(n, np.float32)


def run_qmatmul(be, dtype, raw, rows, k, x, mode="default", layout=0):
    w = be.upload_weight(raw, dtype, (rows, k), layout)
    T = x.size // k
    xb = be.f32_buf(x)
    yb = be.f32_buf(np.full(T * rows + 8, CANARY, np.float32))
    {"default": be.qmatmul, "f32": be.qmatmul_f32, "i8": be.qmatmul_i8}[mode](w, xb, yb)
    y = be.download_f32(yb)
    assert np.all(y[T * rows:] == CANARY), "wrote past the output"
    return y[:T * rows].reshape(T, rows)


def oracle_f32(dtype, raw, rows, k, x):
    """(CPU oracle output, f64 dot of the exact block values) [T, rows]."""
    cpu = ffi.qmatmul(dtype, raw, rows, k, x)
    return cpu, f32_exact(npq.dequantize(dtype, raw, rows, k), x)


KS = {Q4K: (256, 512, 768), Q6K: (256, 512, 768), Q8: (32, 288, 768), F32: (3, 288), F16: (64, 288)}


@pytest.mark.parametrize("dtype", [Q4K, Q6K, Q8])
def test_f32_mode_reference_shapes_and_inputs(backend, dtype):
    for rows in (1, 7, 9, 20):
        for k in KS[dtype]:
            raw = ref_weights(dtype, rows, k)
            for kind in range(3):
                x = x_kind(kind, k)
                got = run_qmatmul(backend, dtype, raw, rows, k, x, "f32")
                cpu, exact = oracle_f32(dtype, raw, rows, k, x)
                assert_parity(got, cpu, exact, 1e-5, what=f"dtype={dtype} rows={rows} k={k} x={kind}", correctly_rounded=True)
                if kind == 2:
                    assert np.all(got == 0)


@pytest.mark.parametrize("dtype", [F32, F16])
def test_f32_mode_float_weights(backend, dtype):
    for rows, k in ((2, 3), (5, 288), (33, 64)):
        raw = synth.weight(dtype, rows, k, 3)
        x = synth.normal_f32(2 * k, 4)
        got = run_qmatmul(backend, dtype, raw, rows, k, x)
        cpu, exact = oracle_f32(dtype, raw, rows, k, x)
        assert_parity(got, cpu, exact, 1e-5, what=f"dtype={dtype}", correctly_rounded=True)
    # src/backend/test_support.rs:254-268 hand-computed batch.
    w = np.array([1.0, -2.0, 3.0, 4.0, 5.0, -6.0], np.float32).view(np.uint8)
    got = run_qmatmul(backend, F32, w, 2, 3, np.array([2.0, -1.0, 0.5, -1.0, 2.0, 1.0], np.float32))
    assert list(got.reshape(-1)) == [5.5, 0.0, -2.0, 0.0]


@pytest.mark.parametrize("dtype", [Q4K, Q6K, Q8])
@pytest.mark.parametrize("T", [1, 2, 3, 4, 5, 8, 9, 17])
def test_f32_mode_batched_tokens(backend, dtype, T):
    rows, k = 37, 1024
    raw = synth.weight(dtype, rows, k, 100 + T)
    x = synth.normal_f32(T * k, 200 + T)
    got = run_qmatmul(backend, dtype, raw, rows, k, x, "f32")
    cpu, exact = oracle_f32(dtype, raw, rows, k, x)
    assert_parity(got, cpu, exact, 1e-5, what=f"dtype={dtype} T={T}", correctly_rounded=True)
    # The single-token call (the decode kernel) meets the same bar on token 0.
    one = run_qmatmul(backend, dtype, raw, rows, k, x[:k], "f32")
    assert_parity(one[0], cpu[0], exact[0], 1e-5, what=f"dtype={dtype} T=1 of {T}", correctly_rounded=True)


SHAPES_8B = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)]


@pytest.mark.parametrize("shape", SHAPES_8B)
def test_q4k_f32_mode_llama3_8b_shapes(backend, shape):
    rows, k = shape
    raw = synth.weight(Q4K, rows, k, 1)
    x = synth.normal_f32(k, 2)
    got = run_qmatmul(backend, Q4K, raw, rows, k, x, "f32")
    cpu, exact = oracle_f32(Q4K, raw, rows, k, x)
    rate = assert_parity(got, cpu, exact, 1e-5, what=f"Q4_K {shape}", correctly_rounded=True)
    print(f"Q4_K {shape}: plain 1e-5/1e-6 pass rate vs sequential oracle {rate:.4f}")


@pytest.mark.parametrize("shape,T", [((4096, 14336), 1), ((4096, 14336), 4), ((4096, 14336), 8),
                                     ((128256, 4096), 1)])
def test_q6k_f32_mode_config3_shapes(backend, shape, T):
    rows, k = shape
    raw = synth.weight(Q6K, rows, k, 3)
    x = synth.normal_f32(T * k, 4)
    got = run_qmatmul(backend, Q6K, raw, rows, k, x, "f32")
    cpu = ffi.qmatmul(Q6K, raw, rows, k, x)
    exact = np.empty_like(cpu, dtype=np.float64)
    for r0 in range(0, rows, 8192):
        r1 = min(rows, r0 + 8192)
        W = npq.dequantize(Q6K, raw[r0 * (k // 256) * 210:r1 * (k // 256) * 210], r1 - r0, k)
        exact[:, r0:r1] = f32_exact(W, x)
    assert_parity(got, cpu, exact, 1e-5, what=f"Q6_K {shape} T={T}", correctly_rounded=True)


# ------------------------------------------------------------ int8 mode ----

def oracle_i8(dtype, raw, rows, k, x):
    q, d, _ = ffi.quantize_act(x, 256)
    xh = ffi.dequantize_act(q, d, 256)
    return oracle_f32(dtype, raw, rows, k, xh)


@pytest.mark.parametrize("dtype", [Q4K, Q6K, Q8])
def test_i8_mode_reference_shapes(backend, dtype):
    for rows in (1, 7, 9, 20):
        for k in (256, 512, 768):
            raw = ref_weights(dtype, rows, k)
            for kind in range(3):
                x = x_kind(kind, k)
                got = run_qmatmul(backend, dtype, raw, rows, k, x, "i8")
                cpu, exact = oracle_i8(dtype, raw, rows, k, x)
                assert_parity(got, cpu, exact, 1e-3, what=f"i8 dtype={dtype} rows={rows} k={k} x={kind}")


@pytest.mark.parametrize("dtype", [Q4K, Q6K, Q8])
@pytest.mark.parametrize("shape", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)])
def test_i8_mode_llama3_8b_shapes(backend, dtype, shape):
    rows, k = shape
    raw = synth.weight(dtype, rows, k, 11)
    x = synth.normal_f32(k, 12)
    got = run_qmatmul(backend, dtype, raw, rows, k, x, "i8")
    cpu, exact = oracle_i8(dtype, raw, rows, k, x)
    assert_parity(got, cpu, exact, 1e-3, what=f"i8 {dtype} {shape}")
    # Quantization error itself, against the unquantized f32 oracle
    # (src/backend/rocm/tests.rs:306-376 requires rel-RMS below 0.03).
    full = ffi.qmatmul(dtype, raw, rows, k, x)
    rel_rms = np.sqrt(np.mean((got - full) ** 2) / np.mean(full ** 2))
    assert rel_rms < 0.03, rel_rms


@pytest.mark.parametrize("T", [2, 5, 8, 11, 16, 17, 35, 64, 70])
def test_i8_mode_batched(backend, T):
    rows, k = 29, 2048
    for dtype in (Q4K, Q6K, Q8):
        raw = synth.weight(dtype, rows, k, T)
        x = synth.normal_f32(T * k, 50 + T)
        got = run_qmatmul(backend, dtype, raw, rows, k, x, "i8")
        # From ffi.GEMM_MIN_TOKENS tokens the prepared weights go to the
        # prefill GEMM, whose activations are quantized per 32 (below: the
        # batch GEMV, 16 tokens per launch, per 256).
        gemm = T >= ffi.GEMM_MIN_TOKENS
        g = 32 if gemm else 256
        q = np.concatenate([ffi.quantize_act(x[t * k:(t + 1) * k], g)[0] for t in range(T)])
        d = np.concatenate([ffi.quantize_act(x[t * k:(t + 1) * k], g)[1] for t in range(T)])
        xq = ffi.dequantize_act(q, d, g)
        cpu, exact = oracle_f32(dtype, raw, rows, k, xq)
        absum = abs_dot(npq.dequantize(dtype, raw, rows, k), xq) if gemm else None
        assert_parity(got, cpu, exact, 1e-3, abs_sum=absum, what=f"i8 batched {dtype} T={T}")


@pytest.mark.parametrize("dtype,shape,T", [(Q6K, (4096, 14336), 4), (Q6K, (4096, 14336), 8),
                                           (Q4K, (14336, 4096), 8), (Q8, (4096, 4096), 3)])
def test_i8_mode_batched_llama3_8b_shapes(backend, dtype, shape, T):
    # The decode-batching case (batch 4 and 8) at Llama-3-8B shapes.
    rows, k = shape
    raw = synth.weight(dtype, rows, k, 21)
    x = synth.normal_f32(T * k, 22)
    got = run_qmatmul(backend, dtype, raw, rows, k, x, "i8")
    xh = np.concatenate([ffi.dequantize_act(*ffi.quantize_act(x[t * k:(t + 1) * k], 256)[:2], 256) for t in range(T)])
    cpu, exact = oracle_f32(dtype, raw, rows, k, xh)
    # atol 1e-5: outputs near zero are differences of per-256 terms of order
    # one, each rounded once in f32 by the single-token kernel.
    assert_parity(got, cpu, exact, 1e-3, atol=1e-5, what=f"i8 batched {dtype} {shape} T={T}")
    # Each token's row equals that token decoded alone, within the same bar.
    one = run_qmatmul(backend, dtype, raw, rows, k, x[(T - 1) * k:], "i8")
    assert_parity(one[0], cpu[T - 1], exact[T - 1], 1e-3, atol=1e-5, what="single token")


@pytest.mark.parametrize("dtype", [Q4K, Q6K, Q8])
def test_batch_ring_equals_staged(backend, dtype):
    """The DMA-ring batch kernel (the default) and the register-staged one
    form the same int32 products and f32 sums in the same order, so their
    outputs are equal bit for bit: token counts 5..15 (8 and 16 staged
    token rows), ragged tiles (rows not a multiple of 16), 2 to 56 column
    blocks (one to eight chunks, one to four waves splitting a tile, chunks
    that start inside a pair of blocks), workgroups of 4 tiles sharing the
    activations (with waves past the last tile, and tiles of two weights in
    one workgroup), the gated gate/up and the fused three-weight call. The
    ring runs twice: on the row planes and, with the batch layout on, on the
    Q6_K weights' tile images (made at each weight's first call here). The
    oracle side of this kernel is test_i8_mode_batched and
    test_i8_mode_batched_llama3_8b_shapes."""
    def both(fn):
        out = []
        for kind, tiles in ((backend_mod.BATCH_AUTO, True), (backend_mod.BATCH_AUTO, False),
                            (backend_mod.BATCH_STAGED, False)):
            backend.set_batch_kernel(kind)
            backend.set_batch_layout(tiles)
            out.append(fn())
        backend.set_batch_kernel(backend_mod.BATCH_AUTO)
        backend.set_batch_layout(False)
        return out

    def same(a, b, c, what):
        assert np.array_equal(a.view(np.uint32), c.view(np.uint32)), ("tile images", what)
        assert np.array_equal(b.view(np.uint32), c.view(np.uint32)), ("row planes", what)

    backend.set_act_mode(backend_mod.ACT_I8)
    try:
        # (40, 768): an odd number of 256-column blocks, which the ring kernel
        # (pairs of blocks) leaves to the staged one. (40008, 512): 2501
        # tiles, four per workgroup.
        for rows, k in ((29, 1024), (80, 4096), (48, 14336), (40008, 512), (40, 768)):
            raw = synth.weight(dtype, rows, k, 60 + rows)
            for T in (5, 8, 9, 15):
                x = synth.normal_f32(T * k, 61 + T)
                a, b, c = both(lambda: run_qmatmul(backend, dtype, raw, rows, k, x, "i8"))
                same(a, b, c, (rows, k, T))
        # Gate/up: 96 rows (one tile per workgroup, waves split its columns)
        # and 24592 rows (1537 tiles, four per workgroup, the last one
        # alone). Fused QKV: 96 rows each, then 16400 + 4104 + 4088 rows
        # (1538 tiles, four per workgroup; one workgroup holds q's last
        # tiles and k's first).
        for shapes, k, T in (((96, 96, 96), 4096, 7), ((24592, 24592, 24592), 512, 8), ((16400, 4104, 4088), 512, 6)):
            raws = [synth.weight(dtype, r, k, 70 + i) for i, r in enumerate(shapes)]
            ws = [backend.upload_weight(raw, dtype, (r, k)) for raw, r in zip(raws, shapes)]
            xb = backend.f32_buf(synth.normal_f32(T * k, 71))

            def gate_up():
                r = shapes[0]
                g, u, y = (backend.alloc(T * r * 4) for _ in range(3))
                backend.ffn_gate_up(ws[0], ws[1], xb, g, u, y)
                return backend.download_f32(y).copy()

            def qkv():
                outs = [backend.alloc(T * r * 4) for r in shapes]
                backend.qmatmul_qkv(ws[0], ws[1], ws[2], xb, *outs)
                return np.concatenate([backend.download_f32(o) for o in outs])

            for fn in ((gate_up, qkv) if shapes[0] == shapes[2] else (qkv,)):
                a, b, c = both(fn)
                same(a, b, c, (fn.__name__, shapes, k, T))
    finally:
        backend.set_act_mode(backend_mod.ACT_F32)


def test_batch_tile_images_follow_rewrites(backend):
    """A Q6_K weight's tile images are made at its first batched call (with
    the batch layout on) and charged to the device ledger by exactly the
    weight's GGUF bytes (16-row tiles of 512-column pairs, rows a multiple of
    16); rewriting the weight's bytes frees them, and the next call reads
    the new bytes (made again from them)."""
    rows, k, T = 64, 2048, 8
    raws = [synth.weight(Q6K, rows, k, 880 + i) for i in range(2)]
    x = synth.normal_f32(T * k, 882)
    want = [run_qmatmul(backend, Q6K, r, rows, k, x, "i8") for r in raws]  # row planes (layout off)
    w = backend.upload_weight(raws[0], Q6K, (rows, k))
    xb, yb = backend.f32_buf(x), backend.alloc(T * rows * 4)
    backend.set_batch_layout(True)
    try:
        before = backend.buffer_usage(DOMAIN_DEVICE)[0]
        backend.qmatmul_i8(w, xb, yb)
        assert backend.buffer_usage(DOMAIN_DEVICE)[0] - before == len(raws[0])
        assert np.array_equal(backend.download_f32(yb).reshape(T, rows), want[0])
        # The prepared bytes of the second weight, written over the first.
        backend.upload(w.buf, 0, backend_mod.pack_weight(raws[1], Q6K, (rows, k)))
        assert backend.buffer_usage(DOMAIN_DEVICE)[0] == before
        backend.qmatmul_i8(w, xb, yb)
        assert np.array_equal(backend.download_f32(yb).reshape(T, rows), want[1])
        w.buf.close()
        assert backend.buffer_usage(DOMAIN_DEVICE)[0] < before
    finally:
        backend.set_batch_layout(False)


@pytest.mark.parametrize("group", [32, 256])
def test_quantize_act_bit_exact(backend, group):
    x = synth.normal_f32(8 * 1024, 77) * 3
    x[:group] = 0
    x[group:2 * group] = np.linspace(-1, 1, group, dtype=np.float32) * 127  # .5 ties
    # Activations whose quantization depends on rounding the product before
    # the half-way offset (a quantizer fusing them into one FMA fails here).
    x[2 * group:18 * group] = near_tie_x(16, group, 78)
    n = x.size
    xb = backend.f32_buf(x)
    qb, db, sb = backend.alloc(n), backend.alloc(n // group * 4), backend.alloc(n // 16 * 4)
    backend.quantize_act(xb, group, qb, db, sb)
    q, d, s = ffi.quantize_act(x, group)
    assert np.array_equal(backend.download(qb, 0, n).view(np.int8), q)
    assert np.array_equal(backend.download(db, 0, n // group * 4).view(np.uint32), d.view(np.uint32))
    assert np.array_equal(backend.download(sb, 0, n // 16 * 4).view(np.int32), s)


@pytest.mark.parametrize("dtype", [Q4K, Q6K, Q8])
def test_block_dot_i32_bit_exact(backend, dtype):
    rows, k, T = 9, 1024, 3
    raw = synth.weight(dtype, rows, k, 31)
    q, _, _ = ffi.quantize_act(synth.normal_f32(T * k, 32), 256)
    q = q.copy()
    q[:64] = 127
    q[64:128] = -128  # extremes the quantizer never emits, still exact
    w = backend.upload_weight(raw, dtype, (rows, k))
    qb = backend.alloc(q.size)
    backend.upload(qb, 0, q)
    sub = 16 if dtype == Q6K else 32
    ob = backend.alloc(T * rows * (k // sub) * 4)
    backend.block_dot_i32(w, qb, ob)
    got = backend.download(ob, 0, ob.len).view(np.int32).reshape(T, rows, k // sub)
    assert np.array_equal(got, ffi.block_dot_i32(dtype, raw, rows, k, q, T))


# ------------------------------------------------------------- fusions ----

@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("dtype", [Q4K, Q6K, Q8])
def test_fused_qkv_equals_separate_calls(backend, dtype, mode):
    backend.set_act_mode(mode)
    try:
        k_in = 512
        shapes = [(96, k_in), (32, k_in), (32, k_in)]
        for T in (1, 3):
            x = backend.f32_buf(synth.normal_f32(T * k_in, 5))
            ws = [backend.upload_weight(synth.weight(dtype, r, c, 40 + i), dtype, (r, c))
                  for i, (r, c) in enumerate(shapes)]
            outs = [backend.alloc(T * r * 4) for r, _ in shapes]
            backend.qmatmul_qkv(ws[0], ws[1], ws[2], x, *outs)
            for w, o, (r, _) in zip(ws, outs, shapes):
                sep = backend.alloc(T * r * 4)
                backend.qmatmul(w, x, sep)
                assert np.array_equal(backend.download_f32(o), backend.download_f32(sep))
    finally:
        backend.set_act_mode(0)


def test_fused_qkv_mixed_dtypes(backend):
    k_in = 256
    x_h = synth.normal_f32(k_in, 5)
    x = backend.f32_buf(x_h)
    specs = [(Q6K, 64), (Q4K, 16), (Q8, 16)]
    ws = [backend.upload_weight(synth.weight(dt, r, k_in, i), dt, (r, k_in)) for i, (dt, r) in enumerate(specs)]
    outs = [backend.alloc(r * 4) for _, r in specs]
    backend.qmatmul_qkv(ws[0], ws[1], ws[2], x, *outs)
    for (dt, r), o, i in zip(specs, outs, range(3)):
        raw = synth.weight(dt, r, k_in, i)
        cpu, exact = oracle_f32(dt, raw, r, k_in, x_h)
        assert_parity(backend.download_f32(o), cpu, exact, 1e-5, correctly_rounded=True)


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("dtype", [Q4K, Q6K, Q8])
def test_ffn_gate_up_matches_oracle_and_unfused(backend, dtype, mode):
    backend.set_act_mode(mode)
    try:
        rows, k, T = 300, 1024, 2
        g_raw, u_raw = synth.weight(dtype, rows, k, 61), synth.weight(dtype, rows, k, 62)
        x_h = synth.normal_f32(T * k, 63)
        g = backend.upload_weight(g_raw, dtype, (rows, k))
        u = backend.upload_weight(u_raw, dtype, (rows, k))
        x = backend.f32_buf(x_h)
        gs, us = backend.alloc(T * rows * 4), backend.alloc(T * rows * 4)
        y = backend.f32_buf(np.full(T * rows + 8, CANARY, np.float32))
        backend.ffn_gate_up(g, u, x, gs, us, y)
        got = backend.download_f32(y)
        assert np.all(got[T * rows:] == CANARY)
        got = got[:T * rows]
        # Unfused on the device: qmatmul, qmatmul, silu_mul (backend.rs:472-489).
        backend.qmatmul(g, x, gs)
        backend.qmatmul(u, x, us)
        y2 = backend.alloc(T * rows * 4)
        backend.silu_mul(gs, us, y2)
        assert np.array_equal(got, backend.download_f32(y2))
        # Oracle: CPU gate/up, CPU silu_mul; exact = f64 chain.
        xx = x_h if mode == 0 else np.concatenate(
            [ffi.dequantize_act(*ffi.quantize_act(x_h[t * k:(t + 1) * k], 256)[:2], 256) for t in range(T)])
        cg, eg = oracle_f32(dtype, g_raw, rows, k, xx)
        cu, eu = oracle_f32(dtype, u_raw, rows, k, xx)
        cpu = ffi.silu_mul(cg.reshape(-1), cu.reshape(-1))
        exact = (eg / (1 + np.exp(-eg)) * eu).reshape(-1)
        assert_parity(got, cpu, exact, 1e-5 if mode == 0 else 1e-3, atol=1e-5, what=f"gate_up {dtype} mode {mode}")
    finally:
        backend.set_act_mode(0)


def test_i8_activation_cache_reuses_and_invalidates(backend):
    # Pattern of src/backend/rocm/decode/tests.rs:134-164: int8 activations are
    # reused across weights of both dtypes until x is written again.
    rows, k = 9, 768
    w4 = backend.upload_weight(synth.weight(Q4K, rows, k, 1), Q4K, (rows, k))
    w6 = backend.upload_weight(synth.weight(Q6K, rows, k, 2), Q6K, (rows, k))
    xa = ((np.arange(k) % 37) - 18.0).astype(np.float32) * 0.1
    x = backend.f32_buf(xa)
    y = backend.alloc(rows * 4)
    backend.qmatmul_i8(w4, x, y)
    backend.qmatmul_i8(w6, x, y)
    reused = backend.download_f32(y).copy()
    fresh = backend.f32_buf(xa)
    backend.qmatmul_i8(w6, fresh, y)
    assert np.array_equal(reused, backend.download_f32(y))
    xb = -xa * 0.5 + 0.25
    backend.upload(x, 0, xb)  # a write to x invalidates
    backend.qmatmul_i8(w6, x, y)
    rewritten = backend.download_f32(y).copy()
    backend.qmatmul_i8(w6, backend.f32_buf(xb), y)
    assert np.array_equal(rewritten, backend.download_f32(y))
    assert not np.array_equal(reused, rewritten)
    # A kernel writing the cached x (here: add into x) also invalidates.
    backend.qmatmul_i8(w6, x, y)
    backend.add(fresh, fresh, x)
    backend.qmatmul_i8(w6, x, y)
    want = backend.alloc(rows * 4)
    backend.qmatmul_i8(w6, backend.f32_buf(xa + xa), want)
    assert np.array_equal(backend.download_f32(y), backend.download_f32(want))


@pytest.mark.parametrize("T", [1, 3, 16, 63, 64])
def test_rmsnorm_int8_activations_bit_exact(backend, T):
    # In the int8 mode an rmsnorm of fewer than 64 rows (ffi.GEMM_MIN_TOKENS,
    # from which the prefill GEMM quantizes per 32 itself) also leaves the int8
    # form of its output in the activation cache; a qmatmul reading y must
    # give the bits of one reading an identical copy of y quantized afresh.
    k, rows = 4096, 40
    w = backend.upload_weight(synth.weight(Q4K, rows, k, 3), Q4K, (rows, k))
    w6 = backend.upload_weight(synth.weight(Q6K, rows, k, 4), Q6K, (rows, k))
    g = backend.f32_buf(synth.normal_f32(k, 5))
    a, b = backend.f32_buf(synth.normal_f32(T * k, 6)), backend.f32_buf(synth.normal_f32(T * k, 7))
    y, s = backend.alloc(T * k * 4), backend.alloc(T * k * 4)
    out, ref = backend.alloc(T * rows * 4), backend.alloc(T * rows * 4)
    backend.set_act_mode(backend_mod.ACT_I8)
    try:
        for fused in (lambda: backend.rmsnorm(g, a, y, 1e-5), lambda: backend.add_rmsnorm(g, a, b, s, y, 1e-5)):
            fused()
            for wt in (w, w6):
                backend.qmatmul(wt, y, out)
                backend.qmatmul(wt, backend.f32_buf(backend.download_f32(y)), ref)
                assert np.array_equal(backend.download_f32(out), backend.download_f32(ref))
        # The normalized values themselves are those of the f32 mode.
        backend.rmsnorm(g, a, y, 1e-5)
        got = backend.download_f32(y)
    finally:
        backend.set_act_mode(backend_mod.ACT_F32)
    backend.rmsnorm(g, a, y, 1e-5)
    assert np.array_equal(got, backend.download_f32(y))


@pytest.mark.parametrize("n_q,kv_len", [(1, 40), (1, 700), (3, 130), (15, 15)])
def test_attention_int8_activations_bit_exact(backend, n_q, kv_len):
    # Same for attention's output (Llama-3-8B heads: 32 query, 8 KV, 128 wide),
    # which then feeds the output projection.
    from mdma_amd.backend import AttnSpec, KvView
    hd, nq, nkv, rows = 128, 32, 8, 40
    k = synth.normal_f32(kv_len * nkv * hd, 8).astype(np.float16)
    v = synth.normal_f32(kv_len * nkv * hd, 9).astype(np.float16)
    kb, vb = backend.alloc(k.size * 2), backend.alloc(v.size * 2)
    backend.upload(kb, 0, k)
    backend.upload(vb, 0, v)
    q = backend.f32_buf(synth.normal_f32(n_q * nq * hd, 10))
    o = backend.alloc(n_q * nq * hd * 4)
    w = backend.upload_weight(synth.weight(Q6K, rows, nq * hd, 11), Q6K, (rows, nq * hd))
    out, ref = backend.alloc(n_q * rows * 4), backend.alloc(n_q * rows * 4)
    backend.set_act_mode(backend_mod.ACT_I8)
    try:
        backend.attn(q, KvView(kb, vb, kv_len), AttnSpec(hd, nq, nkv), o)
        got = backend.download_f32(o)
        backend.qmatmul(w, o, out)
        backend.qmatmul(w, backend.f32_buf(got), ref)
        assert np.array_equal(backend.download_f32(out), backend.download_f32(ref))
    finally:
        backend.set_act_mode(backend_mod.ACT_F32)
    backend.attn(q, KvView(kb, vb, kv_len), AttnSpec(hd, nq, nkv), o)
    assert np.array_equal(got, backend.download_f32(o))


@pytest.mark.parametrize("dtype", [Q4K, Q6K])
@pytest.mark.parametrize("k,rows", [(768, 48), (2048, 48), (4096, 48), (8192, 48), (14336, 48), (8192, 50),
                                    (14336, 50), (14336, 4096)])
def test_one_token_in_kernel_quantization_bit_exact(backend, dtype, k, rows):
    # One int8 token: the GEMV quantizes x itself; the result must be the
    # bits of the GEMV over separately quantized x (x cached by rmsnorm).
    # Rows of more than 4096 columns run two multi-wave teams per workgroup
    # sharing one quantization of x; 50 rows leave the last workgroup with a
    # team past the end, 4096 rows are the down projection's shape.
    w = backend.upload_weight(synth.weight(dtype, rows, k, 41), dtype, (rows, k))
    x = synth.normal_f32(k, 42) * 3
    x[:256] = 0  # an all-zero group
    xb = backend.f32_buf(x)
    y1, y2, yn = backend.alloc(rows * 4), backend.alloc(rows * 4), backend.alloc(k * 4)
    backend.set_act_mode(backend_mod.ACT_I8)
    try:
        backend.qmatmul(w, xb, y1)  # in-kernel quantization
        # rmsnorm with unit weights and eps 0 of (x / rms) reproduces x up to
        # rounding, so quantize explicitly instead: the cache holds yn's int8 form.
        backend.rmsnorm(backend.f32_buf(np.ones(k, np.float32)), xb, yn, 1e-5)
        backend.qmatmul(w, yn, y2)  # reads the cached int8 activations of yn
        yv = backend.download_f32(yn)
        y3 = backend.alloc(rows * 4)
        backend.qmatmul(w, backend.f32_buf(yv), y3)  # in-kernel quantization of the same values
        assert np.array_equal(backend.download_f32(y2), backend.download_f32(y3))
        cpu, exact = oracle_i8(dtype, synth.weight(dtype, rows, k, 41), rows, k, x)
        assert_parity(backend.download_f32(y1), cpu, exact, 1e-3, atol=1e-5)
    finally:
        backend.set_act_mode(backend_mod.ACT_F32)


def test_fused_calls_in_kernel_quantization_bit_exact(backend):
    # qmatmul_qkv and ffn_gate_up of one f32 token quantize x inside the
    # kernel (once per workgroup for rows of 4096): the bits of the same
    # calls over the cached int8 form of the same values.
    k = 4096
    raws = {"q": (Q6K, 64), "k": (Q6K, 32), "v": (Q6K, 32), "gate": (Q4K, 96), "up": (Q4K, 96)}
    ws = {n: backend.upload_weight(synth.weight(dt, r, k, 60 + i), dt, (r, k)) for i, (n, (dt, r)) in enumerate(raws.items())}
    x = synth.normal_f32(k, 61)
    xb = backend.f32_buf(x)
    yn = backend.alloc(k * 4)
    backend.set_act_mode(backend_mod.ACT_I8)
    try:
        backend.rmsnorm(backend.f32_buf(np.ones(k, np.float32)), xb, yn, 1e-5)
        yv = backend.f32_buf(backend.download_f32(yn))  # same values, not cached
        outs = {}
        for name, src in (("cached", yn), ("in_kernel", yv)):
            o = [backend.alloc(raws[n][1] * 4) for n in ("q", "k", "v")]
            backend.qmatmul_qkv(ws["q"], ws["k"], ws["v"], src, *o)
            g, u, a = backend.alloc(96 * 4), backend.alloc(96 * 4), backend.alloc(96 * 4)
            backend.ffn_gate_up(ws["gate"], ws["up"], src, g, u, a)
            outs[name] = [backend.download_f32(b) for b in o + [a]]
        for a_, b_ in zip(outs["cached"], outs["in_kernel"]):
            assert np.array_equal(a_, b_)
    finally:
        backend.set_act_mode(backend_mod.ACT_F32)


def sampled_rows(dtype, raw, rows, k, picks):
    """(row indices, raw bytes of those rows): weight rows are contiguous, so
    a run of rows is a weight of its own for the oracle."""
    rb = len(raw) // rows
    idx = np.concatenate([np.arange(r0, min(rows, r0 + n)) for r0, n in picks])
    return idx, np.concatenate([raw[r * rb:(r + 1) * rb] for r in idx])


def gate_up_oracle(dtype, g_raw, u_raw, rows, k, xq):
    """CPU gate and up GEMVs on the (requantized) input, then CPU silu_mul
    (Backend::ffn_gate_up's default, src/backend.rs:472-489); exact = the
    f64 chain on the oracle's dequantized weights."""
    cg, eg = oracle_f32(dtype, g_raw, rows, k, xq)
    cu, eu = oracle_f32(dtype, u_raw, rows, k, xq)
    cpu = ffi.silu_mul(cg.reshape(-1), cu.reshape(-1))
    return cpu, (eg / (1 + np.exp(-eg)) * eu).reshape(-1)


@pytest.mark.parametrize("dtype", [Q4K, Q6K])
@pytest.mark.parametrize("variant", ["x_lds", "x_quant"])
def test_one_token_gate_up_i8_matches_oracle(backend, dtype, variant):
    """The decode path's dominant kernel: the fused gate/up + SiLU of one
    token in the int8 mode at Llama-3-8B's 14336x4096, in both forms the
    decode path runs. x_lds: x is an rmsnorm output whose int8 form the
    rmsnorm left in the activation cache; the kernel stages it once per
    workgroup in LDS. x_quant: x is a plain f32 buffer; the kernel quantizes
    it in its own prologue. Oracle: requantize x per 256, CPU gate and up,
    CPU silu_mul (src/backend/rocm/decode/tests.rs:68-130), 1e-3 relative."""
    rows, k = 14336, 4096
    g_raw, u_raw = synth.weight(dtype, rows, k, 71), synth.weight(dtype, rows, k, 72)
    g = backend.upload_weight(g_raw, dtype, (rows, k))
    u = backend.upload_weight(u_raw, dtype, (rows, k))
    x_h = synth.normal_f32(k, 73) * 2
    x_h[256:512] = 0  # an all-zero group
    gs, us = backend.alloc(rows * 4), backend.alloc(rows * 4)
    y = backend.f32_buf(np.full(rows + 8, CANARY, np.float32))
    backend.set_act_mode(backend_mod.ACT_I8)
    try:
        if variant == "x_lds":
            xb = backend.alloc(k * 4)
            backend.rmsnorm(backend.f32_buf(np.full(k, 0.5, np.float32)), backend.f32_buf(x_h), xb, 1e-5)
            x_used = backend.download_f32(xb)
        else:
            xb = backend.f32_buf(x_h)
            x_used = x_h
        backend.ffn_gate_up(g, u, xb, gs, us, y)
        got = backend.download_f32(y)
    finally:
        backend.set_act_mode(backend_mod.ACT_F32)
    assert np.all(got[rows:] == CANARY), "wrote past the output"
    q, d, _ = ffi.quantize_act(x_used, 256)
    cpu, exact = gate_up_oracle(dtype, g_raw, u_raw, rows, k, ffi.dequantize_act(q, d, 256))
    rate = assert_parity(got[:rows], cpu, exact, 1e-3, atol=1e-5, what=f"gate/up i8 {dtype} {variant}")
    print(f"gate/up i8 dtype={dtype} {variant}: plain 1e-3/1e-5 pass rate {rate:.5f}")


HEAD = (128256, 4096)
HEAD_PICKS = ((0, 2048), (64128 - 1000, 2000), (128256 - 2048, 2048))


@pytest.mark.parametrize("mode,T", [("i8", 1), ("i8", 4), ("i8", 8), ("f32", 4), ("f32", 8)])
@pytest.mark.parametrize("cached", [False, True])
def test_q6k_head_matches_oracle(backend, mode, T, cached):
    """The Q6_K output head at its full 128256x4096 shape, batch 1 (int8:
    the ITERS16 run of the one-token kernels), 4 and 8 (the decode-batching
    case), in both activation modes. x either comes from an rmsnorm (in the
    int8 mode its int8 form is cached) or is a plain f32 buffer. The oracle
    checks 6096 output rows at the start, middle and end of the vocabulary
    (weight rows are contiguous, so a run of rows is its own weight)."""
    if mode == "f32" and cached:
        pytest.skip("the f32 mode has no int8 cache")
    rows, k = HEAD
    raw = synth.weight(Q6K, rows, k, 81)
    w = backend.upload_weight(raw, Q6K, HEAD)
    x_h = synth.normal_f32(T * k, 82 + T)
    yb = backend.f32_buf(np.full(T * rows + 8, CANARY, np.float32))
    backend.set_act_mode(backend_mod.ACT_I8 if mode == "i8" else backend_mod.ACT_F32)
    try:
        if cached:
            xb = backend.alloc(T * k * 4)
            backend.rmsnorm(backend.f32_buf(np.full(k, 0.7, np.float32)), backend.f32_buf(x_h), xb, 1e-5)
            x_used = backend.download_f32(xb)
        else:
            xb = backend.f32_buf(x_h)
            x_used = x_h
        backend.qmatmul(w, xb, yb)
        got = backend.download_f32(yb)
    finally:
        backend.set_act_mode(backend_mod.ACT_F32)
    assert np.all(got[T * rows:] == CANARY), "wrote past the output"
    got = got[:T * rows].reshape(T, rows)
    idx, sub = sampled_rows(Q6K, raw, rows, k, HEAD_PICKS)
    if mode == "i8":
        xq = np.concatenate([ffi.dequantize_act(*ffi.quantize_act(x_used[t * k:(t + 1) * k], 256)[:2], 256)
                             for t in range(T)])
    else:
        xq = x_used
    cpu, exact = oracle_f32(Q6K, sub, idx.size, k, xq)
    rtol = 1e-3 if mode == "i8" else 1e-5
    rate = assert_parity(got[:, idx], cpu, exact, rtol, atol=1e-5 if mode == "i8" else 1e-6,
                         what=f"head {mode} T={T} cached={cached}", correctly_rounded=mode == "f32")
    print(f"Q6_K head {mode} T={T} cached={cached}: plain pass rate {rate:.5f}")
    w.buf.close()


# ---------------------------------------------------------- shape rules ----

def test_qmatmul_shape_rules(backend):
    raw = synth.weight(Q4K, 4, 512, 1)
    w = backend.upload_weight(raw, Q4K, (4, 512))
    with pytest.raises(ShapeMismatch):
        backend.qmatmul(w, backend.alloc(300 * 4), backend.alloc(64))
    with pytest.raises(ShapeMismatch):
        backend.qmatmul(w, backend.alloc(512 * 4), backend.alloc(12))
    with pytest.raises(ShapeMismatch):
        backend.qmatmul(QWeight(Q4K, (4, 384), w.buf), backend.alloc(384 * 4), backend.alloc(64))
    with pytest.raises(ShapeMismatch):
        backend.qmatmul(QWeight(Q4K, (8, 512), w.buf), backend.alloc(512 * 4), backend.alloc(64))
    with pytest.raises(ShapeMismatch):
        backend.ffn_gate_up(w, QWeight(Q4K, (2, 512), w.buf), backend.alloc(2048), backend.alloc(16),
                            backend.alloc(16), backend.alloc(16))


# ------------------------------------------------------ storage layouts ----

def raw_weight(be, raw, dtype, shape):
    """A weight buffer holding raw GGUF blocks (alloc + upload, as a caller of
    the trait may build one): the backend's GGUF-layout kernels read it."""
    a = np.ascontiguousarray(raw).view(np.uint8).reshape(-1)
    b = be.alloc(a.nbytes, POOL_WEIGHTS)
    be.upload(b, 0, a)
    return QWeight(dtype, tuple(shape), b)


@pytest.mark.parametrize("T", [1, 3])
@pytest.mark.parametrize("dtype", [Q4K, Q6K, Q8])
def test_raw_and_prepared_storage_agree_with_oracle(backend, dtype, T):
    """upload_weight stores Q4_K/Q6_K/Q8_0 in the prepared layout; raw GGUF
    buffers and pre-packed uploads (layout GFX950) must give the oracle's
    results too, in both activation modes."""
    rows, k = 37, 768
    raw = synth.weight(dtype, rows, k, 90 + dtype)
    x = synth.normal_f32(T * k, 91)
    W = ffi.dequantize_row(dtype, raw, rows * k).reshape(rows, k)
    cpu, exact = oracle_f32(dtype, raw, rows, k, x)
    cpu8, exact8 = oracle_i8(dtype, raw, rows, k, x)
    ws = {"prepared": backend.upload_weight(raw, dtype, (rows, k)),
          "packed": backend.upload_weight(pack_weight(raw, dtype, (rows, k)), dtype, (rows, k), LAYOUT_GFX950),
          "raw": raw_weight(backend, raw, dtype, (rows, k))}
    xb = backend.f32_buf(x)
    for name, w in ws.items():
        for mode, fn in (("f32", backend.qmatmul_f32), ("i8", backend.qmatmul_i8)):
            yb = backend.f32_buf(np.full(T * rows + 8, CANARY, np.float32))
            fn(w, xb, yb)
            y = backend.download_f32(yb)
            assert np.all(y[T * rows:] == CANARY), (name, mode)
            if mode == "f32":
                assert_parity(y[:T * rows], cpu, exact, 1e-5, what=f"{name} f32 dtype={dtype} T={T}", correctly_rounded=True)
            else:
                assert_parity(y[:T * rows], cpu8, exact8, 1e-3, what=f"{name} i8 dtype={dtype} T={T}")
    # The embedding gather reads every storage layout the same way.
    ids = np.array([0, rows - 1, 5, 5], np.uint32)
    for name, w in ws.items():
        ob = backend.alloc(ids.size * k * 4)
        backend.embed(w, ids, ob)
        assert np.array_equal(backend.download_f32(ob), W[ids].reshape(-1)), name


def test_packed_upload_rejects_wrong_sizes(backend):
    raw = synth.weight(Q4K, 4, 256, 5)
    with pytest.raises(ShapeMismatch):
        backend.upload_weight(raw[:-16], Q4K, (4, 256), LAYOUT_GFX950)
    with pytest.raises(backend_mod.NotImplemented):
        backend.upload_weight(np.zeros(4 * 256 * 4, np.uint8), F32, (4, 256), LAYOUT_GFX950)


# ------------------------------------------------------- prefill GEMM ----
# int8 mode with T >= 64 tokens on prepared Q8_0 / Q4_K / Q6_K weights runs a
# prefill GEMM on activations quantized per 32 with an f32 scale: the
# f16-path GEMM for Q4_K and Q6_K (default), the int8 MFMA GEMM otherwise or when
# asked. Oracle: the reference's "requantize, then CPU qmatmul"
# (src/backend/rocm/decode/tests.rs:68-130).

def oracle_i8_32(dtype, raw, rows, k, x):
    """(CPU oracle, exact, sum_k |x_k w_k|) of the per-32 requantized product."""
    q, d, _ = ffi.quantize_act(x, 32)
    xq = ffi.dequantize_act(q, d, 32)
    cpu, exact = oracle_f32(dtype, raw, rows, k, xq)
    return cpu, exact, abs_dot(npq.dequantize(dtype, raw, rows, k), xq)


# (dtype, prefill kernel): both kernels for Q4_K and Q6_K, the int8 one for Q8_0.
GEMM_CASES = [(Q8, backend_mod.PREFILL_I8), (Q4K, backend_mod.PREFILL_AUTO), (Q4K, backend_mod.PREFILL_I8),
              (Q6K, backend_mod.PREFILL_AUTO), (Q6K, backend_mod.PREFILL_I8)]
GEMM_IDS = ["q8-i8", "q4k-f16", "q4k-i8", "q6k-f16", "q6k-i8"]


@pytest.fixture
def prefill_kernel(backend, request):
    backend.set_prefill_kernel(request.param)
    yield request.param
    backend.set_prefill_kernel(backend_mod.PREFILL_AUTO)


def gemm_cases(f):
    f = pytest.mark.parametrize("dtype,prefill_kernel", GEMM_CASES, ids=GEMM_IDS, indirect=["prefill_kernel"])(f)
    return f


@pytest.mark.parametrize("shape", [(64, 256, 64), (97, 512, 200), (130, 1024, 257), (64, 4096, 384),
                                   (300, 768, 130), (300, 4096, 384), (520, 1024, 520)])
@gemm_cases
def test_prefill_gemm_i8(backend, dtype, prefill_kernel, shape):
    T, k, rows = shape
    raw = synth.weight(dtype, rows, k, 300 + T)
    x = synth.normal_f32(T * k, 301 + rows)
    got = run_qmatmul(backend, dtype, raw, rows, k, x, "i8")
    cpu, exact, absum = oracle_i8_32(dtype, raw, rows, k, x)
    assert_parity(got, cpu, exact, 1e-3, abs_sum=absum,
                  what=f"gemm dtype={dtype} kernel={prefill_kernel} T={T} k={k} rows={rows}")


@gemm_cases
def test_prefill_gemm_activation_ranges(backend, dtype, prefill_kernel):
    """Token rows over 50 decades of magnitude, an all-zero row, a row of one
    non-zero, rows whose blocks quantize to the int8 extremes +-127 (and a
    block of equal values, all at 127) and mixed block magnitudes within a
    row: the f16-path GEMM rescales each row's block sums by a power of two
    to keep them in f16 range, and must agree with the oracle throughout."""
    T, k, rows = 72, 512, 136
    raw = synth.weight(dtype, rows, k, 320)
    x = synth.normal_f32(T * k, 321).reshape(T, k)
    for t in range(24):
        x[t] *= np.float32(10.0 ** (2 * t - 25))
    x[24] = 0
    x[25] = 0
    x[25, 300] = -3.5
    x[26] = np.sign(x[26]) * 2.0  # every block all at +-127
    x[27] = 1.25                  # equal values: 127 everywhere
    x[28, :256] *= np.float32(1e-6)  # one super-block 10^6 smaller than the next
    x[29, ::32] = 1e4             # one outlier per block
    x = x.reshape(-1)
    got = run_qmatmul(backend, dtype, raw, rows, k, x, "i8")
    cpu, exact, absum = oracle_i8_32(dtype, raw, rows, k, x)
    # The slack of each element scales with its own terms (abs_sum): rows of
    # 1e-25 and of 1e21 are held to the same relative bar.
    assert_parity(got, cpu, exact, 1e-3, atol=0.0, abs_sum=absum, what=f"gemm ranges kernel={prefill_kernel}")
    assert np.all(got[24] == 0)


@gemm_cases
def test_prefill_gemm_config4_shapes_sampled_rows(backend, dtype, prefill_kernel):
    """Full config-4 shapes on the GPU; the oracle checks a sample of output
    rows (the weight rows are contiguous, so a row slice is its own weight)."""
    for T, k, rows in ((512, 4096, 14336), (2048, 14336, 4096)):
        raw = synth.weight(dtype, rows, k, 400 + T)
        x = synth.normal_f32(T * k, 401 + T)
        w = backend.upload_weight(raw, dtype, (rows, k))
        xb, yb = backend.f32_buf(x), backend.alloc(T * rows * 4)
        backend.qmatmul_i8(w, xb, yb)
        y = backend.download_f32(yb).reshape(T, rows)
        rb = len(raw) // rows
        for r0 in (0, rows // 2 + 13, rows - 16):
            sl = raw[r0 * rb:(r0 + 16) * rb]
            tok = np.r_[0:8, 130:133, T - 8:T]
            cpu, exact, absum = oracle_i8_32(dtype, sl, 16, k, x.reshape(T, k)[tok].reshape(-1))
            assert_parity(y[tok, r0:r0 + 16].reshape(-1), cpu, exact, 1e-3, abs_sum=absum,
                          what=f"gemm config4 dtype={dtype} kernel={prefill_kernel} T={T} rows {r0}..")
        w.buf.close(), xb.close(), yb.close()


def q6k_full_scale_range(raw, rows, k, seed):
    """Q6_K blocks whose sub-block scales span the whole int8 range, as real
    Q6_K files have (the quantizer sets a scale of -128 in every super-block):
    each block gets -128 and 127 and random scales in [-128, 127]."""
    rng = np.random.default_rng(seed)
    b = np.frombuffer(raw, np.uint8).copy().reshape(rows * (k // 256), 210)
    n = b.shape[0]
    sc = rng.integers(-128, 128, size=(n, 16)).astype(np.int8)
    lo = rng.integers(0, 16, size=n)
    sc[np.arange(n), lo] = -128
    sc[np.arange(n), (lo + rng.integers(1, 16, size=n)) % 16] = 127
    b[:, 192:208] = sc.view(np.uint8)
    return b.reshape(-1)


@pytest.mark.parametrize("kind", [backend_mod.PREFILL_AUTO, backend_mod.PREFILL_I8], ids=["f16", "i8"])
def test_prefill_gemm_q6k_full_scale_range(backend, kind):
    """Q6_K sub-block scales over all of [-128, 127] (the benchmark
    distribution keeps them in [-64, 63]; weight values sc * q then reach
    4096, past f16's consecutive integers: the f16 path carries them as the
    exact split A1 + A2), at a config-4 shape and a small one."""
    backend.set_prefill_kernel(kind)
    try:
        q6k_full_scale_cases(backend, kind)
    finally:
        backend.set_prefill_kernel(backend_mod.PREFILL_AUTO)


def q6k_full_scale_cases(backend, kind):
    for T, k, rows in ((64, 512, 96), (512, 4096, 14336)):
        raw = q6k_full_scale_range(synth.weight(Q6K, rows, k, 600 + T), rows, k, 601)
        x = synth.normal_f32(T * k, 602 + T)
        w = backend.upload_weight(raw, Q6K, (rows, k))
        xb, yb = backend.f32_buf(x), backend.alloc(T * rows * 4)
        backend.qmatmul_i8(w, xb, yb)
        y = backend.download_f32(yb).reshape(T, rows)
        rb = len(raw) // rows
        for r0 in sorted({0, rows // 2 + 13, rows - 16}):
            sl = raw[r0 * rb:(r0 + 16) * rb]
            tok = np.unique(np.r_[0:8, min(130, T - 3):min(133, T), T - 8:T])
            cpu, exact, absum = oracle_i8_32(Q6K, sl, 16, k, x.reshape(T, k)[tok].reshape(-1))
            assert_parity(y[tok, r0:r0 + 16].reshape(-1), cpu, exact, 1e-3, abs_sum=absum,
                          what=f"gemm q6k full scales kind={kind} T={T} rows {r0}..")
        w.buf.close(), xb.close(), yb.close()


@pytest.mark.parametrize("shape", [(512, 4096, 1024), (300, 14336, 256)])
def test_prefill_gemm_q6k_wide_repeatable(backend, shape):
    """The Q6_K f16-path GEMM over more than 128 tokens (256 tokens per
    workgroup, split K at these row counts) gives the same bits on every
    call, with full-range sub-block scales (A2 terms present) and the
    oracle's values on sampled rows: a read of LDS another wave's loads have
    not filled would show as call-to-call differences."""
    T, k, rows = shape
    backend.set_act_mode(1)
    try:
        raw = q6k_full_scale_range(synth.weight(Q6K, rows, k, 620 + T), rows, k, 621)
        x = synth.normal_f32(T * k, 622 + T)
        w = backend.upload_weight(raw, Q6K, (rows, k))
        xb = backend.f32_buf(x)
        outs = []
        for _ in range(6):
            yb = backend.alloc(T * rows * 4)
            backend.qmatmul_i8(w, xb, yb)
            outs.append(backend.download_f32(yb))
            yb.close()
        for o in outs[1:]:
            assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32)), f"wide Q6_K GEMM not repeatable at {shape}"
        y = outs[0].reshape(T, rows)
        rb = len(raw) // rows
        for r0 in (0, rows - 16):
            sl = raw[r0 * rb:(r0 + 16) * rb]
            tok = np.unique(np.r_[0:4, 255:259, T - 4:T])
            cpu, exact, absum = oracle_i8_32(Q6K, sl, 16, k, x.reshape(T, k)[tok].reshape(-1))
            assert_parity(y[tok, r0:r0 + 16].reshape(-1), cpu, exact, 1e-3, abs_sum=absum,
                          what=f"wide q6k T={T} k={k} rows {r0}..")
        w.buf.close(), xb.close()
    finally:
        backend.set_act_mode(0)


@pytest.mark.parametrize("shape", [(200, 768, 256), (64, 512, 384), (130, 512, 128)])
def test_prefill_gated_gemm_equals_separate(backend, shape):
    """Q4_K ffn_gate_up at prefill size runs one gated GEMM launch whose
    epilogue writes silu(gate) * up. Each output's arithmetic is that of the
    separate GEMMs (K under 1024 columns: no launch splits K), and the SiLU
    is silu_mul's, so the result equals qmatmul(gate), qmatmul(up), then
    silu_mul, bit for bit."""
    T, k, n = shape
    backend.set_act_mode(1)
    try:
        raws = [synth.weight(Q4K, n, k, 530 + i) for i in range(2)]
        ws = [backend.upload_weight(r, Q4K, (n, k)) for r in raws]
        xb = backend.f32_buf(synth.normal_f32(T * k, 540 + T))
        gs, us, y = (backend.alloc(T * n * 4) for _ in range(3))
        backend.ffn_gate_up(ws[0], ws[1], xb, gs, us, y)
        got = backend.download_f32(y)
        og, ou, y2 = (backend.alloc(T * n * 4) for _ in range(3))
        backend.qmatmul(ws[0], xb, og)
        backend.qmatmul(ws[1], xb, ou)
        backend.silu_mul(og, ou, y2)
        want = backend.download_f32(y2)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
            f"gated GEMM differs from separate GEMMs + silu_mul at {shape}: {np.sum(got != want)} elements"
    finally:
        backend.set_act_mode(0)


@pytest.mark.parametrize("shape", [(64, 4096, 1024), (70, 512, 320), (300, 2048, 256)])
def test_prefill_gated_gemm_matches_oracle(backend, shape):
    """The gated launch against the oracle's silu(gate) * up where K is
    split over workgroups (64 x 4096 -> 1024: 16 column tiles) and over
    ragged token counts; 320 rows (not a multiple of 128) take the unfused
    GEMMs and silu_mul."""
    T, k, n = shape
    backend.set_act_mode(1)
    try:
        raws = [synth.weight(Q4K, n, k, 550 + i) for i in range(2)]
        ws = [backend.upload_weight(r, Q4K, (n, k)) for r in raws]
        x = synth.normal_f32(T * k, 560 + n)
        xb = backend.f32_buf(x)
        gs, us = backend.alloc(T * n * 4), backend.alloc(T * n * 4)
        y = backend.f32_buf(np.full(T * n + 16, CANARY, np.float32))
        backend.ffn_gate_up(ws[0], ws[1], xb, gs, us, y)
        out = backend.download_f32(y)
        assert np.all(out[T * n:] == CANARY)
        g = oracle_i8_32(Q4K, raws[0], n, k, x)[0].astype(np.float32)
        u = oracle_i8_32(Q4K, raws[1], n, k, x)[0].astype(np.float32)
        want = ffi.silu_mul(g.reshape(-1), u.reshape(-1))
        np.testing.assert_allclose(out[:T * n], want, rtol=2e-3, atol=1e-3)
    finally:
        backend.set_act_mode(0)


@pytest.mark.parametrize("dtype", [Q8, Q4K, Q6K])
def test_prefill_gemm_fused_calls(backend, dtype):
    backend.set_act_mode(1)
    try:
        T, k, n = 64, 512, 160
        raws = [synth.weight(dtype, n, k, 500 + i) for i in range(3)]
        ws = [backend.upload_weight(r, dtype, (n, k)) for r in raws]
        x = synth.normal_f32(T * k, 510)
        xb = backend.f32_buf(x)
        outs = [backend.alloc(T * n * 4) for _ in range(3)]
        backend.qmatmul_qkv(ws[0], ws[1], ws[2], xb, *outs)
        for i in range(3):
            cpu, exact, absum = oracle_i8_32(dtype, raws[i], n, k, x)
            assert_parity(backend.download_f32(outs[i]), cpu, exact, 1e-3, abs_sum=absum,
                          what=f"gemm qkv {i}")
        y = backend.alloc(T * n * 4)
        backend.ffn_gate_up(ws[0], ws[1], xb, outs[0], outs[1], y)
        g = oracle_i8_32(dtype, raws[0], n, k, x)[0].astype(np.float32)
        u = oracle_i8_32(dtype, raws[1], n, k, x)[0].astype(np.float32)
        want = ffi.silu_mul(g.reshape(-1), u.reshape(-1))
        np.testing.assert_allclose(backend.download_f32(y), want, rtol=2e-3, atol=1e-3)
    finally:
        backend.set_act_mode(0)
