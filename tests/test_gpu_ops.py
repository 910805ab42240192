"""GPU parity of the per-token Llama ops against the CPU oracle
(src/backend/cpu.rs semantics). Bit-exact where the device repeats the CPU's
arithmetic (embedding dequantization, add, RoPE from the same angle table,
f16 KV conversion, greedy); tolerance where the reduction order differs."""
import numpy as np
import pytest

from mdma_amd import synth
from mdma_amd.backend import AttnSpec, KvView, RopeSpec, ShapeMismatch
from oracle import ffi

pytestmark = pytest.mark.gpu
Q8, Q4K, Q6K, F32, F16 = 8, 12, 14, 0, 1


def f16r(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


@pytest.mark.parametrize("dtype,n_embd", [(F32, 288), (F16, 64), (Q8, 288), (Q4K, 512), (Q6K, 512)])
def test_embed_bit_exact(backend, dtype, n_embd):
    vocab = 50
    raw = synth.weight(dtype, vocab, n_embd, 9)
    table = backend.upload_weight(raw, dtype, (vocab, n_embd))
    ids = [0, 49, 7, 7, 31]
    out = backend.f32_buf(np.full(len(ids) * n_embd + 4, 123456.25, np.float32))
    backend.embed(table, ids, out)
    got = backend.download_f32(out)
    assert np.all(got[len(ids) * n_embd:] == np.float32(123456.25))
    want = ffi.embed(dtype, raw, vocab, n_embd, ids).reshape(-1)
    assert np.array_equal(got[:len(ids) * n_embd].view(np.uint32), want.view(np.uint32))
    with pytest.raises(ShapeMismatch):
        backend.embed(table, [vocab], out)
    with pytest.raises(ShapeMismatch):
        backend.embed(table, [], out)


def test_embed_q4k_known_answer_blocks(backend):
    # The reference's every-header-byte Q4_K blocks (src/cache/layout/tests.rs:8-55).
    for seed in (0, 77, 255):
        raw = (((np.arange(144 * 3, dtype=np.uint32) * 73 + seed * 31) & 255)).astype(np.uint8).reshape(3, 144)
        raw[:, 0:2] = np.frombuffer(np.float16(0.125).tobytes(), np.uint8)
        raw[:, 2:4] = np.frombuffer(np.float16(0.0625).tobytes(), np.uint8)
        t = backend.upload_weight(raw.reshape(-1), Q4K, (3, 256))
        out = backend.alloc(3 * 256 * 4)
        backend.embed(t, [0, 1, 2], out)
        assert np.array_equal(backend.download_f32(out), ffi.embed(Q4K, raw.reshape(-1), 3, 256, [0, 1, 2]).reshape(-1))


@pytest.mark.parametrize("dim,rows", [(2, 1), (288, 8), (4096, 3), (1000, 2), (16384, 2), (4098, 2), (5120, 1)])
def test_rmsnorm_and_add_rmsnorm(backend, dim, rows):
    w = synth.normal_f32(dim, 1)
    a = synth.normal_f32(dim * rows, 2)
    b = synth.normal_f32(dim * rows, 3)
    wb, ab, bb = backend.f32_buf(w), backend.f32_buf(a), backend.f32_buf(b)
    y = backend.alloc(dim * rows * 4)
    backend.rmsnorm(wb, ab, y, 1e-5)
    want = ffi.rmsnorm(w, a, 1e-5)
    np.testing.assert_allclose(backend.download_f32(y), want, rtol=2e-6, atol=1e-7)
    s, y2 = backend.alloc(dim * rows * 4), backend.alloc(dim * rows * 4)
    backend.add_rmsnorm(wb, ab, bb, s, y2, 1e-5)
    ws, wy = ffi.add_rmsnorm(w, a, b, 1e-5)
    assert np.array_equal(backend.download_f32(s), ws)
    np.testing.assert_allclose(backend.download_f32(y2), wy, rtol=2e-6, atol=1e-7)
    # Hand-computed (src/backend/cpu/tests.rs:128-140).
    if dim == 2:
        backend.rmsnorm(backend.f32_buf([1.0, 1.0]), backend.f32_buf([3.0, 4.0]), y, 0.0)
        sc = 1 / np.sqrt(12.5)
        np.testing.assert_allclose(backend.download_f32(y)[:2], [3 * sc, 4 * sc], atol=1e-6)


def test_add_and_silu_mul(backend):
    for n in (1, 63, 64, 65, 255, 256, 257, 14336 * 3):
        a, b = synth.normal_f32(n, n) * 4, synth.normal_f32(n, n + 1)
        ab, bb = backend.f32_buf(a), backend.f32_buf(b)
        y = backend.f32_buf(np.full(n + 3, 7.0, np.float32))
        backend.add(ab, bb, y)
        got = backend.download_f32(y)
        assert np.array_equal(got[:n], ffi.add(a, b)) and np.all(got[n:] == 7.0)
        backend.silu_mul(ab, bb, y)
        got = backend.download_f32(y)
        np.testing.assert_allclose(got[:n], ffi.silu_mul(a, b), rtol=1e-6, atol=1e-7)
        assert np.all(got[n:] == 7.0)


@pytest.mark.parametrize("hd,nq,nkv,T,pos,theta", [(2, 1, 1, 1, 1, 10000.0), (48, 6, 6, 3, 5, 10000.0),
                                                   (128, 32, 8, 2, 4000, 500000.0), (64, 4, 2, 7, 0, 10000.0)])
def test_rope_bit_exact(backend, hd, nq, nkv, T, pos, theta):
    q, k = synth.normal_f32(T * nq * hd, 1), synth.normal_f32(T * nkv * hd, 2)
    qb, kb = backend.f32_buf(q), backend.f32_buf(k)
    backend.rope(qb, kb, pos, T, RopeSpec(hd, theta))
    wq, wk = ffi.rope(q, k, pos, T, hd, theta)
    assert np.array_equal(backend.download_f32(qb), wq)
    assert np.array_equal(backend.download_f32(kb), wk)


def test_kv_write_and_fused_rope_kv_write(backend):
    hd, nq, nkv, T, pos, theta = 64, 8, 2, 3, 9, 10000.0
    q, k, v = synth.normal_f32(T * nq * hd, 1), synth.normal_f32(T * nkv * hd, 2), synth.normal_f32(T * nkv * hd, 3)
    ctx_rows = 16
    row = nkv * hd
    dk, dv = backend.alloc(ctx_rows * row * 2), backend.alloc(ctx_rows * row * 2)
    backend.upload(dk, 0, np.zeros(ctx_rows * row, np.uint16))
    backend.upload(dv, 0, np.zeros(ctx_rows * row, np.uint16))
    qb, kb, vb = backend.f32_buf(q), backend.f32_buf(k), backend.f32_buf(v)
    backend.rope_kv_write(qb, kb, vb, dk, dv, pos * row, pos, T, RopeSpec(hd, theta), T * row)
    wq, wk = ffi.rope(q, k, pos, T, hd, theta)
    assert np.array_equal(backend.download_f32(qb), wq)
    gk = backend.download(dk, 0, dk.len).view(np.float16).astype(np.float32)
    gv = backend.download(dv, 0, dv.len).view(np.float16).astype(np.float32)
    assert np.array_equal(gk[pos * row:(pos + T) * row], f16r(wk))
    assert np.array_equal(gv[pos * row:(pos + T) * row], f16r(v))
    assert np.all(gk[:pos * row] == 0) and np.all(gk[(pos + T) * row:] == 0)
    # Plain kv_write.
    backend.kv_write(vb, kb, dk, dv, 0, T * row)
    assert np.array_equal(backend.download(dk, 0, T * row * 2).view(np.float16).astype(np.float32), f16r(v))
    with pytest.raises(ShapeMismatch):
        backend.kv_write(vb, kb, dk, dv, (ctx_rows - 1) * row, T * row)


@pytest.mark.parametrize("hd,nq,nkv,n_q,kv_len", [(2, 1, 1, 1, 2), (48, 6, 6, 1, 9), (48, 6, 6, 8, 8),
                                                  (128, 32, 8, 1, 700), (128, 32, 8, 4, 2500), (64, 4, 1, 5, 5),
                                                  (128, 32, 8, 1, 64), (128, 32, 8, 1, 65), (128, 32, 8, 70, 70),
                                                  (128, 16, 2, 3, 300), (256, 8, 2, 2, 130), (96, 6, 3, 1, 200),
                                                  (64, 12, 4, 2, 129), (128, 32, 8, 8, 2500),
                                                  # prompts of 64 queries and more (the matrix-core kernel):
                                                  # G = 4, 1, 8, 2, hd 128 and 64, with and without a prefix
                                                  (128, 32, 8, 64, 64), (128, 32, 8, 512, 512),
                                                  (128, 32, 8, 200, 300), (64, 8, 8, 128, 128),
                                                  (128, 16, 2, 96, 100), (64, 8, 4, 65, 65)])
def test_attention_over_f16_cache(backend, hd, nq, nkv, n_q, kv_len):
    q = synth.normal_f32(n_q * nq * hd, 1)
    k = f16r(synth.normal_f32(kv_len * nkv * hd, 2))
    v = f16r(synth.normal_f32(kv_len * nkv * hd, 3))
    kb, vb = backend.alloc(k.size * 2), backend.alloc(v.size * 2)
    backend.upload(kb, 0, k.astype(np.float16))
    backend.upload(vb, 0, v.astype(np.float16))
    o = backend.f32_buf(np.full(q.size + 2, -3.0, np.float32))
    backend.attn(backend.f32_buf(q), KvView(kb, vb, kv_len), AttnSpec(hd, nq, nkv), o)
    got = backend.download_f32(o)
    assert np.all(got[q.size:] == -3.0)
    want = ffi.attention(q, k, v, kv_len, hd, nq, nkv)
    np.testing.assert_allclose(got[:q.size], want, rtol=2e-5, atol=2e-6)


@pytest.mark.parametrize("hd,G", [(64, 2), (128, 4)])
def test_attention_head_split_same_bits(backend, hd, G):
    """A launch with few workgroups splits each KV head's query heads over
    two workgroups; one with many does not. The same heads' outputs must be
    the same bits either way: 2 KV heads (split) against 200 KV heads whose
    first 2 hold the same q, K and V (not split), one 64-key tile per run in
    both (384 keys: 6 runs)."""
    kv_len, small, big = 384, 2, 200
    q_b = synth.normal_f32(big * G * hd, 11)
    k_b = f16r(synth.normal_f32(kv_len * big * hd, 12)).reshape(kv_len, big * hd)
    v_b = f16r(synth.normal_f32(kv_len * big * hd, 13)).reshape(kv_len, big * hd)
    outs = []
    for nkv in (small, big):
        q = q_b[:nkv * G * hd]
        k = np.ascontiguousarray(k_b[:, :nkv * hd]).reshape(-1)
        v = np.ascontiguousarray(v_b[:, :nkv * hd]).reshape(-1)
        kb, vb = backend.alloc(k.size * 2), backend.alloc(v.size * 2)
        backend.upload(kb, 0, k.astype(np.float16))
        backend.upload(vb, 0, v.astype(np.float16))
        o = backend.alloc(q.size * 4)
        backend.attn(backend.f32_buf(q), KvView(kb, vb, kv_len), AttnSpec(hd, nkv * G, nkv), o)
        outs.append(backend.download_f32(o))
    assert np.array_equal(outs[0], outs[1][:small * G * hd])
    want = ffi.attention(q_b[:small * G * hd], np.ascontiguousarray(k_b[:, :small * hd]).reshape(-1),
                         np.ascontiguousarray(v_b[:, :small * hd]).reshape(-1), kv_len, hd, small * G, small)
    np.testing.assert_allclose(outs[0], want, rtol=2e-5, atol=2e-6)


def test_attention_hand_computed(backend):
    # src/backend/cpu/tests.rs:186-214 (values exact in f16).
    kb, vb = backend.alloc(8), backend.alloc(8)
    backend.upload(kb, 0, np.array([1, 0, 0, 1], np.float16))
    backend.upload(vb, 0, np.array([10, 20, 30, 40], np.float16))
    o = backend.alloc(8)
    backend.attn(backend.f32_buf([1.0, 0.0]), KvView(kb, vb, 2), AttnSpec(2, 1, 1), o)
    s = 1 / np.sqrt(2)
    w0, w1 = 1 / (1 + np.exp(-s)), np.exp(-s) / (1 + np.exp(-s))
    np.testing.assert_allclose(backend.download_f32(o), [w0 * 10 + w1 * 30, w0 * 20 + w1 * 40], atol=1e-5)


def test_greedy(backend):
    for x in (np.array([1.0, 3.0, 2.0, 3.0, -1.0], np.float32), np.array([-0.0, 0.0, -0.0], np.float32),
              synth.normal_f32(32000, 1), synth.normal_f32(128256, 2), np.full(5000, 2.5, np.float32),
              np.full(12289, -np.float32(3e38), np.float32)):
        assert backend.greedy(backend.f32_buf(x)) == ffi.greedy(x)
    # The maximum, and a tie for it, in different chunks of 4096.
    x = synth.normal_f32(20000, 4)
    x[5000] = x[17000] = 9.0
    assert backend.greedy(backend.f32_buf(x)) == ffi.greedy(x) == 17000
    x[17000] = 8.0
    assert backend.greedy(backend.f32_buf(x)) == 5000
    # Sub-range of a buffer (offset, n).
    assert backend.greedy(backend.f32_buf(x), 4097, 9000) == 5000 - 4097
    from mdma_amd.backend import BackendError
    bad = synth.normal_f32(100, 3)
    bad[17] = np.inf
    with pytest.raises(BackendError):
        backend.greedy(backend.f32_buf(bad))
    bad = synth.normal_f32(10000, 5)
    bad[9999] = np.nan
    with pytest.raises(BackendError):
        backend.greedy(backend.f32_buf(bad))
