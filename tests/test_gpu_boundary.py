"""The drop-in boundary on the GPU: the trait-shaped upload_weight(bytes,
layout), BufferBudget semantics and graph replay safety.

- upload_weight (src/backend.rs:228-237) carries no dtype or shape. GGUF
  bytes are stored raw; the first op that reads the buffer as a QWeight
  repacks it on the device into the prepared layout. The repacked bytes must
  equal the host packer's, results must match the oracle and the typed
  upload's bit for bit, and RocmQ4kV3 bytes are refused as NotImplemented.
- BufferBudget (src/memory/buffers.rs:32-99): device and host quotas,
  installed only before allocations (BufferBudget::replace), requested bytes
  charged, zero forbids a domain, the context's own scratch growth charged.
- A captured graph replays eager results, and refuses to replay once the
  context has replaced a buffer it captured.
"""
import numpy as np
import pytest

import npq
from conftest import assert_parity, f32_exact
from mdma_amd import backend as bm
from mdma_amd import gguf, llama_synth, synth
from mdma_amd.backend import (DOMAIN_DEVICE, DOMAIN_HOST, LAYOUT_GFX950, LAYOUT_GGUF, LAYOUT_ROCM_Q4K_V3,
                              Gfx950Backend, QWeight, pack_weight)
from mdma_amd.model import Model
from oracle import ffi

pytestmark = pytest.mark.gpu
Q8, Q4K, Q6K, F32 = 8, 12, 14, 0


@pytest.mark.parametrize("dtype,rows,k", [(Q4K, 96, 1024), (Q6K, 70, 768), (Q8, 33, 288)])
def test_trait_upload_repacks_on_first_use(backend, dtype, rows, k):
    raw = synth.weight(dtype, rows, k, 700 + dtype)
    x = synth.normal_f32(3 * k, 701)
    buf = backend.upload_weight_bytes(raw, LAYOUT_GGUF)
    assert backend.buf_layout(buf) == LAYOUT_GGUF and buf.len == raw.nbytes
    w = QWeight(dtype, (rows, k), buf)
    xb, yb = backend.f32_buf(x), backend.alloc(3 * rows * 4)
    backend.qmatmul_f32(w, xb, yb)
    # The first op repacked the buffer: it now holds the prepared rows, the
    # device repack byte for byte the host packer's.
    assert backend.buf_layout(buf) == LAYOUT_GFX950
    packed = pack_weight(raw, dtype, (rows, k))
    assert buf.len == packed.nbytes
    assert np.array_equal(backend.download(buf, 0, buf.len), packed)
    got = backend.download_f32(yb)
    cpu = ffi.qmatmul(dtype, raw, rows, k, x)
    exact = f32_exact(npq.dequantize(dtype, raw, rows, k), x)
    assert_parity(got, cpu, exact, 1e-5, what=f"trait upload {dtype}", correctly_rounded=True)
    # The prepared kernels ran: the same bits as a weight uploaded typed.
    typed = backend.upload_weight(raw, dtype, (rows, k))
    y2 = backend.alloc(3 * rows * 4)
    for fn in (backend.qmatmul_f32, backend.qmatmul_i8):
        fn(w, xb, yb)
        fn(typed, xb, y2)
        assert np.array_equal(backend.download_f32(yb), backend.download_f32(y2))


def test_view_of_trait_upload_keeps_the_weight_raw(backend):
    # A view into a weight's raw bytes taken before its first use: the weight
    # stays raw (a repack would free the bytes under the view), the view
    # downloads the uploaded bytes, and ops through the parent and the view
    # both read them.
    rows, k = 96, 1024
    raw = synth.weight(Q4K, rows, k, 711)
    x = synth.normal_f32(2 * k, 712)
    buf = backend.upload_weight_bytes(raw, LAYOUT_GGUF)
    view = backend.view(buf, 0, buf.len)
    xb = backend.f32_buf(x)
    y_parent, y_view = backend.alloc(2 * rows * 4), backend.alloc(2 * rows * 4)
    backend.qmatmul_f32(QWeight(Q4K, (rows, k), buf), xb, y_parent)
    assert backend.buf_layout(buf) == LAYOUT_GGUF and buf.len == raw.nbytes
    assert np.array_equal(backend.download(view, 0, view.len), raw.view(np.uint8))
    backend.qmatmul_f32(QWeight(Q4K, (rows, k), view), xb, y_view)
    a, b = backend.download_f32(y_parent), backend.download_f32(y_view)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    cpu = ffi.qmatmul(Q4K, raw, rows, k, x)
    assert_parity(a, cpu, f32_exact(npq.dequantize(Q4K, raw, rows, k), x), rtol=1e-5, what="view of raw weight",
                  correctly_rounded=True)
    view.close()


def test_trait_upload_layouts(backend):
    raw = synth.weight(Q4K, 8, 256, 710)
    with pytest.raises(bm.NotImplemented):
        backend.upload_weight_bytes(raw, LAYOUT_ROCM_Q4K_V3)
    # Prepared bytes are stored as they are.
    pre = backend.upload_weight_bytes(pack_weight(raw, Q4K, (8, 256)), LAYOUT_GFX950)
    assert backend.buf_layout(pre) == LAYOUT_GFX950
    x = synth.normal_f32(256, 711)
    y = backend.alloc(8 * 4)
    backend.qmatmul_f32(QWeight(Q4K, (8, 256), pre), backend.f32_buf(x), y)
    cpu = ffi.qmatmul(Q4K, raw, 8, 256, x)
    assert_parity(backend.download_f32(y), cpu, f32_exact(npq.dequantize(Q4K, raw, 8, 256), x), 1e-5,
                  correctly_rounded=True)
    # Float weights keep their bytes; a QWeight whose size does not match
    # the raw bytes is a shape error, not a repack.
    f = backend.upload_weight_bytes(synth.weight(F32, 4, 64, 712), LAYOUT_GGUF)
    backend.qmatmul(QWeight(F32, (4, 64), f), backend.f32_buf(synth.normal_f32(64, 1)), backend.alloc(16))
    assert backend.buf_layout(f) == LAYOUT_GGUF
    odd = backend.upload_weight_bytes(raw, LAYOUT_GGUF)
    with pytest.raises(bm.ShapeMismatch):
        backend.qmatmul(QWeight(Q4K, (16, 256), odd), backend.f32_buf(x), backend.alloc(64))
    assert backend.buf_layout(odd) == LAYOUT_GGUF


def test_embed_through_trait_upload(backend):
    raw = synth.weight(Q6K, 40, 512, 720)
    buf = backend.upload_weight_bytes(raw, LAYOUT_GGUF)
    ids = np.array([3, 0, 39, 3], np.uint32)
    out = backend.alloc(ids.size * 512 * 4)
    backend.embed(QWeight(Q6K, (40, 512), buf), ids, out)
    assert backend.buf_layout(buf) == LAYOUT_GFX950
    W = ffi.dequantize_row(Q6K, raw, 40 * 512).reshape(40, 512)
    assert np.array_equal(backend.download_f32(out), W[ids].reshape(-1))


# ---------------------------------------------------------------- budget ----

def fresh():
    return Gfx950Backend(0)


def test_budget_zero_device_quota_forbids_allocation():
    be = fresh()
    try:
        be.set_buffer_budget(device=0)
        with pytest.raises(bm.BufferBudget):
            be.alloc(16)
        assert be.buffer_usage(DOMAIN_DEVICE) == (0, 0)
        assert be.buffer_usage(DOMAIN_HOST)[1] == 2**64 - 1
    finally:
        be.close()


def test_budget_installs_only_before_allocations_and_charges_requested_bytes():
    be = fresh()
    try:
        b = be.alloc(1000)
        assert be.buffer_usage(DOMAIN_DEVICE)[0] == 1000  # requested, not the 1024 allocated
        with pytest.raises(bm.Backend):
            be.set_buffer_budget(device=1 << 30)
        b.close()
        assert be.buffer_usage(DOMAIN_DEVICE)[0] == 0
        be.set_buffer_budget(device=5000)
        keep = [be.alloc(2000), be.alloc(3000)]
        with pytest.raises(bm.BufferBudget):
            be.alloc(1)
        assert be.buffer_usage(DOMAIN_DEVICE) == (5000, 5000)
        keep[0].close()
        be.alloc(1500).close()
    finally:
        be.close()


def test_budget_charges_context_scratch_growth():
    """The int8 activation buffer a 3-token int8 GEMV grows (at least 1 MiB)
    is charged: a quota that holds the buffers but not that growth refuses
    the call with BufferBudget; a larger one accepts it and shows the charge."""
    rows, k = 64, 4096
    raw = synth.weight(Q4K, rows, k, 730)
    x = synth.normal_f32(3 * k, 731)
    for quota, ok in ((1 << 20, False), (8 << 20, True)):
        be = fresh()
        try:
            be.set_buffer_budget(device=quota)
            w = be.upload_weight(raw, Q4K, (rows, k))
            xb, yb = be.f32_buf(x), be.alloc(3 * rows * 4)
            held = be.buffer_usage(DOMAIN_DEVICE)[0]
            if not ok:
                with pytest.raises(bm.BufferBudget):
                    be.qmatmul_i8(w, xb, yb)
                assert be.buffer_usage(DOMAIN_DEVICE)[0] == held
            else:
                be.qmatmul_i8(w, xb, yb)
                assert be.buffer_usage(DOMAIN_DEVICE)[0] >= held + (1 << 20)
                cpu = ffi.qmatmul(Q4K, raw, rows, k, np.concatenate(
                    [ffi.dequantize_act(*ffi.quantize_act(x[t * k:(t + 1) * k], 256)[:2], 256) for t in range(3)]))
                assert np.allclose(be.download_f32(yb), cpu.reshape(-1), rtol=1e-3, atol=1e-4)
        finally:
            be.close()


def test_budget_refusing_tile_images_keeps_row_planes():
    """With the batch layout on, a Q6_K weight's tile images are charged to
    the device budget at its first batched call: a quota one byte short of
    them leaves the call on the row planes (same bits, no error, nothing
    charged for them); a quota that holds them shows their bytes."""
    rows, k, T = 64, 2048, 8
    raw = synth.weight(Q6K, rows, k, 740)
    x = synth.normal_f32(T * k, 741)
    tile = len(raw)  # 16-row tiles of 512-column pairs: the GGUF bytes
    out, grow = [], None
    for extra in (None, -1, 0):
        be = fresh()
        try:
            if extra is not None:
                be.set_buffer_budget(device=held + grow + tile + extra)
            w = be.upload_weight(raw, Q6K, (rows, k))
            xb, yb = be.f32_buf(x), be.alloc(T * rows * 4)
            held = be.buffer_usage(DOMAIN_DEVICE)[0]
            be.set_batch_layout(extra is not None)
            be.qmatmul_i8(w, xb, yb)
            used = be.buffer_usage(DOMAIN_DEVICE)[0] - held
            if extra is None:
                grow = used  # the int8 activation buffer's growth alone
            else:
                assert used == grow + (tile if extra == 0 else 0), (extra, used, grow)
            out.append(be.download_f32(yb).copy())
        finally:
            be.close()
    assert all(np.array_equal(o.view(np.uint32), out[0].view(np.uint32)) for o in out)


def test_insufficient_memory_before_any_allocation(backend, tmp_path):
    p = str(tmp_path / "tiny.gguf")
    llama_synth.write(p, llama_synth.TINYSTORIES, llama_synth.Q8_ALL, 1)
    m = Model(backend, p)
    used = backend.buffer_usage(DOMAIN_DEVICE)[0]
    # 200000 sequences of 256 positions: ~354 GB of KV cache, past the device.
    with pytest.raises(bm.InsufficientMemory):
        m.session(256, 200000, 8)
    assert backend.buffer_usage(DOMAIN_DEVICE)[0] == used
    m.close()


# ---------------------------------------------------------------- graphs ----

def test_graph_replay_equals_eager_and_refuses_after_reallocation(backend):
    """A captured int8 GEMV sequence (rmsnorm writing the int8 form, then the
    GEMVs reading it) replays the eager bits, repeatedly and with eager work
    and synchronisation between replays; after the context replaces its
    scratch the graph refuses to replay."""
    rows, k = 512, 4096
    w = backend.upload_weight(synth.weight(Q4K, rows, k, 740), Q4K, (rows, k))
    w6 = backend.upload_weight(synth.weight(Q6K, rows, k, 741), Q6K, (rows, k))
    g = backend.f32_buf(np.full(k, 0.9, np.float32))
    xr = backend.f32_buf(synth.normal_f32(k, 742))
    xn, y1, y2 = backend.alloc(k * 4), backend.alloc(rows * 4), backend.alloc(rows * 4)
    backend.set_act_mode(bm.ACT_I8)
    try:
        backend.reserve_scratch(16 << 20)

        def step():
            backend.rmsnorm(g, xr, xn, 1e-5)
            backend.qmatmul(w, xn, y1)
            backend.qmatmul(w6, xn, y2)

        step()
        want = (backend.download_f32(y1).copy(), backend.download_f32(y2).copy())
        graph = backend.capture(step)
        x2, o2 = backend.f32_buf(synth.normal_f32(2 * k, 743)), backend.alloc(2 * rows * 4)
        for i in range(4):
            backend.upload(y1, 0, np.zeros(rows, np.float32))
            backend.upload(y2, 0, np.zeros(rows, np.float32))
            backend.qmatmul(w6, x2, o2)  # eager work between replays, through the int8 activation buffer
            graph.launch()
            backend.join_execution()
            assert np.array_equal(backend.download_f32(y1), want[0]), i
            assert np.array_equal(backend.download_f32(y2), want[1]), i
        backend.reserve_scratch(64 << 20)  # replaces the scratch the graph captured
        with pytest.raises(bm.Backend):
            graph.launch()
        graph.close()
    finally:
        backend.set_act_mode(bm.ACT_F32)


def test_graph_of_raw_weight_refuses_after_repack(backend):
    """A weight from the trait-shaped upload captured while still raw (no
    repack under capture): the replay reads the raw bytes; once an eager op
    repacks the weight, the graph refuses to replay."""
    rows, k = 64, 1024
    raw = synth.weight(Q4K, rows, k, 750)
    buf = backend.upload_weight_bytes(raw, LAYOUT_GGUF)
    w = QWeight(Q4K, (rows, k), buf)
    x = synth.normal_f32(k, 751)
    xb, yb = backend.f32_buf(x), backend.alloc(rows * 4)
    backend.reserve_scratch(16 << 20)
    graph = backend.capture(lambda: backend.qmatmul_f32(w, xb, yb))
    assert backend.buf_layout(buf) == LAYOUT_GGUF
    graph.launch()
    backend.join_execution()
    cpu = ffi.qmatmul(Q4K, raw, rows, k, x)
    assert_parity(backend.download_f32(yb), cpu, f32_exact(npq.dequantize(Q4K, raw, rows, k), x), 1e-5,
                  correctly_rounded=True)
    backend.qmatmul_f32(w, xb, yb)
    assert backend.buf_layout(buf) == LAYOUT_GFX950
    with pytest.raises(bm.Backend):
        graph.launch()
    graph.close()
