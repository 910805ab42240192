"""The CPU-order mode (MDMA_ACT_F32_CPU) against the CPU oracle, bit for bit.

CpuBackend::qmatmul (/root/reference/src/backend/cpu.rs:46-48,335-368) sums
every output sequentially in f32 from -0.0 over f32-rounded products of the
dequantized row; the mode's GEMV does the same, one lane per row, so every
output must equal the oracle's exactly (the plain 1e-5 / 1e-6 pass rate is
then 1.0 by construction, and is asserted as equality). Likewise rmsnorm,
add_rmsnorm, silu_mul (with the C library's expf), ffn_gate_up and
attention (cpu.rs:50-60,388-402,447-458,530-590). Both weight layouts (the
prepared planes and raw GGUF blocks) are covered, at the reference's test
shapes (src/backend/rocm/decode/tests.rs:81-96, committed oracle outputs in
tests/golden/qmatmul_small.npz) and at every Llama-3-8B shape of the
benchmark configurations.
"""
import os

import numpy as np
import pytest

from mdma_amd import synth
from mdma_amd.backend import ACT_F32, ACT_F32_CPU, AttnSpec, KvView, QWeight
from oracle import ffi

pytestmark = pytest.mark.gpu
Q8, Q4K, Q6K, F32, F16 = 8, 12, 14, 0, 1
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "qmatmul_small.npz")
CANARY = np.float32(123456.25)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture
def cpu_mode(backend):
    backend.set_act_mode(ACT_F32_CPU)
    yield backend
    backend.set_act_mode(ACT_F32)


def weight(be, dtype, raw, rows, k, layout):
    """layout 'prepared': the gfx950 planes; 'raw': the GGUF bytes as they are."""
    if layout == "prepared":
        return be.upload_weight(raw, dtype, (rows, k))
    a = np.ascontiguousarray(raw).view(np.uint8).reshape(-1)
    b = be.alloc(a.nbytes)
    be.upload(b, 0, a)
    return QWeight(dtype, (rows, k), b)


def gpu_qmatmul(be, w, rows, x, T):
    yb = be.f32_buf(np.full(T * rows + 8, CANARY, np.float32))
    be.qmatmul(w, be.f32_buf(x), yb)
    y = be.download_f32(yb)
    assert np.all(y[T * rows:] == CANARY), "wrote past the output"
    return y[:T * rows].reshape(T, rows)


@pytest.mark.parametrize("layout", ["prepared", "raw"])
def test_reference_shapes_equal_committed_oracle_outputs(cpu_mode, layout):
    g = np.load(GOLDEN)
    n = 0
    for dt in (Q8, Q4K, Q6K):
        for rows in (1, 7, 9, 20):
            for k in (256, 512, 768):
                key = f"{dt}_{rows}_{k}"
                raw, x, want = g[key + "_w"], g[key + "_x"], g[key + "_y"]
                got = gpu_qmatmul(cpu_mode, weight(cpu_mode, dt, raw, rows, k, layout), rows, x, 2)
                assert np.array_equal(bits(got), bits(want)), key
                n += 1
    assert n == 36


LLAMA8B = [(Q4K, 4096, 4096), (Q4K, 1024, 4096), (Q4K, 14336, 4096), (Q4K, 4096, 14336),
           (Q6K, 4096, 14336), (Q6K, 4096, 4096), (Q6K, 1024, 4096), (Q8, 4096, 4096)]


@pytest.mark.parametrize("dtype,rows,k", LLAMA8B)
@pytest.mark.parametrize("T", [1, 4, 8])
def test_llama8b_shapes_bit_equal_oracle(cpu_mode, dtype, rows, k, T):
    raw = synth.weight(dtype, rows, k, rows + k + dtype, True)
    x = synth.normal_f32(T * k, 7 * T + dtype)
    got = gpu_qmatmul(cpu_mode, weight(cpu_mode, dtype, raw, rows, k, "prepared"), rows, x, T)
    want = ffi.qmatmul(dtype, raw, rows, k, x)
    diff = np.count_nonzero(bits(got) != bits(want))
    assert diff == 0, f"{diff} of {got.size} outputs differ"


def test_output_head_bit_equal_oracle(cpu_mode):
    rows, k = 128256, 4096
    raw = synth.weight(Q6K, rows, k, 77, True)
    x = synth.normal_f32(k, 78)
    got = gpu_qmatmul(cpu_mode, weight(cpu_mode, Q6K, raw, rows, k, "prepared"), rows, x, 1)
    assert np.array_equal(bits(got), bits(ffi.qmatmul(Q6K, raw, rows, k, x)))


@pytest.mark.parametrize("T", [3, 19])
def test_ragged_tokens_and_raw_layout(cpu_mode, T):
    # Token counts that are not whole groups of 8 chains; raw GGUF rows of an
    # odd number of blocks (2-byte-aligned Q6_K / Q8_0 blocks).
    for dtype, rows, k in ((Q6K, 70, 768), (Q8, 65, 288), (Q4K, 129, 1280)):
        raw = synth.weight(dtype, rows, k, 5 + rows, True)
        x = synth.normal_f32(T * k, 11 + T)
        want = ffi.qmatmul(dtype, raw, rows, k, x)
        for layout in ("prepared", "raw"):
            got = gpu_qmatmul(cpu_mode, weight(cpu_mode, dtype, raw, rows, k, layout), rows, x, T)
            assert np.array_equal(bits(got), bits(want)), (dtype, layout)


@pytest.mark.parametrize("dtype", [F32, F16])
def test_float_weights_bit_equal_oracle(cpu_mode, dtype):
    rows, k, T = 33, 100, 3
    w = synth.normal_f32(rows * k, 3)
    raw = w.view(np.uint8) if dtype == F32 else w.astype(np.float16).view(np.uint8)
    x = synth.normal_f32(T * k, 4)
    got = gpu_qmatmul(cpu_mode, weight(cpu_mode, dtype, raw, rows, k, "raw"), rows, x, T)
    assert np.array_equal(bits(got), bits(ffi.qmatmul(dtype, raw, rows, k, x)))


def test_cancellation_case_takes_the_sequential_value(cpu_mode):
    # The oracle's own pin (tests/test_oracle.py): the sequential f32 sum of
    # [1e8, 1, -1e8, 1] is 1, the exact sum 2.
    raw = np.array([1e8, 1.0, -1e8, 1.0], np.float32).view(np.uint8)
    got = gpu_qmatmul(cpu_mode, weight(cpu_mode, F32, raw, 1, 4, "raw"), 1, np.ones(4, np.float32), 1)
    assert got[0, 0] == np.float32(1.0)


def test_rmsnorm_and_add_rmsnorm_bit_equal(cpu_mode):
    be = cpu_mode
    for dim, rows in ((4096, 3), (288, 5), (14336, 1)):
        w = synth.normal_f32(dim, dim)
        a = synth.normal_f32(rows * dim, 1) * 3
        b = synth.normal_f32(rows * dim, 2)
        y = be.alloc(rows * dim * 4)
        be.rmsnorm(be.f32_buf(w), be.f32_buf(a), y, 1e-5)
        assert np.array_equal(bits(be.download_f32(y)), bits(ffi.rmsnorm(w, a, 1e-5)))
        s = be.alloc(rows * dim * 4)
        be.add_rmsnorm(be.f32_buf(w), be.f32_buf(a), be.f32_buf(b), s, y, 1e-5)
        ws, wy = ffi.add_rmsnorm(w, a, b, 1e-5)
        assert np.array_equal(bits(be.download_f32(s)), bits(ws))
        assert np.array_equal(bits(be.download_f32(y)), bits(wy))


def silu_inputs():
    # exp(-g) at inputs where the correctly rounded exp and the C library's
    # expf differ (found on the CPU; the device must give the library's),
    # the overflow / underflow edges, signed zeros and a wide random sample.
    hexes = ["0x1.ec0716p-11", "0x1.ec0f18p-11", "0x1.9424fcp-14", "0x1.e2671ap-14", "-0x1.b8d88ap-11",
             "-0x1.fefe02p-16", "-0x1.04845ep+5", "0x1.f8cbb2p+5"]
    hard = np.array([float.fromhex(h) for h in hexes] + [88.0, -88.0, 88.72283, -88.72284, 103.97, -103.97, 104.0,
                                                          0.0, -0.0, 1e-30, -1e-30], np.float32)
    rng = np.random.default_rng(5)
    wide = (rng.standard_normal(1 << 20) * 8).astype(np.float32)
    tiny = (rng.standard_normal(1 << 18) * 1e-3).astype(np.float32)
    return np.concatenate([hard, wide, tiny])


def test_silu_mul_bit_equal_with_c_library_expf(cpu_mode):
    be = cpu_mode
    g = silu_inputs()
    u = synth.normal_f32(g.size, 9)
    y = be.alloc(g.size * 4)
    be.silu_mul(be.f32_buf(g), be.f32_buf(u), y)
    got, want = be.download_f32(y), ffi.silu_mul(g, u)
    diff = np.nonzero(bits(got) != bits(want))[0]
    assert diff.size == 0, f"{diff.size} differ; first g {g[diff[:4]]} gpu {got[diff[:4]]} cpu {want[diff[:4]]}"


def test_ffn_gate_up_bit_equal(cpu_mode):
    be = cpu_mode
    F, E, T = 1536, 512, 2
    gr, ur = synth.weight(Q4K, F, E, 1, True), synth.weight(Q4K, F, E, 2, True)
    x = synth.normal_f32(T * E, 3)
    gw, uw = be.upload_weight(gr, Q4K, (F, E)), be.upload_weight(ur, Q4K, (F, E))
    gs, us, y = be.alloc(T * F * 4), be.alloc(T * F * 4), be.alloc(T * F * 4)
    be.ffn_gate_up(gw, uw, be.f32_buf(x), gs, us, y)
    want = ffi.silu_mul(ffi.qmatmul(Q4K, gr, F, E, x).reshape(-1), ffi.qmatmul(Q4K, ur, F, E, x).reshape(-1))
    assert np.array_equal(bits(be.download_f32(y)), bits(want))


@pytest.mark.parametrize("n_q,kv_len,hd,H,KVH", [(1, 1, 128, 32, 8), (1, 700, 128, 32, 8), (17, 17, 48, 6, 6),
                                                  (5, 300, 64, 8, 2), (1, 2150, 256, 4, 1)])
def test_attention_bit_equal(cpu_mode, n_q, kv_len, hd, H, KVH):
    be = cpu_mode
    q = synth.normal_f32(n_q * H * hd, kv_len + hd)
    kc = synth.normal_f32(kv_len * KVH * hd, 2).astype(np.float16)
    vc = synth.normal_f32(kv_len * KVH * hd, 3).astype(np.float16)
    kb, vb = be.alloc(kc.nbytes), be.alloc(vc.nbytes)
    be.upload(kb, 0, kc.view(np.uint8))
    be.upload(vb, 0, vc.view(np.uint8))
    o = be.alloc(q.nbytes)
    be.attn(be.f32_buf(q), KvView(kb, vb, kv_len), AttnSpec(hd, H, KVH), o)
    want = ffi.attention(q, kc.astype(np.float32), vc.astype(np.float32), kv_len, hd, H, KVH)
    assert np.array_equal(bits(be.download_f32(o)), bits(want))
