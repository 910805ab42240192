"""CPU checks of the gfx950 prepared weight layout (layout.cpp).

The layout is this backend's own (the reference's counterpart is its ROCm
Q4_K plane pack, src/cache/layout.rs:40-79, pinned by the round trip in
src/cache/layout/tests.rs:8-55). It is pinned here by:
  - a lossless round trip GGUF -> prepared -> GGUF on random blocks;
  - an independent numpy statement of where every GGUF byte lands, compared
    byte for byte with the library's packer;
  - the byte counts (every block keeps its size; rows pad to 16 bytes).
"""
import numpy as np
import pytest

from mdma_amd import backend, synth

Q8, Q4K, Q6K = 8, 12, 14
SHAPES = {Q4K: [(1, 256), (3, 512), (7, 4096)], Q6K: [(1, 256), (5, 768), (2, 4096)],
          Q8: [(1, 32), (4, 288), (3, 768), (2, 4096)]}


def random_blocks(dtype, rows, cols, seed):
    n = rows * (cols // synth.BLOCK_SIZE[dtype]) * synth.TYPE_SIZE[dtype]
    return np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8)


def numpy_pack(raw, dtype, rows, cols):
    """Where each GGUF byte goes, restated independently of the C++ packer."""
    nb = cols // synth.BLOCK_SIZE[dtype]
    ts = synth.TYPE_SIZE[dtype]
    rb = -(-(nb * ts) // 16) * 16
    out = np.zeros((rows, rb), np.uint8)
    blk = raw.reshape(rows, nb, ts)
    if dtype == Q4K:
        qs = blk[:, :, 16:].reshape(rows, nb, 4, 2, 16)  # [row, block, pair, half, 16]
        out[:, :64 * nb] = qs[:, :, :, 0, :].reshape(rows, -1)
        out[:, 64 * nb:128 * nb] = qs[:, :, :, 1, :].reshape(rows, -1)
        out[:, 128 * nb:144 * nb] = blk[:, :, :16].reshape(rows, -1)
    elif dtype == Q6K:
        ql, qh, sc, d = blk[:, :, :128], blk[:, :, 128:192], blk[:, :, 192:208], blk[:, :, 208:210]
        A = np.zeros((rows, nb, 4, 16), np.uint8)
        B, H, S = A.copy(), A.copy(), np.zeros((rows, nb, 4, 4), np.uint8)
        for k in range(4):
            n, h = k >> 1, k & 1
            A[:, :, k] = ql[:, :, 64 * n + 16 * h: 64 * n + 16 * h + 16]
            B[:, :, k] = ql[:, :, 64 * n + 32 + 16 * h: 64 * n + 32 + 16 * h + 16]
            H[:, :, k] = qh[:, :, 32 * n + 16 * h: 32 * n + 16 * h + 16]
            for r in range(4):
                S[:, :, k, r] = sc[:, :, 8 * n + 2 * r + h]
        out[:, :64 * nb] = A.reshape(rows, -1)
        out[:, 64 * nb:128 * nb] = B.reshape(rows, -1)
        out[:, 128 * nb:192 * nb] = H.reshape(rows, -1)
        out[:, 192 * nb:208 * nb] = S.reshape(rows, -1)
        out[:, 208 * nb:210 * nb] = d.reshape(rows, -1)
    else:
        out[:, :16 * nb] = blk[:, :, 2:18].reshape(rows, -1)
        out[:, 16 * nb:32 * nb] = blk[:, :, 18:34].reshape(rows, -1)
        out[:, 32 * nb:34 * nb] = blk[:, :, :2].reshape(rows, -1)
    return out.reshape(-1)


@pytest.mark.parametrize("dtype", [Q4K, Q6K, Q8])
def test_pack_matches_numpy_statement_and_round_trips(dtype):
    for i, (rows, cols) in enumerate(SHAPES[dtype]):
        raw = random_blocks(dtype, rows, cols, 100 * dtype + i)
        packed = backend.pack_weight(raw, dtype, (rows, cols))
        assert np.array_equal(packed, numpy_pack(raw, dtype, rows, cols)), (dtype, rows, cols)
        assert np.array_equal(backend.unpack_weight(packed, dtype, (rows, cols)), raw)


@pytest.mark.parametrize("dtype", [Q4K, Q6K, Q8])
def test_prepared_sizes(dtype):
    for rows, cols in SHAPES[dtype]:
        nb = cols // synth.BLOCK_SIZE[dtype]
        row = nb * synth.TYPE_SIZE[dtype]
        assert backend.prepared_bytes(dtype, rows, cols) == rows * (-(-row // 16) * 16)
    # Every Llama-3-8B shape keeps the GGUF byte count exactly.
    for rows, cols in [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336), (128256, 4096)]:
        raw = rows * (cols // synth.BLOCK_SIZE[dtype]) * synth.TYPE_SIZE[dtype]
        assert backend.prepared_bytes(dtype, rows, cols) == raw


def test_pack_rejects_bad_input():
    raw = random_blocks(Q4K, 2, 256, 1)
    assert backend.prepared_bytes(0, 2, 256) == 0  # F32 has no prepared layout
    with pytest.raises(backend.BackendError) as e:
        backend.pack_weight(raw, 0, (2, 256))
    assert e.value.code == 3
    with pytest.raises(backend.BackendError) as e:
        backend.pack_weight(raw[:-1], Q4K, (2, 256))
    assert e.value.code == 2
    with pytest.raises(backend.BackendError) as e:
        backend.pack_weight(raw, Q4K, (2, 300))
    assert e.value.code == 2
