import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def backend():
    from mdma_amd.backend import Gfx950Backend

    b = Gfx950Backend(0)
    yield b
    b.close()


def f32_exact(W: np.ndarray, x: np.ndarray) -> np.ndarray:
    """f64 dot products of the oracle's dequantized rows with x: [T, n_out]."""
    return x.reshape(-1, W.shape[1]).astype(np.float64) @ W.astype(np.float64).T


PARITY_LOG = []


U32 = 2.0 ** -24  # unit roundoff of f32


def abs_dot(W, x):
    """sum_k |x[t, k]| |W[r, k]| in f64, [T, rows]: the scale of a dot
    product's partial sums, which sets its rounding error (the CPU's
    sequential f32 sum is guaranteed only within K * u of it)."""
    k = W.shape[1]
    return np.abs(np.asarray(x, np.float64).reshape(-1, k)) @ np.abs(np.asarray(W, np.float64)).T


def assert_parity(got, cpu, exact, rtol, atol=1e-6, what="", correctly_rounded=False, abs_sum=None, k_u=2.0):
    """Per-element parity against the CPU oracle.

    The oracle sums each dot product sequentially in f32 (reference
    src/backend/cpu.rs:46-48) over weights it dequantized to f32, so it
    carries its own error |cpu - exact| of up to ~1e-4 at K=14336; no parallel
    reduction order can reproduce it bit for bit. An element passes when the
    GPU is within the stated tolerance of the oracle after allowing for that
    error:
        |gpu - cpu| <= atol + rtol*|cpu| + |cpu - exact|
    where exact is the f64 dot product of the exact block values
    (tests/npq.py: d*sc*q - dmin*m with the f32 products d*sc and dmin*m the
    CPU forms exactly; only Q4_K's final subtraction is rounded by the CPU)
    with the same x -- the quantity the f32-mode kernels compute before their
    one rounding. Non-finite values fail. The plain pass rate (no slack term)
    is returned and logged for the session summary.

    correctly_rounded: the f32-mode GEMVs form each dot product exactly (f64
    products and sums) and round once, so every element must be at least as
    close to exact as the CPU's sequential f32 sum, which no rounding of the
    exact value can lose to: |gpu - exact| <= |cpu - exact| everywhere.

    abs_sum (per element sum_k |x_k w_k|, see abs_dot): for kernels that sum
    in f32 at the scale of the partial sums (the prefill GEMMs), the slack
    gains k_u * u * abs_sum, k_u roundings at that scale. Without it an
    output that cancels to near zero would have to match to about 1e-6
    while its terms are ~10: tighter than one ulp of the partial sums, a
    bound the CPU's own sum (within K * u * abs_sum) does not meet either.
    """
    got = np.asarray(got, dtype=np.float64).reshape(-1)
    cpu = np.asarray(cpu, dtype=np.float64).reshape(-1)
    exact = np.asarray(exact, dtype=np.float64).reshape(-1)
    assert got.shape == cpu.shape == exact.shape
    assert np.all(np.isfinite(got)), f"{what}: non-finite GPU output"
    bound = atol + rtol * np.abs(cpu) + np.abs(cpu - exact)
    if abs_sum is not None:
        bound = bound + k_u * U32 * np.asarray(abs_sum, dtype=np.float64).reshape(-1)
    err = np.abs(got - cpu)
    bad = np.nonzero(~(err <= bound))[0]
    assert bad.size == 0, (f"{what}: {bad.size}/{got.size} elements outside tolerance; first {bad[:5]}: "
                           f"gpu {got[bad[:5]]} cpu {cpu[bad[:5]]} exact {exact[bad[:5]]}")
    plain = float(np.mean(err <= atol + rtol * np.abs(cpu)))
    closer = np.abs(got - exact) <= np.abs(cpu - exact)
    gpu_closer = float(np.mean(closer))
    if correctly_rounded:
        far = np.nonzero(~closer)[0]
        assert far.size == 0, (f"{what}: {far.size} elements farther from exact than the CPU; first {far[:5]}: "
                               f"gpu {got[far[:5]]} cpu {cpu[far[:5]]} exact {exact[far[:5]]}")
    PARITY_LOG.append((what, got.size, rtol, atol, plain, gpu_closer))
    return plain


def pytest_terminal_summary(terminalreporter):
    if not PARITY_LOG:
        return
    tr = terminalreporter
    tr.section("parity: plain pass rates (|gpu-cpu| <= atol + rtol|cpu|, no slack) and GPU-closer-to-exact rates")
    for what, n, rtol, atol, plain, closer in PARITY_LOG:
        tr.write_line(f"{what or '-'}: n={n} rtol={rtol:g} atol={atol:g} plain={plain:.5f} gpu_closer={closer:.4f}")
    worst = min(p for _, _, _, _, p, _ in PARITY_LOG)
    tr.write_line(f"parity checks: {len(PARITY_LOG)}, lowest plain pass rate {worst:.5f}")
