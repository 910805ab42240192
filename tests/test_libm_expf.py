"""The device expf of the CPU-order mode (mdma_amd/csrc/libm_expf.h) against
the C library's expf, which the CPU backend's softmax and SiLU call
(/root/reference/src/backend/cpu.rs:50-60,447-458 through f32::exp): the
same source compiled for the host must give the C library's bits on every
one of the 2^32 f32 inputs (NaN payloads aside), and its table of 2^(i/32)
must be the nearest doubles. The GPU performs the same IEEE double
operations; tests/test_gpu_cpu_order.py checks the device results."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_libm_expf_equals_c_library_on_every_input(tmp_path):
    exe = str(tmp_path / "expf_check")
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-pthread", "-o", exe,
                    os.path.join(HERE, "libm_expf_check.cpp"), "-lm"], check=True)
    out = subprocess.run([exe], check=True, capture_output=True, text=True, timeout=600).stdout.split()
    assert out == ["mismatches", "0", "table_errors", "0"], out
