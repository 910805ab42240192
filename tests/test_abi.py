"""CPU-only checks of the drop-in boundary: the C-ABI library loads, exports
every entry point include/mdma_gfx950.h declares, and the Python mirror binds
them; plus the host-side tooling (GGUF writer/reader, synthetic generators)."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from mdma_amd import backend, gguf, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mdma_gfx950.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(mdma_gfx950_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(backend.LIB_PATH)
    names = declared_symbols()
    assert len(names) >= 35
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", backend.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (mdma_gfx950_\w+)", out))
    assert set(names) <= exported


def test_python_mirror_binds_every_declared_symbol():
    from mdma_amd import model

    assert set(backend.exported_symbols()) | set(model.exported_symbols()) == set(declared_symbols())
    model._lib()  # argtypes/restypes resolve against the library


def test_library_is_gfx950_only(tmp_path):
    fb = str(tmp_path / "fatbin")
    bundler = "/opt/rocm/llvm/bin/clang-offload-bundler"
    if subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", backend.LIB_PATH, fb]).returncode \
            or not os.path.exists(bundler):
        pytest.skip("objcopy / clang-offload-bundler unavailable")
    out = subprocess.run([bundler, "--type=o", f"--input={fb}", "--list"], capture_output=True, text=True)
    targets = set(re.findall(r"amdgcn-amd-amdhsa--(gfx\w+)", out.stdout))
    assert targets == {"gfx950"}, targets


def test_create_without_gpu_reports_backend_error():
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is present")
    with pytest.raises(backend.BackendError) as e:
        backend.Gfx950Backend(0)
    assert e.value.code == 10


def test_last_error_is_thread_local_string():
    lib = backend.lib()
    assert isinstance(lib.mdma_gfx950_last_error(), bytes)


def test_gguf_roundtrip(tmp_path):
    p = str(tmp_path / "m.gguf")
    w = synth.weight(synth.GGML_Q4_K, 3, 512, 1)
    n = synth.normal_f32(7, 2)
    gguf.write(p, {"general.architecture": "llama", "llama.block_count": 2, "llama.rope.freq_base": 10000.0},
               [("a.weight", synth.GGML_Q4_K, (3, 512), w), ("n.weight", synth.GGML_F32, (7,), n)])
    r = gguf.Reader(p)
    assert r.metadata["general.architecture"] == "llama" and r.metadata["llama.block_count"] == 2
    assert r.tensors["a.weight"].shape == (3, 512) and r.tensors["a.weight"].dtype == synth.GGML_Q4_K
    assert r.tensors["a.weight"].offset % 32 == 0
    assert np.array_equal(r.bytes_of("a.weight"), w)
    assert np.array_equal(r.bytes_of("n.weight").view(np.float32), n)
    # src/gguf/tests.rs:147-160: Q4_K [2, 256] is 288 bytes.
    assert gguf.tensor_bytes(synth.GGML_Q4_K, (2, 256)) == 288


def test_synthetic_distributions():
    raw = synth.q4k_blocks(4096, 1).reshape(-1, 144)
    d = raw[:, :2].copy().view(np.float16).astype(np.float32)
    assert d.min() >= 0 and 5e-4 < d.mean() < 1.2e-3  # |N(0,1)|*1e-3 has mean 0.8e-3
    s = synth.Stream(1)
    v = s.ints(100000, 0, 63)
    assert v.min() == 0 and v.max() == 63
    x = synth.normal_f32(200000, 3)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1) < 0.01
    q8 = synth.q8_0_blocks(1000, 2).reshape(-1, 34)[:, 2:].view(np.int8)
    assert q8.min() == -127 and q8.max() == 127
    q6 = synth.q6k_blocks(1000, 2).reshape(-1, 210)[:, 192:208].view(np.int8)
    assert q6.min() == -64 and q6.max() == 63
    # Same seed, same bytes.
    assert np.array_equal(synth.q4k_blocks(10, 7), synth.q4k_blocks(10, 7))
