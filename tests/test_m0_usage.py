"""The LDS-DMA helpers (lds_dma16 / lds_dma4, mdma_amd/csrc/kernels.h) set M0
inside inline assembly. The compiler reserves M0 and does not honour it in a
clobber list, so the kernels that use the helpers must contain no other M0
use: compiled for gfx950 exactly as the Makefile builds them, every line of
their assembly that names M0 must be an `s_mov_b32 m0, ...` immediately
followed by a `global_load_lds_*`, and nothing else may name M0."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "mdma_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fno-gpu-flush-denormals-to-zero", "-Xclang",
         "-target-feature", "-Xclang", "-packed-fp32-ops", "-mllvm", "-amdgpu-mfma-vgpr-form", "--cuda-device-only",
         "-S", "-x", "hip"]


def uses_lds_dma(path):
    return "lds_dma16(" in open(path).read() or "lds_dma4(" in open(path).read()


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="needs hipcc")
def test_m0_only_set_for_lds_dma(tmp_path):
    srcs = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip") and uses_lds_dma(os.path.join(CSRC, f)))
    assert srcs, "no kernel uses the LDS-DMA helpers"
    procs = []
    for f in srcs:
        out = str(tmp_path / (f + ".s"))
        procs.append((f, out, subprocess.Popen([HIPCC, *FLAGS, "-o", out, os.path.join(CSRC, f)],
                                               stdout=subprocess.DEVNULL, stderr=subprocess.PIPE)))
    checked = 0
    for f, out, p in procs:
        _, err = p.communicate(timeout=600)
        assert p.returncode == 0, (f, err.decode()[-2000:])
        lines = [l.split(";")[0].strip() for l in open(out)]
        lines = [l for l in lines if l and not l.startswith((".", "//"))]
        for i, l in enumerate(lines):
            if not re.search(r"\bm0\b", l):
                continue
            assert l.startswith("s_mov_b32 m0,"), (f, l)
            assert i + 1 < len(lines) and lines[i + 1].startswith("global_load_lds_dword"), (f, l, lines[i + 1])
            checked += 1
    assert checked > 0
