"""The GEMMs' XCD-aware tile order (grid_tile, mdma_amd/csrc/kernels.h): the
map from a workgroup's (blockIdx.x, blockIdx.y) to its output tile must be a
bijection of the grid onto itself, or tiles would be computed twice and
others never. The function's own source is compiled for the host (its
device qualifiers and the block and grid indices stubbed) and checked over
every grid of up to 64 x 24 tiles and several group sizes; grids whose tile
count is not a multiple of 8, or of one token tile, keep the dispatch order,
and each XCD (dispatch index mod 8) receives a contiguous run of the order,
so its tiles span few token tiles."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KERNELS_H = os.path.join(ROOT, "mdma_amd", "csrc", "kernels.h")

HARNESS = r"""
#include <cstdint>
#include <cstdio>
#include <vector>
#include <algorithm>
using std::min;
#define __device__
#define __forceinline__ inline
struct Idx { uint32_t x, y, z; };
static Idx blockIdx, gridDim;
@GRID_TILE@
int main() {
  long bad = 0, grids = 0;
  for (uint32_t gt : {0u, 1u, 2u, 4u, 16u})
    for (uint32_t nx = 1; nx <= 64; nx++)
      for (uint32_t ny = 1; ny <= 24; ny++) {
        gridDim = Idx{nx, ny, 1};
        const uint32_t n = nx * ny;
        std::vector<int> seen(n, 0);
        std::vector<uint32_t> ymin(8, ~0u), ymax(8, 0);
        for (uint32_t y = 0; y < ny; y++)
          for (uint32_t x = 0; x < nx; x++) {
            blockIdx = Idx{x, y, 0};
            const GridTile t = grid_tile(gt);
            if (t.x >= nx || t.y >= ny) { bad++; continue; }
            seen[t.y * nx + t.x]++;
            const bool keep = gt == 0 || ny < 2 || n % 8;
            if (keep && (t.x != x || t.y != y)) bad++;
            const uint32_t j = (y * nx + x) % 8;
            ymin[j] = min(ymin[j], t.y), ymax[j] = std::max(ymax[j], t.y);
          }
        for (int s : seen) bad += s != 1;
        // Reordered grids: an XCD's run of the order covers at most two groups of gt token tiles.
        if (gt && ny >= 2 && n % 8 == 0)
          for (int j = 0; j < 8; j++)
            if (ymin[j] != ~0u && ymax[j] - ymin[j] + 1 > 2 * gt && ymax[j] - ymin[j] + 1 > (ny + 7) / 8 + 2 * gt) bad++;
        grids++;
      }
  printf("%ld %ld\n", grids, bad);
  return bad != 0;
}
"""


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_grid_tile_is_a_bijection(tmp_path):
    src = open(KERNELS_H).read()
    m = re.search(r"struct GridTile \{.*?\n\};\n.*?__device__ __forceinline__ GridTile grid_tile\(uint32_t gt\) \{.*?\n\}\n",
                  src, re.S)
    assert m, "grid_tile not found in kernels.h"
    cpp = tmp_path / "tile_order.cpp"
    cpp.write_text(HARNESS.replace("@GRID_TILE@", m.group(0)))
    exe = str(tmp_path / "tile_order")
    subprocess.run(["g++", "-O2", "-std=c++17", "-o", exe, str(cpp)], check=True, capture_output=True, timeout=300)
    out = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    grids, bad = map(int, out.stdout.split())
    assert grids == 5 * 64 * 24 and bad == 0 and out.returncode == 0, out.stdout
