"""The movement planner's tile shapes (move_plan in csrc/geometry.h), CPU only:
compiled with g++ from the same header the kernels use and run over random
permuted, reversed, broadcast and padded views of ranks 1-6 and every payload
width. A tile must fit the LDS arena and the offset tables the kernel sizes
for it, the register stage must hold it, and its runs and batch dims must
cover exactly the view's elements."""
import subprocess
from pathlib import Path

REPO = Path(__file__).resolve().parent.parent

PROGRAM = r"""
#include <cstdio>
#include <random>
#include <algorithm>
#include "geometry.h"
using namespace t4a;
int main() {
  std::mt19937_64 rng(7);
  int tiled = 0, checked = 0;
  for (int it = 0; it < 40000; ++it) {
    const int rank = 1 + rng() % 6;
    const int esizes[4] = {1, 4, 8, 16};
    const int es = esizes[rng() % 4];
    long long ext[8];
    for (int k = 0; k < rank; ++k) ext[k] = 1 + rng() % 40;
    int perm[8];
    for (int k = 0; k < rank; ++k) perm[k] = k;
    std::shuffle(perm, perm + rank, rng);
    t4a_cuda_layout src{};
    src.rank = rank;
    long long stride = 1 + (rng() % 3 == 0 ? rng() % 3 : 0);  // sometimes padded
    long long offset = 0;
    for (int i = 0; i < rank; ++i) {
      const int k = perm[i];
      src.extents[k] = ext[k];
      src.strides[k] = stride;
      stride *= ext[k] + (rng() % 4 == 0 ? 1 : 0);
    }
    for (int k = 0; k < rank; ++k) {
      if (rng() % 5 == 0) { offset += (ext[k] - 1) * src.strides[k]; src.strides[k] = -src.strides[k]; }
      else if (rng() % 9 == 0) src.strides[k] = 0;
    }
    src.offset = offset;
    long long len = 1;
    for (int k = 0; k < rank; ++k) len *= ext[k];
    MovePlan p;
    move_plan(&p, src, nullptr, 0, len, es);
    ++checked;
    if (p.mode != kMoveTiled) continue;
    ++tiled;
    const long long budget = es >= 16 ? 1024 : es >= 8 ? 2048 : 4096;
    // register stage of move_tiles
    const long long max_elems = es >= 16 ? 32 * 32 : es >= 8 ? 64 * 32 : 64 * 64;
    bool ok = p.la >= 1 && p.lb >= 1 && p.la <= kMoveRunMax && p.lb <= kMoveRunMax &&
              p.la * p.lb <= budget && p.la * p.lb <= max_elems &&
              p.la * (p.lb + 1) * es <= kMoveTileBytes;
    // runs times tiles times batch extents cover the elements exactly once
    long long a_full = p.a_inner * p.ext[p.a_dims[p.na - 1]];
    long long b_full = p.b_inner * p.ext[p.b_dims[p.nb - 1]];
    long long covered = a_full * b_full;
    for (int i = 0; i < p.nbatch; ++i) covered *= p.ext[p.batch_dims[i]];
    ok = ok && covered == len && p.la == p.a_inner * p.a_tile && p.lb == p.b_inner * p.b_tile;
    if (!ok) {
      std::printf("bad plan it=%d es=%d la=%lld lb=%lld covered=%lld len=%lld\n", it, es, p.la,
                  p.lb, covered, len);
      return 1;
    }
  }
  std::printf("%d %d\n", checked, tiled);
  return 0;
}
"""


def test_move_plan_tiles_fit_lds_tables_and_registers(tmp_path):
    src = tmp_path / "move_plan.cc"
    src.write_text(PROGRAM)
    exe = tmp_path / "move_plan"
    build = subprocess.run(["g++", "-O2", "-std=c++17", f"-I{REPO / 'include'}",
                            f"-I{REPO / 't4a-cuda-kernels_amd' / 'csrc'}", str(src), "-o",
                            str(exe)], capture_output=True, text=True)
    assert build.returncode == 0, build.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stdout + run.stderr
    checked, tiled = map(int, run.stdout.split())
    assert checked == 40000 and tiled > 5000
