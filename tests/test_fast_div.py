"""The kernels' multiply-shift division (FastDiv in csrc/geometry.h), CPU only:
compiled with g++ from the same header and checked against exact division for
every divisor up to 5000, random ones up to 2^31 - 1 and divisors from 2^31 - 2
to 2^32 - 1, at dividends that cover each divisor's multiples and their
neighbours, small values and values just below the 2^31 bound."""
import subprocess
from pathlib import Path

REPO = Path(__file__).resolve().parent.parent

PROGRAM = r"""
#include <cstdio>
#include <cstdint>
#include <random>
#include "geometry.h"
int main() {
  std::mt19937_64 rng(12345);
  long long checked = 0;
  auto check = [&](unsigned d, unsigned x) {
    const t4a::FastDiv f = t4a::fast_div(d);
    if (t4a::div_by(x, f) != x / d) { std::printf("d=%u x=%u got %u\n", d, x, t4a::div_by(x, f)); return false; }
    ++checked;
    return true;
  };
  const unsigned top = 0x7fffffffu;
  for (unsigned d = 1; d <= 5000; ++d) {
    for (unsigned x = 0; x < 3 * d + 3; ++x) if (!check(d, x)) return 1;
    for (unsigned k = 0; k < 64; ++k) {
      const unsigned long long q = rng() % (top / d + 1);
      for (long long e = -1; e <= 1; ++e) {
        const long long x = (long long)(q * d) + e;
        if (x >= 0 && x <= top && !check(d, (unsigned)x)) return 1;
      }
    }
    for (unsigned x = top - 64; x < top; ++x) if (!check(d, x)) return 1;
    if (!check(d, top)) return 1;
  }
  // Divisors from 2^31 up: every dividend below 2^31 has quotient 0 (2^31
  // itself takes the general form, larger ones the special one).
  for (unsigned long long d = 0x7ffffffeull; d <= 0xffffffffull; d += (d < 0x80000010ull ? 1 : 0x0fffffffull)) {
    for (unsigned x : {0u, 1u, 2u, 12345u, top - 1, top}) if (!check((unsigned)d, x)) return 1;
    for (int k = 0; k < 64; ++k) if (!check((unsigned)d, (unsigned)(rng() % ((unsigned long long)top + 1)))) return 1;
  }
  if (!check(0xffffffffu, top) || !check(0x80000001u, top)) return 1;
  for (int i = 0; i < 200000; ++i) {
    const unsigned d = 1 + (unsigned)(rng() % top);
    const unsigned x = (unsigned)(rng() % ((unsigned long long)top + 1));
    if (!check(d, x) || !check(d, d) || !check(d, d - 1) || !check(d, top)) return 1;
  }
  std::printf("%lld\n", checked);
  return 0;
}
"""


def test_fast_div_matches_exact_division(tmp_path):
    src = tmp_path / "fast_div.cc"
    src.write_text(PROGRAM)
    exe = tmp_path / "fast_div"
    build = subprocess.run(["g++", "-O2", "-std=c++17", f"-I{REPO / 'include'}",
                            f"-I{REPO / 't4a-cuda-kernels_amd' / 'csrc'}", str(src), "-o",
                            str(exe)], capture_output=True, text=True)
    assert build.returncode == 0, build.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stdout + run.stderr
    assert int(run.stdout) > 1_000_000
