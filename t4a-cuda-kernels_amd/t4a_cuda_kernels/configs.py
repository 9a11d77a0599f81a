"""The benchmark configurations' seeded inputs.

Every configuration's values come from one generator, the reference's
SplitMix64 (reference tests/gpu_reduce_golden.rs:49-64), seeded with the
configuration's seed:

- `draws(seed, n)`: the first n outputs of SplitMix64(seed) (the state advances
  by 0x9E3779B97F4A7C15 before each output, then is mixed);
- `uniform`: the reference's `unit()`, (next() >> 11) * 2^-52 - 1, uniform in
  [-1, 1) on a 2^-52 grid (exact in f64), rounded to the element type;
- `normal`: Box-Muller on two consecutive draws: u1 = (1 - unit()) / 2 in
  (0, 1], u2 = (unit() + 1) / 2 in [0, 1), z = sqrt(-2 ln u1) cos(2 pi u2),
  one value per pair of draws, computed in f64 and rounded to the element type;
  a complex value takes two consecutive normals (real part first);
- `integers(lo, hi)`: next() % (hi - lo + 1) + lo; `choice(values)`:
  values[next() % len(values)].

Values are produced in flat (memory) order of the configuration's compact
tensor. Large arrays are generated in chunks, so memory stays a small
multiple of the output.
"""
from __future__ import annotations

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 22


def draws(seed: int, n: int, start: int = 0) -> np.ndarray:
    """Outputs start .. start + n - 1 of SplitMix64(seed) (output k is the mix
    of seed + (k + 1) * gamma)."""
    k = np.arange(start + 1, start + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + k * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def unit(d: np.ndarray) -> np.ndarray:
    """The reference's unit(): uniform in [-1, 1) on a 2^-52 grid, exact in f64."""
    return (d >> np.uint64(11)).astype(np.float64) * (1.0 / float(1 << 52)) - 1.0


def _chunked(n: int, out: np.ndarray, per_value: int, fill) -> np.ndarray:
    """Fill `out` (n values) chunk by chunk; value i uses draws
    [i * per_value, (i + 1) * per_value)."""
    for a in range(0, n, _CHUNK):
        b = min(n, a + _CHUNK)
        fill(out[a:b], a * per_value, (b - a) * per_value)
    return out


def uniform(seed: int, n: int, dtype=np.float32) -> np.ndarray:
    """n values of unit(), rounded to `dtype` (f32 or f64)."""
    out = np.empty(n, dtype=dtype)
    return _chunked(n, out, 1, lambda o, s, c: np.copyto(o, unit(draws(seed, c, s)),
                                                         casting="unsafe"))


def _box_muller(d: np.ndarray) -> np.ndarray:
    u = unit(d)
    u1 = (1.0 - u[0::2]) * 0.5  # (0, 1]
    u2 = (u[1::2] + 1.0) * 0.5  # [0, 1)
    return np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)


def normal(seed: int, n: int, dtype=np.float32) -> np.ndarray:
    """n N(0,1) values by Box-Muller (two draws each), rounded to `dtype`. A
    complex dtype takes 2n normals, real and imaginary parts interleaved."""
    dtype = np.dtype(dtype)
    if dtype.kind == "c":
        part = np.float32 if dtype == np.complex64 else np.float64
        return normal(seed, 2 * n, part).view(dtype)
    out = np.empty(n, dtype=dtype)
    return _chunked(n, out, 2, lambda o, s, c: np.copyto(o, _box_muller(draws(seed, c, s)),
                                                         casting="unsafe"))


def integers(seed: int, n: int, lo: int, hi: int, dtype=np.int64) -> np.ndarray:
    """n integers next() % (hi - lo + 1) + lo, inclusive of both ends."""
    span = np.uint64(hi - lo + 1)
    out = np.empty(n, dtype=dtype)

    def fill(o, s, c):
        np.copyto(o, (draws(seed, c, s) % span).astype(np.int64) + lo, casting="unsafe")

    return _chunked(n, out, 1, fill)


def choice(seed: int, n: int, values, dtype=np.int32) -> np.ndarray:
    """n picks values[next() % len(values)]."""
    table = np.asarray(values, dtype=dtype)
    out = np.empty(n, dtype=dtype)

    def fill(o, s, c):
        o[:] = table[(draws(seed, c, s) % np.uint64(len(table))).astype(np.intp)]

    return _chunked(n, out, 1, fill)


# ---- the benchmark configurations' inputs (C-order shapes) ----

def c1_input(m: int = 1024) -> np.ndarray:
    """C1: f32 C-[m, m] uniform[-1, 1), seed 0."""
    return uniform(0, m * m, np.float32)


def c2_inputs() -> tuple[np.ndarray, np.ndarray]:
    """C2: f32 C-[8192, 8192] uniform[-1, 1) seed 1, and i64 integers in
    [-1000, 1000] from the same seed."""
    n = 8192 * 8192
    return uniform(1, n, np.float32), integers(1, n, -1000, 1000, np.int64)


def c3_input(dtype) -> np.ndarray:
    """C3: f64 (or complex64 of two f32 parts) C-[64, 128, 64, 32] N(0,1), seed 2."""
    return normal(2, 64 * 128 * 64 * 32, dtype)


def c4_inputs() -> tuple[np.ndarray, np.ndarray]:
    """C4: f32 C-[32, 1048576, 4] N(0,1) seed 3, and i32 values in {-1, 1, 2}
    from the same seed."""
    n = 32 * 1048576 * 4
    return normal(3, n, np.float32), choice(3, n, [-1, 1, 2], np.int32)


def c5_input() -> np.ndarray:
    """C5: complex128 C-[16]^6, parts N(0,1), seed 4."""
    return normal(4, 16 ** 6, np.complex128)
