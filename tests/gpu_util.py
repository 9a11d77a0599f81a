"""Device-buffer helpers for the GPU parity tests.

Destinations are filled with the reference tests' sentinel byte 0xCD and
followed by GUARD guard bytes (reference tests/gpu_reduce_golden.rs:38-41), so
a write past the end or an element the kernel never wrote is visible. Buffers
and launches go through t4a_cuda_kernels.hipmem, the HIP runtime the kernels'
library is linked against; kernels run on the null stream, so the synchronous
copies order after them.
"""
from __future__ import annotations

import sys

import numpy as np

import t4a_cuda_kernels as t
from t4a_cuda_kernels import hipmem

SENTINEL = 0xCD
GUARD = 256

NUMPY = {
    t.DType.F32: np.float32,
    t.DType.F64: np.float64,
    t.DType.I32: np.int32,
    t.DType.I64: np.int64,
    t.DType.Bool: np.uint8,
    t.DType.C32: np.complex64,
    t.DType.C64: np.complex128,
}


def say(*msg) -> None:
    """Name the case before a GPU step, flushed, so a failing run shows it."""
    print("[gpu]", *msg, flush=True)
    sys.stdout.flush()


def stream():
    """The null stream (hipMemcpy orders after kernels on it)."""
    return None


def to_device(arr: np.ndarray, guard: int = GUARD) -> hipmem.DeviceBuffer:
    return hipmem.DeviceBuffer.from_array(arr, extra=guard, fill=SENTINEL)


def sentinel(nbytes: int, guard: int = GUARD) -> hipmem.DeviceBuffer:
    buf = hipmem.DeviceBuffer(nbytes + guard)
    buf.fill(SENTINEL)
    return buf


def to_host(buf: hipmem.DeviceBuffer, nbytes: int, what: str = "destination") -> np.ndarray:
    hipmem.synchronize()
    host = buf.download()
    assert (host[nbytes:] == SENTINEL).all(), f"{what}: a write landed past the end"
    return host[:nbytes]


def random_elements(dtype: t.DType, count: int, rng: np.random.Generator) -> np.ndarray:
    """Values of the element type (every byte pattern matters for movement;
    reductions get finite values)."""
    if dtype in (t.DType.F32, t.DType.F64):
        return rng.uniform(-1.0, 1.0, count).astype(NUMPY[dtype])
    if dtype in (t.DType.C32, t.DType.C64):
        re = rng.uniform(-1.0, 1.0, count)
        im = rng.uniform(-1.0, 1.0, count)
        return (re + 1j * im).astype(NUMPY[dtype])
    if dtype == t.DType.Bool:
        return rng.integers(0, 2, count).astype(np.uint8)
    if dtype == t.DType.I32:
        return rng.integers(-(2**31), 2**31, count, dtype=np.int64).astype(np.int32)
    return rng.integers(-(2**62), 2**62, count, dtype=np.int64)
