"""ctypes binding of the CPU oracle (oracle/t4a_oracle.c) -- TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module, and only as the checker or the reported CPU baseline; the product path
(t4a-cuda-kernels_amd/) never imports it.

Arrays are numpy buffers; layouts are anything with a `.c` CLayout (the
product's `Layout`) or a CLayout itself. Build with `make -C oracle`.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_double, c_int, c_longlong, c_void_p
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "_build" / "libt4a_oracle.so"
_LIB = None


def load() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} is not built: run `make -C oracle`")
        lib = ctypes.CDLL(str(LIB_PATH))
        lib.t4a_oracle_materialize_strided.argtypes = [c_void_p, c_void_p, c_int, c_void_p,
                                                       c_longlong]
        lib.t4a_oracle_strided_to_strided.argtypes = [c_void_p, c_void_p, c_int, c_void_p,
                                                      c_void_p, c_longlong]
        lib.t4a_oracle_tiled_transpose.argtypes = [c_void_p, c_void_p, c_int, c_longlong,
                                                   c_longlong, c_longlong, c_longlong,
                                                   c_longlong]
        lib.t4a_oracle_reduce.argtypes = [c_void_p, c_void_p, c_int, c_int, c_int, c_int,
                                          c_void_p, c_void_p, c_int, c_longlong]
        lib.t4a_oracle_reduce_partials.argtypes = [c_void_p, c_void_p, c_int, c_int, c_int,
                                                   c_void_p, c_void_p, c_int, c_longlong,
                                                   c_longlong, c_longlong]
        lib.t4a_oracle_reduce_f64.argtypes = [POINTER(c_double), c_void_p, c_int, c_int,
                                              c_void_p, c_int, c_longlong]
        lib.t4a_oracle_fill_zero_view.argtypes = [c_void_p, c_int, c_void_p, c_longlong]
        lib.t4a_oracle_contiguous_to_view.argtypes = [c_void_p, c_void_p, c_int, c_void_p,
                                                      c_longlong]
        lib.t4a_oracle_broadcast_in_dim.argtypes = [c_void_p, c_void_p, c_int, c_void_p,
                                                    c_void_p, POINTER(c_longlong), c_int,
                                                    c_longlong]
        lib.t4a_oracle_concatenate_copy.argtypes = [c_void_p, c_void_p, c_int, c_void_p,
                                                    c_void_p, c_int, c_longlong, c_longlong]
        lib.t4a_oracle_fnv1a64.argtypes = [c_void_p, ctypes.c_ulonglong]
        lib.t4a_oracle_fnv1a64.restype = ctypes.c_ulonglong
        lib.t4a_oracle_dtype_size.argtypes = [c_int]
        lib.t4a_oracle_dtype_size.restype = c_int
        lib.t4a_oracle_set_threads.argtypes = [c_int]
        lib.t4a_oracle_set_threads.restype = None
        lib.t4a_oracle_max_threads.argtypes = []
        lib.t4a_oracle_max_threads.restype = c_int
        for name in ("t4a_oracle_fill_zero_view", "t4a_oracle_contiguous_to_view",
                     "t4a_oracle_broadcast_in_dim", "t4a_oracle_concatenate_copy"):
            getattr(lib, name).restype = None
        for name in ("t4a_oracle_materialize_strided", "t4a_oracle_strided_to_strided",
                     "t4a_oracle_tiled_transpose", "t4a_oracle_reduce",
                     "t4a_oracle_reduce_partials", "t4a_oracle_reduce_f64"):
            getattr(lib, name).restype = None
        _LIB = lib
    return _LIB


def _p(a: np.ndarray) -> c_void_p:
    assert a.flags["C_CONTIGUOUS"]
    return c_void_p(a.ctypes.data)


def _l(layout) -> c_void_p:
    c = layout.c if hasattr(layout, "c") else layout
    return ctypes.cast(ctypes.pointer(c), c_void_p)


def materialize_strided(dst: np.ndarray, src: np.ndarray, dtype: int, src_layout,
                        length: int) -> None:
    load().t4a_oracle_materialize_strided(_p(dst), _p(src), int(dtype), _l(src_layout), length)


def strided_to_strided(dst: np.ndarray, src: np.ndarray, dtype: int, src_layout, dst_layout,
                       length: int) -> None:
    load().t4a_oracle_strided_to_strided(_p(dst), _p(src), int(dtype), _l(src_layout),
                                         _l(dst_layout), length)


def fill_zero_view(out: np.ndarray, dtype: int, layout, length: int) -> None:
    load().t4a_oracle_fill_zero_view(_p(out), int(dtype), _l(layout), length)


def contiguous_to_view(dst: np.ndarray, src: np.ndarray, dtype: int, dst_layout,
                       length: int) -> None:
    load().t4a_oracle_contiguous_to_view(_p(dst), _p(src), int(dtype), _l(dst_layout), length)


def broadcast_in_dim(out: np.ndarray, inp: np.ndarray, dtype: int, out_layout, in_layout,
                     dims, out_len: int) -> None:
    d = (c_longlong * max(len(dims), 1))(*dims)
    load().t4a_oracle_broadcast_in_dim(_p(out), _p(inp), int(dtype), _l(out_layout),
                                       _l(in_layout), d, len(dims), out_len)


def concatenate_copy(out: np.ndarray, inp: np.ndarray, dtype: int, out_layout, in_layout,
                     axis: int, axis_offset: int, in_len: int) -> None:
    load().t4a_oracle_concatenate_copy(_p(out), _p(inp), int(dtype), _l(out_layout),
                                       _l(in_layout), axis, axis_offset, in_len)


def tiled_transpose(dst: np.ndarray, src: np.ndarray, dtype: int, src_offset: int,
                    batch_stride: int, dst_fast_extent: int, src_fast_extent: int,
                    batches: int) -> None:
    load().t4a_oracle_tiled_transpose(_p(dst), _p(src), int(dtype), src_offset, batch_stride,
                                      dst_fast_extent, src_fast_extent, batches)


def reduce(out: np.ndarray, inp: np.ndarray, dtype: int, op: int, strategy: int,
           block_width: int, out_layout, in_layout, axis: int, output_len: int) -> None:
    load().t4a_oracle_reduce(_p(out), _p(inp), int(dtype), int(op), int(strategy), block_width,
                             _l(out_layout), _l(in_layout), axis, output_len)


def reduce_partials(partials: np.ndarray, inp: np.ndarray, dtype: int, op: int,
                    plane_width: int, partials_layout, in_layout, axis: int, output_len: int,
                    splits: int, chunk_len: int) -> None:
    load().t4a_oracle_reduce_partials(_p(partials), _p(inp), int(dtype), int(op), plane_width,
                                      _l(partials_layout), _l(in_layout), axis, output_len,
                                      splits, chunk_len)


def reduce_f64(inp: np.ndarray, dtype: int, op: int, in_layout, axis: int,
               output_len: int, complex_out: bool) -> np.ndarray:
    out = np.zeros(output_len * (2 if complex_out else 1), dtype=np.float64)
    load().t4a_oracle_reduce_f64(out.ctypes.data_as(POINTER(c_double)), _p(inp), int(dtype),
                                 int(op), _l(in_layout), axis, output_len)
    return out


def set_threads(n: int) -> None:
    """OpenMP threads for the loops over independent outputs (default 1);
    every output is still folded serially on one thread."""
    load().t4a_oracle_set_threads(int(n))


def max_threads() -> int:
    return int(load().t4a_oracle_max_threads())


def fnv1a64(a: np.ndarray) -> int:
    a = np.ascontiguousarray(a)
    return load().t4a_oracle_fnv1a64(c_void_p(a.ctypes.data), a.nbytes)
