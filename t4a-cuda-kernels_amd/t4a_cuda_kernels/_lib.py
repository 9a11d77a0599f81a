"""ctypes binding of libt4a_hip.so (the C ABI declared in include/t4a/*.h).

The structures mirror include/t4a/abi.h and include/t4a/t4a.h field for field;
their sizes are checked against the C header's static assertions at load time.
"""
from __future__ import annotations

import ctypes
from ctypes import c_int, c_longlong, c_uint, c_void_p, c_char_p, POINTER
from pathlib import Path

MAX_RANK = 8
LIB_PATH = Path(__file__).with_name("libt4a_hip.so")


class CLayout(ctypes.Structure):
    """t4a_cuda_layout: 144 bytes (reference cuda/include/t4a/abi.cuh:47-57)."""

    _fields_ = [
        ("rank", c_int),
        ("reserved", c_int),
        ("offset", c_longlong),
        ("extents", c_longlong * MAX_RANK),
        ("strides", c_longlong * MAX_RANK),
    ]


class CLayoutAny(ctypes.Structure):
    """t4a_cuda_layout_any: 32 bytes, the arrays by pointer (reference
    cuda/include/t4a/abi.cuh:109-121): host memory for the planners, device
    memory for the launchers and kernels."""

    _fields_ = [
        ("rank", c_int),
        ("reserved", c_int),
        ("offset", c_longlong),
        ("extents", c_void_p),
        ("strides", c_void_p),
    ]


class CAxisValues(ctypes.Structure):
    """t4a_cuda_axis_values: 72 bytes (reference abi.cuh:74-79)."""

    _fields_ = [("rank", c_int), ("reserved", c_int), ("values", c_longlong * MAX_RANK)]


class CAxisValuesAny(ctypes.Structure):
    """t4a_cuda_axis_values_any: 16 bytes, the values by pointer (reference
    abi.cuh:122-126)."""

    _fields_ = [("rank", c_int), ("reserved", c_int), ("values", c_void_p)]


class CTransposeConfig(ctypes.Structure):
    """t4a_cuda_transpose_config: 16 bytes (reference abi.cuh:239-245)."""

    _fields_ = [
        ("tile", c_int),
        ("block_rows", c_int),
        ("padding", c_int),
        ("vector_width", c_int),
    ]


class CLaunch(ctypes.Structure):
    _fields_ = [
        ("grid", c_uint * 3),
        ("block", c_uint * 3),
        ("shared_bytes", c_uint),
        ("variant", c_int),
    ]


class CSplit(ctypes.Structure):
    _fields_ = [("splits", c_longlong), ("chunk_len", c_longlong)]


class CReductionPlan(ctypes.Structure):
    _fields_ = [
        ("kind", c_int),
        ("strategy", c_int),
        ("launch", CLaunch),
        ("split", CSplit),
        ("pass1", CLaunch),
        ("combine_strategy", c_int),
        ("combine_op", c_int),
        ("pass2", CLaunch),
    ]


assert ctypes.sizeof(CLayout) == 144 and ctypes.alignment(CLayout) == 8
assert CLayout.offset.offset == 8 and CLayout.extents.offset == 16 and CLayout.strides.offset == 80
assert ctypes.sizeof(CTransposeConfig) == 16
assert ctypes.sizeof(CLayoutAny) == 32 and CLayoutAny.extents.offset == 16
assert ctypes.sizeof(CAxisValues) == 72 and ctypes.sizeof(CAxisValuesAny) == 16

# Every C symbol declared in include/t4a/t4a.h, with its ctypes signature.
SIGNATURES = {
    "t4a_abi_revision": (c_int, []),
    "t4a_status_name": (c_char_p, [c_int]),
    "t4a_code_object_count": (c_int, []),
    "t4a_code_object_name": (c_char_p, [c_int]),
    "t4a_code_object_file": (c_char_p, [c_int]),
    "t4a_code_object_target": (c_char_p, []),
    "t4a_code_object_entry_count": (c_int, [c_int]),
    "t4a_code_object_entry": (c_char_p, [c_int, c_int]),
    "t4a_code_object_of": (c_int, [c_char_p]),
    "t4a_code_object_path": (c_int, [c_int, c_char_p, ctypes.c_ulong]),
    "t4a_dtype_size": (c_int, [c_int]),
    "t4a_layout_new": (c_int, [POINTER(CLayout), c_int, POINTER(c_longlong),
                               POINTER(c_longlong), c_longlong]),
    "t4a_layout_compact": (c_int, [POINTER(CLayout), c_int, POINTER(c_longlong)]),
    "t4a_layout_element_count": (c_int, [POINTER(CLayout), POINTER(c_longlong)]),
    "t4a_plan_copy_exact": (c_int, [c_int, c_longlong, POINTER(CLaunch)]),
    "t4a_plan_materialize_strided": (c_int, [c_int, POINTER(CLayout), c_longlong,
                                             POINTER(CLaunch)]),
    "t4a_plan_strided_to_strided": (c_int, [c_int, POINTER(CLayout), c_longlong,
                                            POINTER(CLayout), c_longlong, POINTER(CLaunch)]),
    "t4a_plan_move_route": (c_int, [c_int, POINTER(CLayout), POINTER(CLayout),
                                    POINTER(c_int)]),
    "t4a_transpose_config_new": (c_int, [c_int, c_int, c_int, c_int,
                                         POINTER(CTransposeConfig)]),
    "t4a_transpose_config_default": (CTransposeConfig, []),
    "t4a_plan_tiled_transpose": (c_int, [c_int, CTransposeConfig, c_longlong, c_longlong,
                                         c_longlong, c_longlong, c_longlong, c_longlong,
                                         c_longlong, POINTER(CLaunch)]),
    "t4a_split_policy": (c_int, [c_longlong, c_uint, POINTER(c_int), POINTER(CSplit)]),
    "t4a_plan_reduce": (c_int, [c_int, c_int, c_int, POINTER(CLayout), c_longlong,
                                POINTER(CLayout), c_longlong, c_uint, c_uint,
                                POINTER(CLaunch)]),
    "t4a_plan_reduce_partials": (c_int, [c_int, c_int, POINTER(CLayout), c_longlong,
                                         POINTER(CLayout), c_longlong, c_uint, CSplit, c_uint,
                                         POINTER(CLaunch)]),
    "t4a_plan_reduction": (c_int, [c_int, c_int, POINTER(CLayout), c_longlong,
                                   POINTER(CLayout), c_longlong, c_uint, c_uint,
                                   POINTER(CReductionPlan)]),
    "t4a_reduction_partials_layout": (c_int, [POINTER(CLayout), c_uint, c_longlong,
                                              POINTER(CLayout)]),
    "t4a_hip_last_error": (c_int, []),
    "t4a_hip_tiled_transpose": (c_int, [c_void_p, c_void_p, c_int, c_longlong, c_longlong,
                                        c_longlong, c_longlong, CTransposeConfig,
                                        POINTER(CLaunch), c_void_p]),
    "t4a_hip_copy_exact": (c_int, [c_void_p, c_void_p, c_int, c_longlong, POINTER(CLaunch),
                                   c_void_p]),
    "t4a_hip_materialize_strided": (c_int, [c_void_p, c_void_p, c_int, POINTER(CLayout),
                                            c_longlong, POINTER(CLaunch), c_void_p]),
    "t4a_hip_strided_to_strided": (c_int, [c_void_p, c_void_p, c_int, POINTER(CLayout),
                                           POINTER(CLayout), c_longlong, POINTER(CLaunch),
                                           c_void_p]),
    "t4a_hip_reduce": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, POINTER(CLayout),
                               POINTER(CLayout), c_int, c_longlong, POINTER(CLaunch),
                               c_void_p]),
    "t4a_hip_reduce_partials": (c_int, [c_void_p, c_void_p, c_int, c_int, POINTER(CLayout),
                                        POINTER(CLayout), c_int, c_longlong, c_longlong,
                                        c_longlong, POINTER(CLaunch), c_void_p]),
    "t4a_plan_materialize_strided_any": (c_int, [c_int, POINTER(CLayoutAny), c_longlong,
                                                 POINTER(CLaunch)]),
    "t4a_plan_strided_to_strided_any": (c_int, [c_int, POINTER(CLayoutAny), c_longlong,
                                                POINTER(CLayoutAny), c_longlong,
                                                POINTER(CLaunch)]),
    "t4a_plan_reduce_any": (c_int, [c_int, c_int, c_int, POINTER(CLayoutAny), c_longlong,
                                    POINTER(CLayoutAny), c_longlong, c_uint, c_uint,
                                    POINTER(CLaunch)]),
    "t4a_plan_reduce_partials_any": (c_int, [c_int, c_int, POINTER(CLayoutAny), c_longlong,
                                             POINTER(CLayoutAny), c_longlong, c_uint, CSplit,
                                             c_uint, POINTER(CLaunch)]),
    "t4a_plan_reduction_any": (c_int, [c_int, c_int, POINTER(CLayoutAny), c_longlong,
                                       POINTER(CLayoutAny), c_longlong, c_uint, c_uint,
                                       POINTER(CReductionPlan)]),
    "t4a_reduction_partials_layout_any": (c_int, [POINTER(CLayoutAny), c_uint, c_longlong,
                                                  POINTER(c_longlong), POINTER(c_longlong)]),
    "t4a_hip_materialize_strided_any": (c_int, [c_void_p, c_void_p, c_int, POINTER(CLayoutAny),
                                                c_longlong, POINTER(CLaunch), c_void_p]),
    "t4a_hip_strided_to_strided_any": (c_int, [c_void_p, c_void_p, c_int, POINTER(CLayoutAny),
                                               POINTER(CLayoutAny), c_longlong,
                                               POINTER(CLaunch), c_void_p]),
    "t4a_hip_reduce_any": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, POINTER(CLayoutAny),
                                   POINTER(CLayoutAny), c_int, c_longlong, POINTER(CLaunch),
                                   c_void_p]),
    "t4a_hip_reduce_partials_any": (c_int, [c_void_p, c_void_p, c_int, c_int,
                                            POINTER(CLayoutAny), POINTER(CLayoutAny), c_int,
                                            c_longlong, c_longlong, c_longlong,
                                            POINTER(CLaunch), c_void_p]),
    "t4a_plan_fill_zero": (c_int, [c_int, c_longlong, POINTER(CLaunch)]),
    "t4a_plan_fill_zero_view": (c_int, [c_int, POINTER(CLayout), c_longlong, POINTER(CLaunch)]),
    "t4a_plan_contiguous_to_view": (c_int, [c_int, POINTER(CLayout), c_longlong,
                                            POINTER(CLaunch)]),
    "t4a_plan_broadcast_in_dim": (c_int, [c_int, POINTER(CLayout), c_longlong, POINTER(CLayout),
                                          c_longlong, POINTER(CAxisValues), POINTER(CLaunch)]),
    "t4a_plan_concatenate_copy": (c_int, [c_int, POINTER(CLayout), c_longlong, POINTER(CLayout),
                                          c_longlong, c_uint, c_longlong, POINTER(CLaunch)]),
    "t4a_plan_fill_zero_view_any": (c_int, [c_int, POINTER(CLayoutAny), c_longlong,
                                            POINTER(CLaunch)]),
    "t4a_plan_contiguous_to_view_any": (c_int, [c_int, POINTER(CLayoutAny), c_longlong,
                                                POINTER(CLaunch)]),
    "t4a_plan_broadcast_in_dim_any": (c_int, [c_int, POINTER(CLayoutAny), c_longlong,
                                              POINTER(CLayoutAny), c_longlong,
                                              POINTER(CAxisValuesAny), POINTER(CLaunch)]),
    "t4a_plan_concatenate_copy_any": (c_int, [c_int, POINTER(CLayoutAny), c_longlong,
                                              POINTER(CLayoutAny), c_longlong, c_uint,
                                              c_longlong, POINTER(CLaunch)]),
    "t4a_hip_fill_zero": (c_int, [c_void_p, c_int, c_longlong, POINTER(CLaunch), c_void_p]),
    "t4a_hip_fill_zero_view": (c_int, [c_void_p, c_int, POINTER(CLayout), c_longlong,
                                       POINTER(CLaunch), c_void_p]),
    "t4a_hip_contiguous_to_view": (c_int, [c_void_p, c_void_p, c_int, POINTER(CLayout),
                                           c_longlong, POINTER(CLaunch), c_void_p]),
    "t4a_hip_broadcast_in_dim": (c_int, [c_void_p, c_void_p, c_int, POINTER(CLayout),
                                         POINTER(CLayout), POINTER(CAxisValues), c_longlong,
                                         POINTER(CLaunch), c_void_p]),
    "t4a_hip_concatenate_copy": (c_int, [c_void_p, c_void_p, c_int, POINTER(CLayout),
                                         POINTER(CLayout), c_int, c_longlong, c_longlong,
                                         POINTER(CLaunch), c_void_p]),
    "t4a_hip_fill_zero_view_any": (c_int, [c_void_p, c_int, POINTER(CLayoutAny), c_longlong,
                                           POINTER(CLaunch), c_void_p]),
    "t4a_hip_contiguous_to_view_any": (c_int, [c_void_p, c_void_p, c_int, POINTER(CLayoutAny),
                                               c_longlong, POINTER(CLaunch), c_void_p]),
    "t4a_hip_broadcast_in_dim_any": (c_int, [c_void_p, c_void_p, c_int, POINTER(CLayoutAny),
                                             POINTER(CLayoutAny), POINTER(CAxisValuesAny),
                                             c_longlong, POINTER(CLaunch), c_void_p]),
    "t4a_hip_concatenate_copy_any": (c_int, [c_void_p, c_void_p, c_int, POINTER(CLayoutAny),
                                             POINTER(CLayoutAny), c_int, c_longlong,
                                             c_longlong, POINTER(CLaunch), c_void_p]),
    "t4a_hip_reduction": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int,
                                  POINTER(CLayout), POINTER(CLayout), c_int, c_longlong,
                                  POINTER(CReductionPlan), c_void_p]),
    "t4a_hip_launch_count": (ctypes.c_ulonglong, []),
    "t4a_hip_reduction_scratch": (c_int, [c_void_p, c_void_p, c_int, c_int, POINTER(CLayout),
                                          POINTER(CLayout), c_int, c_longlong,
                                          POINTER(CReductionPlan), c_void_p]),
    "t4a_hip_reduction_joins": (c_int, [c_void_p, c_int, c_int, POINTER(CLayout),
                                        POINTER(CLayout), c_int, c_longlong,
                                        POINTER(CReductionPlan)]),
}

_LIB = None


def load() -> ctypes.CDLL:
    """Load the shared library once. A missing build is an error, never a fallback."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is not built: run `python t4a-cuda-kernels_amd/build.py` "
            "(or __graft_entry__.build()) first")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _LIB = lib
    return lib
