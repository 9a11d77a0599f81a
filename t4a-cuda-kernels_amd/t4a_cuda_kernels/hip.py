"""Launch the gfx950 kernels through the C ABI (include/t4a/t4a.h, t4a_hip_*).

Pointers are device addresses (ints, or objects with `data_ptr()` such as torch
tensors); `stream` is a HIP stream handle (int), an object with `cuda_stream`
(a torch stream), or None for the null stream. The caller owns every buffer,
the stream and completion, as with the reference entries
(reference docs/abi/c-kernel-abi.md:3-14). Nothing here synchronizes.
"""
from __future__ import annotations

from ctypes import byref, c_void_p
from typing import Optional

from . import (DType, Launch, Layout, ReduceOp, ReduceStrategy, ReductionPlan,
               T4aError, TransposeConfig, _lib, reduction_partials_layout)


def _ptr(x) -> c_void_p:
    if hasattr(x, "data_ptr"):
        return c_void_p(x.data_ptr())
    return c_void_p(int(x))


def _stream(stream) -> c_void_p:
    if stream is None:
        return c_void_p(0)
    if hasattr(stream, "cuda_stream"):
        return c_void_p(stream.cuda_stream)
    return c_void_p(int(stream))


def _check(status: int) -> None:
    if status != 0:
        raise T4aError(status)


def tiled_transpose(dst, src, dtype: DType, src_offset: int, batch_stride: int,
                    dst_fast_extent: int, src_fast_extent: int, config: TransposeConfig,
                    launch: Launch, stream=None) -> None:
    """Reference t4a_cuda_tiled_transpose (cuda/src/movement.cu:571-573)."""
    _check(_lib.load().t4a_hip_tiled_transpose(
        _ptr(dst), _ptr(src), int(dtype), src_offset, batch_stride, dst_fast_extent,
        src_fast_extent, config.c, byref(launch.to_c()), _stream(stream)))


def copy_exact(dst, src, dtype: DType, length: int, launch: Launch, stream=None) -> None:
    """Reference t4a_cuda_copy_exact (cuda/src/movement.cu:528-533)."""
    _check(_lib.load().t4a_hip_copy_exact(_ptr(dst), _ptr(src), int(dtype), length,
                                          byref(launch.to_c()), _stream(stream)))


def materialize_strided(dst, src, dtype: DType, src_layout: Layout, length: int,
                        launch: Launch, stream=None) -> None:
    """Reference t4a_cuda_materialize_strided (cuda/src/movement.cu:535-537)."""
    _check(_lib.load().t4a_hip_materialize_strided(
        _ptr(dst), _ptr(src), int(dtype), byref(src_layout.c), length, byref(launch.to_c()),
        _stream(stream)))


def strided_to_strided(dst, src, dtype: DType, src_layout: Layout, dst_layout: Layout,
                       length: int, launch: Launch, stream=None) -> None:
    """Reference t4a_cuda_strided_to_strided (cuda/src/movement.cu:553-556)."""
    _check(_lib.load().t4a_hip_strided_to_strided(
        _ptr(dst), _ptr(src), int(dtype), byref(src_layout.c), byref(dst_layout.c), length,
        byref(launch.to_c()), _stream(stream)))


def fill_zero(out, dtype: DType, length: int, launch: Launch, stream=None) -> None:
    """Reference t4a_cuda_fill_zero (cuda/src/movement.cu:514-518)."""
    _check(_lib.load().t4a_hip_fill_zero(_ptr(out), int(dtype), length, byref(launch.to_c()),
                                         _stream(stream)))


def fill_zero_view(out, dtype: DType, layout: Layout, length: int, launch: Launch,
                   stream=None) -> None:
    """Reference t4a_cuda_fill_zero_view (cuda/src/movement.cu:520-526)."""
    _check(_lib.load().t4a_hip_fill_zero_view(_ptr(out), int(dtype), byref(layout.c), length,
                                              byref(launch.to_c()), _stream(stream)))


def contiguous_to_view(dst, src, dtype: DType, dst_layout: Layout, length: int,
                       launch: Launch, stream=None) -> None:
    """Reference t4a_cuda_contiguous_to_view (cuda/src/movement.cu:544-551)."""
    _check(_lib.load().t4a_hip_contiguous_to_view(
        _ptr(dst), _ptr(src), int(dtype), byref(dst_layout.c), length, byref(launch.to_c()),
        _stream(stream)))


def broadcast_in_dim(out, inp, dtype: DType, out_layout: Layout, in_layout: Layout, dims,
                     out_len: int, launch: Launch, stream=None) -> None:
    """Reference t4a_cuda_broadcast_in_dim (cuda/src/movement.cu:648-656)."""
    from . import axis_values
    _check(_lib.load().t4a_hip_broadcast_in_dim(
        _ptr(out), _ptr(inp), int(dtype), byref(out_layout.c), byref(in_layout.c),
        byref(axis_values(dims)), out_len, byref(launch.to_c()), _stream(stream)))


def concatenate_copy(out, inp, dtype: DType, out_layout: Layout, in_layout: Layout, axis: int,
                     axis_offset: int, in_len: int, launch: Launch, stream=None) -> None:
    """Reference t4a_cuda_concatenate_copy (cuda/src/movement.cu:668-676)."""
    _check(_lib.load().t4a_hip_concatenate_copy(
        _ptr(out), _ptr(inp), int(dtype), byref(out_layout.c), byref(in_layout.c), axis,
        axis_offset, in_len, byref(launch.to_c()), _stream(stream)))


def reduce(out, inp, dtype: DType, op: ReduceOp, strategy: ReduceStrategy,
           out_layout: Layout, in_layout: Layout, axis: int, output_len: int, launch: Launch,
           stream=None) -> None:
    """Reference t4a_cuda_reduce (cuda/src/reduce.cu:765-768)."""
    _check(_lib.load().t4a_hip_reduce(
        _ptr(out), _ptr(inp), int(dtype), int(op), int(strategy), byref(out_layout.c),
        byref(in_layout.c), axis, output_len, byref(launch.to_c()), _stream(stream)))


def reduce_partials(partials, inp, dtype: DType, op: ReduceOp, partials_layout: Layout,
                    in_layout: Layout, axis: int, output_len: int, splits: int,
                    chunk_len: int, launch: Launch, stream=None) -> None:
    """Reference t4a_cuda_reduce_partials (cuda/src/reduce.cu:813-817)."""
    _check(_lib.load().t4a_hip_reduce_partials(
        _ptr(partials), _ptr(inp), int(dtype), int(op), byref(partials_layout.c),
        byref(in_layout.c), axis, output_len, splits, chunk_len, byref(launch.to_c()),
        _stream(stream)))


# ---- general-rank twins: layouts are t4a_cuda_layout_any structs whose arrays
# live in device memory (WideLayout.device_c over device copies of
# WideLayout.extents / .strides), ordered before the launch on `stream`.

def materialize_strided_any(dst, src, dtype: DType, src_layout, length: int, launch: Launch,
                            stream=None) -> None:
    """Reference t4a_cuda_materialize_strided_any (cuda/src/movement.cu:620-626)."""
    _check(_lib.load().t4a_hip_materialize_strided_any(
        _ptr(dst), _ptr(src), int(dtype), byref(src_layout), length, byref(launch.to_c()),
        _stream(stream)))


def strided_to_strided_any(dst, src, dtype: DType, src_layout, dst_layout, length: int,
                           launch: Launch, stream=None) -> None:
    """Reference t4a_cuda_strided_to_strided_any (cuda/src/movement.cu:638-646)."""
    _check(_lib.load().t4a_hip_strided_to_strided_any(
        _ptr(dst), _ptr(src), int(dtype), byref(src_layout), byref(dst_layout), length,
        byref(launch.to_c()), _stream(stream)))


def fill_zero_view_any(out, dtype: DType, layout, length: int, launch: Launch,
                       stream=None) -> None:
    """Reference t4a_cuda_fill_zero_view_any (cuda/src/movement.cu:612-618)."""
    _check(_lib.load().t4a_hip_fill_zero_view_any(_ptr(out), int(dtype), byref(layout), length,
                                                  byref(launch.to_c()), _stream(stream)))


def contiguous_to_view_any(dst, src, dtype: DType, dst_layout, length: int, launch: Launch,
                           stream=None) -> None:
    """Reference t4a_cuda_contiguous_to_view_any (cuda/src/movement.cu:629-635)."""
    _check(_lib.load().t4a_hip_contiguous_to_view_any(
        _ptr(dst), _ptr(src), int(dtype), byref(dst_layout), length, byref(launch.to_c()),
        _stream(stream)))


def broadcast_in_dim_any(out, inp, dtype: DType, out_layout, in_layout, dims, out_len: int,
                         launch: Launch, stream=None) -> None:
    """Reference t4a_cuda_broadcast_in_dim_any (cuda/src/movement.cu:658-666); `dims` a
    t4a_cuda_axis_values_any over device memory."""
    _check(_lib.load().t4a_hip_broadcast_in_dim_any(
        _ptr(out), _ptr(inp), int(dtype), byref(out_layout), byref(in_layout), byref(dims),
        out_len, byref(launch.to_c()), _stream(stream)))


def concatenate_copy_any(out, inp, dtype: DType, out_layout, in_layout, axis: int,
                         axis_offset: int, in_len: int, launch: Launch, stream=None) -> None:
    """Reference t4a_cuda_concatenate_copy_any (cuda/src/movement.cu:678-685)."""
    _check(_lib.load().t4a_hip_concatenate_copy_any(
        _ptr(out), _ptr(inp), int(dtype), byref(out_layout), byref(in_layout), axis,
        axis_offset, in_len, byref(launch.to_c()), _stream(stream)))


def reduce_any(out, inp, dtype: DType, op: ReduceOp, strategy: ReduceStrategy, out_layout,
               in_layout, axis: int, output_len: int, launch: Launch, stream=None) -> None:
    """Reference t4a_cuda_reduce_any (cuda/src/reduce.cu:854-900)."""
    _check(_lib.load().t4a_hip_reduce_any(
        _ptr(out), _ptr(inp), int(dtype), int(op), int(strategy), byref(out_layout),
        byref(in_layout), axis, output_len, byref(launch.to_c()), _stream(stream)))


def reduce_partials_any(partials, inp, dtype: DType, op: ReduceOp, partials_layout, in_layout,
                        axis: int, output_len: int, splits: int, chunk_len: int,
                        launch: Launch, stream=None) -> None:
    """Reference t4a_cuda_reduce_partials_any (cuda/src/reduce.cu:902-940)."""
    _check(_lib.load().t4a_hip_reduce_partials_any(
        _ptr(partials), _ptr(inp), int(dtype), int(op), byref(partials_layout),
        byref(in_layout), axis, output_len, splits, chunk_len, byref(launch.to_c()),
        _stream(stream)))


def enqueue_reduction(plan: ReductionPlan, out, inp, partials, dtype: DType, op: ReduceOp,
                      out_layout: Layout, in_layout: Layout, axis: int, output_len: int,
                      stream=None) -> Optional[Layout]:
    """Enqueue a planned reduction: the direct pass, or pass 1 then the combine
    pass on the same stream with no host wait between them (the reference
    caller's sequence, tests/gpu_reduce_golden.rs:416-441). `partials` must hold
    the element count of `reduction_partials_layout(in_layout, axis, splits)`.
    Returns the partials layout of a split plan."""
    if plan.kind == "Direct":
        reduce(out, inp, dtype, op, plan.strategy, out_layout, in_layout, axis, output_len,
               plan.launch, stream)
        return None
    partials_layout = reduction_partials_layout(in_layout, axis, plan.split.splits)
    reduce_partials(partials, inp, dtype, op, partials_layout, in_layout, axis, output_len,
                    plan.split.splits, plan.split.chunk_len, plan.pass1, stream)
    reduce(out, partials, dtype, plan.combine_op, plan.combine_strategy, out_layout,
           partials_layout, axis, output_len, plan.pass2, stream)
    return partials_layout


def reduction(plan: ReductionPlan, out, inp, partials, dtype: DType, op: ReduceOp,
              out_layout: Layout, in_layout: Layout, axis: int, output_len: int,
              stream=None) -> None:
    """A whole planned reduction through t4a_hip_reduction: one launch where
    each block can hold all of an output's chunks (a unit combine over at most
    32 partials of a contiguous axis), else pass 1 and the combine. `partials`
    (the plan's partials layout) is written either way; None for Direct plans."""
    _check(_lib.load().t4a_hip_reduction(
        _ptr(out), _ptr(inp), _ptr(partials) if partials is not None else c_void_p(0),
        int(dtype), int(op), byref(out_layout.c), byref(in_layout.c), axis, output_len,
        byref(plan.to_c()), _stream(stream)))


# Bytes of the library's per-GPU partials array (T4A_HIP_SCRATCH_BYTES).
SCRATCH_BYTES = 8 * 1024 * 1024


def reduction_scratch(plan: ReductionPlan, out, inp, dtype: DType, op: ReduceOp,
                      out_layout: Layout, in_layout: Layout, axis: int, output_len: int,
                      stream=None) -> None:
    """`reduction` without a partials workspace, allocating nothing: a Split
    plan's partials live in the library's per-GPU array of SCRATCH_BYTES
    (ScratchLimit when they do not fit). Calls that overlap on one GPU race."""
    _check(_lib.load().t4a_hip_reduction_scratch(
        _ptr(out), _ptr(inp), int(dtype), int(op), byref(out_layout.c), byref(in_layout.c), axis,
        output_len, byref(plan.to_c()), _stream(stream)))


def reduction_joins(plan: ReductionPlan, inp, dtype: DType, op: ReduceOp, out_layout: Layout,
                    in_layout: Layout, axis: int, output_len: int) -> bool:
    """Whether `reduction` runs `plan` over `inp` as one launch."""
    return bool(_lib.load().t4a_hip_reduction_joins(
        _ptr(inp), int(dtype), int(op), byref(out_layout.c), byref(in_layout.c), axis,
        output_len, byref(plan.to_c())))
