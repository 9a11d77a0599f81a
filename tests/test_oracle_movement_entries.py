"""Pins for the oracle's fill_zero_view, contiguous_to_view, broadcast_in_dim and
concatenate_copy (oracle/t4a_oracle.c, restating reference cuda/src/movement.cu:
79-125, 397-466) against NumPy's own semantics, not a retyped index formula:

- fill_zero_view zeroes exactly the view's addresses (a prefilled pattern
  survives everywhere else), with reversed, extent-1 and offset views;
- contiguous_to_view is NumPy's scatter through the view's index map;
- broadcast_in_dim equals np.broadcast_to of the input with its axes moved to
  their destination positions (reference axis 0 fastest = NumPy Fortran order);
- two concatenate_copy calls give np.concatenate along the axis.
"""
import numpy as np
import pytest

import t4a_cuda_kernels as t
from oracle import t4a_oracle as orc

F32, F64, C64, BOOL = t.DType.F32, t.DType.F64, t.DType.C64, t.DType.Bool
NP = {F32: np.float32, F64: np.float64, C64: np.complex128, BOOL: np.uint8}


def view_indices(ext, st, offset=0):
    idx = np.array([offset], dtype=np.int64)
    for k in reversed(range(len(ext))):
        idx = (idx[:, None] + np.arange(ext[k], dtype=np.int64)[None, :] * st[k]).ravel()
    return idx


def values(dtype, n, rng):
    if dtype == BOOL:
        return rng.integers(0, 2, n).astype(np.uint8)
    if dtype == C64:
        return (rng.standard_normal(n) + 1j * rng.standard_normal(n)).astype(np.complex128)
    return rng.standard_normal(n).astype(NP[dtype])


VIEWS = [([4, 3, 5], [15, 5, 1], 0), ([4, 1, 6], [1, 99, 8], 3), ([7, 3], [-3, 1], 18),
         ([2, 2, 2, 2], [8, 1, 4, 2], 0), ([], [], 5)]


@pytest.mark.parametrize("dtype", [F32, F64, C64, BOOL], ids=lambda d: d.name)
def test_fill_zero_view_zeroes_exactly_the_view(dtype):
    rng = np.random.default_rng(1)
    for ext, st, off in VIEWS:
        layout = t.Layout(ext, st, off)
        n = layout.max_reachable_offset() + 1
        out = values(dtype, n + 4, rng)
        keep = out.copy()
        orc.fill_zero_view(out, dtype, layout, layout.element_count())
        touched = np.zeros(n + 4, bool)
        touched[view_indices(ext, st, off)] = True
        assert not out.view(np.uint8).reshape(n + 4, -1)[touched].any()
        assert np.array_equal(out[~touched], keep[~touched])


@pytest.mark.parametrize("dtype", [F32, C64, BOOL], ids=lambda d: d.name)
def test_contiguous_to_view_is_the_view_scatter(dtype):
    rng = np.random.default_rng(2)
    for ext, st, off in VIEWS:
        layout = t.Layout(ext, st, off)
        n = layout.element_count()
        src = values(dtype, n, rng)
        dst = np.zeros(layout.max_reachable_offset() + 1, NP[dtype])
        want = dst.copy()
        want[view_indices(ext, st, off)] = src
        orc.contiguous_to_view(dst, src, dtype, layout, n)
        assert np.array_equal(dst, want)


def numpy_broadcast(inp_f, out_ext, dims):
    """np.broadcast_to of a Fortran-order input whose axis i lands on output
    axis dims[i]."""
    order = sorted(range(len(dims)), key=lambda i: dims[i])
    moved = np.transpose(inp_f, order) if order else inp_f
    shape = [1] * len(out_ext)
    for i in order:
        shape[dims[i]] = inp_f.shape[i]
    return np.broadcast_to(moved.reshape(shape, order="F"), out_ext)


@pytest.mark.parametrize("dtype", [F32, F64, C64, BOOL], ids=lambda d: d.name)
def test_broadcast_in_dim_is_numpy_broadcasting(dtype):
    rng = np.random.default_rng(3)
    cases = [([3, 4, 5], [4, 1], [1, 2]), ([3, 4, 5], [5, 3], [2, 0]), ([6, 2], [], []),
             ([2, 3, 4, 5], [1, 5, 1], [0, 3, 1]), ([7], [7], [0]), ([5, 4], [4, 5], [1, 0])]
    for out_ext, in_ext, dims in cases:
        n_in = int(np.prod(in_ext)) if in_ext else 1
        inp = values(dtype, n_in, rng)
        inp_f = inp.reshape(in_ext, order="F") if in_ext else inp.reshape(())
        out_l = t.Layout.compact(out_ext)
        in_l = t.Layout.compact(in_ext)
        n = out_l.element_count()
        out = np.zeros(n, NP[dtype])
        orc.broadcast_in_dim(out, inp, dtype, out_l, in_l, dims, n)
        want = numpy_broadcast(inp_f, out_ext, dims).ravel(order="F")
        assert np.array_equal(out, want), (out_ext, in_ext, dims)
    # a strided, offset input view: the same as its materialized copy
    big = values(dtype, 200, rng)
    in_l = t.Layout([4, 1], [3, 50], 7)
    inp = big[view_indices([4, 1], [3, 50], 7)]
    out_l = t.Layout.compact([5, 4])
    out = np.zeros(20, NP[dtype])
    orc.broadcast_in_dim(out, big, dtype, out_l, in_l, [1, 0], 20)
    assert np.array_equal(out, numpy_broadcast(inp.reshape([4, 1], order="F"), [5, 4],
                                               [1, 0]).ravel(order="F"))


@pytest.mark.parametrize("dtype", [F32, C64], ids=lambda d: d.name)
def test_concatenate_copy_pairs_are_numpy_concatenate(dtype):
    rng = np.random.default_rng(4)
    for ext_a, ext_b, axis in [([3, 4, 5], [3, 2, 5], 1), ([2, 3], [5, 3], 0),
                               ([4, 2, 3], [4, 2, 6], 2)]:
        a, b = values(dtype, int(np.prod(ext_a)), rng), values(dtype, int(np.prod(ext_b)), rng)
        out_ext = list(ext_a)
        out_ext[axis] += ext_b[axis]
        out_l = t.Layout.compact(out_ext)
        n = out_l.element_count()
        out = np.zeros(n, NP[dtype])
        orc.concatenate_copy(out, a, dtype, out_l, t.Layout.compact(ext_a), axis, 0, a.size)
        orc.concatenate_copy(out, b, dtype, out_l, t.Layout.compact(ext_b), axis, ext_a[axis],
                             b.size)
        want = np.concatenate([a.reshape(ext_a, order="F"), b.reshape(ext_b, order="F")],
                              axis=axis).ravel(order="F")
        assert np.array_equal(out, want)
    # into a strided destination view: the same bytes as the compact case scattered
    a = values(dtype, 12, rng)
    out_l = t.Layout([3, 6], [7, 1], 2)
    out = np.zeros(out_l.max_reachable_offset() + 1, NP[dtype])
    orc.concatenate_copy(out, a, dtype, out_l, t.Layout.compact([3, 4]), 1, 2, 12)
    want = np.zeros_like(out)
    want[view_indices([3, 4], [7, 1], 2 + 2 * 1)] = a
    assert np.array_equal(out, want)
