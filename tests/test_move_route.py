"""Route selection of the movement launchers (t4a_plan_move_route), CPU only.

The planner fuses axes (extent-1 axes dropped, axes chained on both sides
merged) and then picks the kernel: the copy kernel for one run contiguous on
both sides (the reference consumer's "linear" class), 16-byte row units when a
dim is contiguous on both sides, the tiled transpose's kernel for one compact
2-D transpose, the tile walk when each run's chain has at most two dims and
the tile is one of the walk's shapes, the general tiled kernel otherwise, and a
per-element decode when no dim is contiguous on one of the sides
(reference docs/design/cubecl-performance-parity.md:57-63 asks for exactly
this linear / strided / tiled classification after fusion).
"""
import pytest

import t4a_cuda_kernels as t
from t4a_cuda_kernels import DType, Error, Layout, MoveRoute, T4aError

F32, F64, C32, C64, BOOL = DType.F32, DType.F64, DType.C32, DType.C64, DType.Bool


def route(dtype, src, dst=None):
    return t.move_route(dtype, src, dst)


def transposed(m, n, offset=0):
    """The [m, n] view of a compact [n, m] buffer (axis 0 fastest)."""
    return Layout([m, n], [n, 1], offset)


def test_benchmark_configurations_take_their_fast_routes():
    # C1-shaped transpose through materialize_strided: the routed transpose
    assert route(F32, transposed(1024, 1024)) == MoveRoute.Transpose
    assert route(F32, transposed(8192, 8192)) == MoveRoute.Transpose
    # C3: rank-4 reversed-view permute, one 64 x 32 tile per block (8-byte)
    c3 = Layout([64, 64, 128, 32], [32, 262144, -2048, 1], 260096)
    assert route(F64, c3) == MoveRoute.TileOnce
    assert route(C32, c3) == MoveRoute.TileOnce
    # C5: the rank-6 c64 permute, one 32 x 32 tile per block
    c5 = Layout([16] * 6, [256, 65536, 16, 1048576, 4096, 1], 0)
    assert route(C64, c5) == MoveRoute.TileOnce


def test_linear_and_row_routes():
    # identical compact layouts, with offsets: one run
    assert route(F32, Layout.compact([300, 40])) == MoveRoute.Linear
    assert route(F32, Layout([300, 40], [1, 300], 7), Layout([300, 40], [1, 300], 5)) == \
        MoveRoute.Linear
    # extent-1 axes and chained axes fuse away
    assert route(F64, Layout([1, 64, 1, 8], [99, 1, 5, 64], 0)) == MoveRoute.Linear
    # rows of 1000 into a destination with row pitch 1500 (concatenate, outer rows)
    assert route(F32, Layout.compact([1000, 300]), Layout([1000, 300], [1, 1500], 200)) == \
        MoveRoute.Rows
    # one row broadcast down 8192 rows (broadcast_in_dim's source view)
    assert route(F32, Layout([8192, 8192], [1, 0], 0)) == MoveRoute.Rows
    # Bool rows, and c64 rows (16-byte elements are one unit each)
    assert route(BOOL, Layout([256, 7], [1, 300], 0)) == MoveRoute.Rows
    assert route(C64, Layout([16, 9], [1, 20], 0)) == MoveRoute.Rows


def test_transpose_route_conditions():
    # offsets on both sides keep the route
    assert route(F32, Layout([97, 131], [1, 97], 5), Layout([97, 131], [131, 1], 3)) == \
        MoveRoute.Transpose
    # a padded (non-compact) source row pitch is not a compact transpose
    assert route(F32, Layout([64, 64], [72, 1], 0)) != MoveRoute.Transpose
    # a batched transpose (third dim) takes the tile walk
    assert route(F32, Layout([64, 64, 3], [64, 1, 4096], 0)) in (MoveRoute.TileOnce,
                                                                 MoveRoute.Tiles)
    # every dtype
    for dt in DType:
        assert route(dt, transposed(300, 257)) == MoveRoute.Transpose, dt


def test_tile_and_element_routes():
    # no source dim of stride 1 (a reversed fast axis): per-element decode
    assert route(F32, Layout([1000], [-1], 999)) == MoveRoute.Elements
    # a broadcast fast axis with the destination fast elsewhere: tiles or elements
    assert route(F32, Layout([300, 7], [0, 1], 0)) in (MoveRoute.Tiles, MoveRoute.TileOnce,
                                                        MoveRoute.Elements)
    # one-byte elements never take the one-tile kernels
    c3 = Layout([64, 64, 128, 32], [32, 262144, -2048, 1], 260096)
    assert route(BOOL, c3) == MoveRoute.Tiles
    # empty and single-element moves
    assert route(F32, Layout([0, 5], [1, 1], 0)) == MoveRoute.Empty
    assert route(F32, Layout([], [], 3)) == MoveRoute.Elements


def _strides(ext, order):
    """Strides of a compact buffer whose axes, fastest first, are `order`."""
    st, c = [0] * len(ext), 1
    for k in order:
        st[k] = c
        c *= ext[k]
    return st


# Moves whose run ends at 16 or 32 elements on one side (the next dim of that
# side's chain belongs to the other chain), so the planner hands the tile budget
# to the other run: 128 x 16, 128 x 32, 32 x 128, 16 x 128 tiles for 4-byte
# elements, 128 x 16, 32 x 64, 16 x 128 for 8-byte, 64 x 16, 16 x 64 for 16-byte.
LONG_SHORT = [
    ([64, 32, 16, 8], [2, 0, 3, 1], [0, 1, 2, 3]),
    ([64, 32, 32, 8], [2, 0, 3, 1], [0, 1, 2, 3]),
    ([32, 64, 32, 8], [1, 2, 0, 3], [0, 1, 3, 2]),
    ([16, 64, 32, 8], [1, 2, 0, 3], [0, 1, 3, 2]),
    ([64, 33, 16, 5], [2, 0, 3, 1], [0, 1, 2, 3]),
    ([16, 64, 33, 7], [1, 2, 0, 3], [0, 1, 3, 2]),
]


def test_long_and_short_tiles_take_the_tile_walk():
    for ext, so, do in LONG_SHORT:
        src, dst = Layout(ext, _strides(ext, so), 0), Layout(ext, _strides(ext, do), 0)
        for dt in (F32, F64, C32, C64):
            assert route(dt, src, dst) == MoveRoute.TileOnce, (ext, dt)


def test_route_validates_like_the_planners():
    with pytest.raises(T4aError) as e:
        route(F32, Layout.compact([3, 4]), Layout.compact([4, 3]))
    assert e.value.error == Error.CountMismatch
    with pytest.raises(T4aError) as e:
        route(F32, Layout.compact([3, 4]), Layout([3, 4], [1, 0], 0))
    assert e.value.error == Error.BroadcastDestination
    with pytest.raises(T4aError) as e:
        route(99, Layout.compact([3, 4]))
    assert e.value.error == Error.UnsupportedDType
