"""Host planning: validation and geometry, CPU only.

Ported from the reference's planner tests (reference tests/planning.rs): every
refusal is the same `Error` variant for the same input. Geometry assertions
state this library's MI355X plans where they differ from the reference's
(256-thread unit, pass-1 and movement blocks; 512-thread transpose blocks; the
batch in grid z), and the reference's wherever the geometry carries the fold
topology (a PLANE block is its plane width, a pass-1 block of at most 32
threads is one plane).
"""
import pytest

import t4a_cuda_kernels as t
from t4a_cuda_kernels import (DType, Error, Layout, ReduceOp, ReduceStrategy, Split, T4aError,
                              TransposeConfig)


def err(fn, *args):
    with pytest.raises(T4aError) as info:
        fn(*args)
    return info.value.error


def reduced(extents, axis):
    inp = Layout.compact(extents)
    out = list(extents)
    out[axis] = 1
    return inp, Layout.compact(out)


# ---- layouts (reference tests/planning.rs:36-80) -----------------------------------

def test_layout_rejects_bad_inputs():
    assert err(Layout, [1] * 9, [1] * 9, 0) == Error.RankOutOfRange
    assert err(Layout, [1, 2], [1], 0) == Error.RankLength
    assert err(Layout, [-1], [1], 0) == Error.NegativeExtent


def test_rank_zero_is_a_scalar_view():
    layout = Layout([], [], 7)
    assert layout.rank == 0 and layout.element_count() == 1
    assert layout.min_reachable_offset() == 7 and layout.max_reachable_offset() == 7
    launch = t.plan_materialize_strided(DType.F64, layout, 8)
    assert not launch.is_empty()


def test_compact_layout_has_axis_zero_fastest():
    layout = Layout.compact([2, 3, 4])
    assert layout.strides == [1, 2, 6]
    assert layout.element_count() == 24 and layout.max_reachable_offset() == 23


def test_negative_strides_report_the_reachable_span():
    layout = Layout([3], [-2], 4)
    assert (layout.min_reachable_offset(), layout.max_reachable_offset()) == (0, 4)
    reversed_ = Layout([3], [-1], 2)
    assert (reversed_.min_reachable_offset(), reversed_.max_reachable_offset()) == (0, 2)


def test_extent_product_overflow_is_rejected():
    layout = Layout([2**63 - 1, 2], [1, 1], 0)
    assert err(layout.element_count) == Error.Overflow
    assert err(Layout.compact, [2**63 - 1, 2]) == Error.Overflow


def test_broadcast_read_is_fine_broadcast_write_is_not():
    broadcast = Layout([3, 4], [1, 0], 0)
    assert not t.plan_materialize_strided(DType.F32, broadcast, 12).is_empty()
    assert err(t.plan_strided_to_strided, DType.F32, Layout.compact([3, 4]), 12, broadcast,
               12) == Error.BroadcastDestination


# ---- movement (reference tests/planning.rs:114-166, 3198-3240) -----------------------

def test_view_entries_derive_the_count_and_reject_out_of_span():
    layout = Layout([3], [2], 0)
    assert not t.plan_materialize_strided(DType.F32, layout, 5).is_empty()
    assert err(t.plan_materialize_strided, DType.F32, layout, 4) == Error.OffsetOutOfSpan
    sparse, compact = Layout([3], [3], 0), Layout([3], [1], 0)
    assert err(t.plan_strided_to_strided, DType.F32, compact, 3, sparse, 3) == \
        Error.OffsetOutOfSpan
    assert err(t.plan_strided_to_strided, DType.F32, compact, 3, sparse, 6) == \
        Error.OffsetOutOfSpan
    negative = Layout([3], [-1], 1)
    assert err(t.plan_materialize_strided, DType.F32, negative, 3) == Error.OffsetOutOfSpan
    assert err(t.plan_materialize_strided, DType.F32, layout, -1) == Error.NegativeCount


def test_strided_to_strided_requires_equal_extents():
    assert err(t.plan_strided_to_strided, DType.F32, Layout.compact([2, 2]), 4,
               Layout.compact([4]), 4) == Error.CountMismatch


def test_a_reversed_layout_is_a_strided_movement_plan():
    ext, strides = [3, 4], [1, 3]
    off = sum((e - 1) * s for e, s in zip(ext, strides))
    reversed_ = Layout(ext, [-s for s in strides], off)
    assert not t.plan_materialize_strided(DType.F64, reversed_, 12).is_empty()
    assert not t.plan_strided_to_strided(DType.F64, reversed_, 12, Layout.compact(ext),
                                         12).is_empty()


def test_movement_unknown_dtype_and_empty():
    assert err(t.plan_materialize_strided, 9, Layout.compact([4]), 4) == Error.UnsupportedDType
    assert t.plan_materialize_strided(DType.F32, Layout.compact([0, 3]), 0).is_empty()
    assert t.plan_copy_exact(DType.Bool, 0).is_empty()
    assert err(t.plan_copy_exact, DType.F32, -1) == Error.NegativeCount
    too_many = (2**31 - 1) * 256 + 1
    assert err(t.plan_copy_exact, DType.F32, too_many) == Error.LaunchLimit


def test_movement_geometry():
    launch = t.plan_materialize_strided(DType.F64, Layout([64, 64, 128, 32],
                                                          [32, 262144, -2048, 1], 260096),
                                        64 * 128 * 64 * 32)
    assert launch.block == (256, 1, 1) and launch.grid[0] >= 1 and launch.shared_bytes == 0


# ---- tiled transpose (reference tests/planning.rs:180-280) ---------------------------

def test_transpose_configuration_range():
    for bad in [(12, 8, 1, 1), (16, 3, 1, 1), (16, 8, 2, 1), (16, 8, 1, 8)]:
        assert err(TransposeConfig, *bad) == Error.InvalidTransposeConfig
    TransposeConfig(8, 16, 0, 4)
    assert TransposeConfig.DEFAULT.tile == 16
    assert TransposeConfig(32, 8, 1, 1).shared_bytes(DType.C64.size) <= t.DEFAULT_SHARED_BYTES


def test_transpose_plans_batches_in_grid_z():
    cfg = TransposeConfig.DEFAULT
    span = 512 * 1024 * 3
    launch = t.plan_tiled_transpose(DType.F64, cfg, 0, 512 * 1024, 512, 1024, 3, span, span)
    assert launch.grid[2] == 3 and launch.block == (512, 1, 1)
    # 128 x 64 tiles of f64: 4 x 16 per matrix
    assert launch.grid[0] == 64
    launch = t.plan_tiled_transpose(DType.F32, cfg, 0, 35, 5, 7, 1, 35, 35)
    assert launch.grid == (1, 1, 1)


def test_transpose_rejects_bad_batches_and_limits():
    cfg = TransposeConfig.DEFAULT
    assert err(t.plan_tiled_transpose, DType.F32, cfg, 0, 5, 2, 3, 1, 6, 6) == \
        Error.InvalidTransposeConfig
    assert err(t.plan_tiled_transpose, DType.F32, cfg, -1, 6, 2, 3, 1, 6, 6) == \
        Error.NegativeCount
    assert err(t.plan_tiled_transpose, DType.F32, cfg, 1, 6, 2, 3, 1, 6, 6) == \
        Error.OffsetOutOfSpan
    wide_rows = 65_535 * 16 + 1  # the reference's grid.y bound at tile 16
    assert err(t.plan_tiled_transpose, DType.F32, cfg, 0, wide_rows, 1, wide_rows, 1,
               wide_rows, wide_rows) == Error.LaunchLimit
    long_columns = 65_535 * 16 + 1
    assert not t.plan_tiled_transpose(DType.F32, cfg, 0, long_columns, long_columns, 1, 1,
                                      long_columns, long_columns).is_empty()
    assert err(t.plan_tiled_transpose, DType.F32, cfg, 0, 6, 2, 3, 65_536, 6 * 65_536,
               6 * 65_536) == Error.LaunchLimit
    assert t.plan_tiled_transpose(DType.F32, cfg, 0, 0, 0, 8, 4, 0, 0).is_empty()


# ---- reductions (reference tests/planning.rs:685-1155, 3567-3662, 3881-3964) -----------

def test_split_policy_matches_the_baseline():
    assert t.split_policy(255, 32) is None
    assert t.split_policy(256, 32) is None
    assert t.split_policy(512, 32) == Split(2, 256)
    assert t.split_policy(513, 32) == Split(2, 256)
    assert t.split_policy(1000, 32) == Split(3, 333)
    assert t.split_policy(8448, 32) == Split(33, 256)
    capped = t.split_policy(10_000_000, 32)
    assert capped == Split(t.MAX_SPLITS, 10_000_000 // t.MAX_SPLITS)
    assert t.split_policy(256, 16) == Split(2, 128)
    assert t.split_policy(255, 8) == Split(3, 85)
    assert t.split_policy(0, 32) is None
    assert err(t.split_policy, 512, 0) == Error.InvalidPlaneWidth


def test_strategy_boundary_is_the_plane_width():
    inp, out = reduced([32, 3], 0)
    t.plan_reduce(DType.F32, ReduceOp.Sum, ReduceStrategy.Unit, out, 3, inp, 96, 0, 32)
    t.plan_reduce(DType.F32, ReduceOp.Sum, ReduceStrategy.Plane, out, 3, inp, 96, 0, 32)
    si, so = reduced([31, 3], 0)
    assert err(t.plan_reduce, DType.F32, ReduceOp.Sum, ReduceStrategy.Plane, so, 3, si, 93, 0,
               32) == Error.StrategyMismatch
    inp, out = reduced([33, 3], 0)
    assert err(t.plan_reduce, DType.F32, ReduceOp.Sum, ReduceStrategy.Unit, out, 3, inp, 99, 0,
               32) == Error.StrategyMismatch
    t.plan_reduce(DType.F32, ReduceOp.Sum, ReduceStrategy.Plane, out, 3, inp, 99, 0, 32)
    assert err(t.plan_reduce, DType.F32, ReduceOp.Sum, ReduceStrategy.Plane, out, 3, inp, 99, 0,
               24) == Error.InvalidPlaneWidth


def test_reduction_geometry_and_shapes():
    inp, out = reduced([4, 64, 2], 1)
    launch = t.plan_reduce(DType.F32, ReduceOp.Max, ReduceStrategy.Plane, out, 8, inp, 512, 1, 32)
    # this build's plane geometry: 256 / W planes of W lanes a block (block.y)
    assert launch.grid == (1, 1, 1) and launch.block == (32, 8, 1)
    inp, out = reduced([64, 100_000], 0)
    launch = t.plan_reduce(DType.F32, ReduceOp.Sum, ReduceStrategy.Plane, out, 100_000, inp,
                           6_400_000, 0, 16)
    assert launch.grid == (4096, 1, 1) and launch.block == (16, 16, 1)
    inp, out = reduced([4, 4, 2], 1)
    launch = t.plan_reduce(DType.F32, ReduceOp.Sum, ReduceStrategy.Unit, out, 8, inp, 32, 1, 8)
    # this build's unit geometry: one-wavefront blocks below 1024 * 256 outputs
    assert launch.grid == (1, 1, 1) and launch.block == (64, 1, 1)
    inp, out = reduced([4, 4, 300_000], 1)
    launch = t.plan_reduce(DType.F32, ReduceOp.Sum, ReduceStrategy.Unit, out, 1_200_000, inp,
                           4_800_000, 1, 8)
    assert launch.grid == (4688, 1, 1) and launch.block == (256, 1, 1)
    inp, _ = reduced([4, 64], 1)
    assert err(t.plan_reduce, DType.F32, ReduceOp.Sum, ReduceStrategy.Plane,
               Layout.compact([4]), 4, inp, 256, 1, 32) == Error.RankLength
    assert err(t.plan_reduce, DType.F32, ReduceOp.Sum, ReduceStrategy.Plane,
               Layout.compact([5, 1]), 5, inp, 256, 1, 32) == Error.ShapeMismatch
    zi, zo = reduced([4, 0], 1)
    assert err(t.plan_reduce, DType.F32, ReduceOp.Sum, ReduceStrategy.Unit, zo, 4, zi, 0, 1,
               32) == Error.NegativeCount
    ei, eo = reduced([0, 64], 1)
    assert t.plan_reduce(DType.F32, ReduceOp.Sum, ReduceStrategy.Plane, eo, 0, ei, 0, 1,
                         32).is_empty()
    assert err(t.plan_reduce, DType.F32, ReduceOp.Sum, ReduceStrategy.Plane, out, 8, inp, 256, 2,
               32) == Error.InvalidAxis


def test_reduction_dtype_gates_follow_the_operation():
    inp, out = reduced([64, 2], 0)
    assert err(t.plan_reduce, DType.C64, ReduceOp.Max, ReduceStrategy.Plane, out, 2, inp, 128,
               0, 32) == Error.UnsupportedDType
    assert err(t.plan_reduce, DType.I32, ReduceOp.SumSquares, ReduceStrategy.Plane, out, 2, inp,
               128, 0, 32) == Error.UnsupportedDType
    assert err(t.plan_reduce, DType.Bool, ReduceOp.Sum, ReduceStrategy.Plane, out, 2, inp, 128,
               0, 32) == Error.UnsupportedDType
    t.plan_reduce(DType.C64, ReduceOp.Prod, ReduceStrategy.Plane, out, 2, inp, 128, 0, 32)
    assert ReduceOp.SumSquares.combine() == ReduceOp.Sum
    assert ReduceOp.Max.combine() == ReduceOp.Max


def test_reduction_plan_applies_the_auto_policy():
    inp, out = reduced([64, 4], 0)
    plan = t.plan_reduction(DType.F64, ReduceOp.Sum, out, 4, inp, 256, 0, 32)
    assert plan.kind == "Direct" and plan.strategy == ReduceStrategy.Plane
    assert plan.launch.grid == (1, 1, 1) and plan.launch.block == (32, 8, 1)
    inp, out = reduced([512, 4], 0)
    plan = t.plan_reduction(DType.F64, ReduceOp.Sum, out, 4, inp, 2048, 0, 32)
    assert plan.kind == "Split" and plan.split == Split(2, 256)
    assert plan.pass1.block == (256, 1, 1) and plan.pass1.grid[0] >= 1
    assert plan.combine_strategy == ReduceStrategy.Unit and plan.combine_op == ReduceOp.Sum
    inp, out = reduced([8448, 2], 0)
    plan = t.plan_reduction(DType.F32, ReduceOp.SumSquares, out, 2, inp, 16896, 0, 32)
    assert plan.split.splits == 33 and plan.combine_strategy == ReduceStrategy.Plane
    assert plan.combine_op == ReduceOp.Sum and plan.pass2.grid == (1, 1, 1)
    assert plan.pass2.block == (32, 8, 1)


def test_partials_plans_enforce_the_floor_split():
    inp, _ = reduced([512, 4], 0)
    partials = Layout.compact([2, 4])
    t.plan_reduce_partials(DType.F32, ReduceOp.Sum, partials, 8, inp, 2048, 0, Split(2, 256), 32)
    for bad in (Split(64, 1), Split(2, 200), Split(1, 512)):
        assert err(t.plan_reduce_partials, DType.F32, ReduceOp.Sum, partials, 8, inp, 2048, 0,
                   bad, 32) == Error.InvalidSplit
    assert err(t.plan_reduce_partials, DType.F32, ReduceOp.Sum, Layout.compact([3, 4]), 12, inp,
               2048, 0, Split(2, 256), 32) == Error.ShapeMismatch


def test_combine_pass_widens_only_for_long_partials_and_not_for_prod():
    out = Layout.compact([1])
    for length, want_splits, want_block in [(8448, 33, 32), (16384, 64, 64),
                                            (1_048_576, 4096, 512)]:
        inp = Layout.compact([length])
        for op in (ReduceOp.Sum, ReduceOp.Max, ReduceOp.Min, ReduceOp.SumSquares):
            plan = t.plan_reduction(DType.F64, op, out, 1, inp, length, 0, 32)
            assert plan.split.splits == want_splits
            assert plan.combine_strategy == ReduceStrategy.Plane
            # a 32-lane combine plane is packed with seven idle ones (block.y)
            assert plan.pass2.block == ((32, 8, 1) if want_block == 32 else (want_block, 1, 1))
        plan = t.plan_reduction(DType.F64, ReduceOp.Prod, out, 1, inp, length, 0, 32)
        assert plan.pass2.block == (32, 8, 1)


def test_wide_combine_widths_are_plane_only_and_bounded():
    out, inp = Layout.compact([1]), Layout.compact([1024])
    t.plan_reduce(DType.F64, ReduceOp.Sum, ReduceStrategy.Plane, out, 1, inp, 1024, 0, 512)
    assert err(t.plan_reduce, DType.F64, ReduceOp.Sum, ReduceStrategy.Unit, out, 1, inp, 1024, 0,
               64) == Error.InvalidPlaneWidth
    assert err(t.plan_reduce, DType.F64, ReduceOp.Sum, ReduceStrategy.Plane, out, 1, inp, 1024, 0,
               1024) == Error.InvalidPlaneWidth


def test_pass1_blocks_are_one_dimensional_and_narrow_planes_keep_one_per_block():
    splits = 390
    for width in (32, 16, 8):
        axis_len = splits * width * 8 + 3
        inp = Layout.compact([3, axis_len])
        partials = Layout.compact([3, splits])
        launch = t.plan_reduce_partials(DType.F64, ReduceOp.Sum, partials, 3 * splits, inp,
                                        3 * axis_len, 1, Split(splits, axis_len // splits),
                                        width)
        assert launch.block[1:] == (1, 1) and launch.shared_bytes == 0
        if width == 32:
            assert launch.block[0] == 256
        else:  # a block of at most 32 threads is one plane of that width
            assert launch.block == (width, 1, 1) and launch.grid == (3 * splits, 1, 1)


def test_reduction_partials_layout_is_compact_with_the_split_axis():
    inp = Layout([5, 100, 7], [700, 7, 1], 3)
    partials = t.reduction_partials_layout(inp, 1, 4)
    assert partials.extents == [5, 4, 7] and partials.is_compact()
    assert err(t.reduction_partials_layout, inp, 3, 4) == Error.InvalidAxis


def test_configuration_plans():
    """The plans of the benchmark configurations C1-C5 (reference axis order)."""
    inp = Layout.compact([8192, 8192])
    plan = t.plan_reduction(DType.F32, ReduceOp.Sum, Layout.compact([1, 8192]), 8192, inp,
                            8192 * 8192, 0, 32)
    assert plan.split == Split(32, 256) and plan.combine_strategy == ReduceStrategy.Unit
    inp = Layout.compact([4, 1048576, 32])
    plan = t.plan_reduction(DType.F32, ReduceOp.SumSquares, Layout.compact([4, 1, 32]), 128, inp,
                            4 * 1048576 * 32, 1, 32)
    assert plan.split == Split(4096, 256) and plan.pass2.block == (512, 1, 1)
    plan = t.plan_reduction(DType.I32, ReduceOp.Prod, Layout.compact([1, 1048576, 32]),
                            1048576 * 32, inp, 4 * 1048576 * 32, 0, 32)
    assert plan.kind == "Direct" and plan.strategy == ReduceStrategy.Unit


def test_reduction_joins_only_unit_combines_of_whole_chunks():
    """Which Split plans t4a_hip_reduction runs as one launch (host logic only:
    the input address is a number, nothing is dereferenced)."""
    from t4a_cuda_kernels import hip
    F32, I64 = t.DType.F32, t.DType.I64

    def joins(dtype, n, rows, addr=0x10000, out_l=None, op=t.ReduceOp.Sum):
        in_l = t.Layout.compact([n, rows])
        out_l = out_l or t.Layout.compact([1, rows])
        plan = t.plan_reduction(dtype, op, out_l, out_l.max_reachable_offset() + 1, in_l,
                                n * rows, 0, 32)
        assert plan.kind == "Split"
        return hip.reduction_joins(plan, addr, dtype, op, out_l, in_l, 0, rows)

    for n in (512, 1024, 1536, 3072, 4096, 6144, 8192):  # splits 2 .. 32, unit combines
        assert joins(F32, n, 7)
    for n in (512, 1024, 1536, 2048, 3072, 4096):  # splits 2 .. 16: at most 8 loads a lane
        assert joins(I64, n, 3)
    for n in (6144, 8192):  # 24 or 32 splits of 2 KiB chunks: 12 or 16 loads a lane
        assert not joins(I64, n, 3)
    assert joins(F32, 8192, 5, op=t.ReduceOp.Max)
    assert joins(F32, 8192, 10, out_l=t.Layout([1, 10], [0, 3], 5))  # strided finals
    assert not joins(F32, 8192, 7, addr=0x10004)  # input not 16-byte aligned
    assert not joins(F32, 8960, 3)  # 35 splits: a plane combine
    assert not joins(F32, 5000, 4)  # a longer last chunk
