"""The general-rank planners (t4a_plan_*_any over WideLayout), CPU only.

At rank <= 8 each must return the by-value planner's geometry (variant FAST);
past rank 8 the variant is GENERAL (reference RankVariant::select,
src/lib.rs:817-838) and validation follows the same order and errors
(reference LayoutRef::new and the planners, src/lib.rs:908-928, 1628-1679,
3193-3557). Extent-1 axes and chained axes fuse away, so a wide layout that
fuses to at most eight axes gets the narrow layout's movement geometry.
"""
import itertools
import random

import pytest

import t4a_cuda_kernels as t
from t4a_cuda_kernels import DType, Error, Layout, ReduceOp, ReduceStrategy, T4aError, WideLayout

F32, F64 = DType.F32, DType.F64


def err(fn, *args):
    with pytest.raises(T4aError) as e:
        fn(*args)
    return e.value.error


def permuted(extents, order):
    """Strides of a compact layout whose axes are laid out in `order` (the
    first listed axis fastest)."""
    strides = [0] * len(extents)
    s = 1
    for k in order:
        strides[k] = s
        s *= extents[k]
    return strides


def launch_tuple(l):
    return (tuple(l.grid), tuple(l.block), l.shared_bytes)


def test_wide_layout_validation_and_pack():
    assert err(WideLayout, [2, 3], [1]) == Error.RankLength
    assert err(WideLayout, [2, -1], [1, 2]) == Error.NegativeExtent
    w = WideLayout.compact([2, 3, 4])
    assert w.strides == [1, 2, 6] and w.pack() == [2, 3, 4, 1, 2, 6]
    assert WideLayout.compact([1] * 20).element_count() == 1
    assert err(WideLayout.compact, [2**40, 2**40]) == Error.Overflow


def test_movement_geometry_matches_the_by_value_planner_up_to_rank_eight():
    rng = random.Random(5)
    for rank in range(0, 9):
        for _ in range(6):
            ext = [rng.randint(1, 6) for _ in range(rank)]
            order = list(range(rank))
            rng.shuffle(order)
            st = permuted(ext, order)
            n = 1
            for e in ext:
                n *= e
            for dt in (F32, F64, DType.C64, DType.Bool):
                fast = t.plan_materialize_strided(dt, Layout(ext, st), n)
                wide = t.plan_materialize_strided(dt, WideLayout(ext, st), n)
                assert launch_tuple(fast) == launch_tuple(wide), (ext, st, dt)
                assert wide.variant == t.RankVariant.Fast
                dst = Layout.compact(ext)
                fast = t.plan_strided_to_strided(dt, Layout(ext, st), n, dst, n)
                wide = t.plan_strided_to_strided(dt, WideLayout(ext, st), n, WideLayout.of(dst), n)
                assert launch_tuple(fast) == launch_tuple(wide)


def test_wide_movement_variant_and_fused_geometry():
    # rank 12 with extent-1 axes: fuses to the rank-3 permute of the same data
    ext8 = [16, 8, 32]
    st8 = permuted(ext8, [2, 0, 1])
    ext, st = [], []
    for e, s in zip(ext8, st8):
        ext += [e, 1, 1, 1]
        st += [s, 7, 0, 123]
    n = 16 * 8 * 32
    wide = t.plan_materialize_strided(F64, WideLayout(ext, st), n)
    fast = t.plan_materialize_strided(F64, Layout(ext8, st8), n)
    assert wide.variant == t.RankVariant.General
    assert launch_tuple(wide) == launch_tuple(fast)
    # eleven axes of extent 2, scrambled: nothing fuses, a flat geometry
    ext = [2] * 11
    st = permuted(ext, [3, 9, 0, 6, 1, 10, 4, 7, 2, 8, 5])
    l = t.plan_materialize_strided(F32, WideLayout(ext, st), 2**11)
    assert l.variant == t.RankVariant.General and l.grid[0] >= 1 and l.block[0] == 256


def test_wide_movement_errors():
    ext = [2] * 10
    st = permuted(ext, list(range(10)))
    w = WideLayout(ext, st)
    assert err(t.plan_materialize_strided, DType.F32, w, 2**10 - 1) == Error.OffsetOutOfSpan
    assert err(t.plan_materialize_strided, DType.F32, w, -1) == Error.NegativeCount
    assert err(t.plan_strided_to_strided, DType.F32, w, 2**10,
               WideLayout(ext[:9], st[:9]), 2**10) == Error.CountMismatch
    bcast = WideLayout(ext, st[:9] + [0])
    assert err(t.plan_strided_to_strided, DType.F32, w, 2**10, bcast,
               2**10) == Error.BroadcastDestination
    assert t.plan_materialize_strided(DType.F32, WideLayout([3] * 9 + [0], [1] * 10), 0).is_empty()


def reduce_pair(ext, axis, wide):
    out_ext = list(ext)
    out_ext[axis] = 1
    mk = WideLayout.compact if wide else Layout.compact
    return mk(out_ext), mk(ext)


def test_reduction_plans_match_the_by_value_planner_up_to_rank_eight():
    for rank in range(1, 9):
        for axis in range(rank):
            for L in (3, 40, 6000):
                ext = [2 + (k % 3) for k in range(rank)]
                ext[axis] = L
                n = 1
                for e in ext:
                    n *= e
                on = n // L
                fo, fi = reduce_pair(ext, axis, False)
                wo, wi = reduce_pair(ext, axis, True)
                for op in (ReduceOp.Sum, ReduceOp.Max):
                    fp = t.plan_reduction(F32, op, fo, on, fi, n, axis, 32)
                    wp = t.plan_reduction(F32, op, wo, on, wi, n, axis, 32)
                    assert fp.kind == wp.kind
                    if fp.kind == "Direct":
                        assert launch_tuple(fp.launch) == launch_tuple(wp.launch)
                        assert fp.strategy == wp.strategy
                    else:
                        assert fp.split == wp.split
                        assert launch_tuple(fp.pass1) == launch_tuple(wp.pass1)
                        assert launch_tuple(fp.pass2) == launch_tuple(wp.pass2)
                        assert (fp.combine_strategy, fp.combine_op) == (wp.combine_strategy,
                                                                        wp.combine_op)
                fpl = t.reduction_partials_layout(fi, axis, 4)
                wpl = t.reduction_partials_layout(wi, axis, 4)
                assert fpl.extents == wpl.extents and fpl.strides == wpl.strides


def test_rank_nine_split_plan_and_variants():
    # the reference's rank-9 wide-combine case (tests/gpu_dynamic_rank.rs:2880-2960)
    ext = [2, 131072] + [1] * 7
    wo, wi = reduce_pair(ext, 1, True)
    p = t.plan_reduction(F32, ReduceOp.Max, wo, 2, wi, 2 * 131072, 1, 32)
    assert p.kind == "Split" and p.split.splits == 512
    assert p.combine_strategy == ReduceStrategy.Plane and p.pass2.block[0] >= 64
    assert p.pass1.variant == t.RankVariant.General and p.pass2.variant == t.RankVariant.General
    pl = t.reduction_partials_layout(wi, 1, 512)
    assert pl.extents == [2, 512] + [1] * 7 and pl.strides[:3] == [1, 2, 1024]
    # the same plan as the rank-2 layout it fuses to
    fo, fi = reduce_pair([2, 131072], 1, False)
    q = t.plan_reduction(F32, ReduceOp.Max, fo, 2, fi, 2 * 131072, 1, 32)
    assert q.split == p.split
    assert launch_tuple(q.pass1) == launch_tuple(p.pass1)
    assert launch_tuple(q.pass2) == launch_tuple(p.pass2)


def test_wide_reduction_errors():
    ext = [3] * 10
    wo, wi = reduce_pair(ext, 4, True)
    on, n = 3**9, 3**10
    assert err(t.plan_reduce, F32, ReduceOp.Sum, ReduceStrategy.Unit, wo, on, wi, n, 10,
               32) == Error.InvalidAxis
    assert err(t.plan_reduce, F32, ReduceOp.Sum, ReduceStrategy.Unit, WideLayout.compact([3] * 9),
               on, wi, n, 4, 32) == Error.RankLength
    bad = WideLayout.compact([3] * 4 + [2] + [3] * 5)
    assert err(t.plan_reduce, F32, ReduceOp.Sum, ReduceStrategy.Unit, bad, on, wi, n, 4,
               32) == Error.ShapeMismatch
    assert err(t.plan_reduce, F32, ReduceOp.Sum, ReduceStrategy.Plane, wo, on, wi, n, 4,
               32) == Error.StrategyMismatch
    assert err(t.plan_reduce, DType.Bool, ReduceOp.Sum, ReduceStrategy.Unit, wo, on, wi, n, 4,
               32) == Error.UnsupportedDType
    assert err(t.plan_reduce, F32, ReduceOp.Sum, ReduceStrategy.Unit, wo, on, wi, n - 1, 4,
               32) == Error.OffsetOutOfSpan
    l = t.plan_reduce(F32, ReduceOp.Sum, ReduceStrategy.Unit, wo, on, wi, n, 4, 32)
    assert l.variant == t.RankVariant.General and not l.is_empty()


@pytest.mark.parametrize("rank", [9, 12, 16])
def test_wide_unfused_reduction_geometry(rank):
    """Non-axis dims that do not fuse (more than seven left): UNIT, PLANE and
    pass-1 plans still come back, for the general twins' decode."""
    ext = [2] * rank
    axis = 3
    order = list(range(rank))
    random.Random(rank).shuffle(order)
    st = permuted(ext, order)
    out_ext = list(ext)
    out_ext[axis] = 1
    out_st = [s if k != axis else 0 for k, s in enumerate(permuted(out_ext, order))]
    wi = WideLayout(ext, st)
    wo = WideLayout(out_ext, out_st)
    n = 2**rank
    l = t.plan_reduce(F32, ReduceOp.Sum, ReduceStrategy.Unit, wo, wo.max_reachable_offset() + 1,
                      wi, n, axis, 32)
    assert l.variant == t.RankVariant.General and l.grid[0] >= 1
    ext[axis] = 64 * 8
    st = permuted(ext, order)
    wi = WideLayout(ext, st)
    p = t.plan_reduction(F32, ReduceOp.Sum, wo, wo.max_reachable_offset() + 1, wi,
                         wi.max_reachable_offset() + 1, axis, 32)
    assert p.kind == "Split" and p.pass1.grid[0] >= 1 and p.pass1.block[0] == 256
