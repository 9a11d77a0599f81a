"""Planners of fill_zero, fill_zero_view, contiguous_to_view, broadcast_in_dim
and concatenate_copy (and their general-rank twins), CPU only.

Validation order and errors follow the reference planners
(src/lib.rs:1484-1589 broadcast_in_dim / concatenate_copy, 1591-1658
fill_zero / fill_zero_view / contiguous_to_view) and the reference's own
planning tests (tests/planning.rs:43-52 rank-0 view, 80-102 broadcast
destination and fill_zero counts, 113-121 span, 3104-3196 rank maps and
axis offsets). Grid sizes are this build's own (one 16-byte vector per thread
where the view allows it); the tests pin what the launch covers, not the
reference's 256-element blocks.
"""
import random

import pytest

import t4a_cuda_kernels as t
from t4a_cuda_kernels import DType, Error, Layout, RankVariant, T4aError, WideLayout

F32, F64, C64 = DType.F32, DType.F64, DType.C64
ALL_DTYPES = list(DType)


def err(fn, *args):
    with pytest.raises(T4aError) as e:
        fn(*args)
    return e.value.error


def launch_tuple(l):
    return (tuple(l.grid), tuple(l.block), l.shared_bytes)


def threads(l):
    return l.grid[0] * l.grid[1] * l.grid[2] * l.block[0] * l.block[1] * l.block[2]


# ---------------------------------------------------------------- fill_zero

def test_fill_zero_counts_and_refusals():
    # tests/planning.rs:95-102, 105-111
    assert t.plan_fill_zero(F32, 0).is_empty()
    for n in (1, 256, 257, 1_000_000):
        for dt in ALL_DTYPES:
            l = t.plan_fill_zero(dt, n)
            assert l.variant == RankVariant.Fast
            # Every element is owned by some thread: a 16-byte vector each.
            per_thread = max(1, 16 // dt.size)
            assert threads(l) * per_thread >= n
    assert err(t.plan_fill_zero, F32, -1) == Error.NegativeCount
    # The flat launch limit (2^31 - 1 blocks of the flat block) is refused the
    # way copy_exact refuses it.
    huge = (2**31 - 1) * 256 * 64 + 1
    assert err(t.plan_fill_zero, DType.Bool, huge) == err(t.plan_copy_exact, DType.Bool, huge)
    assert err(t.plan_fill_zero, 99, 4) == Error.UnsupportedDType


# ---------------------------------------------------------- fill_zero_view

def test_fill_zero_view_rank_zero_and_span():
    # tests/planning.rs:43-52: a rank-0 view at offset 7 in an 8-element span.
    scalar = Layout([], [], 7)
    l = t.plan_fill_zero_view(F64, scalar, 8)
    assert tuple(l.grid) == (1, 1, 1)
    assert err(t.plan_fill_zero_view, F64, scalar, 7) == Error.OffsetOutOfSpan
    # tests/planning.rs:113-131: three elements spaced by two.
    spaced = Layout([3], [2], 0)
    assert tuple(t.plan_fill_zero_view(F32, spaced, 5).grid) == (1, 1, 1)
    assert err(t.plan_fill_zero_view, F32, spaced, 4) == Error.OffsetOutOfSpan
    negative = Layout([3], [-1], 1)
    assert err(t.plan_fill_zero_view, F32, negative, 8) == Error.OffsetOutOfSpan
    # An empty view plans an empty launch but still validates the dtype.
    assert t.plan_fill_zero_view(F32, Layout([0, 3], [1, 1], 0), 0).is_empty()
    assert err(t.plan_fill_zero_view, 99, spaced, 5) == Error.UnsupportedDType


def test_fill_zero_view_refuses_broadcast_destinations():
    # tests/planning.rs:80-91: stride 0 on an axis of extent > 1 is no destination.
    bc = Layout([3, 4], [1, 0], 0)
    assert err(t.plan_fill_zero_view, F32, bc, 12) == Error.BroadcastDestination
    assert err(t.plan_contiguous_to_view, F32, bc, 12) == Error.BroadcastDestination
    # Extent 1 with stride 0 is fine.
    ok = Layout([3, 1], [1, 0], 0)
    assert not t.plan_fill_zero_view(F32, ok, 3).is_empty()
    assert not t.plan_contiguous_to_view(F32, ok, 3).is_empty()


def test_fill_zero_view_covers_the_logical_count():
    rng = random.Random(11)
    for _ in range(60):
        rank = rng.randint(1, 5)
        ext = [rng.randint(1, 40) for _ in range(rank)]
        gaps = [rng.randint(1, 3) for _ in range(rank)]
        st, s = [], 1
        for e, g in zip(ext, gaps):
            st.append(s * g)
            s *= e * g
        layout = Layout(ext, st, rng.randint(0, 5))
        n = layout.element_count()
        span = layout.max_reachable_offset() + 1
        for dt in (DType.Bool, F32, F64, C64):
            l = t.plan_fill_zero_view(dt, layout, span)
            assert l.variant == RankVariant.Fast
            assert 0 < threads(l)
            # A thread per element, or per 16-byte vector of the stride-1 axis.
            per = 1 if dt.size in (1, 2, 16) else 16 // dt.size
            assert threads(l) * per >= n


# ------------------------------------------------------- contiguous_to_view

def test_contiguous_to_view_validation():
    v = Layout([3, 4], [4, 1], 0)  # a transposed view of a 12-element buffer
    assert not t.plan_contiguous_to_view(F64, v, 12).is_empty()
    assert err(t.plan_contiguous_to_view, F64, v, 11) == Error.OffsetOutOfSpan
    assert err(t.plan_contiguous_to_view, 77, v, 12) == Error.UnsupportedDType
    assert t.plan_contiguous_to_view(F64, Layout([0], [1], 0), 0).is_empty()
    # A reversed destination (tests/gpu_remaining_families.rs:822-870).
    rev = Layout([3, 5, 2, 4], [-1, 3, -15, -30], 2 + 15 + 90)
    assert rev.min_reachable_offset() == 0
    assert not t.plan_contiguous_to_view(F64, rev, 120).is_empty()


# ----------------------------------------------------------- broadcast_in_dim

def test_broadcast_in_dim_rank_map_errors():
    # tests/planning.rs:3104-3153
    out = Layout.compact([2, 3])
    inp = Layout.compact([2])
    assert t.plan_broadcast_in_dim(F64, out, 6, inp, 2, [0]).variant == RankVariant.Fast
    assert err(t.plan_broadcast_in_dim, F64, out, 6, inp, 2, [2]) == Error.InvalidAxis
    assert err(t.plan_broadcast_in_dim, F64, out, 6, inp, 2, [-1]) == Error.InvalidAxis
    inp2 = Layout.compact([2, 2])
    assert err(t.plan_broadcast_in_dim, F64, out, 6, inp2, 4, [0, 0]) == Error.DuplicateAxis
    assert err(t.plan_broadcast_in_dim, F64, out, 6, inp, 2, [1]) == Error.ShapeMismatch
    inp3 = Layout.compact([3])
    assert not t.plan_broadcast_in_dim(F64, out, 6, inp3, 3, [1]).is_empty()
    assert err(t.plan_broadcast_in_dim, F64, out, 6, inp2, 4, [0]) == Error.RankLength
    scalar = Layout.compact([])
    assert not t.plan_broadcast_in_dim(F64, out, 6, scalar, 1, []).is_empty()
    # The destination must be compact and not a broadcast.
    strided = Layout([2, 3], [1, 3], 0)
    assert err(t.plan_broadcast_in_dim, F64, strided, 9, inp, 2, [0]) == Error.NotCompact
    shifted = Layout([2, 3], [1, 2], 1)
    assert err(t.plan_broadcast_in_dim, F64, shifted, 7, inp, 2, [0]) == Error.NotCompact
    # Spans: the input is checked before the destination.
    assert err(t.plan_broadcast_in_dim, F64, out, 6, inp, 1, [0]) == Error.OffsetOutOfSpan
    assert err(t.plan_broadcast_in_dim, F64, out, 5, inp, 2, [0]) == Error.OffsetOutOfSpan
    # A strided (non-compact) input is a read and is fine
    # (tests/gpu_remaining_families.rs:620-660).
    src = Layout([2, 3], [1, 5], 0)
    assert not t.plan_broadcast_in_dim(F64, out, 6, src, 12, [0, 1]).is_empty()
    assert err(t.plan_broadcast_in_dim, 42, out, 6, inp, 2, [0]) == Error.UnsupportedDType
    # More than eight dims cannot travel by value.
    assert err(t.axis_values, list(range(9))) == Error.RankLength


def test_broadcast_in_dim_general_rank_and_overflow():
    wide_out = WideLayout.compact([2] * 9)
    wide_in = WideLayout.compact([2] * 9)
    n = wide_out.element_count()
    l = t.plan_broadcast_in_dim(F64, wide_out, n, wide_in, n, list(range(9)))
    assert l.variant == RankVariant.General
    huge = WideLayout([1 << 40, 1 << 40], [1, 1 << 40], 0)
    huge_in = WideLayout.compact([1, 1])
    assert err(t.plan_broadcast_in_dim, F64, huge, 1, huge_in, 1, [0, 1]) in (
        Error.Overflow, Error.NotCompact)
    # Rank 16 with two broadcast input axes (tests/gpu_remaining_families.rs:352-370).
    ext = [2 + k % 2 for k in range(16)]
    ie = list(ext)
    ie[1] = ie[15] = 1
    out = WideLayout.compact(ext)
    inp = WideLayout.compact(ie)
    l = t.plan_broadcast_in_dim(F64, out, out.element_count(), inp, inp.element_count(),
                                list(range(16)))
    assert l.variant == RankVariant.General and not l.is_empty()


def test_broadcast_in_dim_any_agrees_with_the_by_value_planner():
    rng = random.Random(3)
    for _ in range(80):
        out_rank = rng.randint(0, 6)
        out_ext = [rng.randint(1, 5) for _ in range(out_rank)]
        in_rank = rng.randint(0, out_rank)
        dims = rng.sample(range(out_rank), in_rank)
        in_ext = [out_ext[d] if rng.random() < 0.7 else 1 for d in dims]
        out = Layout.compact(out_ext)
        inp = Layout.compact(in_ext)
        on, inn = out.element_count(), inp.element_count()
        for dt in (F32, F64, C64):
            a = t.plan_broadcast_in_dim(dt, out, on, inp, inn, dims)
            b = t.plan_broadcast_in_dim(dt, WideLayout.of(out), on, WideLayout.of(inp), inn,
                                        dims)
            assert launch_tuple(a) == launch_tuple(b)
            assert a.variant == b.variant == RankVariant.Fast


# ---------------------------------------------------------- concatenate_copy

def test_concatenate_copy_axis_offset_errors():
    # tests/planning.rs:3155-3196
    out = Layout.compact([2, 5])
    inp = Layout.compact([2, 3])
    assert t.plan_concatenate_copy(F64, out, 10, inp, 6, 1, 2).variant == RankVariant.Fast
    assert err(t.plan_concatenate_copy, F64, out, 10, inp, 6, 1, 3) == Error.ShapeMismatch
    assert err(t.plan_concatenate_copy, F64, out, 10, inp, 6, 1, -1) == Error.NegativeCount
    assert err(t.plan_concatenate_copy, F64, out, 10, inp, 6, 2, 0) == Error.InvalidAxis
    other = Layout.compact([3, 3])
    assert err(t.plan_concatenate_copy, F64, out, 10, other, 9, 1, 0) == Error.ShapeMismatch
    assert err(t.plan_concatenate_copy, F64, out, 10, Layout.compact([2]), 2, 0, 0) == \
        Error.RankLength
    # The input must be compact; the destination may be any injective view.
    assert err(t.plan_concatenate_copy, F64, out, 10, Layout([2, 3], [3, 1], 0), 6, 1, 0) == \
        Error.NotCompact
    strided = Layout([2, 4, 2], [1, 3, 12], 0)
    assert not t.plan_concatenate_copy(F64, strided, 23, Layout.compact([2, 2, 2]), 8, 1,
                                       1).is_empty()
    assert err(t.plan_concatenate_copy, F64, strided, 22, Layout.compact([2, 2, 2]), 8, 1,
               1) == Error.OffsetOutOfSpan
    bc = Layout([2, 5], [1, 0], 0)
    assert err(t.plan_concatenate_copy, F64, bc, 10, inp, 6, 1, 0) == Error.BroadcastDestination
    # Spans: the input before the destination.
    assert err(t.plan_concatenate_copy, F64, out, 10, inp, 5, 1, 0) == Error.OffsetOutOfSpan
    assert err(t.plan_concatenate_copy, F64, out, 9, inp, 6, 1, 0) == Error.OffsetOutOfSpan
    assert err(t.plan_concatenate_copy, 13, out, 10, inp, 6, 1, 0) == Error.UnsupportedDType


def test_concatenate_copy_general_rank_and_overflow():
    wide_out = WideLayout.compact([2] * 16)
    wide_in = WideLayout.compact([2] * 16)
    n = wide_in.element_count()
    l = t.plan_concatenate_copy(F64, wide_out, wide_out.element_count(), wide_in, n, 3, 0)
    assert l.variant == RankVariant.General
    big = 2**63 - 1
    edge = WideLayout([big // 2, 2], [1, big // 2], 0)
    assert err(t.plan_concatenate_copy, F64, edge, 1, edge, 1, 0, 1) in (
        Error.Overflow, Error.ShapeMismatch, Error.NotCompact)
    # The shifted end itself overflows.
    out = WideLayout([4], [1], 0)
    inp = WideLayout.compact([2])
    assert err(t.plan_concatenate_copy, F64, out, 4, inp, 2, 0, big) in (
        Error.Overflow, Error.ShapeMismatch)


def test_concatenate_copy_any_agrees_with_the_by_value_planner():
    rng = random.Random(9)
    for _ in range(80):
        rank = rng.randint(1, 6)
        in_ext = [rng.randint(1, 5) for _ in range(rank)]
        axis = rng.randrange(rank)
        out_ext = list(in_ext)
        out_ext[axis] += rng.randint(0, 4)
        off = rng.randint(0, out_ext[axis] - in_ext[axis])
        out = Layout.compact(out_ext)
        inp = Layout.compact(in_ext)
        for dt in (F32, F64):
            a = t.plan_concatenate_copy(dt, out, out.element_count(), inp, inp.element_count(),
                                        axis, off)
            b = t.plan_concatenate_copy(dt, WideLayout.of(out), out.element_count(),
                                        WideLayout.of(inp), inp.element_count(), axis, off)
            assert launch_tuple(a) == launch_tuple(b)


def test_view_entries_any_agree_with_the_by_value_planners():
    rng = random.Random(17)
    for _ in range(60):
        rank = rng.randint(0, 8)
        ext = [rng.randint(1, 4) for _ in range(rank)]
        order = list(range(rank))
        rng.shuffle(order)
        st = [0] * rank
        s = 1
        for k in order:
            st[k] = s
            s *= ext[k]
        neg = [k for k in range(rank) if rng.random() < 0.3]
        off = 0
        for k in neg:
            off += (ext[k] - 1) * st[k]
            st[k] = -st[k]
        layout = Layout(ext, st, off)
        span = layout.max_reachable_offset() + 1
        for dt in (F32, F64, C64, DType.Bool):
            for plan in (t.plan_fill_zero_view, t.plan_contiguous_to_view):
                a = plan(dt, layout, span)
                b = plan(dt, WideLayout.of(layout), span)
                assert launch_tuple(a) == launch_tuple(b)
                assert a.variant == b.variant == RankVariant.Fast
    w = WideLayout.compact([2] * 10)
    for plan in (t.plan_fill_zero_view, t.plan_contiguous_to_view):
        assert plan(F32, w, 1024).variant == RankVariant.General
        assert err(plan, F32, w, 1023) == Error.OffsetOutOfSpan
