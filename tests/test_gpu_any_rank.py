"""The general-rank `_any` twins on the GPU (reference tests/gpu_dynamic_rank.rs:
114-210, 316-414, 1190-1336, 2880-3214): geometry arrays in device memory.

- up to rank 8 the twins return the by-value entries' bytes, under the
  by-value planner's geometry;
- at rank 9 and 16 (extent-1 and chained axes fuse away) they match a CPU
  gather and a CPU fold in the reference's order;
- layouts that stay wider than eight axes after fusion (scrambled extent-2
  axes) take the LDS-resident decode, checked the same way;
- the reference's rank-9 split Max reaches every partial through the wide
  combine, and a rank-9 split gives the bytes of the rank-2 layout it fuses to.
"""
import random

import numpy as np
import pytest

import t4a_cuda_kernels as t
from t4a_cuda_kernels import DType, Layout, ReduceOp, ReduceStrategy, WideLayout, hip, hipmem
from gpu_util import NUMPY, random_elements, say, sentinel, stream, to_device, to_host
from oracle import t4a_oracle as orc

pytestmark = pytest.mark.gpu

F32, F64 = DType.F32, DType.F64


def permuted(extents, order):
    strides = [0] * len(extents)
    s = 1
    for k in order:
        strides[k] = s
        s *= extents[k]
    return strides


class Geometry:
    """A WideLayout's arrays copied to the device, and its device struct."""

    def __init__(self, w: WideLayout):
        self.ext = to_device(np.array(w.extents or [0], dtype=np.int64))
        self.st = to_device(np.array(w.strides or [0], dtype=np.int64))
        self.c = w.device_c(self.ext.ptr, self.st.ptr)


def view_indices(ext, st, offset=0):
    """Element offsets of a view in flat logical order (axis 0 fastest)."""
    idx = np.array([offset], dtype=np.int64)
    for k in reversed(range(len(ext))):
        idx = (idx[:, None] + np.arange(ext[k], dtype=np.int64)[None, :] * st[k]).ravel()
    return idx


def count(ext):
    n = 1
    for e in ext:
        n *= e
    return n


def test_movement_twins_agree_up_to_rank_eight():
    rng = np.random.default_rng(50)
    for rank in range(2, 9):
        ext = [2 + k % 3 for k in range(rank)]
        n = count(ext)
        st = permuted(ext, list(reversed(range(rank))))
        src = random_elements(F64, n, rng)
        d_src = to_device(src)
        fast_l, wide = Layout(ext, st), WideLayout(ext, st)
        g = Geometry(wide)
        plan = t.plan_materialize_strided(F64, fast_l, n)
        say("materialize twins rank", rank, "plan", plan.grid, plan.block)
        a, b = sentinel(n * 8), sentinel(n * 8)
        hip.materialize_strided(a, d_src, F64, fast_l, n, plan, stream())
        hip.materialize_strided_any(b, d_src, F64, g.c, n, plan, stream())
        want = np.zeros(n, dtype=np.float64)
        orc.materialize_strided(want, src, F64, fast_l, n)
        ga, gb = to_host(a, n * 8), to_host(b, n * 8)
        assert np.array_equal(ga, want.view(np.uint8)), rank
        assert np.array_equal(gb, want.view(np.uint8)), rank
        # strided_to_strided with the first and last axes swapped on the destination
        order = list(reversed(range(rank)))
        order[0], order[-1] = order[-1], order[0]
        dst_st = permuted(ext, order)
        dst_fast, dst_wide = Layout(ext, dst_st), WideLayout(ext, dst_st)
        gd = Geometry(dst_wide)
        plan = t.plan_strided_to_strided(F64, fast_l, n, dst_fast, n)
        a, b = sentinel(n * 8), sentinel(n * 8)
        hip.strided_to_strided(a, d_src, F64, fast_l, dst_fast, n, plan, stream())
        hip.strided_to_strided_any(b, d_src, F64, g.c, gd.c, n, plan, stream())
        assert np.array_equal(to_host(a, n * 8), to_host(b, n * 8)), rank


@pytest.mark.parametrize("dtype", [F64, DType.C64, DType.Bool], ids=lambda d: d.name)
def test_rank_nine_and_sixteen_match_a_cpu_gather(dtype):
    rng = np.random.default_rng(51)
    for rank in (9, 16):
        ext = [2 + k % 3 for k in range(rank)]
        n = count(ext)
        if dtype != F64 and rank == 16:
            continue
        st = permuted(ext, list(reversed(range(rank))))
        wide = WideLayout(ext, st)
        src = random_elements(dtype, n, rng)
        plan = t.plan_materialize_strided(dtype, wide, n)
        assert plan.variant == t.RankVariant.General
        g = Geometry(wide)
        say("materialize_any rank", rank, dtype.name, "len", n, "plan", plan.grid)
        d = sentinel(n * dtype.size)
        hip.materialize_strided_any(d, to_device(src), dtype, g.c, n, plan, stream())
        want = np.ascontiguousarray(src[view_indices(ext, st)])
        assert np.array_equal(to_host(d, n * dtype.size), want.view(np.uint8)), rank


@pytest.mark.parametrize("rank", [9, 11, 13])
def test_layouts_wider_than_eight_after_fusion(rank):
    """Extent-2 axes in a scrambled order fuse nowhere: the per-element
    decode over LDS-resident axes, for materialize and strided_to_strided."""
    rng = np.random.default_rng(52 + rank)
    ext = [2] * rank
    order = list(range(rank))
    random.Random(rank).shuffle(order)
    st = permuted(ext, order)
    n = 2**rank
    src = random_elements(F32, n, rng)
    wide = WideLayout(ext, st, 3)
    plan = t.plan_materialize_strided(F32, wide, n + 3)
    g = Geometry(wide)
    say("wide materialize rank", rank, "plan", plan.grid)
    d_src = to_device(np.concatenate([np.zeros(3, np.float32), src]))
    d = sentinel(n * 4)
    hip.materialize_strided_any(d, d_src, F32, g.c, n, plan, stream())
    full = np.concatenate([np.zeros(3, np.float32), src])
    assert np.array_equal(to_host(d, n * 4), full[view_indices(ext, st, 3)].view(np.uint8))
    # into a second scrambled destination
    order2 = list(range(rank))
    random.Random(rank + 100).shuffle(order2)
    dst_st = permuted(ext, order2)
    dst = WideLayout(ext, dst_st)
    gd = Geometry(dst)
    plan = t.plan_strided_to_strided(F32, wide, n + 3, dst, n)
    d = sentinel(n * 4)
    hip.strided_to_strided_any(d, d_src, F32, g.c, gd.c, n, plan, stream())
    want = np.zeros(n, np.float32)
    want[view_indices(ext, dst_st)] = full[view_indices(ext, st, 3)]
    assert np.array_equal(to_host(d, n * 4), want.view(np.uint8))


def serial_sum(x):
    """The unit fold: element 0 seeds, the rest join in axis order (float64)."""
    acc = x[:, 0].copy()
    for i in range(1, x.shape[1]):
        acc = acc + x[:, i]
    return acc


def plane_sum(x, w=32):
    """The plane fold: lane t seeds element t and folds t + w, t + 2w, ...;
    then the own-left xor tree over the w lanes."""
    outs, L = x.shape
    acc = np.empty((outs, w))
    for lane in range(w):
        a = x[:, lane].copy()
        for i in range(lane + w, L, w):
            a = a + x[:, i]
        acc[:, lane] = a
    off = 1
    while off < w:
        acc = acc + acc[:, np.arange(w) ^ off]
        off *= 2
    return acc[:, 0]


def axis_rows(src, ext, st, axis, offset=0):
    """[outputs, axis_len] of the input's values, outputs in flat order."""
    out_ext = list(ext)
    out_ext[axis] = 1
    base = view_indices(out_ext, st, offset)
    return src[base[:, None] + np.arange(ext[axis])[None, :] * st[axis]]


def test_reduction_twins_agree_up_to_rank_eight():
    rng = np.random.default_rng(53)
    for rank in range(2, 9):
        ext = [3 + k % 2 for k in range(rank)]
        axis = rank // 2
        n = count(ext)
        src = rng.standard_normal(n)
        d_src = to_device(src)
        out_ext = list(ext)
        out_ext[axis] = 1
        on = n // ext[axis]
        fo, fi = Layout.compact(out_ext), Layout.compact(ext)
        go, gi = Geometry(WideLayout.compact(out_ext)), Geometry(WideLayout.compact(ext))
        for strategy, w in ((ReduceStrategy.Unit, 32), (ReduceStrategy.Plane, 8)):
            if strategy == ReduceStrategy.Plane and ext[axis] < w:
                continue
            plan = t.plan_reduce(F64, ReduceOp.Sum, strategy, fo, on, fi, n, axis, w)
            say("reduce twins rank", rank, strategy.name)
            a, b = sentinel(on * 8), sentinel(on * 8)
            hip.reduce(a, d_src, F64, ReduceOp.Sum, strategy, fo, fi, axis, on, plan, stream())
            hip.reduce_any(b, d_src, F64, ReduceOp.Sum, strategy, go.c, gi.c, axis, on, plan,
                           stream())
            assert np.array_equal(to_host(a, on * 8), to_host(b, on * 8)), (rank, strategy)
        # pass 1 with the axis splits x 32 long
        lext = [2 + k % 2 for k in range(rank)]
        splits = 3
        lext[axis] = splits * 32
        ln = count(lext)
        lsrc = rng.standard_normal(ln)
        li = Layout.compact(lext)
        pl = t.reduction_partials_layout(li, axis, splits)
        pn = pl.element_count()
        lon = ln // lext[axis]
        split = t.Split(splits, lext[axis] // splits)
        plan = t.plan_reduce_partials(F64, ReduceOp.Sum, pl, pn, li, ln, axis, split, 32)
        gpl, gli = Geometry(WideLayout.of(pl)), Geometry(WideLayout.of(li))
        d_l = to_device(lsrc)
        a, b = sentinel(pn * 8), sentinel(pn * 8)
        say("partials twins rank", rank)
        hip.reduce_partials(a, d_l, F64, ReduceOp.Sum, pl, li, axis, lon, splits,
                            split.chunk_len, plan, stream())
        hip.reduce_partials_any(b, d_l, F64, ReduceOp.Sum, gpl.c, gli.c, axis, lon, splits,
                                split.chunk_len, plan, stream())
        want = np.zeros(pn)
        orc.reduce_partials(want, lsrc, F64, ReduceOp.Sum, 32, pl, li, axis, lon, splits,
                            split.chunk_len)
        assert np.array_equal(to_host(a, pn * 8), want.view(np.uint8)), rank
        assert np.array_equal(to_host(b, pn * 8), want.view(np.uint8)), rank


@pytest.mark.parametrize("rank", [9, 16])
def test_rank_nine_and_sixteen_reduce_match_the_cpu_fold(rank):
    ext = [2 + k % 3 for k in range(rank)]
    axis = 4
    n = count(ext)
    st = permuted(ext, list(range(rank)))
    src = (np.arange(n, dtype=np.float64) + 0.5)
    out_ext = list(ext)
    out_ext[axis] = 1
    wo, wi = WideLayout.compact(out_ext), WideLayout.compact(ext)
    on = n // ext[axis]
    plan = t.plan_reduce(F64, ReduceOp.Sum, ReduceStrategy.Unit, wo, on, wi, n, axis, 32)
    assert plan.variant == t.RankVariant.General
    go, gi = Geometry(wo), Geometry(wi)
    say("reduce_any rank", rank, "outputs", on)
    d = sentinel(on * 8)
    hip.reduce_any(d, to_device(src), F64, ReduceOp.Sum, ReduceStrategy.Unit, go.c, gi.c, axis,
                   on, plan, stream())
    want = serial_sum(axis_rows(src, ext, st, axis))
    assert np.array_equal(to_host(d, on * 8), want.view(np.uint8))


@pytest.mark.parametrize("rank", [10, 12])
def test_reductions_wider_than_eight_after_fusion(rank):
    """Non-axis extent-2 axes in a scrambled order (none fuse) around a
    strided axis: UNIT and PLANE reduce_any and pass 1 against CPU folds in
    the reference topology, and Max exactly."""
    rng = np.random.default_rng(54 + rank)
    axis = 2
    order = list(range(rank))
    random.Random(rank).shuffle(order)
    if order[0] == axis:
        order[0], order[1] = order[1], order[0]
    for L, strategy, w in ((5, ReduceStrategy.Unit, 32), (80, ReduceStrategy.Plane, 32)):
        ext = [2] * rank
        ext[axis] = L
        st = permuted(ext, order)
        n = count(ext)
        src = rng.standard_normal(n)
        out_ext = list(ext)
        out_ext[axis] = 1
        out_st = permuted(out_ext, order)
        wi, wo = WideLayout(ext, st), WideLayout(out_ext, out_st)
        on = n // L
        gi, go = Geometry(wi), Geometry(wo)
        rows = axis_rows(src, ext, st, axis)
        out_pos = view_indices(out_ext, out_st)
        for op in (ReduceOp.Sum, ReduceOp.Max):
            plan = t.plan_reduce(F64, op, strategy, wo, on, wi, n, axis, w)
            say("wide reduce rank", rank, strategy.name, op.name)
            d = sentinel(on * 8)
            hip.reduce_any(d, to_device(src), F64, op, strategy, go.c, gi.c, axis, on, plan,
                           stream())
            got = to_host(d, on * 8).view(np.float64)
            fold = rows.max(axis=1) if op == ReduceOp.Max else (
                serial_sum(rows) if strategy == ReduceStrategy.Unit else plane_sum(rows, w))
            want = np.zeros(on)
            want[out_pos] = fold
            assert np.array_equal(got, want), (rank, strategy, op)
    # pass 1: 4 splits of 64 along the strided axis
    ext = [2] * rank
    ext[axis] = 256
    st = permuted(ext, order)
    n = count(ext)
    src = rng.standard_normal(n)
    wi = WideLayout(ext, st)
    pl = t.reduction_partials_layout(wi, axis, 4)
    pn = pl.element_count()
    on = n // 256
    split = t.Split(4, 64)
    plan = t.plan_reduce_partials(F64, ReduceOp.Sum, pl, pn, wi, n, axis, split, 32)
    gi, gp = Geometry(wi), Geometry(pl)
    d = sentinel(pn * 8)
    say("wide partials rank", rank)
    hip.reduce_partials_any(d, to_device(src), F64, ReduceOp.Sum, gp.c, gi.c, axis, on, 4, 64,
                            plan, stream())
    got = to_host(d, pn * 8).view(np.float64)
    rows = axis_rows(src, ext, st, axis)
    p_out = list(pl.extents)
    p_out[axis] = 1
    base = view_indices(p_out, pl.strides)
    for s in range(4):
        want = plane_sum(rows[:, s * 64:(s + 1) * 64])
        assert np.array_equal(got[base + s * pl.strides[axis]], want), (rank, s)


def test_rank_nine_split_reaches_every_partial_through_the_wide_combine():
    """Reference tests/gpu_dynamic_rank.rs:2880-3000: a 131072-long axis is 512
    partials; each output's maximum sits in a different late partial."""
    rank, axis = 9, 1
    ext = [2, 131072] + [1] * 7
    n = count(ext)
    idx = np.arange(n)
    output, position = idx // ext[axis], idx % ext[axis]
    spike = ext[axis] - 1 - 97 * output
    values = np.where(position == spike, 1000.0 + output,
                      position * 1e-3 + output * 1e-6).astype(np.float32)
    # reference axis 0 is the fastest: element (o, p) at o + 2 p
    src = np.empty(n, np.float32)
    src[output + 2 * position] = values
    wi = WideLayout.compact(ext)
    out_ext = list(ext)
    out_ext[axis] = 1
    wo = WideLayout.compact(out_ext)
    on = 2
    plan = t.plan_reduction(F32, ReduceOp.Max, wo, on, wi, n, axis, 32)
    assert plan.kind == "Split" and plan.split.splits == 512
    assert plan.combine_strategy == ReduceStrategy.Plane
    pl = t.reduction_partials_layout(wi, axis, 512)
    pn = pl.element_count()
    gi, go, gp = Geometry(wi), Geometry(wo), Geometry(pl)
    d_src = to_device(src)
    part, out = sentinel(pn * 4), sentinel(on * 4)
    say("rank-9 split max", plan.pass1.grid, plan.pass2.grid, plan.pass2.block)
    hip.reduce_partials_any(part, d_src, F32, ReduceOp.Max, gp.c, gi.c, axis, on, 512,
                            plan.split.chunk_len, plan.pass1, stream())
    hip.reduce_any(out, part, F32, plan.combine_op, plan.combine_strategy, go.c, gp.c, axis, on,
                   plan.pass2, stream())
    got = to_host(out, on * 4).view(np.float32)
    assert list(got) == [1000.0, 1001.0]
    # the bytes of the rank-2 layout it fuses to, through the by-value path
    fi, fo = Layout.compact([2, 131072]), Layout.compact([2, 1])
    fplan = t.plan_reduction(F32, ReduceOp.Max, fo, on, fi, n, 1, 32)
    fout, fpart = sentinel(on * 4), sentinel(pn * 4)
    hip.enqueue_reduction(fplan, fout, d_src, fpart, F32, ReduceOp.Max, fo, fi, 1, on, stream())
    assert np.array_equal(to_host(fpart, pn * 4), to_host(part, pn * 4))
    assert np.array_equal(to_host(fout, on * 4), to_host(out, on * 4))


@pytest.mark.parametrize("dtype", [F32, F64, DType.I32, DType.I64], ids=lambda d: d.name)
def test_strided_axis_pass1_twin_takes_the_column_mapping(dtype):
    """A pass 1 over a strided axis with neighbouring output columns: the twin
    plans the launchers' column mapping inside the kernel. At rank 9 (extent-1
    axes appended: a GENERAL plan) and rank 3 through the twin, its partials are
    the by-value launcher's and the oracle's bytes, for every op the dtype has,
    full and ragged column blocks, aligned and shifted inputs."""
    rng = np.random.default_rng(90)
    ops = [ReduceOp.Sum, ReduceOp.Max, ReduceOp.Min, ReduceOp.Prod]
    if dtype in (F32, F64):
        ops.append(ReduceOp.SumSquares)
    for cols, rows, other, shift in ((256, 1024, 1, 0), (300, 768, 2, 0), (129, 512, 1, 1)):
        ext = [cols, rows, other]
        axis = 1
        n = count(ext)
        if dtype in (DType.I32, DType.I64):
            src = rng.integers(-3, 4, n + shift).astype(NUMPY[dtype])
        else:
            src = rng.uniform(-1, 1, n + shift).astype(NUMPY[dtype])
        d_src = to_device(src)
        fi = Layout([cols, rows, other], [1, cols, cols * rows], shift)
        out_ext = [cols, 1, other]
        fo = Layout.compact(out_ext)
        on = count(out_ext)
        split = t.split_policy(rows, 32)
        pl = t.reduction_partials_layout(Layout.compact(ext), axis, split.splits)
        pn = pl.element_count()
        for rank in (3, 9):
            k = rank - 3
            wi = WideLayout(ext + [1] * k, fi.strides + [5] * k, shift)
            wp = WideLayout(pl.extents + [1] * k, pl.strides + [5] * k, 0)
            gi, gp = Geometry(wi), Geometry(wp)
            for op in ops:
                plan = t.plan_reduce_partials(dtype, op, pl, pn, fi, n + shift, axis, split, 32)
                aplan = t.plan_reduce_partials(dtype, op, wp, pn, wi, n + shift, axis, split, 32)
                if rank == 9:
                    assert aplan.variant == t.RankVariant.General
                say("strided pass-1 twin", dtype.name, ext, shift, rank, op.name, aplan.grid)
                a, b = sentinel(pn * dtype.size), sentinel(pn * dtype.size)
                hip.reduce_partials(a, d_src, dtype, op, pl, fi, axis, on, split.splits,
                                    split.chunk_len, plan, stream())
                hip.reduce_partials_any(b, d_src, dtype, op, gp.c, gi.c, axis, on, split.splits,
                                        split.chunk_len, aplan, stream())
                want = np.zeros(pn, dtype=NUMPY[dtype])
                orc.reduce_partials(want, src, dtype, op, 32, pl, fi, axis, on, split.splits,
                                    split.chunk_len)
                ga, gb = to_host(a, pn * dtype.size), to_host(b, pn * dtype.size)
                assert np.array_equal(gb, ga), (ext, shift, rank, op)
                assert np.array_equal(ga, want.view(np.uint8)), (ext, shift, rank, op)


@pytest.mark.parametrize("dtype", [F32, F64, DType.I32, DType.I64], ids=lambda d: d.name)
def test_contiguous_axis_pass1_twin_takes_the_lean_mapping(dtype):
    """A pass 1 over a contiguous axis in short chunks: the twin plans the lean
    mapping inside the kernel (several chunks' loads in flight per plane). At
    rank 9 and rank 2 through the twin, its partials are the by-value
    launcher's and the oracle's bytes, for every op the dtype has, equal and
    ragged last chunks, aligned and shifted (no lean) inputs, one and several
    fused output dims."""
    rng = np.random.default_rng(91)
    ops = [ReduceOp.Sum, ReduceOp.Max, ReduceOp.Min, ReduceOp.Prod]
    if dtype in (F32, F64):
        ops.append(ReduceOp.SumSquares)
    for ext, shift in (([8192, 96], 0), ([5000, 64], 0), ([8192, 24, 5], 0), ([4096, 80], 1)):
        axis = 0
        n = count(ext)
        if dtype in (DType.I32, DType.I64):
            src = rng.integers(-3, 4, n + shift).astype(NUMPY[dtype])
        else:
            src = rng.uniform(-1, 1, n + shift).astype(NUMPY[dtype])
        d_src = to_device(src)
        fi = Layout(list(ext), Layout.compact(ext).strides, shift)
        out_ext = [1] + list(ext[1:])
        on = count(out_ext)
        split = t.split_policy(ext[0], 32)
        pl = t.reduction_partials_layout(Layout.compact(ext), axis, split.splits)
        pn = pl.element_count()
        r0 = len(ext)
        for rank in (r0, 9):
            k = rank - r0
            wi = WideLayout(list(ext) + [1] * k, fi.strides + [5] * k, shift)
            wp = WideLayout(pl.extents + [1] * k, pl.strides + [5] * k, 0)
            gi, gp = Geometry(wi), Geometry(wp)
            for op in ops:
                plan = t.plan_reduce_partials(dtype, op, pl, pn, fi, n + shift, axis, split, 32)
                aplan = t.plan_reduce_partials(dtype, op, wp, pn, wi, n + shift, axis, split, 32)
                if rank == 9:
                    assert aplan.variant == t.RankVariant.General
                say("contiguous pass-1 twin", dtype.name, ext, shift, rank, op.name,
                    split.splits, split.chunk_len, aplan.grid)
                a, b = sentinel(pn * dtype.size), sentinel(pn * dtype.size)
                hip.reduce_partials(a, d_src, dtype, op, pl, fi, axis, on, split.splits,
                                    split.chunk_len, plan, stream())
                hip.reduce_partials_any(b, d_src, dtype, op, gp.c, gi.c, axis, on, split.splits,
                                        split.chunk_len, aplan, stream())
                want = np.zeros(pn, dtype=NUMPY[dtype])
                orc.reduce_partials(want, src, dtype, op, 32, pl, fi, axis, on, split.splits,
                                    split.chunk_len)
                ga, gb = to_host(a, pn * dtype.size), to_host(b, pn * dtype.size)
                assert np.array_equal(gb, ga), (ext, shift, rank, op)
                assert np.array_equal(ga, want.view(np.uint8)), (ext, shift, rank, op)
