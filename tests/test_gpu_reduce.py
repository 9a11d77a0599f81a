"""Single-axis reductions on the GPU against the CPU oracle.

The kernels keep the reference's fold topology, so for NaN-free inputs every
partial and every final must equal the oracle's bit for bit -- floats included.
Where a NaN comes out of an add or multiply only its NaN-ness is compared (the
payload is the hardware's; reference docs/abi/c-kernel-abi.md:364-366); max/min
select an operand and stay bit-exact. Independently of the topology, float
finals are also checked against the reference tests' f64 sequential sum within
the stated tolerance: relative 1e-5 (f32/c32) or 1e-12 (f64/c64) scaled by
sqrt(n) (reference tests/gpu_reduce.rs:40-130).

Covered: unit and plane direct passes at plane widths 8/16/32, the wide combine
widths 64..512, split reductions over contiguous axes (grouped walk, aligned and
not), strided axes in all three pass-1 mappings (planes, 64+ columns, 2..32
columns), complex and integer types, non-compact outputs, and the configuration
shapes C2, C4 and C5.
"""
import math

import numpy as np
import pytest

import t4a_cuda_kernels as t
from t4a_cuda_kernels import configs, hip
from gpu_util import NUMPY, say, sentinel, stream, to_device, to_host
from oracle import t4a_oracle as orc

pytestmark = pytest.mark.gpu

Sum, Prod, SumSq, Max, Min = (t.ReduceOp.Sum, t.ReduceOp.Prod, t.ReduceOp.SumSquares,
                              t.ReduceOp.Max, t.ReduceOp.Min)
F32, F64, I32, I64, C32, C64 = (t.DType.F32, t.DType.F64, t.DType.I32, t.DType.I64,
                                t.DType.C32, t.DType.C64)

PAIRS = [(d, op) for op in t.ReduceOp for d in (F32, F64, I32, I64, C32, C64) if op.supports(d)]


def values(dtype, op, count, rng):
    """Finite inputs; products stay near one so they neither overflow nor vanish."""
    if dtype in (I32, I64):
        if op == Prod:
            return rng.choice(np.array([-1, 1, 1, 2, 3], dtype=NUMPY[dtype]), count)
        return rng.integers(-1000, 1001, count).astype(NUMPY[dtype])
    if op == Prod:
        re = 1.0 + rng.uniform(-1, 1, count) / 256.0
        im = rng.uniform(-1, 1, count) / 256.0
    else:
        re = rng.uniform(-1.0, 1.0, count)
        im = rng.uniform(-1.0, 1.0, count)
    if dtype in (C32, C64):
        return (re + 1j * im).astype(NUMPY[dtype])
    return re.astype(NUMPY[dtype])


def _nan_equal(dtype, a: np.ndarray, b: np.ndarray) -> bool:
    """Element bytes equal, or both NaN in every NaN component."""
    if dtype in (I32, I64):
        return np.array_equal(a, b)
    comp = np.float32 if dtype in (F32, C32) else np.float64
    x = np.ascontiguousarray(a).view(comp)
    y = np.ascontiguousarray(b).view(comp)
    xi = x.view(np.uint32 if comp == np.float32 else np.uint64)
    yi = y.view(np.uint32 if comp == np.float32 else np.uint64)
    return bool(((xi == yi) | (np.isnan(x) & np.isnan(y))).all())


def check_f64_reference(dtype, op, data, in_l, axis, out_l, finals):
    """Tolerance check of the finals against the sequential f64 reference."""
    if dtype in (I32, I64) or op in (Max, Min):
        return
    on = out_l.element_count()
    cplx = dtype in (C32, C64)
    ref = orc.reduce_f64(data, dtype, op, in_l, axis, on, cplx)
    # finals are in output-layout order; gather them in logical output order
    got = []
    for o in range(on):
        rest, off = o, out_l.offset
        for e, s in zip(out_l.extents, out_l.strides):
            off += (rest % e) * s
            rest //= e
        got.append(finals[off])
    got = np.array(got)
    if cplx:
        got = np.stack([got.real, got.imag], axis=1).reshape(-1)
    n = in_l.extents[axis]
    tol = (1e-5 if dtype in (F32, C32) else 1e-12) * math.sqrt(n)
    scale = np.maximum(np.abs(ref), 1.0)
    if op == Sum:  # cancellation: scale by the sum of magnitudes
        absref = orc.reduce_f64(np.abs(data) if not cplx else
                                (np.abs(data.real) + 1j * np.abs(data.imag)).astype(data.dtype),
                                dtype, op, in_l, axis, on, cplx)
        scale = np.maximum(absref, 1.0)
    err = np.abs(got.astype(np.float64) - ref)
    assert (err <= tol * scale).all(), f"max rel err {(err / scale).max()} > {tol}"


def run(dtype, op, in_l, axis, out_l, width, data, *, plan=None, explicit=None):
    """Plan (or take `explicit` = (strategy, block width) for a direct pass),
    run the passes on the GPU and in the oracle, compare."""
    in_len = max(in_l.max_reachable_offset() + 1, 1)
    out_len = max(out_l.max_reachable_offset() + 1, 1)
    on = out_l.element_count()
    es = dtype.size
    say("reduce", dtype.name, op.name, in_l, "axis", axis, "->", out_l, "w", width, explicit)
    if explicit is None:
        plan = plan or t.plan_reduction(dtype, op, out_l, out_len, in_l, in_len, axis, width)
    else:
        strategy, bw = explicit
        plan = t.ReductionPlan("Direct", strategy=strategy,
                               launch=t.plan_reduce(dtype, op, strategy, out_l, out_len, in_l,
                                                    in_len, axis, bw))
    d_in = to_device(data)
    d_out = sentinel(out_len * es)
    want_out = np.frombuffer(bytes([0xCD]) * (out_len * es), dtype=NUMPY[dtype]).copy()
    if plan.kind == "Direct":
        hip.reduce(d_out, d_in, dtype, op, plan.strategy, out_l, in_l, axis, on, plan.launch,
                   stream())
        bw = plan.launch.block[0] if plan.strategy == t.ReduceStrategy.Plane else width
        orc.reduce(want_out, data, dtype, op, plan.strategy, bw, out_l, in_l, axis, on)
    else:
        pl = t.reduction_partials_layout(in_l, axis, plan.split.splits)
        pn = pl.element_count()
        want_part = np.zeros(pn, dtype=NUMPY[dtype])
        orc.reduce_partials(want_part, data, dtype, op, width, pl, in_l, axis, on,
                            plan.split.splits, plan.split.chunk_len)
        bw = plan.pass2.block[0] if plan.combine_strategy == t.ReduceStrategy.Plane else width
        orc.reduce(want_out, want_part, dtype, plan.combine_op, plan.combine_strategy, bw,
                   out_l, pl, axis, on)
        # Both doors of a split plan: the caller's two launches, and the whole
        # plan through t4a_hip_reduction (one joined launch where it joins).
        joins = hip.reduction_joins(plan, d_in, dtype, op, out_l, in_l, axis, on)
        for door in ("two launches", "t4a_hip_reduction"):
            say("  door:", door, "(joined)" if door != "two launches" and joins else "")
            d_part = sentinel(pn * es)
            d_out = sentinel(out_len * es)
            if door == "two launches":
                hip.enqueue_reduction(plan, d_out, d_in, d_part, dtype, op, out_l, in_l, axis,
                                      on, stream())
            else:
                hip.reduction(plan, d_out, d_in, d_part, dtype, op, out_l, in_l, axis, on,
                              stream())
            got_part = to_host(d_part, pn * es, "partials")
            assert _nan_equal(dtype, got_part, want_part.view(np.uint8)), \
                f"pass-1 partials differ ({door})"
            got = to_host(d_out, out_len * es, "output")
            assert _nan_equal(dtype, got, want_out.view(np.uint8)), f"finals differ ({door})"
        return plan, got.view(NUMPY[dtype])
    got = to_host(d_out, out_len * es, "output")
    assert _nan_equal(dtype, got, want_out.view(np.uint8)), "finals differ"
    return plan, got.view(NUMPY[dtype])


def compact_case(dtype, op, c_shape, c_axis, width, rng, *, explicit=None):
    """A C-order shape reduced over C-axis `c_axis` (reference axis r-1-c_axis)."""
    ext = list(reversed(c_shape))
    axis = len(c_shape) - 1 - c_axis
    in_l = t.Layout.compact(ext)
    oe = list(ext)
    oe[axis] = 1
    out_l = t.Layout.compact(oe)
    data = values(dtype, op, in_l.element_count(), rng)
    plan, finals = run(dtype, op, in_l, axis, out_l, width, data, explicit=explicit)
    check_f64_reference(dtype, op, data, in_l, axis, out_l, finals)
    return plan


@pytest.mark.parametrize("dtype,op", PAIRS, ids=[f"{d.name}-{o.name}" for d, o in PAIRS])
def test_direct_unit_and_plane(dtype, op):
    rng = np.random.default_rng(100 + 10 * int(dtype) + int(op))
    for width in (8, 16, 32):
        for c_shape, c_axis in [((37, 5), 1), ((5, 37), 0), ((3, 7, 11), 1), ((1, 1), 0),
                                ((300, width), 1), ((width + 3, 9), 0), ((2, 255, 3), 1)]:
            compact_case(dtype, op, c_shape, c_axis, width, rng)


@pytest.mark.parametrize("dtype,op", PAIRS, ids=[f"{d.name}-{o.name}" for d, o in PAIRS])
def test_wide_plane_widths(dtype, op):
    """Widths 64-512, with axis lengths on both sides of the plane body's switch
    from loads issued up front (a lane walks at most 16 elements: length 16 *
    width) to the serial walk joined across wavefronts through LDS (16 * width +
    1, about 40 * width), on a contiguous and on a strided axis."""
    rng = np.random.default_rng(200 + 10 * int(dtype) + int(op))
    for bw in (64, 128, 256, 512):
        plane = (t.ReduceStrategy.Plane, bw)
        compact_case(dtype, op, (3, bw * 5 + 7), 1, 32, rng, explicit=plane)
        compact_case(dtype, op, (bw + 1, 2), 0, 32, rng, explicit=plane)
        for length in (16 * bw, 16 * bw + 1, 40 * bw + 3):
            compact_case(dtype, op, (2, length), 1, 32, rng, explicit=plane)
        compact_case(dtype, op, (16 * bw + 1, 3), 0, 32, rng, explicit=plane)


@pytest.mark.parametrize("dtype,op", PAIRS, ids=[f"{d.name}-{o.name}" for d, o in PAIRS])
def test_split_contiguous_axis(dtype, op):
    rng = np.random.default_rng(300 + 10 * int(dtype) + int(op))
    for width in (8, 16, 32):
        for n in (8 * width * 2, 8195, 65541, 100_003):
            plan = compact_case(dtype, op, (n,), 0, width, rng)
            assert plan.kind == "Split"
    compact_case(dtype, op, (3, 20_001), 1, 32, rng)


@pytest.mark.parametrize("dtype,op", PAIRS, ids=[f"{d.name}-{o.name}" for d, o in PAIRS])
def test_split_strided_axis(dtype, op):
    """Outer axes: 2..32 columns (ROWS), 64+ columns incl. a ragged block
    (COLUMNS), 3 columns and complex types (plane mapping)."""
    rng = np.random.default_rng(400 + 10 * int(dtype) + int(op))
    for cols in (2, 3, 4, 8, 16, 32, 64, 100, 256):
        compact_case(dtype, op, (2, 1031, cols), 1, 32, rng)
    compact_case(dtype, op, (700, 5), 0, 16, rng)
    compact_case(dtype, op, (600, 70), 0, 8, rng)


def test_split_unaligned_and_non_compact_output():
    rng = np.random.default_rng(5)
    # input at an odd element offset: the grouped walk loads element by element
    ext = [20_000, 3]
    in_l = t.Layout(ext, [1, 20_000], 1)
    out_l = t.Layout([1, 3], [0, 5], 2)  # gaps between outputs
    for dtype, op in [(F32, Sum), (F64, SumSq), (I32, Max), (I64, Sum)]:
        data = values(dtype, op, 60_001, rng)
        run(dtype, op, in_l, 0, out_l, 32, data)
    # reversed reduce axis (negative stride): serial walk
    in_l = t.Layout([9000, 4], [-1, 9000], 8999)
    for dtype, op in [(F32, Sum), (C64, Prod), (I64, Min)]:
        data = values(dtype, op, 36_000, rng)
        run(dtype, op, in_l, 0, t.Layout.compact([1, 4]), 32, data)


def test_special_values():
    """NaN wins max/min (bit-exact payloads); an arithmetic NaN stays NaN; signed
    zeros and infinities."""
    rng = np.random.default_rng(6)
    n = 50_000
    for dtype in (F32, F64):
        for op in (Sum, Prod, SumSq, Max, Min):
            data = values(dtype, op, 3 * n, rng)
            data[5] = np.nan
            data[n + 17] = np.inf
            data[n + 4000] = -np.inf
            data[2 * n:] = -0.0
            data[2 * n + 77] = 0.0
            ext = [n, 3]
            run(dtype, op, t.Layout.compact(ext), 0, t.Layout.compact([1, 3]), 32, data)


@pytest.mark.parametrize("dtype", [F32, F64, I32, I64], ids=lambda d: d.name)
def test_unit_one_group_axes_many_outputs(dtype):
    """Unit reductions over a one-group axis (4..7 elements of 4 bytes, 2..3 of 8)
    with enough outputs for the four-outputs-per-thread mapping, ragged count."""
    rng = np.random.default_rng(12 + int(dtype))
    v = 16 // dtype.size
    for length in range(v, 2 * v):
        for op in (Sum, Prod, Max, Min):
            if not op.supports(dtype):
                continue
            compact_case(dtype, op, (300_007, length), 1, 32, rng,
                         explicit=(t.ReduceStrategy.Unit, 32))


@pytest.mark.parametrize("dtype,op", [(F32, Sum), (F32, Max), (F64, Prod), (I32, Sum),
                                      (C32, Sum), (C64, Sum), (I64, Min)],
                         ids=lambda x: x.name)
def test_direct_plane_packed_planes(dtype, op):
    """Direct PLANE under this build's geometry: 256 / W planes of W = 8, 16, 32
    lanes a block (block.y), a grid of at most 4096 blocks striding over more
    outputs than it holds planes, runs of four outputs a plane when a lane
    holds few elements, one at a time with every load ahead, and the serial
    walk past that, on a contiguous and on a strided axis; 32-lane planes of
    at most 8-byte elements over a strided axis run one thread per output
    (lane 0's fold and tree)."""
    rng = np.random.default_rng(60 + int(dtype) + 7 * int(op))
    ahead = 4 if dtype.size >= 16 else 8 if dtype.size >= 8 else 16
    for w in (8, 16, 32):
        direct_max = 16 * w - 1  # below two chunks of 8 planes: no split
        cand = {w + 1, w * ahead // 4, w * ahead // 4 + 1, w * ahead + 1, direct_max}
        lengths = sorted(n for n in cand if w <= n <= direct_max)
        for length in lengths:
            outputs = 40_000 if length <= 64 else 9_000
            plan = compact_case(dtype, op, (outputs, length), 1, w, rng,
                                explicit=(t.ReduceStrategy.Plane, w))
            assert plan.launch.block == (w, 256 // w, 1), plan.launch
            compact_case(dtype, op, (length, outputs), 0, w, rng,
                         explicit=(t.ReduceStrategy.Plane, w))


@pytest.mark.parametrize("dtype", [F32, F64, I32, I64], ids=lambda d: d.name)
def test_unit_short_contiguous_axes_many_outputs(dtype):
    """Unit reductions over contiguous axes of 2 to 9 16-byte groups with
    enough outputs for 256-thread blocks: up to 8 groups every load before the
    first fold, past that group by group, tails after the last whole group."""
    rng = np.random.default_rng(70 + int(dtype))
    v = 16 // dtype.size
    for length in sorted({2 * v, 3 * v + 1, min(8 * v, 32), 8 * v + 3, 9 * v}):
        if length > 32:
            continue
        for op in (Sum, Max):
            compact_case(dtype, op, (300_007, length), 1, 32, rng,
                         explicit=(t.ReduceStrategy.Unit, 32))


@pytest.mark.parametrize("dtype,op", [(F32, Sum), (F64, SumSq), (I64, Sum), (C64, Sum),
                                      (F32, Max), (I32, Prod)], ids=lambda x: x.name)
def test_single_output_long_chunks(dtype, op):
    """One output over 2^22 + 13 elements (4096 chunks of about 1024, one plane
    each, whole 4-group batches with the next batch's loads in flight, then the
    partial batch and the tail), and over 2^20 + 5 (4096 chunks of 256)."""
    rng = np.random.default_rng(30 + int(dtype) + 5 * int(op))
    for n in ((1 << 22) + 13, (1 << 20) + 5):
        compact_case(dtype, op, (n,), 0, 32, rng)


@pytest.mark.parametrize("dtype", [F32, F64, I32, I64], ids=lambda d: d.name)
def test_unit_one_group_output_decodes(dtype):
    """The one-group kernel's two output decodes: one fused output dim with a
    non-unit output stride (the linear decode), two and three unfused output
    dims over a padded input (the general decode), each with more than 262,144
    outputs so the planner's 256-thread Unit launch takes that kernel; and one
    output under a caller's 256-thread launch (the linear decode with no dim)."""
    rng = np.random.default_rng(40 + int(dtype))
    v = 16 // dtype.size
    length, lp = v + 1, 2 * v  # one group plus one element; rows padded to 2 groups
    s2 = 67 * lp + v
    cases = [
        (t.Layout.compact([length, 300_001]), t.Layout([1, 300_001], [1, 3], 0)),
        (t.Layout([length, 1001, 300], [1, lp, 1001 * lp + v], 0),
         t.Layout.compact([1, 1001, 300])),
        (t.Layout([length, 67, 71, 73], [1, lp, s2, s2 * 71 + v], 0),
         t.Layout.compact([1, 67, 71, 73])),
    ]
    for op in (Sum, Prod, Max):
        for in_l, out_l in cases:
            span = in_l.max_reachable_offset() + 1
            data = values(dtype, op, span, rng)
            run(dtype, op, in_l, 0, out_l, 32, data, explicit=(t.ReduceStrategy.Unit, 32))
        # one output, the caller's own 256-thread launch
        in_l, out_l = t.Layout.compact([length]), t.Layout.compact([1])
        data = values(dtype, op, length, rng)
        say("reduce one output", dtype.name, op.name, "length", length)
        d_in = to_device(data)
        d_out = sentinel(dtype.size)
        launch = t.Launch((1, 1, 1), (256, 1, 1), 0)
        hip.reduce(d_out, d_in, dtype, op, t.ReduceStrategy.Unit, out_l, in_l, 0, 1, launch,
                   stream())
        want = np.zeros(1, dtype=NUMPY[dtype])
        orc.reduce(want, data, dtype, op, t.ReduceStrategy.Unit, 32, out_l, in_l, 0, 1)
        assert _nan_equal(dtype, to_host(d_out, dtype.size, "output"), want.view(np.uint8))


def test_extrema_nan_payloads_bit_exact():
    """Max / Min select an operand, so their results are exact bytes even for NaN
    payloads: several payloads (quiet, signalling, negative) in one chunk, in
    the tail, rows of signed zeros only, infinities -- on the contiguous-axis
    pass 1 whose any-order fast fold hands NaN results to the exact order."""
    rng = np.random.default_rng(11)
    rows, n = 24, 8192
    payloads = {F32: [0x7FC00001, 0x7F800001, 0xFFC00123, 0x7FFFFFFF, 0xFF800002],
                F64: [0x7FF8000000000001, 0x7FF0000000000001, 0xFFF8000000000123,
                      0x7FFFFFFFFFFFFFFF, 0xFFF0000000000002]}
    for dtype in (F32, F64):
        bits = np.uint32 if dtype == F32 else np.uint64
        for op in (Max, Min):
            data = values(dtype, op, rows * n, rng)
            raw = data.view(bits)
            pl = payloads[dtype]
            raw[3] = pl[0]                                  # row 0, chunk 0
            raw[n + 10], raw[n + 200], raw[n + 201] = pl[1], pl[2], pl[0]  # row 1, one chunk
            raw[2 * n + 255] = pl[3]                        # last element of a chunk
            raw[3 * n + n - 1] = pl[4]                      # last element of the row
            raw[4 * n + 7], raw[4 * n + 4000] = pl[2], pl[1]  # two chunks of one row
            data[5 * n:6 * n] = -0.0                        # signed zeros only
            data[5 * n + 1234] = 0.0
            data[6 * n:7 * n] = 0.0
            data[6 * n + 99] = -0.0
            data[7 * n + 50] = np.inf
            data[8 * n + 60] = -np.inf
            in_l = t.Layout.compact([n, rows])
            out_l = t.Layout.compact([1, rows])
            plan = t.plan_reduction(dtype, op, out_l, rows, in_l, rows * n, 0, 32)
            assert plan.kind == "Split" and plan.split.chunk_len == 256
            say("extrema payloads", dtype.name, op.name)
            pl_l = t.reduction_partials_layout(in_l, 0, plan.split.splits)
            pn = pl_l.element_count()
            d_in, d_out, d_part = to_device(data), sentinel(rows * dtype.size), sentinel(
                pn * dtype.size)
            hip.enqueue_reduction(plan, d_out, d_in, d_part, dtype, op, out_l, in_l, 0, rows,
                                  stream())
            want_part = np.zeros(pn, dtype=NUMPY[dtype])
            orc.reduce_partials(want_part, data, dtype, op, 32, pl_l, in_l, 0, rows,
                                plan.split.splits, plan.split.chunk_len)
            want = np.zeros(rows, dtype=NUMPY[dtype])
            orc.reduce(want, want_part, dtype, plan.combine_op, plan.combine_strategy, 32, out_l,
                       pl_l, 0, rows)
            got_part = to_host(d_part, pn * dtype.size, "partials")
            got = to_host(d_out, rows * dtype.size, "output")
            assert np.array_equal(got_part, want_part.view(np.uint8)), (dtype, op, "partials")
            assert np.array_equal(got, want.view(np.uint8)), (dtype, op, "finals")
            assert np.isnan(want[:5]).all() and not np.isnan(want[5:]).any()
            zero_sign = np.signbit(want[5:7])
            assert list(zero_sign) == ([False, False] if op == Max else [True, True])


def test_extrema_nan_payloads_outer_axis_bit_exact():
    """The strided-axis pass 1 (one block per 128 columns of a split) folds f32
    Max / Min in any order and redoes a unit in the exact order when one of its
    columns comes out NaN: payloads in one column, two payloads in one column
    (their order decides the result), a NaN in a split's last row, signed
    zeros, infinities, every other column finite."""
    rng = np.random.default_rng(12)
    cols, n = 256, 8192
    for dtype, bits, pl in ((F32, np.uint32, [0x7FC00001, 0x7F800001, 0xFFC00123, 0x7FFFFFFF]),
                            (F64, np.uint64, [0x7FF8000000000001, 0x7FF0000000000001,
                                              0xFFF8000000000123, 0x7FFFFFFFFFFFFFFF])):
        for op in (Max, Min):
            data = values(dtype, op, cols * n, rng)
            raw = data.view(bits)
            at = lambda c, r: r * cols + c                       # column c, row r
            raw[at(3, 17)] = pl[0]
            raw[at(130, 5)], raw[at(130, 4000)] = pl[2], pl[1]  # two in one column
            raw[at(131, 4000)], raw[at(131, 5)] = pl[2], pl[1]  # the same, swapped rows
            raw[at(200, 255)] = pl[3]                           # a split's last row
            data[at(7, 0):at(7, n):cols] = -0.0                 # signed zeros only
            data[at(7, 900)] = 0.0
            data[at(8, 60)] = np.inf
            data[at(9, 61)] = -np.inf
            in_l = t.Layout.compact([cols, n])
            out_l = t.Layout.compact([cols, 1])
            plan = t.plan_reduction(dtype, op, out_l, cols, in_l, cols * n, 1, 32)
            assert plan.kind == "Split"
            say("outer extrema payloads", dtype.name, op.name, plan.split)
            pl_l = t.reduction_partials_layout(in_l, 1, plan.split.splits)
            pn = pl_l.element_count()
            d_in, d_out, d_part = to_device(data), sentinel(cols * dtype.size), sentinel(
                pn * dtype.size)
            hip.enqueue_reduction(plan, d_out, d_in, d_part, dtype, op, out_l, in_l, 1, cols,
                                  stream())
            want_part = np.zeros(pn, dtype=NUMPY[dtype])
            orc.reduce_partials(want_part, data, dtype, op, 32, pl_l, in_l, 1, cols,
                                plan.split.splits, plan.split.chunk_len)
            want = np.zeros(cols, dtype=NUMPY[dtype])
            bw = plan.pass2.block[0] if plan.combine_strategy == t.ReduceStrategy.Plane else 32
            orc.reduce(want, want_part, dtype, plan.combine_op, plan.combine_strategy, bw, out_l,
                       pl_l, 1, cols)
            got_part = to_host(d_part, pn * dtype.size, "partials")
            got = to_host(d_out, cols * dtype.size, "output")
            assert np.array_equal(got_part, want_part.view(np.uint8)), (dtype, op, "partials")
            assert np.array_equal(got, want.view(np.uint8)), (dtype, op, "finals")
            assert np.isnan(want[[3, 130, 131, 200]]).all()
            assert np.signbit(want[7]) == (op == Min)


def test_empty_output_is_no_launch():
    in_l = t.Layout.compact([5, 0])
    out_l = t.Layout.compact([1, 0])
    plan = t.plan_reduction(F32, Sum, out_l, 1, in_l, 1, 0, 32)
    assert plan.kind == "Direct" and plan.launch.is_empty()
    d = sentinel(4)
    hip.reduce(d, d, F32, Sum, plan.strategy, out_l, in_l, 0, 0, plan.launch, stream())
    to_host(d, 0)


# ---- configuration shapes -----------------------------------------------------------

# Inputs are the configurations' own (t4a_cuda_kernels.configs: SplitMix64 of the
# config's seed), the ones bench.py times. Every split plan runs through both
# doors (see run()): C2's inner-axis f32 Sum and Max through t4a_hip_reduction
# are the joined kernel over all 8192 outputs.

def test_config_c2_f32_inner_and_outer_sum_max_and_i64_sum():
    x, xi = configs.c2_inputs()
    in_l = t.Layout.compact([8192, 8192])
    for axis, out_ext in ((0, [1, 8192]), (1, [8192, 1])):
        out_l = t.Layout.compact(out_ext)
        for op in (Sum, Max):
            plan = t.plan_reduction(F32, op, out_l, 8192, in_l, x.size, axis, 32)
            assert hip.reduction_joins(plan, 1 << 20, F32, op, out_l, in_l, axis, 8192) == \
                (axis == 0), (axis, op)
            plan, finals = run(F32, op, in_l, axis, out_l, 32, x)
            assert plan.kind == "Split" and plan.split.splits == 32
            check_f64_reference(F32, op, x, in_l, axis, out_l, finals)
    run(I64, Sum, in_l, 0, t.Layout.compact([1, 8192]), 32, xi)


def test_config_c4_middle_axis_and_i32_product():
    ext = [4, 1048576, 32]  # C-shape [32, 1048576, 4]
    in_l = t.Layout.compact(ext)
    x, xi = configs.c4_inputs()
    for op in (SumSq, Min):
        plan, finals = run(F32, op, in_l, 1, t.Layout.compact([4, 1, 32]), 32, x)
        assert plan.split.splits == 4096
        check_f64_reference(F32, op, x, in_l, 1, t.Layout.compact([4, 1, 32]), finals)
    plan, _ = run(I32, Prod, in_l, 0, t.Layout.compact([1, 1048576, 32]), 32, xi)
    assert plan.kind == "Direct" and plan.strategy == t.ReduceStrategy.Unit


def test_config_c5_sum_over_permuted_axis():
    """Sum over C-axis 3 of the (5,2,0,4,1,3)-permuted c64 [16]^6 tensor (stored
    compact after the permute): reference axis 2, stride 256, length 16."""
    ext = [16] * 6
    in_l = t.Layout.compact(ext)
    x = configs.c5_input()
    out_ext = list(ext)
    out_ext[2] = 1
    out_l = t.Layout.compact(out_ext)
    plan, finals = run(C64, Sum, in_l, 2, out_l, 32, x)
    assert plan.kind == "Direct" and plan.strategy == t.ReduceStrategy.Unit
    check_f64_reference(C64, Sum, x, in_l, 2, out_l, finals)
