"""t4a_hip_reduction, the whole-plan launcher, on the GPU against the CPU oracle.

A split plan whose combine is a unit fold over at most 32 partials of an
end-to-end chunk layout, with at most eight 16-byte loads a lane, runs as one
launch: each 256-thread block holds all of an output's chunks (each 32-lane
plane up to four of them; more than one output per block for fewer than five
splits) and folds their partials from LDS in the unit order. Its finals and partials must be the two-launch path's
bytes, i.e. the oracle's; plans outside that shape take the two launches.
"""
import numpy as np
import pytest

import t4a_cuda_kernels as t
from t4a_cuda_kernels import hip, hipmem
from gpu_util import NUMPY, say, sentinel, stream, to_device, to_host
from oracle import t4a_oracle as orc

pytestmark = pytest.mark.gpu

Sum, SumSq, Max, Min = t.ReduceOp.Sum, t.ReduceOp.SumSquares, t.ReduceOp.Max, t.ReduceOp.Min
F32, F64, I32, I64 = t.DType.F32, t.DType.F64, t.DType.I32, t.DType.I64


def values(dtype, n, rng):
    if dtype in (I32, I64):
        return rng.integers(-1000, 1001, n).astype(NUMPY[dtype])
    return rng.uniform(-1.0, 1.0, n).astype(NUMPY[dtype])


def oracle_finals(dtype, op, data, in_l, axis, out_l, plan):
    on = out_l.element_count()
    out_len = out_l.max_reachable_offset() + 1
    want = np.frombuffer(bytes([0xCD]) * (out_len * dtype.size), dtype=NUMPY[dtype]).copy()
    pl = t.reduction_partials_layout(in_l, axis, plan.split.splits)
    part = np.zeros(pl.element_count(), dtype=NUMPY[dtype])
    orc.reduce_partials(part, data, dtype, op, 32, pl, in_l, axis, on, plan.split.splits,
                        plan.split.chunk_len)
    bw = plan.pass2.block[0] if plan.combine_strategy == t.ReduceStrategy.Plane else 32
    orc.reduce(want, part, dtype, plan.combine_op, plan.combine_strategy, bw, out_l, pl, axis, on)
    return want, pl


def joined_shape(dtype, plan):
    """Whether the plan is one t4a_hip_reduction joins: a unit combine and, with
    ceil(splits / 8) chunks on each 32-lane plane, at most eight 16-byte loads
    a lane (the input being contiguous, end to end and aligned)."""
    loads = -(-plan.split.chunk_len * dtype.size // (16 * 32))
    return (plan.combine_strategy == t.ReduceStrategy.Unit and plan.split.splits <= 32
            and loads * -(-plan.split.splits // 8) <= 8)


def run(dtype, op, in_l, axis, out_l, data, *, joins, calls=2):
    on = out_l.element_count()
    out_len = out_l.max_reachable_offset() + 1
    plan = t.plan_reduction(dtype, op, out_l, out_len, in_l, data.size, axis, 32)
    assert plan.kind == "Split"
    want, pl = oracle_finals(dtype, op, data, in_l, axis, out_l, plan)
    want_part = np.zeros(pl.element_count(), dtype=NUMPY[dtype])
    orc.reduce_partials(want_part, data, dtype, op, 32, pl, in_l, axis, on, plan.split.splits,
                        plan.split.chunk_len)
    d_in = to_device(data)
    assert hip.reduction_joins(plan, d_in, dtype, op, out_l, in_l, axis, on) == joins, \
        (plan.split, plan.combine_strategy)
    for call in range(calls):
        say("reduction", dtype.name, op.name, in_l, "axis", axis, "->", out_l, "splits",
            plan.split.splits, "joined" if joins else "two launches", "call", call)
        d_out = sentinel(out_len * dtype.size)
        d_part = sentinel(pl.element_count() * dtype.size)
        hip.reduction(plan, d_out, d_in, d_part, dtype, op, out_l, in_l, axis, on, stream())
        got = to_host(d_out, out_len * dtype.size, "output")
        assert np.array_equal(got, want.view(np.uint8)), (dtype, op, in_l, call)
        got_part = to_host(d_part, pl.element_count() * dtype.size, "partials")
        assert np.array_equal(got_part, want_part.view(np.uint8)), (dtype, op, in_l, call)
    return plan


@pytest.mark.parametrize("dtype", [F32, F64, I32, I64], ids=lambda d: d.name)
def test_joined_inner_axis_matches_two_launches(dtype):
    rng = np.random.default_rng(40 + int(dtype))
    ops = [Sum, Max, Min] + ([SumSq] if dtype in (F32, F64) else [])
    # splits 32, 32, 16, 2 (four outputs a block, the last block short), 4,
    # 6 (two planes idle), 12 (two chunks on some planes, one on others), 24
    for rows, n in [(24, 8192), (1, 8192), (7, 4096), (7, 512), (3, 1024), (5, 1536),
                    (9, 3072), (4, 6144)]:
        in_l = t.Layout.compact([n, rows])
        out_l = t.Layout.compact([1, rows])
        plan = t.plan_reduction(dtype, Sum, out_l, rows, in_l, rows * n, 0, 32)
        for op in ops:
            run(dtype, op, in_l, 0, out_l, values(dtype, rows * n, rng),
                joins=joined_shape(dtype, plan))


def test_joined_non_compact_and_offset_outputs():
    rng = np.random.default_rng(41)
    rows, n = 10, 8192
    data = values(F32, rows * n, rng)
    in_l = t.Layout.compact([n, rows])
    for out_l in (t.Layout([1, rows], [0, 3], 5), t.Layout([1, rows], [0, 1], 7)):
        run(F32, Sum, in_l, 0, out_l, data, joins=True)
        run(F32, Max, in_l, 0, out_l, data, joins=True)


def test_joined_extrema_keep_nan_payloads():
    rng = np.random.default_rng(42)
    for dtype, bits, pl in ((F32, np.uint32, [0x7FC00001, 0xFFC00123, 0x7F800001]),
                            (F64, np.uint64, [0x7FF8000000000001, 0xFFF8000000000123])):
        rows, n = (6, 8192) if dtype == F32 else (6, 4096)
        for op in (Max, Min):
            data = values(dtype, rows * n, rng)
            raw = data.view(bits)
            raw[5], raw[n + 300], raw[n + 7000] = pl[0], pl[1], pl[-1]
            raw[3 * n + n - 1] = pl[0]
            in_l = t.Layout.compact([n, rows])
            run(dtype, op, in_l, 0, t.Layout.compact([1, rows]), data, joins=True)


def test_two_launch_fallbacks():
    """Plans outside the joined shape still give the oracle's bytes through pass
    1 and the combine."""
    rng = np.random.default_rng(43)
    # a longer last chunk (5000 = 19 x 263 + 3): chunks not end to end
    run(F32, Sum, t.Layout.compact([5000, 4]), 0, t.Layout.compact([1, 4]),
        values(F32, 20_000, rng), joins=False)
    # 35 splits: a plane combine
    run(F32, Max, t.Layout.compact([8960, 3]), 0, t.Layout.compact([1, 3]),
        values(F32, 26_880, rng), joins=False)
    # a strided axis (TILES pass 1)
    run(F64, Sum, t.Layout.compact([64, 8192]), 1, t.Layout.compact([64, 1]),
        values(F64, 64 * 8192, rng), joins=False)
    # eight-byte elements over 32 splits: sixteen loads a lane
    run(I64, Sum, t.Layout.compact([8192, 5]), 0, t.Layout.compact([1, 5]),
        values(I64, 40_960, rng), joins=False)
    # outputs on two dims that do not merge
    run(I64, Sum, t.Layout.compact([8192, 3, 2]), 0, t.Layout([1, 3, 2], [0, 1, 4], 0),
        values(I64, 8192 * 6, rng), joins=False)
