"""t4a_hip_reduction_scratch, the reduction entry that allocates nothing.

Its partials live in the library's per-GPU device array (T4A_HIP_SCRATCH_BYTES)
instead of a caller's workspace, so its finals must be t4a_hip_reduction's
bytes with a workspace of the caller's own, for every route the whole-plan
launcher takes: the joined launch, pass 1 plus a unit or a plane combine, and
a Direct plan. Each case calls the entry twice in a row, the second time on a
smaller input, since every call on a GPU shares the array and the second call
finds the first one's partials in it. A plan whose partials exceed the array
is refused before the device is touched (a CPU test).
"""
import ctypes

import numpy as np
import pytest

import t4a_cuda_kernels as t
from t4a_cuda_kernels import _lib, hip, hipmem
from gpu_util import NUMPY, say, sentinel, stream, to_device, to_host

Sum, SumSq, Max, Min, Prod = (t.ReduceOp.Sum, t.ReduceOp.SumSquares, t.ReduceOp.Max,
                              t.ReduceOp.Min, t.ReduceOp.Prod)
F32, F64, I32, I64, C64 = t.DType.F32, t.DType.F64, t.DType.I32, t.DType.I64, t.DType.C64
SCRATCH_LIMIT = 104  # T4A_HIP_ERR_SCRATCH_LIMIT


def values(dtype, n, rng):
    if dtype in (I32, I64):
        return rng.integers(-1000, 1001, n).astype(NUMPY[dtype])
    if dtype == C64:
        return (rng.standard_normal(n) + 1j * rng.standard_normal(n)).astype(np.complex128)
    return rng.standard_normal(n).astype(NUMPY[dtype])


def layouts(ext, axis):
    in_l = t.Layout.compact(ext)
    oe = list(ext)
    oe[axis] = 1
    return in_l, t.Layout.compact(oe)


def check_route(dtype, op, ext, axis, route, inp):
    """The plan of `ext` takes `route` through t4a_hip_reduction for an input
    at `inp` (only its alignment matters)."""
    in_l, out_l = layouts(ext, axis)
    on = out_l.element_count()
    plan = t.plan_reduction(dtype, op, out_l, on, in_l, in_l.element_count(), axis, 32)
    if route == "direct":
        assert plan.kind == "Direct"
        return plan
    assert plan.kind == "Split"
    joins = hip.reduction_joins(plan, inp, dtype, op, out_l, in_l, axis, on)
    assert joins == (route == "joined"), (ext, axis, plan.split)
    if route in ("unit", "plane"):
        want = t.ReduceStrategy.Unit if route == "unit" else t.ReduceStrategy.Plane
        assert plan.combine_strategy == want, (ext, axis, plan.combine_strategy)
    return plan


def both(dtype, op, ext, axis, data, route):
    """The finals of t4a_hip_reduction (caller's workspace) and of
    t4a_hip_reduction_scratch on the same input."""
    in_l, out_l = layouts(ext, axis)
    on = out_l.element_count()
    d_in = to_device(data)
    plan = check_route(dtype, op, ext, axis, route, d_in)
    nbytes = on * dtype.size
    d_want = sentinel(nbytes)
    d_part = None
    if plan.kind == "Split":
        pl = t.reduction_partials_layout(in_l, axis, plan.split.splits)
        d_part = hipmem.DeviceBuffer(pl.element_count() * dtype.size)
    say("reduction with a workspace", dtype.name, op.name, ext, "axis", axis, route)
    hip.reduction(plan, d_want, d_in, d_part, dtype, op, out_l, in_l, axis, on, stream())
    want = to_host(d_want, nbytes, "workspace entry output")
    d_got = sentinel(nbytes)
    say("reduction_scratch", dtype.name, op.name, ext, "axis", axis, route)
    hip.reduction_scratch(plan, d_got, d_in, dtype, op, out_l, in_l, axis, on, stream())
    got = to_host(d_got, nbytes, "scratch entry output")
    return want, got


# (route, dtype, op, first extents, second (smaller) extents, axis), extents in
# the reference's axis-0-fastest order.
CASES = [
    ("joined", F32, Sum, [8192, 2048], [4096, 96], 0),
    ("joined", F32, Max, [8192, 512], [2048, 40], 0),
    ("unit", I64, Sum, [8192, 2048], [8192, 100], 0),
    ("unit", F32, Sum, [1024, 8192], [600, 1000], 1),
    ("unit", F64, Min, [64, 8192], [64, 7000], 1),
    ("plane", F32, SumSq, [4, 262144, 8], [4, 131072, 3], 1),
    ("plane", C64, Sum, [4, 200000], [2, 70000], 1),
    ("unit", I32, Prod, [8000, 64], [4000, 16], 0),
    ("plane", I32, Prod, [40000, 64], [9000, 16], 0),
    ("direct", F32, Sum, [16, 100000], [16, 1000], 0),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}-{c[1].name}-{c[2].name}")
def test_scratch_entry_matches_the_workspace_entry_twice(case):
    route, dtype, op, first, second, axis = case
    rng = np.random.default_rng(7000 + CASES.index(case))
    for ext in (first, second):
        data = values(dtype, int(np.prod(ext)), rng)
        want, got = both(dtype, op, ext, axis, data, route)
        assert np.array_equal(got, want), (route, dtype, op, ext)


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}-{c[1].name}-{c[2].name}")
def test_cases_take_their_routes(case):
    """CPU: the planner sends both inputs of each case down the labelled route
    (the joined launch needs a 16-byte aligned input, as device buffers are)."""
    route, dtype, op, first, second, axis = case
    for ext in (first, second):
        check_route(dtype, op, ext, axis, route, 1 << 20)


@pytest.mark.gpu
def test_scratch_entry_at_its_limit():
    """Partials of exactly T4A_HIP_SCRATCH_BYTES are accepted (f32 [262144, 2048]
    over axis 0: 1024 splits x 2048 outputs x 4 bytes), then a small call."""
    ext = [262144, 2048]
    in_l, out_l = layouts(ext, 0)
    on = out_l.element_count()
    plan = t.plan_reduction(F32, Sum, out_l, on, in_l, in_l.element_count(), 0, 32)
    assert plan.split.splits * on * 4 == hip.SCRATCH_BYTES
    d_in = hipmem.DeviceBuffer(in_l.element_count() * 4)
    d_in.fill(0x3C)  # every element 0x3C3C3C3C
    pl = t.reduction_partials_layout(in_l, 0, plan.split.splits)
    d_part = hipmem.DeviceBuffer(pl.element_count() * 4)
    d_want, d_got = sentinel(on * 4), sentinel(on * 4)
    say("reduction with a workspace at the scratch limit", ext)
    hip.reduction(plan, d_want, d_in, d_part, F32, Sum, out_l, in_l, 0, on, stream())
    say("reduction_scratch at the scratch limit", ext)
    hip.reduction_scratch(plan, d_got, d_in, F32, Sum, out_l, in_l, 0, on, stream())
    want = to_host(d_want, on * 4, "workspace entry output")
    got = to_host(d_got, on * 4, "scratch entry output")
    assert np.array_equal(got, want)
    assert np.all(np.isfinite(got.view(np.float32)))
    del d_in, d_part
    data = values(F32, 4096 * 30, np.random.default_rng(7100))
    want, got = both(F32, Sum, [4096, 30], 0, data, "joined")
    assert np.array_equal(got, want)


def test_scratch_entry_refuses_partials_past_its_limit():
    """Refused before any device call (so this runs without a GPU): f32 [262144,
    2049] over axis 0 needs 1024 x 2049 partials, 4 KiB past the array."""
    ext = [262144, 2049]
    in_l, out_l = layouts(ext, 0)
    on = out_l.element_count()
    plan = t.plan_reduction(F32, Sum, out_l, on, in_l, in_l.element_count(), 0, 32)
    assert plan.kind == "Split" and plan.split.splits * on * 4 > hip.SCRATCH_BYTES
    lib = _lib.load()
    dummy = ctypes.c_void_p(0x1000)  # never dereferenced: the size check comes first
    status = lib.t4a_hip_reduction_scratch(dummy, dummy, int(F32), int(Sum),
                                           ctypes.byref(out_l.c), ctypes.byref(in_l.c), 0, on,
                                           ctypes.byref(plan.to_c()), ctypes.c_void_p(0))
    assert status == SCRATCH_LIMIT
    assert lib.t4a_status_name(status).decode() == "ScratchLimit"
    with pytest.raises(t.T4aError, match="ScratchLimit"):
        hip.reduction_scratch(plan, 0x1000, 0x1000, F32, Sum, out_l, in_l, 0, on, None)


def test_scratch_size_agrees_with_the_header():
    from pathlib import Path
    import re
    text = (Path(__file__).resolve().parent.parent / "include" / "t4a" / "t4a.h").read_text()
    m = re.search(r"#define T4A_HIP_SCRATCH_BYTES \((\d+)u \* (\d+)u \* (\d+)u\)", text)
    assert m and int(m.group(1)) * int(m.group(2)) * int(m.group(3)) == hip.SCRATCH_BYTES
    assert "T4A_HIP_ERR_SCRATCH_LIMIT = 104" in text
