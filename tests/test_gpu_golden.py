"""The reference's A100 golden split reductions, run through the MI355X kernels.

Every case of tests/golden/reduce-golden.tsv is planned, pass 1 and the combine
run on the GPU through the C ABI, and the partials hash and the final bytes are
compared with the reference GPU's own capture. The fixture holds each case
twice (reference tests/gpu_reduce_golden.rs:316-470, 562-671): the `fast` rows
run through the by-value launchers, the `any` rows through the general-rank
`_any` launchers with the layouts' extents and strides in device memory. Where a NaN comes out of an add
or multiply, the payload is the hardware's (the reference GPU returns the f32
canonical NaN, gfx950 propagates an operand's payload): such NaN components are
compared by NaN-ness, the partials hash is not compared when a partial is NaN,
and every other bit must match. Max/min are compared bit for bit in every class.
"""
import numpy as np
import pytest

import reduce_golden as rg
import t4a_cuda_kernels as t
from t4a_cuda_kernels import hip
from gpu_util import say, sentinel, stream, to_device, to_host
from oracle import t4a_oracle as orc

pytestmark = pytest.mark.gpu

PATHS = {"fast": rg.load_cases(), "any": rg.load_cases(path_kind="any")}
SHAPES = sorted({c.shape for c in PATHS["fast"]})


def device_layout(layout: t.WideLayout, keep: list):
    """`layout` as a t4a_cuda_layout_any over device copies of its arrays."""
    ext = to_device(np.array(layout.extents, dtype=np.int64), guard=0)
    st = to_device(np.array(layout.strides, dtype=np.int64), guard=0)
    keep += [ext, st]
    return layout.device_c(ext.ptr, st.ptr)


def test_both_paths_hold_every_case():
    assert len(PATHS["fast"]) == len(PATHS["any"]) == 666
    fast = {c.key.rsplit("|", 1)[0]: c for c in PATHS["fast"]}
    for c in PATHS["any"]:
        f = fast[c.key.rsplit("|", 1)[0]]
        assert (f.plan, f.partials_bytes, f.partials_fnv, f.finals) == \
            (c.plan, c.partials_bytes, c.partials_fnv, c.finals), c.key


@pytest.mark.parametrize("path", ["fast", "any"])
@pytest.mark.parametrize("shape", SHAPES)
def test_gpu_matches_reference_golden(shape, path):
    failures = []
    for case in (c for c in PATHS[path] if c.shape == shape):
        extents, axis = rg.SHAPE_BY_NAME[case.shape]
        code, width, comps = rg.DTYPES[case.dtype]
        dtype, op = t.DType(code), t.ReduceOp(rg.OPS[case.op])
        oe = list(extents)
        oe[axis] = 1
        if path == "fast":
            in_l, out_l = t.Layout.compact(list(extents)), t.Layout.compact(oe)
        else:
            in_l, out_l = t.WideLayout.compact(list(extents)), t.WideLayout.compact(oe)
        n, on = in_l.element_count(), out_l.element_count()
        plan = t.plan_reduction(dtype, op, out_l, on, in_l, n, axis, case.width)
        arr = rg.input_array(case.shape, case.dtype, case.op, case.cls, plan.split.splits)
        pl = t.reduction_partials_layout(in_l, axis, plan.split.splits)
        pbytes = pl.element_count() * dtype.size
        say(case.key)
        d_in = to_device(arr)
        d_part = sentinel(pbytes)
        d_out = sentinel(on * dtype.size)
        if path == "fast":
            hip.enqueue_reduction(plan, d_out, d_in, d_part, dtype, op, out_l, in_l, axis, on,
                                  stream())
        else:
            keep = []
            c_in, c_out, c_part = (device_layout(x, keep) for x in (in_l, out_l, pl))
            hip.reduce_partials_any(d_part, d_in, dtype, op, c_part, c_in, axis, on,
                                    plan.split.splits, plan.split.chunk_len, plan.pass1,
                                    stream())
            hip.reduce_any(d_out, d_part, dtype, plan.combine_op, plan.combine_strategy, c_out,
                           c_part, axis, on, plan.pass2, stream())
        partials = to_host(d_part, pbytes, "partials")
        finals = to_host(d_out, on * dtype.size, "finals").tobytes()
        ft = np.float32 if width == 4 else np.float64
        partials_nan = np.isnan(partials.view(ft)).any()
        arithmetic_nan = rg.payloads_decided_by_arithmetic(case)
        ok = partials.nbytes == case.partials_bytes
        if not (arithmetic_nan and partials_nan):
            ok = ok and orc.fnv1a64(partials) == case.partials_fnv
        ok = ok and rg.components_equal(case.dtype, case.finals, finals,
                                        payload_free=arithmetic_nan)
        if not ok:
            failures.append(f"{case.key}: golden {case.finals.hex()} got {finals.hex()}")
    assert not failures, "\n".join(failures[:20])
