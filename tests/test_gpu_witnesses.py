"""The reference's known-answer witnesses of the pass-1 topology, on the GPU.

Restated from reference tests/gpu_reduce.rs:
- 2191-2248: PROD is never regrouped -- lane t multiplies start + t + 32k in k
  order, then the plane folds its lanes with the xor tree; emulated here in f32
  with numpy and required bit for bit on a contiguous axis (where the
  regroupable ops take the grouped walk);
- 2277-2345: the topology does not depend on the input address -- the same
  values placed 0..3 elements past a 16-byte boundary give the same partials
  and result bits, for the witness [A, A, -A, -A, 0, ...] (A = 2^127; a walk
  that grouped by address would pair A + A on one alignment and A + -A on
  another) and for ordinary data at several lengths, plane widths and ops;
- 2567-2600: the two revision-13 overflow witnesses (groups of four consecutive
  elements share a lane): A + A and -A + -A in groups 0 and 8 overflow to NaN;
  A + -A in both groups cancel to +0; at every lead.

Each case runs through both doors of a split plan (the caller's two launches
and t4a_hip_reduction), which must agree bit for bit.
"""
import numpy as np
import pytest

import t4a_cuda_kernels as t
from t4a_cuda_kernels import hip
from gpu_util import NUMPY, say, sentinel, stream, to_device, to_host

pytestmark = pytest.mark.gpu

F32, F64 = t.DType.F32, t.DType.F64
Sum, SumSq, Max, Prod = t.ReduceOp.Sum, t.ReduceOp.SumSquares, t.ReduceOp.Max, t.ReduceOp.Prod
A = np.float32(2.0 ** 127)


def from_index(index: np.ndarray, dtype) -> np.ndarray:
    """Reference WalkValue::from_index (gpu_reduce.rs:1828-1843):
    ((i * 7919) % 1009) / 1009 - 0.5, in the element type's arithmetic."""
    v = ((index.astype(np.int64) * 7919) % 1009).astype(dtype)
    return v / dtype(1009.0) - dtype(0.5)


def run_walk(values: np.ndarray, lead: int, op, width: int):
    """A rank-1 reduction of `values` placed `lead` elements into a fresh
    buffer (reference reduce_at_lead / run_walk, gpu_reduce.rs:1927-2010,
    2250-2275): returns (partials, result) as arrays of the element type, the
    same from both doors."""
    dtype = F32 if values.dtype == np.float32 else F64
    host = np.concatenate([np.full(lead, values[0], values.dtype), values])
    length = values.size
    in_l = t.Layout([length], [1], lead)
    out_l = t.Layout.compact([1])
    plan = t.plan_reduction(dtype, op, out_l, 1, in_l, host.size, 0, width)
    d_in = to_device(host)
    es = dtype.size
    results = []
    for door in ("two launches", "t4a_hip_reduction"):
        say("walk", dtype.name, op.name, "len", length, "lead", lead, "width", width, door)
        d_out = sentinel(es)
        if plan.kind == "Direct":
            hip.reduce(d_out, d_in, dtype, op, plan.strategy, out_l, in_l, 0, 1, plan.launch,
                       stream())
            results.append((np.zeros(0, values.dtype),
                            to_host(d_out, es).view(values.dtype)[0]))
            continue
        splits = plan.split.splits
        d_part = sentinel(splits * es)
        if door == "two launches":
            hip.enqueue_reduction(plan, d_out, d_in, d_part, dtype, op, out_l, in_l, 0, 1,
                                  stream())
        else:
            hip.reduction(plan, d_out, d_in, d_part, dtype, op, out_l, in_l, 0, 1, stream())
        results.append((to_host(d_part, splits * es).view(values.dtype).copy(),
                        to_host(d_out, es).view(values.dtype)[0]))
    (p0, r0), (p1, r1) = results
    assert p0.tobytes() == p1.tobytes() and r0.tobytes() == r1.tobytes(), "the doors differ"
    return p0, r0, plan


@pytest.mark.parametrize("length,offset", [(1028, 1), (65549, 0), (65549, 3)])
def test_product_partials_keep_the_serial_lane_walk(length, offset):
    index = np.arange(length + offset)
    host = np.float32(1.0) + from_index(index, np.float32) * np.float32(1e-3)
    partials, _, plan = run_walk(host[offset:], offset, Prod, 32)
    assert plan.kind == "Split"
    splits, chunk = plan.split.splits, plan.split.chunk_len
    view = host[offset:]
    for c in range(splits):
        start = c * chunk
        end = length if c + 1 == splits else start + chunk
        lanes = view[start:start + 32].copy()  # lane t seeds start + t
        k = 1
        while start + 32 * k < end:
            idx = start + 32 * k + np.arange(32)
            more = idx < end
            lanes[more] = lanes[more] * view[idx[more]]
            k += 1
        step = 1
        while step < 32:
            lanes = lanes * lanes[np.arange(32) ^ step]
            step <<= 1
        assert partials[c].view(np.uint32) == lanes[0].view(np.uint32), (length, offset, c)


def test_topology_does_not_depend_on_the_input_address():
    witness = np.zeros(1024, np.float32)
    witness[:4] = [A, A, -A, -A]
    p0, r0, _ = run_walk(witness, 0, Sum, 32)
    for lead in range(1, 4):
        p, r, _ = run_walk(witness, lead, Sum, 32)
        assert r.view(np.uint32) == r0.view(np.uint32), lead
        assert p.view(np.uint32).tolist() == p0.view(np.uint32).tolist(), lead
    for length in (1028, 4099, 65549):
        f32 = from_index(np.arange(length), np.float32)
        f64 = from_index(np.arange(length), np.float64)
        for width in (8, 32):
            for op in (Sum, SumSq, Max):
                p0, r0, _ = run_walk(f32, 0, op, width)
                for lead in range(1, 4):
                    p, r, _ = run_walk(f32, lead, op, width)
                    assert (p.tobytes(), r.tobytes()) == (p0.tobytes(), r0.tobytes()), \
                        ("F32", op, length, width, lead)
                p0, r0, _ = run_walk(f64, 0, op, width)
                p, r, _ = run_walk(f64, 1, op, width)
                assert (p.tobytes(), r.tobytes()) == (p0.tobytes(), r0.tobytes()), \
                    ("F64", op, length, width)


def test_pass1_overflow_follows_the_revision_13_grouping():
    def witness(placement):
        values = np.zeros(1024, np.float32)
        for index, value in placement:
            values[index] = value
        return values

    same_group = witness([(0, A), (1, A), (32, -A), (33, -A)])
    cancelling = witness([(0, A), (1, -A), (32, A), (33, -A)])
    for lead in range(4):
        _, total, _ = run_walk(same_group, lead, Sum, 32)
        assert np.isnan(total), (lead, total)
        _, total, _ = run_walk(cancelling, lead, Sum, 32)
        assert total.view(np.uint32) == np.float32(0.0).view(np.uint32), (lead, total)
