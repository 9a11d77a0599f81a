"""Seeded random movement cases on the GPU, bit for bit against the CPU oracle.

Each case draws an entry (materialize_strided, strided_to_strided,
contiguous_to_view, fill_zero_view, broadcast_in_dim, concatenate_copy), a
dtype, layouts of rank 0-6 (random axis orders, gaps, reversed axes, extent-1
and broadcast axes on read-only sides) and whether the buffers start one
element past a 16-byte boundary, so that every route the launchers choose
(tiled walk, one tile per block, routed transpose, 16-byte row units, the copy
kernel, per-element decode) meets layouts the hand-written cases do not.
Destinations are sentinel-filled and guarded, so a write outside the layout
fails the comparison.
"""
import numpy as np
import pytest

import t4a_cuda_kernels as t
from t4a_cuda_kernels import DType, Layout, T4aError, hip
from gpu_util import NUMPY, SENTINEL, random_elements, say, sentinel, stream, to_device, to_host
from oracle import t4a_oracle as orc

pytestmark = pytest.mark.gpu

ENTRIES = ["materialize", "strided", "contiguous", "fill", "broadcast", "concatenate"]


def injective(rng, ext, gap=0.3, neg=0.3):
    """Strides and offset of an injective view over `ext`: a random axis
    order, optional gaps, reversed axes."""
    rank = len(ext)
    order = list(rng.permutation(rank))
    st = [0] * rank
    s = 1
    for k in order:
        st[k] = s
        s *= ext[k] * (2 if rng.random() < gap else 1)
    off = int(rng.integers(0, 4))
    for k in range(rank):
        if rng.random() < neg:
            off += (ext[k] - 1) * st[k]
            st[k] = -st[k]
    return st, off


def extents(rng, rank, budget=40000):
    while True:
        ext = [int(rng.integers(1, 48 if rank <= 2 else 12 if rank <= 4 else 6))
               for _ in range(rank)]
        n = int(np.prod(ext)) if ext else 1
        if n <= budget:
            return ext


def sentinel_array(dtype, n):
    return np.frombuffer(bytes([SENTINEL]) * (n * dtype.size), dtype=NUMPY[dtype]).copy()


def run_case(rng, case):
    entry = ENTRIES[case % len(ENTRIES)]
    dtype = list(DType)[int(rng.integers(0, len(DType)))]
    es = dtype.size
    shift = int(rng.random() < 0.3)  # both buffers one element past 16 bytes
    rank = int(rng.integers(0, 7))
    ext = extents(rng, rank)
    n = int(np.prod(ext)) if ext else 1
    say("random movement case", case, entry, dtype.name, ext, "shift", shift)

    if entry in ("materialize", "strided"):
        st, off = injective(rng, ext)
        # read-only side: a broadcast axis now and then
        for k in range(rank):
            if ext[k] > 1 and rng.random() < 0.15:
                st[k] = 0
        src_l = Layout(ext, st, off)
        src_len = src_l.max_reachable_offset() + 1
        src = random_elements(dtype, src_len + shift, rng)
        if entry == "materialize":
            dst_len = n
            want = np.zeros(dst_len, dtype=NUMPY[dtype])
            orc.materialize_strided(want, src[shift:], dtype, src_l, n)
            plan = t.plan_materialize_strided(dtype, src_l, src_len)
            d, ds = sentinel((dst_len + shift) * es), to_device(src)
            hip.materialize_strided(d.ptr + shift * es, ds.ptr + shift * es, dtype, src_l, n,
                                    plan, stream())
        else:
            dst_st, dst_off = injective(rng, ext)
            dst_l = Layout(ext, dst_st, dst_off)
            dst_len = dst_l.max_reachable_offset() + 1
            want = sentinel_array(dtype, dst_len)
            orc.strided_to_strided(want, src[shift:], dtype, src_l, dst_l, n)
            plan = t.plan_strided_to_strided(dtype, src_l, src_len, dst_l, dst_len)
            d, ds = sentinel((dst_len + shift) * es), to_device(src)
            hip.strided_to_strided(d.ptr + shift * es, ds.ptr + shift * es, dtype, src_l, dst_l,
                                   n, plan, stream())
    elif entry in ("contiguous", "fill"):
        st, off = injective(rng, ext)
        dst_l = Layout(ext, st, off)
        dst_len = dst_l.max_reachable_offset() + 1
        if entry == "contiguous":
            src = random_elements(dtype, n + shift, rng)
            want = sentinel_array(dtype, dst_len)
            orc.contiguous_to_view(want, src[shift:], dtype, dst_l, n)
            plan = t.plan_contiguous_to_view(dtype, dst_l, dst_len)
            d, ds = sentinel((dst_len + shift) * es), to_device(src)
            hip.contiguous_to_view(d.ptr + shift * es, ds.ptr + shift * es, dtype, dst_l, n,
                                   plan, stream())
        else:
            base = random_elements(dtype, dst_len + shift, rng)
            want = base[shift:].copy()
            orc.fill_zero_view(want, dtype, dst_l, n)
            plan = t.plan_fill_zero_view(dtype, dst_l, dst_len)
            d = to_device(base)
            hip.fill_zero_view(d.ptr + shift * es, dtype, dst_l, n, plan, stream())
    elif entry == "broadcast":
        out_l = Layout.compact(ext)
        in_rank = int(rng.integers(0, rank + 1))
        dims = [int(x) for x in rng.permutation(rank)[:in_rank]]
        in_ext = [ext[d] if rng.random() < 0.75 else 1 for d in dims]
        in_st, in_off = injective(rng, in_ext)
        in_l = Layout(in_ext, in_st, in_off)
        in_len = in_l.max_reachable_offset() + 1
        src = random_elements(dtype, in_len + shift, rng)
        dst_len = n
        want = np.zeros(n, dtype=NUMPY[dtype])
        orc.broadcast_in_dim(want, src[shift:], dtype, out_l, in_l, dims, n)
        plan = t.plan_broadcast_in_dim(dtype, out_l, n, in_l, in_len, dims)
        d, ds = sentinel((dst_len + shift) * es), to_device(src)
        hip.broadcast_in_dim(d.ptr + shift * es, ds.ptr + shift * es, dtype, out_l, in_l, dims,
                             n, plan, stream())
    else:  # concatenate
        if rank == 0:
            ext, rank, n = [3], 1, 3
        axis = int(rng.integers(0, rank))
        out_ext = list(ext)
        out_ext[axis] += int(rng.integers(0, 9))
        axis_offset = int(rng.integers(0, out_ext[axis] - ext[axis] + 1))
        out_st, out_off = injective(rng, out_ext)
        out_l = Layout(out_ext, out_st, out_off)
        in_l = Layout.compact(ext)
        dst_len = out_l.max_reachable_offset() + 1
        src = random_elements(dtype, n + shift, rng)
        base = random_elements(dtype, dst_len + shift, rng)
        want = base[shift:].copy()
        orc.concatenate_copy(want, src[shift:], dtype, out_l, in_l, axis, axis_offset, n)
        plan = t.plan_concatenate_copy(dtype, out_l, dst_len, in_l, n, axis, axis_offset)
        d, ds = to_device(base), to_device(src)
        hip.concatenate_copy(d.ptr + shift * es, ds.ptr + shift * es, dtype, out_l, in_l, axis,
                             axis_offset, n, plan, stream())
    got = to_host(d, (dst_len + shift) * es)[shift * es:]
    assert np.array_equal(got, want.view(np.uint8)), (case, entry, dtype.name, ext, shift)


@pytest.mark.parametrize("block", range(6))
def test_random_movement_matches_the_oracle(block):
    rng = np.random.default_rng(900 + block)
    for case in range(block * 60, block * 60 + 60):
        try:
            run_case(rng, case)
        except T4aError as e:
            # A drawn layout the planner refuses (e.g. a span past 2^31 elements
            # for a 32-bit path) is skipped; the planners' refusals have their
            # own tests.
            pytest.fail(f"case {case}: planner refused a drawn layout: {e}")
