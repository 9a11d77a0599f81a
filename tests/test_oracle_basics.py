"""Pins of the CPU oracle beyond the golden vectors, CPU only.

- tiled_transpose against the closed form (numpy's transpose of each batch),
- materialize_strided / strided_to_strided against a brute-force restatement
  of the reference tests' `view_indices` (reference tests/gpu_kernels.rs:36-51)
  on small random views (reversed, broadcast, permuted),
- reductions of integers (wrapping) and max/min, whose result does not depend
  on the fold order, against numpy, for the unit, plane, wide-plane and split
  passes over random layouts,
- the f64 sequential reference against numpy in float64,
- that the golden vectors discriminate fold order: a serial f32 sum of a golden
  input does not reproduce the golden bytes, so the golden pins the topology.
"""
import numpy as np
import pytest

import reduce_golden as rg
import t4a_cuda_kernels as t
from oracle import t4a_oracle as orc

NUMPY = {t.DType.F32: np.float32, t.DType.F64: np.float64, t.DType.I32: np.int32,
         t.DType.I64: np.int64, t.DType.Bool: np.uint8, t.DType.C32: np.complex64,
         t.DType.C64: np.complex128}


def view_indices(extents, strides, offset):
    """reference tests/gpu_kernels.rs:36-51, restated."""
    count = int(np.prod(extents)) if extents else 1
    out = []
    for flat in range(count):
        index = offset
        for e, s in zip(extents, strides):
            index += (flat % e) * s
            flat //= e
        out.append(index)
    return out


@pytest.mark.parametrize("dtype", list(t.DType), ids=[d.name for d in t.DType])
def test_transpose_closed_form(dtype):
    rng = np.random.default_rng(int(dtype))
    for m, n, b, off in [(5, 7, 1, 0), (16, 3, 2, 3), (1, 9, 3, 1), (33, 65, 1, 0)]:
        src = rng.integers(0, 255, (off + m * n * b) * dtype.size, dtype=np.uint8)
        dst = np.zeros(m * n * b * dtype.size, dtype=np.uint8)
        orc.tiled_transpose(dst, src, dtype, off, m * n, m, n, b)
        # compare elements as opaque byte records: random bits hold NaNs
        rec = np.dtype((np.void, dtype.size))
        s = src[off * dtype.size:].view(rec)
        d = dst.view(rec)
        for k in range(b):
            block = s[k * m * n:(k + 1) * m * n].reshape(m, n)  # src[i*N + j]
            # dst[i + j*M] = src[i*N + j]  <=>  dst viewed (N, M) is src (M, N) transposed
            assert np.array_equal(d[k * m * n:(k + 1) * m * n].reshape(n, m), block.T)


def random_view(rng, rank):
    ext = [int(e) for e in rng.integers(1, 5, rank)]
    perm = rng.permutation(rank)
    st_p = t.Layout.compact([ext[p] for p in perm]).strides
    st = [0] * rank
    for i, p in enumerate(perm):
        st[p] = st_p[i]
    off = int(rng.integers(0, 3))
    for k in range(rank):
        if rng.random() < 0.3:
            off += (ext[k] - 1) * st[k]
            st[k] = -st[k]
        elif rng.random() < 0.15:
            st[k] = 0
    return t.Layout(ext, st, off)


def test_movement_matches_view_indices():
    rng = np.random.default_rng(1)
    for _ in range(60):
        rank = int(rng.integers(0, 6))
        src_l = random_view(rng, rank)
        count = src_l.element_count()
        src_len = max(src_l.max_reachable_offset() + 1, 1)
        src = rng.integers(-2**31, 2**31, src_len, dtype=np.int64).astype(np.int32)
        got = np.zeros(count, dtype=np.int32)
        orc.materialize_strided(got, src, t.DType.I32, src_l, count)
        want = src[view_indices(src_l.extents, src_l.strides, src_l.offset)]
        assert np.array_equal(got, want)
        # strided_to_strided into a permuted destination with gaps
        dperm = rng.permutation(rank)
        pad = [e + 1 for e in src_l.extents]
        st_p = t.Layout.compact([pad[p] for p in dperm]).strides if rank else []
        dst_st = [0] * rank
        for i, p in enumerate(dperm):
            dst_st[p] = st_p[i]
        dst_l = t.Layout(src_l.extents, dst_st, 2)
        dst_len = dst_l.max_reachable_offset() + 1
        got = np.full(dst_len, -7, dtype=np.int32)
        orc.strided_to_strided(got, src, t.DType.I32, src_l, dst_l, count)
        want = np.full(dst_len, -7, dtype=np.int32)
        want[view_indices(src_l.extents, dst_st, 2)] = src[
            view_indices(src_l.extents, src_l.strides, src_l.offset)]
        assert np.array_equal(got, want)


def numpy_reduce(x, extents, axis, op, dtype):
    """Order-independent reference: numpy over the logical array (axis 0 fastest)."""
    arr = x.reshape(list(reversed(extents)))  # C order: last numpy axis = reference axis 0
    ax = len(extents) - 1 - axis
    if op == t.ReduceOp.Sum:
        r = arr.sum(axis=ax, dtype=NUMPY[dtype])
    elif op == t.ReduceOp.Prod:
        r = arr.prod(axis=ax, dtype=NUMPY[dtype])
    elif op == t.ReduceOp.Max:
        r = arr.max(axis=ax)
    else:
        r = arr.min(axis=ax)
    return np.ascontiguousarray(r).reshape(-1)


@pytest.mark.parametrize("dtype", [t.DType.I32, t.DType.I64, t.DType.F32, t.DType.F64])
def test_order_independent_reductions_match_numpy(dtype):
    rng = np.random.default_rng(10 + int(dtype))
    ops = [t.ReduceOp.Max, t.ReduceOp.Min]
    if dtype in (t.DType.I32, t.DType.I64):
        ops += [t.ReduceOp.Sum, t.ReduceOp.Prod]
    for extents, axis in [([37, 5], 0), ([5, 600], 1), ([3, 2100, 2], 1), ([9000], 0),
                          ([4, 300, 3], 1), ([70, 3, 65], 2)]:
        n = int(np.prod(extents))
        if dtype in (t.DType.I32, t.DType.I64):
            x = rng.integers(-2**31, 2**31, n, dtype=np.int64).astype(NUMPY[dtype])
        else:
            x = rng.standard_normal(n).astype(NUMPY[dtype])
        in_l = t.Layout.compact(extents)
        oe = list(extents)
        oe[axis] = 1
        out_l = t.Layout.compact(oe)
        on = out_l.element_count()
        for op in ops:
            with np.errstate(over="ignore"):
                want = numpy_reduce(x, extents, axis, op, dtype)
            for width in (8, 16, 32):
                plan = t.plan_reduction(dtype, op, out_l, on, in_l, n, axis, width)
                out = np.zeros(on, dtype=NUMPY[dtype])
                if plan.kind == "Direct":
                    bw = plan.launch.block[0] if plan.strategy == t.ReduceStrategy.Plane else width
                    orc.reduce(out, x, dtype, op, plan.strategy, bw, out_l, in_l, axis, on)
                else:
                    pl = t.reduction_partials_layout(in_l, axis, plan.split.splits)
                    part = np.zeros(pl.element_count(), dtype=NUMPY[dtype])
                    orc.reduce_partials(part, x, dtype, op, width, pl, in_l, axis, on,
                                        plan.split.splits, plan.split.chunk_len)
                    bw = (plan.pass2.block[0] if plan.combine_strategy == t.ReduceStrategy.Plane
                          else width)
                    orc.reduce(out, part, dtype, plan.combine_op, plan.combine_strategy, bw,
                               out_l, pl, axis, on)
                assert np.array_equal(out, want), (extents, axis, op, width)
            # every wide combine width, as a direct plane pass
            if extents[axis] >= 512:
                for bw in (64, 128, 256, 512):
                    out = np.zeros(on, dtype=NUMPY[dtype])
                    orc.reduce(out, x, dtype, op, t.ReduceStrategy.Plane, bw, out_l, in_l, axis,
                               on)
                    assert np.array_equal(out, want)


def test_nan_wins_extrema_and_signed_zeros():
    x = np.array([1.0, -0.0, 0.0, np.nan, 5.0], dtype=np.float32)
    in_l, out_l = t.Layout.compact([5]), t.Layout.compact([1])
    for op in (t.ReduceOp.Max, t.ReduceOp.Min):
        out = np.zeros(1, dtype=np.float32)
        orc.reduce(out, x, t.DType.F32, op, t.ReduceStrategy.Unit, 32, out_l, in_l, 0, 1)
        assert np.isnan(out[0])
    z = np.array([-0.0, 0.0, -0.0], dtype=np.float64)
    in_l, out_l = t.Layout.compact([3]), t.Layout.compact([1])
    out = np.zeros(1)
    orc.reduce(out, z, t.DType.F64, t.ReduceOp.Max, t.ReduceStrategy.Unit, 32, out_l, in_l, 0, 1)
    assert out[0] == 0.0 and not np.signbit(out[0])
    orc.reduce(out, z, t.DType.F64, t.ReduceOp.Min, t.ReduceStrategy.Unit, 32, out_l, in_l, 0, 1)
    assert out[0] == 0.0 and np.signbit(out[0])
    # a sum over one -0.0 keeps the sign (first-element seeding)
    orc.reduce(out, z[:1].copy(), t.DType.F64, t.ReduceOp.Sum, t.ReduceStrategy.Unit, 32,
               out_l, t.Layout.compact([1]), 0, 1)
    assert np.signbit(out[0])


def test_f64_reference_matches_numpy():
    rng = np.random.default_rng(3)
    x = rng.standard_normal(7 * 300)
    in_l = t.Layout.compact([7, 300])
    for op, fn in ((t.ReduceOp.Sum, np.sum), (t.ReduceOp.SumSquares, lambda a, axis: (a * a).sum(axis))):
        got = orc.reduce_f64(x, t.DType.F64, op, in_l, 1, 7, False)
        want = fn(x.reshape(300, 7), axis=0)
        assert np.allclose(got, want, rtol=1e-12)


def test_golden_discriminates_fold_order():
    """A serial fold of a golden input misses the golden bytes: the vectors pin
    which elements are combined in which order, not just the sum."""
    case = next(c for c in rg.load_cases() if c.key == "n1048576|w32|F32|Sum|Random|fast")
    x = rg.input_array(case.shape, case.dtype, case.op, case.cls, 4096)
    out = np.zeros(1, dtype=np.float32)
    in_l, out_l = t.Layout.compact([1048576]), t.Layout.compact([1])
    orc.reduce(out, x, t.DType.F32, t.ReduceOp.Sum, t.ReduceStrategy.Unit, 32, out_l, in_l, 0, 1)
    assert out.tobytes() != case.finals
    pairwise = np.float32(x.astype(np.float32).sum(dtype=np.float32))
    assert pairwise.tobytes() != case.finals
