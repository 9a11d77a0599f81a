"""The launchers under block shapes their planners never return.

A launcher accepts any geometry (the reference's raw entries take whatever the
caller launches). Its block-size-specialised kernels number their threads along
x alone, so they may only run 1-D blocks of that size: a 2-D block with the
same thread count (128 x 2 = 256, 32 x 16 = 512, the reference transpose
config tile 32 x 16 rows) must take the kernels that read blockDim, and every
output must still equal the oracle's. Grids with a second dimension are
covered too (blocks past the first row redo work already done, writing the
same values)."""
import numpy as np
import pytest

import t4a_cuda_kernels as t
from t4a_cuda_kernels import hip
from gpu_util import NUMPY, random_elements, say, sentinel, stream, to_device, to_host
from oracle import t4a_oracle as orc

pytestmark = pytest.mark.gpu

F32, F64, C64, Bool = t.DType.F32, t.DType.F64, t.DType.C64, t.DType.Bool
SHAPES_256 = [((97, 1, 1), (128, 2, 1)), ((31, 1, 1), (64, 4, 1)), ((13, 3, 1), (256, 1, 1))]


@pytest.mark.parametrize("dtype", [Bool, F32, C64], ids=lambda d: d.name)
def test_copy_and_fill_under_2d_blocks(dtype):
    rng = np.random.default_rng(601)
    n = 40_003
    src = random_elements(dtype, n, rng)
    d_src = to_device(src)
    for grid, block in SHAPES_256:
        launch = t.Launch(grid, block, 0)
        say("copy_exact", dtype.name, grid, block)
        d_dst = sentinel(src.nbytes)
        hip.copy_exact(d_dst, d_src, dtype, n, launch, stream())
        assert np.array_equal(to_host(d_dst, src.nbytes), src.view(np.uint8)), (grid, block)
        say("fill_zero", dtype.name, grid, block)
        hip.fill_zero(d_dst, dtype, n, launch, stream())
        assert not to_host(d_dst, src.nbytes).any(), (grid, block)
        view = t.Layout([101, 300], [1, 131], 7)
        span = view.max_reachable_offset() + 1
        say("fill_zero_view", dtype.name, grid, block)
        d_v = to_device(src[:span])
        hip.fill_zero_view(d_v, dtype, view, view.element_count(), launch, stream())
        want = src[:span].copy()
        orc.fill_zero_view(want, dtype, view, view.element_count())
        assert np.array_equal(to_host(d_v, want.nbytes), want.view(np.uint8)), (grid, block)


@pytest.mark.parametrize("dtype", [Bool, F32, F64, C64], ids=lambda d: d.name)
def test_moves_under_2d_blocks(dtype):
    rng = np.random.default_rng(602)
    cases = [
        (t.Layout([300, 70], [-1, 300], 299), None),                 # reversed rows: elements
        (t.Layout.compact([33, 500]), t.Layout([33, 500], [1, 40], 3)),  # rows
        (t.Layout([64, 64, 40], [64, 1, 4096], 0), None),             # tiled
    ]
    for src_l, dst_l in cases:
        span = src_l.max_reachable_offset() + 1
        src = random_elements(dtype, span, rng)
        d_src = to_device(src)
        dst_l = dst_l or t.Layout.compact(src_l.extents)
        dst_len = dst_l.max_reachable_offset() + 1
        want = np.frombuffer(bytes([0xCD]) * (dst_len * dtype.size), dtype=NUMPY[dtype]).copy()
        orc.strided_to_strided(want, src, dtype, src_l, dst_l, src_l.element_count())
        for grid, block in SHAPES_256:
            say("strided_to_strided", dtype.name, src_l, grid, block)
            d_dst = sentinel(want.nbytes)
            hip.strided_to_strided(d_dst, d_src, dtype, src_l, dst_l, src_l.element_count(),
                                   t.Launch(grid, block, 0), stream())
            assert np.array_equal(to_host(d_dst, want.nbytes), want.view(np.uint8)), \
                (src_l, grid, block)


@pytest.mark.parametrize("dtype", [Bool, F32, F64, C64], ids=lambda d: d.name)
def test_transpose_under_2d_blocks(dtype):
    """512 threads as 32 x 16 (the reference's tile-32, 16-row block), 256 x 2
    and 16 x 32, under 1-D and 2-D grids."""
    rng = np.random.default_rng(603)
    m, n, batches = 260, 333, 2
    src = random_elements(dtype, m * n * batches, rng)
    d_src = to_device(src)
    want = np.zeros(m * n * batches, dtype=NUMPY[dtype])
    orc.tiled_transpose(want, src, dtype, 0, m * n, m, n, batches)
    for grid, block in [((9, 1, 2), (32, 16, 1)), ((9, 11, 2), (32, 16, 1)),
                        ((5, 1, 2), (256, 2, 1)), ((17, 1, 2), (16, 32, 1)),
                        ((9, 11, 2), (512, 1, 1))]:
        say("tiled_transpose", dtype.name, m, n, batches, grid, block)
        d_dst = sentinel(want.nbytes)
        hip.tiled_transpose(d_dst, d_src, dtype, 0, m * n, m, n, t.TransposeConfig.DEFAULT,
                            t.Launch(grid, block, 0), stream())
        assert np.array_equal(to_host(d_dst, want.nbytes), want.view(np.uint8)), (grid, block)


@pytest.mark.parametrize("dtype", [F32, t.DType.I64, C64], ids=lambda d: d.name)
def test_reduce_under_2d_blocks(dtype):
    """Unit reductions whose block holds the specialised 256 or 64 threads in
    two dimensions, and pass 1 under a 2-D block."""
    rng = np.random.default_rng(604)
    ext, axis = [6, 4001], 0
    x = random_elements(dtype, 6 * 4001, rng) if dtype != t.DType.I64 else \
        rng.integers(-1000, 1001, 6 * 4001).astype(np.int64)
    d_in = to_device(x)
    in_l = t.Layout.compact(ext)
    out_l = t.Layout.compact([1, 4001])
    on = 4001
    want = np.zeros(on, dtype=NUMPY[dtype])
    orc.reduce(want, x, dtype, t.ReduceOp.Sum, t.ReduceStrategy.Unit, 32, out_l, in_l, axis, on)
    for grid, block in [((16, 1, 1), (128, 2, 1)), ((63, 1, 1), (32, 2, 1)),
                        ((8, 2, 1), (256, 1, 1)), ((4, 1, 1), (64, 1, 1))]:
        say("reduce unit", dtype.name, ext, grid, block)
        d_out = sentinel(want.nbytes)
        hip.reduce(d_out, d_in, dtype, t.ReduceOp.Sum, t.ReduceStrategy.Unit, out_l, in_l, axis,
                   on, t.Launch(grid, block, 0), stream())
        assert np.array_equal(to_host(d_out, want.nbytes), want.view(np.uint8)), (grid, block)
    # pass 1 over a contiguous axis of 3 x 20000 with 2-D blocks
    ext, axis = [20000, 3], 0
    x = random_elements(dtype, 60000, rng) if dtype != t.DType.I64 else \
        rng.integers(-1000, 1001, 60000).astype(np.int64)
    d_in = to_device(x)
    in_l = t.Layout.compact(ext)
    out_l = t.Layout.compact([1, 3])
    plan = t.plan_reduction(dtype, t.ReduceOp.Sum, out_l, 3, in_l, 60000, axis, 32)
    pl = t.reduction_partials_layout(in_l, axis, plan.split.splits)
    want = np.zeros(pl.element_count(), dtype=NUMPY[dtype])
    orc.reduce_partials(want, x, dtype, t.ReduceOp.Sum, 32, pl, in_l, axis, 3,
                        plan.split.splits, plan.split.chunk_len)
    for grid, block in [((20, 1, 1), (128, 2, 1)), ((9, 2, 1), (256, 1, 1))]:
        say("reduce_partials", dtype.name, ext, grid, block)
        d_part = sentinel(want.nbytes)
        hip.reduce_partials(d_part, d_in, dtype, t.ReduceOp.Sum, pl, in_l, axis, 3,
                            plan.split.splits, plan.split.chunk_len, t.Launch(grid, block, 0),
                            stream())
        assert np.array_equal(to_host(d_part, want.nbytes), want.view(np.uint8)), (grid, block)
