"""The reference-named kernel entries, loaded by name from the gfx950 code
objects and launched with `hipModuleLaunchKernel` + `kernelParams`, the way
the reference's callers launch its cubins (reference tests/gpu/mod.rs:81-111,
297-324), bit for bit against the CPU oracle.

Each entry runs under two geometries: the one the reference's own planner
returns (restated below from src/lib.rs) -- a caller that keeps the reference
crate's planning and swaps only the kernel module -- and the one this build's
planner returns.
"""
from pathlib import Path

import numpy as np
import pytest

import t4a_cuda_kernels as t
from t4a_cuda_kernels import hipmem
from gpu_util import NUMPY, random_elements, say, sentinel, to_device, to_host
from oracle import t4a_oracle as orc

pytestmark = pytest.mark.gpu

PKG = Path(t.__file__).resolve().parent
REAL = [t.DType.F32, t.DType.F64, t.DType.I32, t.DType.I64, t.DType.C32, t.DType.C64]
OPS = list(t.ReduceOp)


@pytest.fixture(scope="module")
def modules():
    mods = {"movement": hipmem.Module(PKG / "t4a_movement.gfx950.hsaco"),
            "reduce": hipmem.Module(PKG / "t4a_reduce.gfx950.hsaco")}
    yield mods
    hipmem.synchronize()
    for m in mods.values():
        m.unload()


# ---- the reference planner's geometry (src/lib.rs), restated -------------------------

def ceil_div(a, b):
    return -(-a // b)


def ref_flat(length):
    """flat_launch (src/lib.rs:1465-1482): 256-thread blocks, one thread per element."""
    return (ceil_div(length, 256), 1, 1), (256, 1, 1), 0


def ref_transpose(cfg, m, n, batches, esize):
    """plan_tiled_transpose (src/lib.rs:1685-1737)."""
    grid = (ceil_div(m, cfg.tile), ceil_div(n, cfg.tile), batches)
    block = (cfg.tile // cfg.vector_width, cfg.block_rows, 1)
    return grid, block, cfg.tile * (cfg.tile + cfg.padding) * esize


def ref_reduce(strategy, output_len, width):
    """launch_for (src/lib.rs:3242-3286)."""
    if strategy == t.ReduceStrategy.Unit:
        return (ceil_div(output_len, width), 1, 1), (width, 1, 1), 0
    return (output_len, 1, 1), (width, 1, 1), 0


def ref_partials(cubes, chunk_len, width):
    """plan_reduce_partials (src/lib.rs:3412-3430): four 32-lane planes per block
    up to 8192 cubes of at most 1024 elements, else one plane per block."""
    planes = 4 if width == 32 and cubes <= 8192 and chunk_len <= 1024 else 1
    return (ceil_div(cubes, planes), 1, 1), (width * planes, 1, 1), 0


def ours(launch):
    return tuple(launch.grid), tuple(launch.block), launch.shared_bytes


def ptr(buf, offset=0):
    import ctypes
    return ctypes.c_void_p(buf.ptr + offset)


def c_int(v):
    import ctypes
    return ctypes.c_int(int(v))


def c_ll(v):
    import ctypes
    return ctypes.c_longlong(int(v))


# ---- movement --------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", list(t.DType), ids=[d.name for d in t.DType])
def test_module_tiled_transpose(modules, dtype):
    rng = np.random.default_rng(31)
    configs = [t.TransposeConfig.DEFAULT, t.TransposeConfig(32, 8, 1, 4),
               t.TransposeConfig(8, 4, 0, 1)]
    for m, n, batches, offset in [(97, 131, 1, 0), (64, 96, 3, 0), (33, 65, 2, 5),
                                  (1024, 1024, 1, 0)]:
        src = random_elements(dtype, offset + m * n * batches, rng)
        d_src = to_device(src)
        want = np.zeros(m * n * batches, dtype=NUMPY[dtype])
        orc.tiled_transpose(want, src, dtype, offset, m * n, m, n, batches)
        for cfg in configs:
            plan = t.plan_tiled_transpose(dtype, cfg, offset, m * n, m, n, batches, src.size,
                                          want.size)
            for who, geo in (("reference", ref_transpose(cfg, m, n, batches, dtype.size)),
                             ("ours", ours(plan))):
                say("module transpose", dtype.name, m, n, batches, offset, cfg, who, geo)
                d_dst = sentinel(want.nbytes)
                modules["movement"].launch(
                    "t4a_cuda_tiled_transpose", *geo, None,
                    [ptr(d_dst), ptr(d_src), c_int(dtype), c_ll(offset), c_ll(m * n), c_ll(m),
                     c_ll(n), cfg.c])
                got = to_host(d_dst, want.nbytes)
                assert np.array_equal(got, want.view(np.uint8)), (m, n, batches, cfg, who)


@pytest.mark.parametrize("dtype", [t.DType.Bool, t.DType.F32, t.DType.F64, t.DType.C64],
                         ids=lambda d: d.name)
def test_module_copy_exact(modules, dtype):
    rng = np.random.default_rng(32)
    for count in (1, 1000, 1000003):
        src = random_elements(dtype, count + 4, rng)
        d_src = to_device(src)
        # aligned buffers, then both pointers one element past a 16-byte boundary
        for shift in (0, 1):
            want = src[shift:shift + count]
            plan = t.plan_copy_exact(dtype, count)
            for who, geo in (("reference", ref_flat(count)), ("ours", ours(plan))):
                say("module copy_exact", dtype.name, count, shift, who, geo)
                d_dst = sentinel((count + 1) * dtype.size)
                off = shift * dtype.size
                modules["movement"].launch("t4a_cuda_copy_exact", *geo, None,
                                           [ptr(d_dst, off), ptr(d_src, off), c_int(dtype),
                                            c_ll(count)])
                got = to_host(d_dst, off + count * dtype.size)[off:]
                assert np.array_equal(got, np.ascontiguousarray(want).view(np.uint8))


def permuted_views(rng):
    """(src view, dst layout) pairs: the C3 and C5 structures at reduced size, a
    reversed axis, a broadcast axis, rank 0 and 1, and random permutations."""
    views = []
    views.append((t.Layout([16, 8, 32, 8], [8, 4096, -128, 1], 31 * 128),
                  t.Layout.compact([16, 8, 32, 8])))
    views.append((t.Layout([8] * 6, [64, 4096, 8, 32768, 512, 1], 0), t.Layout.compact([8] * 6)))
    views.append((t.Layout([300, 7], [0, 1], 0), t.Layout.compact([300, 7])))
    views.append((t.Layout([], [], 3), t.Layout.compact([])))
    views.append((t.Layout([1000], [-1], 999), t.Layout.compact([1000])))
    for _ in range(6):
        rank = int(rng.integers(2, 6))
        ext = [int(e) for e in rng.integers(2, 24, rank)]
        perm = rng.permutation(rank)
        cst = t.Layout.compact([ext[p] for p in perm]).strides
        st = [0] * rank
        for i, p in enumerate(perm):
            st[p] = cst[i]
        views.append((t.Layout(ext, st, 0), t.Layout.compact(ext)))
    return views


@pytest.mark.parametrize("dtype", [t.DType.Bool, t.DType.F32, t.DType.F64, t.DType.C64],
                         ids=lambda d: d.name)
def test_module_strided_movement(modules, dtype):
    rng = np.random.default_rng(33)
    for src_l, dst_l in permuted_views(rng):
        count = src_l.element_count()
        src_len = src_l.max_reachable_offset() + 1
        src = random_elements(dtype, src_len, rng)
        d_src = to_device(src)
        want = np.zeros(count, dtype=NUMPY[dtype])
        orc.materialize_strided(want, src, dtype, src_l, count)
        plan_m = t.plan_materialize_strided(dtype, src_l, src_len)
        for who, geo in (("reference", ref_flat(count)), ("ours", ours(plan_m))):
            say("module materialize", dtype.name, src_l.extents, src_l.strides, who, geo)
            d_dst = sentinel(want.nbytes)
            modules["movement"].launch("t4a_cuda_materialize_strided", *geo, None,
                                       [ptr(d_dst), ptr(d_src), c_int(dtype), src_l.c,
                                        c_ll(count)])
            assert np.array_equal(to_host(d_dst, want.nbytes), want.view(np.uint8)), who
        # strided_to_strided into the transposed (reversed-order) compact layout
        rank = len(src_l.extents)
        rev = t.Layout.compact(list(reversed(src_l.extents))).strides
        dst2 = t.Layout(src_l.extents, list(reversed(rev)), 0) if rank else dst_l
        dst_len = dst2.max_reachable_offset() + 1
        want2 = np.zeros(dst_len, dtype=NUMPY[dtype])
        orc.strided_to_strided(want2, src, dtype, src_l, dst2, count)
        plan_s = t.plan_strided_to_strided(dtype, src_l, src_len, dst2, dst_len)
        for who, geo in (("reference", ref_flat(count)), ("ours", ours(plan_s))):
            say("module strided_to_strided", dtype.name, src_l.extents, who, geo)
            d_dst = sentinel(want2.nbytes)
            modules["movement"].launch("t4a_cuda_strided_to_strided", *geo, None,
                                       [ptr(d_dst), ptr(d_src), c_int(dtype), src_l.c,
                                        dst2.c, c_ll(count)])
            assert np.array_equal(to_host(d_dst, want2.nbytes), want2.view(np.uint8)), who


# ---- reductions ------------------------------------------------------------------------

def reduce_inputs(dtype, n, rng):
    if dtype in (t.DType.I32, t.DType.I64):
        return rng.integers(-3, 4, n).astype(NUMPY[dtype])
    return random_elements(dtype, n, rng)


def supported(dtype, op):
    try:
        t.plan_reduce(dtype, op, t.ReduceStrategy.Unit, t.Layout.compact([1]), 1,
                      t.Layout.compact([4]), 4, 0, 32)
        return True
    except t.T4aError:
        return False


@pytest.mark.parametrize("dtype", REAL, ids=[d.name for d in REAL])
def test_module_reduce(modules, dtype):
    rng = np.random.default_rng(34)
    for extents, axis in [([4, 300], 0), ([300, 16, 3], 1), ([37, 5], 0), ([5, 600], 1),
                          ([3, 70, 2], 1), ([1, 1], 0)]:
        n = int(np.prod(extents))
        x = reduce_inputs(dtype, n, rng)
        d_in = to_device(x)
        in_l = t.Layout.compact(extents)
        oe = list(extents)
        oe[axis] = 1
        out_l = t.Layout.compact(oe)
        on = out_l.element_count()
        length = extents[axis]
        for op in OPS:
            if not supported(dtype, op):
                continue
            # every (strategy, width) the planner accepts for this axis length
            cases = [(s, w) for w in (8, 16, 32) for s in t.ReduceStrategy]
            if length >= 512:
                cases += [(t.ReduceStrategy.Plane, w) for w in (64, 128, 256, 512)]
            for strategy, width in cases:
                try:
                    plan = t.plan_reduce(dtype, op, strategy, out_l, on, in_l, n, axis, width)
                except t.T4aError as e:
                    assert e.error == t.Error.StrategyMismatch, e
                    continue
                want = np.zeros(on, dtype=NUMPY[dtype])
                orc.reduce(want, x, dtype, op, strategy, width, out_l, in_l, axis, on)
                for who, geo in (("reference", ref_reduce(strategy, on, width)),
                                 ("ours", ours(plan))):
                    say("module reduce", dtype.name, op.name, extents, axis, strategy.name,
                        width, who, geo)
                    d_out = sentinel(want.nbytes)
                    modules["reduce"].launch(
                        "t4a_cuda_reduce", *geo, None,
                        [ptr(d_out), ptr(d_in), c_int(dtype), c_int(op), c_int(strategy),
                         out_l.c, in_l.c, c_int(axis), c_ll(on)])
                    got = to_host(d_out, want.nbytes)
                    assert np.array_equal(got, want.view(np.uint8)), (extents, axis, op,
                                                                      strategy, width, who)


@pytest.mark.parametrize("dtype", REAL, ids=[d.name for d in REAL])
def test_module_wide_plane_boundaries(modules, dtype):
    """The entry's wide plane folds (widths 64-512) at axis lengths on both sides
    of the plane body's switch from up-front loads (16 * width) to the serial
    walk (16 * width + 1, about 40 * width), under both geometries."""
    rng = np.random.default_rng(36)
    for width in (64, 128, 256, 512):
        for extents, axis in [([16 * width, 2], 0), ([16 * width + 1, 2], 0),
                              ([40 * width + 3, 1], 0), ([3, 16 * width + 1], 1)]:
            n = int(np.prod(extents))
            x = reduce_inputs(dtype, n, rng)
            d_in = to_device(x)
            in_l = t.Layout.compact(extents)
            oe = list(extents)
            oe[axis] = 1
            out_l = t.Layout.compact(oe)
            on = out_l.element_count()
            for op in (t.ReduceOp.Sum, t.ReduceOp.Max):
                if not supported(dtype, op):
                    continue
                plan = t.plan_reduce(dtype, op, t.ReduceStrategy.Plane, out_l, on, in_l, n, axis,
                                     width)
                want = np.zeros(on, dtype=NUMPY[dtype])
                orc.reduce(want, x, dtype, op, t.ReduceStrategy.Plane, width, out_l, in_l, axis,
                           on)
                for who, geo in (("reference", ref_reduce(t.ReduceStrategy.Plane, on, width)),
                                 ("ours", ours(plan))):
                    say("module wide plane", dtype.name, op.name, extents, axis, width, who, geo)
                    d_out = sentinel(want.nbytes)
                    modules["reduce"].launch(
                        "t4a_cuda_reduce", *geo, None,
                        [ptr(d_out), ptr(d_in), c_int(dtype), c_int(op),
                         c_int(t.ReduceStrategy.Plane), out_l.c, in_l.c, c_int(axis), c_ll(on)])
                    got = to_host(d_out, want.nbytes)
                    assert np.array_equal(got, want.view(np.uint8)), (extents, axis, op, width,
                                                                      who)


@pytest.mark.parametrize("dtype", REAL, ids=[d.name for d in REAL])
def test_module_reduce_partials(modules, dtype):
    rng = np.random.default_rng(35)
    shapes = [([3, 5000], 1), ([40000], 0), ([2600, 3], 0), ([64, 3000], 1)]
    if dtype in (t.DType.F32, t.DType.I32):
        shapes.append(([5000000], 0))  # 4096 splits of 1220: one plane per block
    for extents, axis in shapes:
        n = int(np.prod(extents))
        x = reduce_inputs(dtype, n, rng)
        d_in = to_device(x)
        in_l = t.Layout.compact(extents)
        oe = list(extents)
        oe[axis] = 1
        on = t.Layout.compact(oe).element_count()
        for op in OPS:
            if not supported(dtype, op):
                continue
            for width in (8, 16, 32):
                split = t.split_policy(extents[axis], width)
                if split is None:
                    continue
                pl = t.reduction_partials_layout(in_l, axis, split.splits)
                want = np.zeros(pl.element_count(), dtype=NUMPY[dtype])
                orc.reduce_partials(want, x, dtype, op, width, pl, in_l, axis, on,
                                    split.splits, split.chunk_len)
                plan = t.plan_reduce_partials(dtype, op, pl, pl.element_count(), in_l, n, axis,
                                              split, width)
                for who, geo in (("reference", ref_partials(on * split.splits,
                                                            split.chunk_len, width)),
                                 ("ours", ours(plan))):
                    say("module reduce_partials", dtype.name, op.name, extents, axis, width,
                        split.splits, split.chunk_len, who, geo)
                    d_part = sentinel(want.nbytes)
                    modules["reduce"].launch(
                        "t4a_cuda_reduce_partials", *geo, None,
                        [ptr(d_part), ptr(d_in), c_int(dtype), c_int(op), pl.c, in_l.c,
                         c_int(axis), c_ll(on), c_ll(split.splits), c_ll(split.chunk_len)])
                    got = to_host(d_part, want.nbytes)
                    assert np.array_equal(got, want.view(np.uint8)), (extents, axis, op, width,
                                                                      who)


# Pass-1 shapes that take the entry's column and lean mappings under both
# geometries: a strided axis with 8192 / 256 / 96 neighbouring columns (the
# reference's one-plane 32-thread blocks, its four-plane 128-thread blocks, and
# ours), and a contiguous axis in 256-element chunks (lean, one and four planes
# per block), with a 4-byte-misaligned input (no lean, no paired columns) and a
# partial last column block.
ROUTE_SHAPES = [([8192, 700], 1, 0), ([256, 2000], 1, 0), ([96, 3000], 1, 0),
                ([8192, 512], 0, 0), ([8192, 64], 0, 0), ([8192, 600], 1, 1),
                ([8192, 512], 0, 1), ([200, 900], 1, 0)]


@pytest.mark.parametrize("dtype", REAL, ids=[d.name for d in REAL])
def test_module_reduce_partials_routes(modules, dtype):
    rng = np.random.default_rng(36)
    es = dtype.size
    for extents, axis, lead in ROUTE_SHAPES:
        n = int(np.prod(extents))
        x = reduce_inputs(dtype, n + lead, rng)
        d_in = to_device(x)
        in_l = t.Layout(list(extents), t.Layout.compact(extents).strides, lead)
        oe = list(extents)
        oe[axis] = 1
        on = t.Layout.compact(oe).element_count()
        split = t.split_policy(extents[axis], 32)
        assert split is not None, extents
        pl = t.reduction_partials_layout(in_l, axis, split.splits)
        for op in OPS:
            if not supported(dtype, op):
                continue
            want = np.zeros(pl.element_count(), dtype=NUMPY[dtype])
            orc.reduce_partials(want, x, dtype, op, 32, pl, in_l, axis, on, split.splits,
                                split.chunk_len)
            plan = t.plan_reduce_partials(dtype, op, pl, pl.element_count(), in_l, n + lead,
                                          axis, split, 32)
            for who, geo in (("reference", ref_partials(on * split.splits, split.chunk_len, 32)),
                             ("ours", ours(plan))):
                say("module reduce_partials route", dtype.name, op.name, extents, axis, lead,
                    split.splits, split.chunk_len, who, geo)
                d_part = sentinel(want.nbytes)
                modules["reduce"].launch(
                    "t4a_cuda_reduce_partials", *geo, None,
                    [ptr(d_part), ptr(d_in), c_int(dtype), c_int(op), pl.c, in_l.c,
                     c_int(axis), c_ll(on), c_ll(split.splits), c_ll(split.chunk_len)])
                got = to_host(d_part, want.nbytes)
                assert np.array_equal(got, want.view(np.uint8)), (extents, axis, lead, op, who)
