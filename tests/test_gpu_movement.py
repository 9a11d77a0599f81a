"""Movement entries on the GPU against the CPU oracle, bit for bit.

tiled_transpose, materialize_strided and strided_to_strided copy element bits,
so every destination byte must equal the oracle's (reference
tests/gpu_kernels.rs:193-522): sentinel-filled destinations with guard bytes,
ragged, batched and offset transposes for every dtype, reversed and broadcast
source views, non-compact destinations, rank 0 and empty views, and the
configuration shapes C1 (transpose), C3 (rank-4 permute of a reversed view, f64
and c32) and C5 (rank-6 c64 permute).
"""
import numpy as np
import pytest

import t4a_cuda_kernels as t
from t4a_cuda_kernels import configs, hip
from gpu_util import (NUMPY, SENTINEL, random_elements, say, sentinel, stream, to_device,
                      to_host)
from oracle import t4a_oracle as orc

pytestmark = pytest.mark.gpu

ALL_DTYPES = list(t.DType)


def c_order_permute_view(c_shape, perm, dtype_size=None):
    """Source view (reference axis order) of numpy `transpose(perm)` of a
    C-contiguous array of shape `c_shape`: the output's reference axis k is
    source reference axis r-1-perm[r-1-k]."""
    r = len(c_shape)
    ref_ext = list(reversed(c_shape))
    ref_str = t.Layout.compact(ref_ext).strides
    ext = [ref_ext[r - 1 - perm[r - 1 - k]] for k in range(r)]
    st = [ref_str[r - 1 - perm[r - 1 - k]] for k in range(r)]
    return ext, st


def run_transpose(dtype, m, n, batches, offset, rng, src=None):
    es = dtype.size
    src_len = offset + m * n * batches
    src = random_elements(dtype, src_len, rng) if src is None else src
    dst_len = m * n * batches
    say("transpose", dtype.name, m, n, batches, offset)
    plan = t.plan_tiled_transpose(dtype, t.TransposeConfig.DEFAULT, offset, m * n, m, n,
                                  batches, src_len, dst_len)
    d_src = to_device(src)
    d_dst = sentinel(dst_len * es)
    hip.tiled_transpose(d_dst, d_src, dtype, offset, m * n, m, n, t.TransposeConfig.DEFAULT,
                        plan, stream())
    got = to_host(d_dst, dst_len * es)
    want = np.zeros(dst_len, dtype=NUMPY[dtype])
    orc.tiled_transpose(want, src, dtype, offset, m * n, m, n, batches)
    assert np.array_equal(got, want.view(np.uint8)), f"transpose {dtype.name} {m}x{n}x{batches}+{offset}"


@pytest.mark.parametrize("dtype", ALL_DTYPES, ids=[d.name for d in ALL_DTYPES])
def test_tiled_transpose_matches_coordinate_map(dtype):
    rng = np.random.default_rng(7)
    for m, n, batches, offset in [(1024, 1024, 1, 0), (97, 131, 1, 0), (64, 96, 3, 0),
                                  (33, 65, 2, 5), (1, 1000, 1, 0), (1000, 1, 1, 0),
                                  (256, 64, 4, 1), (130, 260, 2, 4)]:
        run_transpose(dtype, m, n, batches, offset, rng)


def test_tiled_transpose_ragged_large_and_configs():
    rng = np.random.default_rng(8)
    run_transpose(t.DType.F32, 4093, 4099, 1, 0, rng)
    run_transpose(t.DType.C64, 515, 257, 2, 3, rng)
    # Every accepted configuration computes the same map.
    src = random_elements(t.DType.F32, 200 * 300, rng)
    d_src = to_device(src)
    want = np.zeros(200 * 300, dtype=np.float32)
    orc.tiled_transpose(want, src, t.DType.F32, 0, 200 * 300, 200, 300, 1)
    for tile in (8, 16, 32):
        for rows in (4, 8, 16):
            cfg = t.TransposeConfig(tile, rows, 0, 2)
            plan = t.plan_tiled_transpose(t.DType.F32, cfg, 0, 60000, 200, 300, 1, 60000, 60000)
            d_dst = sentinel(60000 * 4)
            hip.tiled_transpose(d_dst, d_src, t.DType.F32, 0, 60000, 200, 300, cfg, plan,
                                stream())
            assert np.array_equal(to_host(d_dst, 240000), want.view(np.uint8))


def test_tiled_transpose_empty_is_no_launch():
    plan = t.plan_tiled_transpose(t.DType.F32, t.TransposeConfig.DEFAULT, 0, 0, 0, 17, 1, 0, 0)
    assert plan.is_empty()
    d = sentinel(64)
    hip.tiled_transpose(d, d, t.DType.F32, 0, 0, 0, 17, t.TransposeConfig.DEFAULT, plan,
                        stream())
    to_host(d, 0)  # every byte is still the sentinel


def test_tiled_transpose_full_size_round_trip():
    """8192^2 f32 (256 MiB a side): transposing twice is the identity."""
    m = n = 8192
    say("transpose round trip", m, n)
    host = np.random.default_rng(9).integers(-2**31, 2**31, m * n, dtype=np.int64)
    host = host.astype(np.int32)
    x = to_device(host)
    y = sentinel(m * n * 4)
    z = sentinel(m * n * 4)
    p1 = t.plan_tiled_transpose(t.DType.F32, t.TransposeConfig.DEFAULT, 0, m * n, m, n, 1,
                                m * n, m * n)
    hip.tiled_transpose(y, x, t.DType.F32, 0, m * n, m, n, t.TransposeConfig.DEFAULT, p1,
                        stream())
    hip.tiled_transpose(z, y, t.DType.F32, 0, m * n, n, m, t.TransposeConfig.DEFAULT, p1,
                        stream())
    assert np.array_equal(to_host(z, m * n * 4).view(np.int32), host)
    # dst[i + j*M] = src[i*N + j]: the first pass is the matrix transpose
    got = to_host(y, m * n * 4).view(np.int32).reshape(n, m)
    assert np.array_equal(got, host.reshape(m, n).T)


@pytest.mark.parametrize("dtype", ALL_DTYPES, ids=[d.name for d in ALL_DTYPES])
def test_copy_exact_aligned_shifted_and_tails(dtype):
    """t4a_hip_copy_exact under its plan: 16-byte aligned buffers (whole vectors
    plus a tail) and both pointers one element past a boundary (element path)."""
    rng = np.random.default_rng(11)
    for count in (1, 3, 17, 4096, 1_000_003):
        src = random_elements(dtype, count + 4, rng)
        d_src = to_device(src)
        plan = t.plan_copy_exact(dtype, count)
        for shift in (0, 1):
            say("copy_exact", dtype.name, count, "shift", shift, "grid", plan.grid)
            off = shift * dtype.size
            d_dst = sentinel((count + 1) * dtype.size)
            hip.copy_exact(d_dst.ptr + off, d_src.ptr + off, dtype, count, plan, stream())
            got = to_host(d_dst, off + count * dtype.size)
            assert (got[:off] == SENTINEL).all(), "a write landed before the destination"
            want = np.ascontiguousarray(src[shift:shift + count]).view(np.uint8)
            assert np.array_equal(got[off:], want), (dtype.name, count, shift)


def test_copy_exact_full_size():
    """256 MiB of f32 plus a three-element tail (the bench's copy, every vector
    and the element path in one launch)."""
    rng = np.random.default_rng(12)
    count = (1 << 26) + 3
    src = random_elements(t.DType.F32, count, rng)
    plan = t.plan_copy_exact(t.DType.F32, count)
    say("copy_exact full size", count, "grid", plan.grid)
    d_src = to_device(src)
    d_dst = sentinel(count * 4)
    hip.copy_exact(d_dst, d_src, t.DType.F32, count, plan, stream())
    assert np.array_equal(to_host(d_dst, count * 4), src.view(np.uint8))


def run_materialize(dtype, layout, rng, src_len=None, src=None):
    count = layout.element_count()
    src_len = src_len if src_len is not None else max(layout.max_reachable_offset() + 1, 1)
    src = random_elements(dtype, src_len, rng) if src is None else src
    say("materialize", dtype.name, layout)
    plan = t.plan_materialize_strided(dtype, layout, src_len)
    d_src = to_device(src)
    d_dst = sentinel(count * dtype.size)
    hip.materialize_strided(d_dst, d_src, dtype, layout, count, plan, stream())
    got = to_host(d_dst, count * dtype.size)
    want = np.zeros(count, dtype=NUMPY[dtype])
    orc.materialize_strided(want, src, dtype, layout, count)
    assert np.array_equal(got, want.view(np.uint8)), f"materialize {dtype.name} {layout}"


def run_strided(dtype, src_layout, dst_layout, rng, dst_len=None, src=None):
    count = src_layout.element_count()
    src_len = max(src_layout.max_reachable_offset() + 1, 1)
    dst_len = dst_len if dst_len is not None else max(dst_layout.max_reachable_offset() + 1, 1)
    src = random_elements(dtype, src_len, rng) if src is None else src
    say("strided_to_strided", dtype.name, src_layout, dst_layout)
    plan = t.plan_strided_to_strided(dtype, src_layout, src_len, dst_layout, dst_len)
    d_src = to_device(src)
    d_dst = sentinel(dst_len * dtype.size)
    hip.strided_to_strided(d_dst, d_src, dtype, src_layout, dst_layout, count, plan, stream())
    got = to_host(d_dst, dst_len * dtype.size)
    want = np.full(dst_len * dtype.size, 0xCD, dtype=np.uint8)
    orc.strided_to_strided(want, src, dtype, src_layout, dst_layout, count)
    assert np.array_equal(got, want), f"strided_to_strided {dtype.name} {src_layout} -> {dst_layout}"


def random_view(rng, rank, max_extent=9):
    """A random source view: permuted compact strides, some axes reversed (the
    offset rebased), some broadcast, a leading gap."""
    ext = [int(e) for e in rng.integers(1, max_extent + 1, rank)]
    perm = rng.permutation(rank)
    # strides of a compact layout over permuted extents keep the view injective
    ext2 = [ext[p] for p in perm]
    st = t.Layout.compact(ext2).strides
    inv = np.argsort(perm)
    ext = [ext2[i] for i in inv]
    st = [st[i] for i in inv]
    offset = int(rng.integers(0, 5))
    for k in range(rank):
        if rng.random() < 0.3 and ext[k] > 1:
            offset += (ext[k] - 1) * st[k]
            st[k] = -st[k]
        elif rng.random() < 0.1:
            st[k] = 0
    return t.Layout(ext, st, offset)


@pytest.mark.parametrize("dtype", ALL_DTYPES, ids=[d.name for d in ALL_DTYPES])
def test_materialize_strided_random_views(dtype):
    rng = np.random.default_rng(11 + int(dtype))
    run_materialize(dtype, t.Layout([], [], 3), rng, src_len=4)  # rank 0: one element
    run_materialize(dtype, t.Layout([0, 5], [1, 0], 0), rng, src_len=1)  # empty
    run_materialize(dtype, t.Layout([37, 21], [21, 1], 0), rng)  # transpose view
    run_materialize(dtype, t.Layout([64, 48], [-1, 64], 63), rng)  # reversed fast axis
    for _ in range(12):
        run_materialize(dtype, random_view(rng, int(rng.integers(1, 7))), rng)


@pytest.mark.parametrize("dtype", ALL_DTYPES, ids=[d.name for d in ALL_DTYPES])
def test_strided_to_strided_random_views(dtype):
    rng = np.random.default_rng(23 + int(dtype))
    for _ in range(12):
        src = random_view(rng, int(rng.integers(1, 7)))
        # destination: a permuted compact layout with gaps and an offset (no
        # broadcast: destinations are injective)
        ext = src.extents
        perm = rng.permutation(len(ext))
        pad = [e + int(rng.integers(0, 3)) for e in ext]
        st_p = t.Layout.compact([pad[p] for p in perm]).strides
        st = [0] * len(ext)
        for i, p in enumerate(perm):
            st[p] = st_p[i]
        run_strided(dtype, src, t.Layout(ext, st, int(rng.integers(0, 7))), rng)


def _strides(ext, order):
    st, c = [0] * len(ext), 1
    for k in order:
        st[k] = c
        c *= ext[k]
    return st


@pytest.mark.parametrize("dtype", [t.DType.F32, t.DType.I32, t.DType.F64, t.DType.C32,
                                   t.DType.C64], ids=lambda d: d.name)
def test_long_and_short_tiles(dtype):
    """Moves whose run ends at 16 or 32 elements on one side, walked with the
    long-and-short tiles (128 x 16 ... 16 x 128), full and ragged, with aligned
    buffers (16-byte vectors on both sides) and with the source or the
    destination one element off (one side element by element)."""
    rng = np.random.default_rng(90 + int(dtype))
    cases = [([64, 32, 16, 8], [2, 0, 3, 1], [0, 1, 2, 3]),
             ([64, 32, 32, 8], [2, 0, 3, 1], [0, 1, 2, 3]),
             ([32, 64, 32, 8], [1, 2, 0, 3], [0, 1, 3, 2]),
             ([16, 64, 32, 8], [1, 2, 0, 3], [0, 1, 3, 2]),
             ([64, 33, 16, 5], [2, 0, 3, 1], [0, 1, 2, 3]),
             ([16, 64, 33, 7], [1, 2, 0, 3], [0, 1, 3, 2])]
    for ext, so, do in cases:
        for s_off, d_off in ((0, 0), (1, 0), (0, 1)):
            src = t.Layout(ext, _strides(ext, so), s_off)
            dst = t.Layout(ext, _strides(ext, do), d_off)
            assert t.move_route(dtype, src, dst) == t.MoveRoute.TileOnce
            run_strided(dtype, src, dst, rng)


def test_general_routes():
    """The per-element route (tiles below 256 elements, as an [8]^6 permute
    swapping axis pairs has; a reversed fast axis) and the general tiled kernel
    (1-byte elements; chains of more than two dims), each on its route, with
    aligned and shifted buffers."""
    rng = np.random.default_rng(78)
    e6, e8 = [8] * 6, [2] * 6 + [64, 64]
    swap = t.Layout(e6, _strides(e6, [1, 0, 3, 2, 5, 4]), 0)
    long_chains = t.Layout(e8, _strides(e8, [7, 6, 5, 4, 3, 2, 1, 0]), 0)
    cases = [(t.DType.F32, swap, t.MoveRoute.Elements),
             (t.DType.C64, swap, t.MoveRoute.Elements),
             (t.DType.F32, t.Layout([512, 300], [-1, 512], 511), t.MoveRoute.Elements),
             (t.DType.Bool, t.Layout([64, 64, 128, 32], [32, 262144, -2048, 1], 260096),
              t.MoveRoute.Tiles),
             (t.DType.F32, long_chains, t.MoveRoute.Tiles),
             (t.DType.F64, long_chains, t.MoveRoute.Tiles)]
    for dtype, src, want in cases:
        dst = t.Layout.compact(src.extents)
        assert t.move_route(dtype, src, dst) == want, (dtype, src)
        for s_off, d_off in ((0, 0), (1, 3)):
            run_strided(dtype, t.Layout(src.extents, src.strides, src.offset + s_off),
                        t.Layout(dst.extents, dst.strides, d_off), rng)


def test_config_c1_transpose_and_its_8192_twin():
    """C1: f32 C-[1024, 1024] transposed (1,0), and the 8192^2 roofline twin, on
    the configuration's seeded inputs (t4a_cuda_kernels.configs)."""
    for m in (1024, 8192):
        run_transpose(t.DType.F32, m, m, 1, 0, None, src=configs.c1_input(m))


def test_config_c3_reversed_rank4_permute_f64_and_c32():
    """C3: C-shape [64,128,64,32], permutation (3,1,0,2), source axis 1 reversed,
    on the configuration's seeded N(0,1) inputs."""
    src_l = t.Layout([64, 64, 128, 32], [32, 262144, -2048, 1], 260096)
    dst_l = t.Layout.compact([64, 64, 128, 32])
    assert src_l.max_reachable_offset() + 1 == 1 << 24
    for dtype, npt in ((t.DType.F64, np.float64), (t.DType.C32, np.complex64)):
        x = configs.c3_input(npt)
        run_strided(dtype, src_l, dst_l, None, src=x)
        run_materialize(dtype, src_l, None, src=x)


def test_config_c5_rank6_c64_permute():
    """C5: c64 C-shape [16]^6 permuted by (5,2,0,4,1,3) into a compact output."""
    ext, st = c_order_permute_view([16] * 6, (5, 2, 0, 4, 1, 3))
    assert st == [256, 65536, 16, 1048576, 4096, 1]
    src_l = t.Layout(ext, st, 0)
    x = configs.c5_input()
    run_materialize(t.DType.C64, src_l, None, src=x)
    run_strided(t.DType.C64, src_l, t.Layout.compact(ext), None, src=x)
