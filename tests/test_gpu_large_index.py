"""GPU cases past the 32-bit index limits, where the kernels leave their 32-bit
fast paths: transposes, moves and reductions over more than 2^31 elements, and
a reduction with more than 2^32 outputs. Each is checked on the host against
the closed form of its map (the transpose's, the reversal's, the row copy's),
or against exact integer sums of a periodic input.

- The reference's own limit test (tests/gpu_kernels.rs:466-522): a Bool
  transpose of a 2^31 x 1 and a (2^31 - 1) x 1 matrix, a byte copy compared
  with the whole source, and the byte past the shape keeping the sentinel. It
  runs through this library's launcher and through the reference-named entry
  under the reference planner's geometry (grid (2^27, 1, 1), blocks 16 x 8).
- A Bool transpose of 65552 x 32784 (2^31 + 1,572,864 elements): whole 128 x 128
  tiles with 64-bit addresses past 2^31, and edge tiles on both sides.
- The launcher's unordered tile walk (planned blocks under a 2-D grid).
- A reversed-view Bool materialize of 2^31 + 17 elements (the per-element
  route) and a row copy of 2^26 rows of 33 bytes into 40-byte pitches (2^31 +
  67M units: the row route's 64-bit fallback).
- An I32 sum over one axis of 2^31 + 33 elements (4096 splits; partials and
  the final checked against exact sums).
- A unit reduction over an extent-1 axis with 65537 x 65537 outputs in a padded
  layout (two output dims, extent product past 2^32: 64-bit output digits).

Device memory: at most ~35 GB at once. The inputs are periodic blocks of a
prime length, so a misplaced element cannot land on an equal value.
"""
import ctypes
from pathlib import Path

import numpy as np
import pytest

import t4a_cuda_kernels as t
from t4a_cuda_kernels import configs, hip, hipmem
from gpu_util import SENTINEL, say

pytestmark = pytest.mark.gpu

Bool, I32 = t.DType.Bool, t.DType.I32
PKG = Path(t.__file__).resolve().parent
PRIME = 1_000_003  # period of the byte patterns


def pattern_bytes(n: int, seed: int) -> np.ndarray:
    """n bytes repeating a random block of PRIME bytes."""
    block = configs.integers(seed, PRIME, 0, 255, np.uint8)
    return np.resize(block, n)


def sentinel_buffer(nbytes: int, guard: int = 256) -> hipmem.DeviceBuffer:
    buf = hipmem.DeviceBuffer(nbytes + guard)
    buf.fill(SENTINEL)
    return buf


@pytest.fixture(scope="module")
def movement_module():
    mod = hipmem.Module(PKG / "t4a_movement.gfx950.hsaco")
    yield mod
    hipmem.synchronize()
    mod.unload()


@pytest.fixture(scope="module")
def reduce_module():
    mod = hipmem.Module(PKG / "t4a_reduce.gfx950.hsaco")
    yield mod
    hipmem.synchronize()
    mod.unload()


def ref_transpose_geometry(m: int, n: int, batches: int = 1):
    """The reference plan_tiled_transpose's geometry for the default config
    (tile 16, 8 block rows, padding 1, vector width 1; src/lib.rs:1685-1737)."""
    cfg = t.TransposeConfig.DEFAULT
    grid = (-(-m // cfg.tile), -(-n // cfg.tile), batches)
    block = (cfg.tile // cfg.vector_width, cfg.block_rows, 1)
    return grid, block, cfg.tile * (cfg.tile + cfg.padding)


def transpose(who, mod, d_dst, d_src, dtype, m, n):
    cfg = t.TransposeConfig.DEFAULT
    if who == "launcher":
        plan = t.plan_tiled_transpose(dtype, cfg, 0, m * n, m, n, 1, m * n, m * n)
        hip.tiled_transpose(d_dst, d_src, dtype, 0, m * n, m, n, cfg, plan, None)
    else:
        mod.launch("t4a_cuda_tiled_transpose", *ref_transpose_geometry(m, n), None,
                   [ctypes.c_void_p(d_dst.ptr), ctypes.c_void_p(d_src.ptr), ctypes.c_int(dtype),
                    ctypes.c_longlong(0), ctypes.c_longlong(m * n), ctypes.c_longlong(m),
                    ctypes.c_longlong(n), cfg.c])
    hipmem.synchronize()


@pytest.mark.parametrize("who", ["launcher", "reference geometry"])
def test_bool_transpose_crosses_the_narrow_index_limit(movement_module, who):
    length = (1 << 31) + 1  # one byte past the wider shape
    values = np.resize((np.arange(4096) % 251).astype(np.uint8), length)
    d_src = hipmem.DeviceBuffer.from_array(values)
    for dst_fast in (1 << 31, (1 << 31) - 1):
        say("Bool transpose", dst_fast, "x 1", who)
        d_dst = sentinel_buffer(length, guard=0)
        transpose(who, movement_module, d_dst, d_src, Bool, dst_fast, 1)
        got = d_dst.download()
        assert np.array_equal(got[:dst_fast], values[:dst_fast]), (dst_fast, who)
        assert got[dst_fast] == SENTINEL, (dst_fast, who)
        del d_dst


@pytest.mark.parametrize("who", ["launcher", "reference geometry"])
def test_bool_transpose_of_more_than_2_31_elements(movement_module, who):
    m, n = 65552, 32784  # 513 x 257 tiles of 128 x 128, partial on both sides
    assert m * n > (1 << 31)
    src = pattern_bytes(m * n, 501)
    d_src = hipmem.DeviceBuffer.from_array(src)
    d_dst = sentinel_buffer(m * n)
    say("Bool transpose", m, "x", n, who)
    transpose(who, movement_module, d_dst, d_src, Bool, m, n)
    got = d_dst.download()
    assert (got[m * n:] == SENTINEL).all(), "a write past the matrix"
    dst2 = got[:m * n].reshape(n, m)  # dst[j, i] = src[i, j]
    src2 = src.reshape(m, n)
    for j0 in range(0, n, 2048):
        j1 = min(n, j0 + 2048)
        assert np.array_equal(dst2[j0:j1], src2[:, j0:j1].T), (who, j0)


@pytest.mark.parametrize("dtype", list(t.DType), ids=[d.name for d in t.DType])
def test_launcher_unordered_tile_walk(dtype):
    """Planned 512-thread blocks under a grid with a second dimension take the
    launcher's unordered (64-bit) tile walk; its map must be the transpose."""
    m, n = 300, 517
    from gpu_util import random_elements
    src = random_elements(dtype, m * n, np.random.default_rng(502))
    want = np.ascontiguousarray(src.reshape(m, n).T)
    d_src = hipmem.DeviceBuffer.from_array(src)
    for grid in ((3, 2, 1), (7, 5, 1), (40, 1, 1)):
        d_dst = sentinel_buffer(src.nbytes)
        launch = t.Launch(grid, (512, 1, 1), 0)
        say("unordered tile walk", dtype.name, m, n, grid)
        hip.tiled_transpose(d_dst, d_src, dtype, 0, m * n, m, n, t.TransposeConfig.DEFAULT,
                            launch, None)
        got = d_dst.download()
        assert np.array_equal(got[:src.nbytes], want.view(np.uint8).reshape(-1)), grid
        assert (got[src.nbytes:] == SENTINEL).all()


@pytest.mark.parametrize("who", ["launcher", "reference geometry"])
def test_reversed_bool_view_past_2_31(movement_module, who):
    n = (1 << 31) + 17
    src_l = t.Layout([n], [-1], n - 1)
    assert t.move_route(Bool, src_l) == t.MoveRoute.Elements
    src = pattern_bytes(n, 503)
    d_src = hipmem.DeviceBuffer.from_array(src)
    d_dst = sentinel_buffer(n)
    say("reversed Bool materialize", n, who)
    if who == "launcher":
        plan = t.plan_materialize_strided(Bool, src_l, n)
        hip.materialize_strided(d_dst, d_src, Bool, src_l, n, plan, None)
    else:
        movement_module.launch("t4a_cuda_materialize_strided", (-(-n // 256), 1, 1),
                               (256, 1, 1), 0, None,
                               [ctypes.c_void_p(d_dst.ptr), ctypes.c_void_p(d_src.ptr),
                                ctypes.c_int(Bool), src_l.c, ctypes.c_longlong(n)])
    hipmem.synchronize()
    got = d_dst.download()
    assert np.array_equal(got[:n], src[::-1]), who
    assert (got[n:] == SENTINEL).all()


def test_row_copy_past_2_31_units():
    rows, width, pitch = 1 << 26, 33, 40
    src_l = t.Layout.compact([width, rows])
    dst_l = t.Layout([width, rows], [1, pitch], 0)
    assert t.move_route(Bool, src_l, dst_l) == t.MoveRoute.Elements
    count = width * rows
    assert count > (1 << 31)
    src = pattern_bytes(count, 504)
    d_src = hipmem.DeviceBuffer.from_array(src)
    d_dst = sentinel_buffer(pitch * rows)
    dst_len = dst_l.max_reachable_offset() + 1
    plan = t.plan_strided_to_strided(Bool, src_l, count, dst_l, dst_len)
    say("Bool rows", rows, "x", width, "into pitch", pitch)
    hip.strided_to_strided(d_dst, d_src, Bool, src_l, dst_l, count, plan, None)
    hipmem.synchronize()
    got = d_dst.download()
    body = got[:pitch * rows].reshape(rows, pitch)
    assert np.array_equal(body[:, :width], src.reshape(rows, width))
    assert (body[:, width:] == SENTINEL).all(), "a write between the rows"
    assert (got[pitch * rows:] == SENTINEL).all()


def periodic_sum(prefix: np.ndarray, a: int, b: int) -> int:
    """Exact sum of x[a:b] for x[i] = block[i % P], `prefix` the block's int64
    prefix sums (length P + 1)."""
    p = len(prefix) - 1
    return int((b // p - a // p) * int(prefix[p]) + int(prefix[b % p]) - int(prefix[a % p]))


def wrap32(v: int) -> int:
    return (v + (1 << 31)) % (1 << 32) - (1 << 31)


def upload_periodic(buf: hipmem.DeviceBuffer, block: np.ndarray, count: int,
                    chunk: int = 1 << 24) -> None:
    """x[i] = block[i % len(block)] for i < count, uploaded chunk by chunk."""
    p = len(block)
    doubled = np.resize(block, chunk + p)
    for a in range(0, count, chunk):
        b = min(count, a + chunk)
        buf.upload(doubled[a % p:a % p + (b - a)], offset=a * block.itemsize)


def test_i32_sum_over_more_than_2_31_elements():
    n = (1 << 31) + 33
    in_l, out_l = t.Layout.compact([n]), t.Layout.compact([1])
    plan = t.plan_reduction(I32, t.ReduceOp.Sum, out_l, 1, in_l, n, 0, 32)
    assert plan.kind == "Split"
    splits, chunk = plan.split.splits, plan.split.chunk_len
    block = configs.integers(505, PRIME, -1000, 1000, np.int32)
    prefix = np.concatenate([[0], np.cumsum(block, dtype=np.int64)])
    bounds = [(c * chunk, (c + 1) * chunk if c + 1 < splits else n) for c in range(splits)]
    want_part = np.array([wrap32(periodic_sum(prefix, a, b)) for a, b in bounds], np.int64)
    want = wrap32(periodic_sum(prefix, 0, n))
    d_in = hipmem.DeviceBuffer(n * 4)
    upload_periodic(d_in, block, n)
    pl = t.reduction_partials_layout(in_l, 0, splits)
    for how in ("reduction", "two launches"):
        d_out, d_part = sentinel_buffer(4), sentinel_buffer(splits * 4)
        say("I32 sum over", n, "elements,", splits, "splits,", how)
        if how == "reduction":
            hip.reduction(plan, d_out, d_in, d_part, I32, t.ReduceOp.Sum, out_l, in_l, 0, 1,
                          None)
        else:
            hip.enqueue_reduction(plan, d_out, d_in, d_part, I32, t.ReduceOp.Sum, out_l, in_l,
                                  0, 1, None)
        hipmem.synchronize()
        part = d_part.download(splits * 4).view(np.int32)
        assert np.array_equal(part.astype(np.int64), want_part), how
        assert d_out.download(4).view(np.int32)[0] == want, how
        assert (d_out.download(256, 4) == SENTINEL).all()
        assert pl.element_count() == splits


def test_unit_reduce_with_more_than_2_32_outputs():
    a = 65537  # outputs a x a in rows of pitch a + 1: two output digits, 64-bit
    in_l = t.Layout.compact([1, a, a])
    out_l = t.Layout([1, a, a], [1, 1, a + 1], 0)
    outputs = a * a
    assert outputs > (1 << 32)
    out_len = out_l.max_reachable_offset() + 1
    plan = t.plan_reduce(I32, t.ReduceOp.Sum, t.ReduceStrategy.Unit, out_l, out_len, in_l,
                         outputs, 0, 32)
    block = configs.integers(506, PRIME, -(1 << 31), (1 << 31) - 1, np.int32)
    d_in = hipmem.DeviceBuffer(outputs * 4)
    upload_periodic(d_in, block, outputs)
    d_out = sentinel_buffer(out_len * 4 + 4)
    say("I32 unit reduce over an extent-1 axis,", outputs, "outputs")
    hip.reduce(d_out, d_in, I32, t.ReduceOp.Sum, t.ReduceStrategy.Unit, out_l, in_l, 0,
               outputs, plan, None)
    hipmem.synchronize()
    # Rows around the 2^31 and 2^32 output indices, the first and the last.
    rows = sorted({0, 1, 2, (1 << 31) // a - 1, (1 << 31) // a, (1 << 31) // a + 1,
                   (1 << 32) // a - 1, (1 << 32) // a, (1 << 32) // a + 1, a - 2, a - 1}
                  | set(np.random.default_rng(507).integers(0, a, 40).tolist()))
    for r in rows:
        got = d_out.download((a + 1) * 4, r * (a + 1) * 4).view(np.int32)
        idx = (r * a + np.arange(a)) % PRIME
        assert np.array_equal(got[:a], block[idx]), r
        assert got[a].view(np.uint32) == 0xCDCDCDCD, ("a write into the row pad", r)
