"""fill_zero, fill_zero_view, contiguous_to_view, broadcast_in_dim and
concatenate_copy on the GPU, bit for bit against the CPU oracle (rank <= 8)
or a numpy gather (wider), through three doors each:

- the C-ABI launchers (t4a_hip_*) under this build's planned geometry;
- the reference-named kernel entries from the code object, launched with
  hipModuleLaunchKernel under the reference planner's flat geometry
  (src/lib.rs:1465-1482: 256-thread blocks, one thread per element) and
  under ours;
- the general-rank `_any` twins with their geometry arrays in device memory.

Cases follow the reference's own tests: tests/gpu_kernels.rs:100-140, 260-290,
745-815 (fill counts, views, reversed destinations), tests/gpu_remaining_families.rs:
270-370 (broadcast identity map for every dtype, a broadcast axis, a
non-self-inverse permutation, a scalar input, rank 9 and 16), 400-600
(concatenate in stream order for every dtype, a non-compact destination,
rank 16), 600-680 (NaN payloads, signed zeros, a strided source), 720-800
(the twins agree up to rank 8), 810-900 (reverse as a scatter).
"""
import ctypes
import random
from pathlib import Path

import numpy as np
import pytest

import t4a_cuda_kernels as t
from t4a_cuda_kernels import DType, Layout, WideLayout, hip, hipmem
from gpu_util import NUMPY, SENTINEL, random_elements, say, sentinel, stream, to_device, to_host
from oracle import t4a_oracle as orc

pytestmark = pytest.mark.gpu

PKG = Path(t.__file__).resolve().parent
F32, F64 = DType.F32, DType.F64
ALL = list(DType)


@pytest.fixture(scope="module")
def movement():
    mod = hipmem.Module(PKG / "t4a_movement.gfx950.hsaco")
    yield mod
    hipmem.synchronize()
    mod.unload()


def ptr(buf, offset=0):
    return ctypes.c_void_p(buf.ptr + offset)


def c_int(v):
    return ctypes.c_int(int(v))


def c_ll(v):
    return ctypes.c_longlong(int(v))


def ref_flat(length):
    """The reference's flat_launch (src/lib.rs:1465-1482)."""
    return (-(-length // 256), 1, 1), (256, 1, 1), 0


def ours(launch):
    return tuple(launch.grid), tuple(launch.block), launch.shared_bytes


class Geometry:
    """A layout's arrays in device memory and its t4a_cuda_layout_any."""

    def __init__(self, layout):
        w = layout if isinstance(layout, WideLayout) else WideLayout.of(layout)
        self.ext = to_device(np.array(w.extents or [0], dtype=np.int64))
        self.st = to_device(np.array(w.strides or [0], dtype=np.int64))
        self.c = w.device_c(self.ext.ptr, self.st.ptr)


class DeviceDims:
    def __init__(self, dims):
        self.buf = to_device(np.array(list(dims) or [0], dtype=np.int64))
        self.c = t.axis_values_any(list(dims), self.buf.ptr)


def view_indices(ext, st, offset=0):
    """Element offsets of a view in flat logical order (axis 0 fastest)."""
    idx = np.array([offset], dtype=np.int64)
    for k in reversed(range(len(ext))):
        idx = (idx[:, None] + np.arange(ext[k], dtype=np.int64)[None, :] * st[k]).ravel()
    return idx


def count(ext):
    n = 1
    for e in ext:
        n *= e
    return n


def strided_view(rng, rank, max_ext=6, neg=0.3, gap=0.3):
    """An injective view: a random axis order, optional gaps between axes and
    reversed axes (offset moved to keep every index >= 0). Extents shrink with
    the rank so that a view spans at most a few million elements."""
    max_ext = min(max_ext, 6 if rank <= 3 else 4 if rank <= 5 else 3)
    ext = [int(rng.integers(1, max_ext + 1)) for _ in range(rank)]
    order = list(rng.permutation(rank))
    st = [0] * rank
    s = 1
    for k in order:
        st[k] = s
        s *= ext[k] * (2 if rng.random() < gap else 1)
    off = int(rng.integers(0, 3))
    for k in range(rank):
        if rng.random() < neg:
            off += (ext[k] - 1) * st[k]
            st[k] = -st[k]
    return ext, st, off


# ----------------------------------------------------------------- fill_zero

@pytest.mark.parametrize("dtype", ALL, ids=lambda d: d.name)
def test_fill_zero_counts_and_alignments(movement, dtype):
    rng = np.random.default_rng(60)
    es = dtype.size
    for n in (1, 255, 256, 257, 1000, 1000003):
        for shift in (0, 1):
            plan = t.plan_fill_zero(dtype, n)
            for who in ("launcher", "reference", "ours"):
                say("fill_zero", dtype.name, n, shift, who)
                base = random_elements(dtype, n + 2, rng)
                d = to_device(base)
                off = shift * es
                if who == "launcher":
                    hip.fill_zero(d.ptr + off, dtype, n, plan, stream())
                else:
                    geo = ref_flat(n) if who == "reference" else ours(plan)
                    movement.launch("t4a_cuda_fill_zero", *geo, None,
                                    [ptr(d, off), c_int(dtype), c_ll(n)])
                got = to_host(d, (n + 2) * es, "fill_zero")
                want = base.copy().view(np.uint8)
                want[off:off + n * es] = 0
                assert np.array_equal(got, want), (n, shift, who)


# ------------------------------------------------------------ fill_zero_view

@pytest.mark.parametrize("dtype", ALL, ids=lambda d: d.name)
def test_fill_zero_view_matches_the_oracle(movement, dtype):
    rng = np.random.default_rng(61)
    views = [([3], [2], 0), ([], [], 7), ([1000, 37], [1, 1024], 3),
             ([64, 48], [49, 1], 0), ([256, 64], [1, 512], 0), ([128, 96], [1, -128], 95 * 128)]
    for rank in (1, 2, 3, 4, 6, 8):
        views.append(strided_view(rng, rank))
    for ext, st, off in views:
        layout = Layout(ext, st, off)
        n = layout.element_count()
        span = layout.max_reachable_offset() + 1
        base = random_elements(dtype, span + 1, rng)
        want = base.copy()
        orc.fill_zero_view(want, dtype, layout, n)
        plan = t.plan_fill_zero_view(dtype, layout, span)
        g = Geometry(layout)
        for shift in (0, 1):
            for who in ("launcher", "reference", "ours", "any"):
                say("fill_zero_view", dtype.name, ext, st, off, shift, who)
                d = to_device(base)
                # A shifted buffer: the view one element further in.
                lay = Layout(ext, st, off + shift) if shift else layout
                w = want
                if shift:
                    w = base.copy()
                    orc.fill_zero_view(w, dtype, lay, n)
                p = t.plan_fill_zero_view(dtype, lay, span + 1) if shift else plan
                if who == "launcher":
                    hip.fill_zero_view(d, dtype, lay, n, p, stream())
                elif who == "any":
                    ga = Geometry(lay) if shift else g
                    hip.fill_zero_view_any(d, dtype, ga.c, n, p, stream())
                else:
                    geo = ref_flat(n) if who == "reference" else ours(p)
                    movement.launch("t4a_cuda_fill_zero_view", *geo, None,
                                    [ptr(d), c_int(dtype), lay.c, c_ll(n)])
                got = to_host(d, (span + 1) * dtype.size, "fill_zero_view")
                assert np.array_equal(got, w.view(np.uint8)), (ext, st, off, shift, who)


def test_fill_zero_view_general_rank():
    rng = np.random.default_rng(62)
    for rank in (9, 12, 16):
        ext = [2 + k % 2 for k in range(rank)]
        order = list(rng.permutation(rank))
        st = [0] * rank
        s = 1
        for k in order:
            st[k] = s
            s *= ext[k] + (1 if k % 3 == 0 else 0)
        w = WideLayout(ext, st, 1)
        span = w.max_reachable_offset() + 1
        n = w.element_count()
        plan = t.plan_fill_zero_view(F64, w, span)
        assert plan.variant == t.RankVariant.General
        base = random_elements(F64, span, rng)
        want = base.copy()
        want[view_indices(ext, st, 1)] = 0
        g = Geometry(w)
        say("fill_zero_view_any rank", rank, "len", n)
        d = to_device(base)
        hip.fill_zero_view_any(d, F64, g.c, n, plan, stream())
        assert np.array_equal(to_host(d, span * 8), want.view(np.uint8)), rank


# -------------------------------------------------------- contiguous_to_view

@pytest.mark.parametrize("dtype", ALL, ids=lambda d: d.name)
def test_contiguous_to_view_matches_the_oracle(movement, dtype):
    rng = np.random.default_rng(63)
    views = [([3, 5, 2, 4], [-1, 3, -15, -30], 2 + 15 + 90),  # reverse, gpu_remaining_families.rs:822
             ([512, 384], [384, 1], 0), ([300, 7], [1, 301], 0), ([], [], 4),
             ([16, 8, 32, 8], [8, 4096, -128, 1], 31 * 128)]
    for rank in (1, 2, 3, 5, 8):
        views.append(strided_view(rng, rank))
    for ext, st, off in views:
        layout = Layout(ext, st, off)
        n = layout.element_count()
        span = layout.max_reachable_offset() + 1
        src = random_elements(dtype, n, rng)
        d_src = to_device(src)
        want = np.frombuffer(bytes([SENTINEL]) * (span * dtype.size), dtype=NUMPY[dtype]).copy()
        orc.contiguous_to_view(want, src, dtype, layout, n)
        plan = t.plan_contiguous_to_view(dtype, layout, span)
        g = Geometry(layout)
        for who in ("launcher", "reference", "ours", "any"):
            say("contiguous_to_view", dtype.name, ext, st, off, who, plan.grid)
            d = sentinel(span * dtype.size)
            if who == "launcher":
                hip.contiguous_to_view(d, d_src, dtype, layout, n, plan, stream())
            elif who == "any":
                hip.contiguous_to_view_any(d, d_src, dtype, g.c, n, plan, stream())
            else:
                geo = ref_flat(n) if who == "reference" else ours(plan)
                movement.launch("t4a_cuda_contiguous_to_view", *geo, None,
                                [ptr(d), ptr(d_src), c_int(dtype), layout.c, c_ll(n)])
            got = to_host(d, span * dtype.size)
            assert np.array_equal(got, want.view(np.uint8)), (ext, st, off, who)


def test_contiguous_to_view_general_rank():
    rng = np.random.default_rng(64)
    for rank in (9, 11, 16):
        ext = [2 + k % 2 if rank == 16 else 2 for k in range(rank)]
        order = list(rng.permutation(rank))
        st = [0] * rank
        s = 1
        for k in order:
            st[k] = s
            s *= ext[k]
        w = WideLayout(ext, st, 0)
        n = w.element_count()
        plan = t.plan_contiguous_to_view(F64, w, n)
        src = random_elements(F64, n, rng)
        want = np.empty(n, dtype=np.float64)
        want[view_indices(ext, st)] = src
        g = Geometry(w)
        say("contiguous_to_view_any rank", rank, "len", n, plan.grid)
        d = sentinel(n * 8)
        hip.contiguous_to_view_any(d, to_device(src), F64, g.c, n, plan, stream())
        assert np.array_equal(to_host(d, n * 8), want.view(np.uint8)), rank


# ----------------------------------------------------------- broadcast_in_dim

def broadcast_expected(src, out_ext, in_ext, in_st, in_off, dims):
    """out[f] = src[in_off + sum_i coord(f, dims[i]) * in_st[i]], coordinate 0
    on input axes of extent 1 (reference movement.cu:409-434)."""
    n = count(out_ext)
    flat = np.arange(n, dtype=np.int64)
    coords = []
    rest = flat
    for e in out_ext:
        coords.append(rest % e)
        rest = rest // e
    idx = np.full(n, in_off, dtype=np.int64)
    for i, d in enumerate(dims):
        if in_ext[i] != 1:
            idx += coords[d] * in_st[i]
    return np.ascontiguousarray(src[idx])


def run_broadcast(movement, who, dtype, out, inp, dims, d_src, n, in_len):
    plan = t.plan_broadcast_in_dim(dtype, out, n, inp, in_len, dims)
    d = sentinel(n * dtype.size)
    if who == "launcher":
        hip.broadcast_in_dim(d, d_src, dtype, out, inp, dims, n, plan, stream())
    elif who == "any":
        go, gi, dd = Geometry(out), Geometry(inp), DeviceDims(dims)
        hip.broadcast_in_dim_any(d, d_src, dtype, go.c, gi.c, dd.c, n, plan, stream())
        hipmem.synchronize()
    else:
        geo = ref_flat(n) if who == "reference" else ours(plan)
        movement.launch("t4a_cuda_broadcast_in_dim", *geo, None,
                        [ptr(d), ptr(d_src), c_int(dtype), out.c, inp.c, t.axis_values(dims),
                         c_ll(n)])
    return d


BROADCAST_CASES = [
    # (out extents, in extents, in strides, in offset, dims)
    ([2, 3], [2, 3], None, 0, [0, 1]),              # identity map
    ([2, 3, 4], [2, 1, 4], None, 0, [0, 1, 2]),     # a broadcast axis
    ([3, 2, 2], [2, 3, 2], None, 0, [2, 0, 1]),     # non-self-inverse permutation
    ([2, 3, 4], [], None, 0, []),                   # scalar input
    ([2, 3], [2, 3], [1, 5], 0, [0, 1]),            # strided source
    ([2, 4, 3], [2, 3], None, 0, [0, 2]),           # an inserted axis
    ([1000, 257], [257], None, 0, [1]),             # row broadcast
    ([257, 1000], [257], None, 0, [0]),             # column broadcast
    ([64, 3, 128], [128, 64], None, 0, [2, 0]),     # inserted axis and a transpose
    ([7, 5, 3, 2], [3, 1, 7], [1, 0, 3], 2, [2, 3, 0]),
    ([256, 300], [256], None, 0, [0]),              # whole rows read again: 16-byte units
    ([64, 5, 48], [64, 48], None, 0, [0, 2]),       # rows decoded over two dims
]


@pytest.mark.parametrize("dtype", ALL, ids=lambda d: d.name)
def test_broadcast_in_dim_matches_the_oracle(movement, dtype):
    rng = np.random.default_rng(65)
    for out_ext, in_ext, in_st, in_off, dims in BROADCAST_CASES:
        inp = Layout(in_ext, in_st, in_off) if in_st else Layout.compact(in_ext)
        out = Layout.compact(out_ext)
        n = out.element_count()
        in_len = inp.max_reachable_offset() + 1
        src = random_elements(dtype, in_len, rng)
        d_src = to_device(src)
        want = np.zeros(n, dtype=NUMPY[dtype])
        orc.broadcast_in_dim(want, src, dtype, out, inp, dims, n)
        alt = broadcast_expected(src, out_ext, in_ext, inp.strides, inp.offset, dims)
        assert np.array_equal(want.view(np.uint8), alt.view(np.uint8))
        for who in ("launcher", "reference", "ours", "any"):
            say("broadcast_in_dim", dtype.name, out_ext, in_ext, dims, who)
            d = run_broadcast(movement, who, dtype, out, inp, dims, d_src, n, in_len)
            got = to_host(d, n * dtype.size)
            assert np.array_equal(got, want.view(np.uint8)), (out_ext, in_ext, dims, who)


def test_broadcast_in_dim_general_rank():
    rng = np.random.default_rng(66)
    for rank in (9, 16):
        ext = [2 + k % 2 for k in range(rank)]
        ie = list(ext)
        ie[1] = 1
        ie[rank - 1] = 1
        out, inp = WideLayout.compact(ext), WideLayout.compact(ie)
        n, m = out.element_count(), inp.element_count()
        dims = list(range(rank))
        src = random_elements(F64, m, rng)
        want = broadcast_expected(src, ext, ie, inp.strides, 0, dims)
        plan = t.plan_broadcast_in_dim(F64, out, n, inp, m, dims)
        assert plan.variant == t.RankVariant.General
        say("broadcast_in_dim_any rank", rank, "len", n)
        d = run_broadcast(None, "any", F64, out, inp, dims, to_device(src), n, m)
        assert np.array_equal(to_host(d, n * 8), want.view(np.uint8)), rank
    # A permuted rank-10 map: input axis i lands on destination axis 9 - i.
    ext = [2, 3, 2, 2, 3, 2, 2, 2, 3, 2]
    ie = list(reversed(ext))
    ie[4] = 1
    out, inp = WideLayout.compact(ext), WideLayout.compact(ie)
    dims = [9 - i for i in range(10)]
    n, m = out.element_count(), inp.element_count()
    src = random_elements(F64, m, rng)
    want = broadcast_expected(src, ext, ie, inp.strides, 0, dims)
    say("broadcast_in_dim_any reversed map rank 10")
    d = run_broadcast(None, "any", F64, out, inp, dims, to_device(src), n, m)
    assert np.array_equal(to_host(d, n * 8), want.view(np.uint8))


# ----------------------------------------------------------- concatenate_copy

def run_concat(movement, who, dtype, d, out, out_len, inp, axis, off, d_src):
    n = inp.element_count()
    plan = t.plan_concatenate_copy(dtype, out, out_len, inp, n, axis, off)
    if who == "launcher":
        hip.concatenate_copy(d, d_src, dtype, out, inp, axis, off, n, plan, stream())
    elif who == "any":
        go, gi = Geometry(out), Geometry(inp)
        hip.concatenate_copy_any(d, d_src, dtype, go.c, gi.c, axis, off, n, plan, stream())
        hipmem.synchronize()
    else:
        geo = ref_flat(n) if who == "reference" else ours(plan)
        movement.launch("t4a_cuda_concatenate_copy", *geo, None,
                        [ptr(d), ptr(d_src), c_int(dtype), out.c, inp.c, c_int(axis), c_ll(off),
                         c_ll(n)])


@pytest.mark.parametrize("dtype", ALL, ids=lambda d: d.name)
def test_concatenate_copy_in_stream_order(movement, dtype):
    """Three launches into one [2, 6] destination: two halves, then the first
    half again, so the final image proves stream order
    (tests/gpu_remaining_families.rs:422-505)."""
    rng = np.random.default_rng(67)
    out, inp = Layout.compact([2, 6]), Layout.compact([2, 3])
    parts = [random_elements(dtype, 6, rng) for _ in range(3)]
    want = np.zeros(12, dtype=NUMPY[dtype])
    for part, off in zip(parts, (0, 3, 0)):
        orc.concatenate_copy(want, part, dtype, out, inp, 1, off, 6)
    for who in ("launcher", "reference", "ours", "any"):
        say("concatenate_copy stream order", dtype.name, who)
        d = to_device(np.zeros(12, dtype=NUMPY[dtype]))
        for part, off in zip(parts, (0, 3, 0)):
            run_concat(movement, who, dtype, d, out, 12, inp, 1, off, to_device(part))
        assert np.array_equal(to_host(d, 12 * dtype.size), want.view(np.uint8)), who


CONCAT_CASES = [
    # (out extents, out strides (None: compact), out offset, in extents, axis, offset)
    ([2, 4, 2], [1, 3, 12], 0, [2, 2, 2], 1, 1),    # non-compact destination
    ([1500, 300], None, 0, [1000, 300], 0, 200),    # rows of a wider destination
    ([300, 1500], None, 0, [300, 1000], 1, 500),    # a block of whole rows
    ([256, 512], [512, 1], 0, [256, 200], 1, 100),  # transposed destination
    ([5, 7, 3], None, 0, [5, 2, 3], 1, 5),
    ([4, 6], [-1, 4], 3, [4, 3], 1, 2),             # reversed destination axis
]


@pytest.mark.parametrize("dtype", ALL, ids=lambda d: d.name)
def test_concatenate_copy_matches_the_oracle(movement, dtype):
    rng = np.random.default_rng(68)
    for out_ext, out_st, out_off, in_ext, axis, off in CONCAT_CASES:
        out = Layout(out_ext, out_st, out_off) if out_st else Layout.compact(out_ext)
        inp = Layout.compact(in_ext)
        span = out.max_reachable_offset() + 1
        n = inp.element_count()
        src = random_elements(dtype, n, rng)
        d_src = to_device(src)
        base = random_elements(dtype, span, rng)
        want = base.copy()
        orc.concatenate_copy(want, src, dtype, out, inp, axis, off, n)
        # The same scatter by numpy: the input's coordinates shifted along axis.
        alt = base.copy()
        ost = out.strides
        shift_st = list(ost)
        alt[view_indices(in_ext, shift_st, out.offset + off * ost[axis])] = src
        assert np.array_equal(want.view(np.uint8), alt.view(np.uint8))
        for who in ("launcher", "reference", "ours", "any"):
            say("concatenate_copy", dtype.name, out_ext, out_st, in_ext, axis, off, who)
            d = to_device(base)
            run_concat(movement, who, dtype, d, out, span, inp, axis, off, d_src)
            got = to_host(d, span * dtype.size)
            assert np.array_equal(got, want.view(np.uint8)), (out_ext, in_ext, axis, off, who)


def test_concatenate_copy_general_rank():
    rng = np.random.default_rng(69)
    rank = 16
    ext = [2 + k % 2 for k in range(rank)]
    ie = list(ext)
    ie[9] = 2
    for axis, off in ((9, 0), (9, 1), (3, 2)):
        oe = list(ext)
        if axis == 3:
            ie2 = list(ext)
            ie2[3] = 1
        else:
            ie2 = ie
        out, inp = WideLayout.compact(oe), WideLayout.compact(ie2)
        n, on = inp.element_count(), out.element_count()
        src = random_elements(F64, n, rng)
        base = random_elements(F64, on, rng)
        want = base.copy()
        want[view_indices(ie2, out.strides, off * out.strides[axis])] = src
        plan = t.plan_concatenate_copy(F64, out, on, inp, n, axis, off)
        assert plan.variant == t.RankVariant.General
        say("concatenate_copy_any rank 16 axis", axis, "offset", off)
        d = to_device(base)
        run_concat(None, "any", F64, d, out, on, inp, axis, off, to_device(src))
        assert np.array_equal(to_host(d, on * 8), want.view(np.uint8)), (axis, off)


# ------------------------------------------------------------- payload bits

def test_copy_entries_preserve_nonfinite_payloads(movement):
    """NaN payloads, signed zeros and infinities survive bit for bit
    (tests/gpu_remaining_families.rs:608-660)."""
    vals = np.array([0x7FF8000000000001, 0xFFF8000000000002, 0x8000000000000000, 0,
                     0x7FF0000000000000, 0xFFF0000000000000], dtype=np.uint64).view(np.float64)
    d_src = to_device(vals)
    lay = Layout.compact([6])
    for who in ("launcher", "reference", "any"):
        say("nonfinite payloads", who)
        d = run_broadcast(movement, who, F64, lay, lay, [0], d_src, 6, 6)
        assert np.array_equal(to_host(d, 48), vals.view(np.uint8)), who
        d = to_device(np.zeros(6))
        run_concat(movement, who, F64, d, lay, 6, lay, 0, 0, d_src)
        assert np.array_equal(to_host(d, 48), vals.view(np.uint8)), who
        plan = t.plan_contiguous_to_view(F64, lay, 6)
        d = sentinel(48)
        hip.contiguous_to_view(d, d_src, F64, lay, 6, plan, stream())
        assert np.array_equal(to_host(d, 48), vals.view(np.uint8)), who


def test_twins_agree_up_to_rank_eight():
    """tests/gpu_remaining_families.rs:720-800: broadcast and concatenate by
    value and general give the same bytes at ranks 1..8; so do the view
    entries over permuted, reversed views."""
    rng = np.random.default_rng(70)
    for rank in range(1, 9):
        ext = [2 + k % 3 for k in range(rank)]
        lay = Layout.compact(ext)
        n = lay.element_count()
        src = random_elements(F64, n, rng)
        d_src = to_device(src)
        dims = list(range(rank))
        say("twins rank", rank)
        a = run_broadcast(None, "launcher", F64, lay, lay, dims, d_src, n, n)
        b = run_broadcast(None, "any", F64, lay, lay, dims, d_src, n, n)
        assert np.array_equal(to_host(a, n * 8), to_host(b, n * 8)), rank
        a, b = to_device(np.zeros(n)), to_device(np.zeros(n))
        run_concat(None, "launcher", F64, a, lay, n, lay, 0, 0, d_src)
        run_concat(None, "any", F64, b, lay, n, lay, 0, 0, d_src)
        assert np.array_equal(to_host(a, n * 8), to_host(b, n * 8)), rank
        e, st, off = strided_view(rng, rank, max_ext=4)
        view = Layout(e, st, off)
        m = view.element_count()
        span = view.max_reachable_offset() + 1
        g = Geometry(view)
        src2 = to_device(random_elements(F64, m, rng))
        plan = t.plan_contiguous_to_view(F64, view, span)
        a, b = sentinel(span * 8), sentinel(span * 8)
        hip.contiguous_to_view(a, src2, F64, view, m, plan, stream())
        hip.contiguous_to_view_any(b, src2, F64, g.c, m, plan, stream())
        assert np.array_equal(to_host(a, span * 8), to_host(b, span * 8)), rank
        plan = t.plan_fill_zero_view(F64, view, span)
        base = random_elements(F64, span, rng)
        a, b = to_device(base), to_device(base)
        hip.fill_zero_view(a, F64, view, m, plan, stream())
        hip.fill_zero_view_any(b, F64, g.c, m, plan, stream())
        assert np.array_equal(to_host(a, span * 8), to_host(b, span * 8)), rank


def test_counts_past_the_layout_stop_at_its_elements():
    """A kernel count larger than the layout's element count touches only the
    layout's elements (the planners never pass one; the kernels still bound
    their walk by the extents)."""
    rng = np.random.default_rng(71)
    lay = Layout([64, 32], [1, 128], 0)  # every other 64-element row of a 4096 span
    span = lay.max_reachable_offset() + 1
    n = lay.element_count()
    base = random_elements(F32, span, rng)
    want = base.copy()
    orc.fill_zero_view(want, F32, lay, n)
    plan = t.plan_fill_zero_view(F32, lay, span)
    say("fill_zero_view count past the layout")
    d = to_device(base)
    hip.fill_zero_view(d, F32, lay, n + 4096, plan, stream())
    assert np.array_equal(to_host(d, span * 4), want.view(np.uint8))
    src = random_elements(F32, n, rng)
    want = np.frombuffer(bytes([SENTINEL]) * (span * 4), dtype=np.float32).copy()
    orc.contiguous_to_view(want, src, F32, lay, n)
    plan = t.plan_contiguous_to_view(F32, lay, span)
    say("contiguous_to_view count past the layout")
    d = sentinel(span * 4)
    # The source holds n + 4096 elements, so every read stays in its buffer.
    d_src = to_device(np.concatenate([src, np.zeros(4096, dtype=np.float32)]))
    hip.contiguous_to_view(d, d_src, F32, lay, n + 4096, plan, stream())
    assert np.array_equal(to_host(d, span * 4), want.view(np.uint8))


def test_row_copies_from_unaligned_buffers():
    """Row copies (a dim contiguous on both sides) through the launchers with
    both pointers one element past a 16-byte boundary: the element-wise form
    of the row walk."""
    rng = np.random.default_rng(72)
    for dtype in (DType.Bool, F32, F64, DType.C64):
        es = dtype.size
        out, inp = Layout.compact([1500, 300]), Layout.compact([1000, 300])
        n, on = inp.element_count(), out.element_count()
        src = random_elements(dtype, n + 1, rng)
        base = random_elements(dtype, on + 1, rng)
        want = base[1:].copy()
        orc.concatenate_copy(want, src[1:], dtype, out, inp, 0, 200, n)
        plan = t.plan_concatenate_copy(dtype, out, on, inp, n, 0, 200)
        say("concatenate_copy unaligned", dtype.name, plan.grid)
        d, d_src = to_device(base), to_device(src)
        hip.concatenate_copy(d.ptr + es, d_src.ptr + es, dtype, out, inp, 0, 200, n, plan,
                             stream())
        got = to_host(d, (on + 1) * es)
        assert np.array_equal(got[:es], base[:1].view(np.uint8)), dtype
        assert np.array_equal(got[es:], want.view(np.uint8)), dtype
        # A row broadcast into a shifted destination.
        o2, row = Layout.compact([256, 40]), Layout.compact([256])
        want2 = np.zeros(256 * 40, dtype=NUMPY[dtype])
        orc.broadcast_in_dim(want2, src[1:], dtype, o2, row, [0], 256 * 40)
        plan = t.plan_broadcast_in_dim(dtype, o2, 256 * 40, row, 256, [0])
        say("broadcast_in_dim unaligned", dtype.name, plan.grid)
        d = sentinel((256 * 40 + 1) * es)
        hip.broadcast_in_dim(d.ptr + es, d_src.ptr + es, dtype, o2, row, [0], 256 * 40, plan,
                             stream())
        got = to_host(d, (256 * 40 + 1) * es)
        assert np.array_equal(got[es:], want2.view(np.uint8)), dtype


@pytest.mark.parametrize("dtype", ALL, ids=lambda d: d.name)
def test_compact_transposes_route_to_the_transpose_kernel(dtype):
    """A movement whose fused plan is one compact 2-D transpose runs on the
    tiled transpose's kernel through the launchers: materialize_strided of a
    transposed view, strided_to_strided and contiguous_to_view into one (with
    a destination offset), broadcast_in_dim with a swapped map and
    concatenate_copy into a transposed destination; full and edge tiles,
    vector and element paths (odd extents, odd offsets)."""
    rng = np.random.default_rng(73)
    for m, n, so, do in ((1, 7, 0, 0), (97, 131, 5, 3), (128, 128, 0, 0), (300, 257, 4, 8),
                         (1024, 768, 0, 4), (64, 2000, 1, 0)):
        count = m * n
        src = random_elements(dtype, so + count, rng)
        d_src = to_device(src)
        view = Layout([m, n], [n, 1], so)  # the source read as its transpose
        want = np.zeros(count, dtype=NUMPY[dtype])
        orc.materialize_strided(want, src, dtype, view, count)
        plan = t.plan_materialize_strided(dtype, view, so + count)
        say("route materialize", dtype.name, m, n, so, plan.grid)
        d = sentinel(count * dtype.size)
        hip.materialize_strided(d, d_src, dtype, view, count, plan, stream())
        assert np.array_equal(to_host(d, count * dtype.size), want.view(np.uint8)), (m, n)

        comp = Layout([n, m], [1, n], so)  # compact [n, m] from the offset
        dst_v = Layout([n, m], [m, 1], do)
        want = np.frombuffer(bytes([SENTINEL]) * ((do + count) * dtype.size),
                             dtype=NUMPY[dtype]).copy()
        orc.strided_to_strided(want, src, dtype, comp, dst_v, count)
        plan = t.plan_strided_to_strided(dtype, comp, so + count, dst_v, do + count)
        say("route strided_to_strided", dtype.name, m, n, so, do, plan.grid)
        d = sentinel((do + count) * dtype.size)
        hip.strided_to_strided(d, d_src, dtype, comp, dst_v, count, plan, stream())
        assert np.array_equal(to_host(d, (do + count) * dtype.size), want.view(np.uint8))

        want = np.frombuffer(bytes([SENTINEL]) * ((do + count) * dtype.size),
                             dtype=NUMPY[dtype]).copy()
        orc.contiguous_to_view(want, src, dtype, dst_v, count)
        plan = t.plan_contiguous_to_view(dtype, dst_v, do + count)
        say("route contiguous_to_view", dtype.name, m, n, do, plan.grid)
        d = sentinel((do + count) * dtype.size)
        hip.contiguous_to_view(d, d_src, dtype, dst_v, count, plan, stream())
        assert np.array_equal(to_host(d, (do + count) * dtype.size), want.view(np.uint8))

        out, inp = Layout.compact([m, n]), Layout.compact([n, m])
        want = np.zeros(count, dtype=NUMPY[dtype])
        orc.broadcast_in_dim(want, src, dtype, out, inp, [1, 0], count)
        plan = t.plan_broadcast_in_dim(dtype, out, count, inp, count + so, [1, 0])
        say("route broadcast_in_dim", dtype.name, m, n, plan.grid)
        d = sentinel(count * dtype.size)
        hip.broadcast_in_dim(d, d_src, dtype, out, inp, [1, 0], count, plan, stream())
        assert np.array_equal(to_host(d, count * dtype.size), want.view(np.uint8))

        # concatenate into columns [2, 2 + n) of a [m, n + 3] destination seen
        # transposed: out extents [n + 3, m] strides [m, 1]
        o2 = Layout([n + 3, m], [m, 1], 0)
        i2 = Layout.compact([n, m])
        span = (n + 3) * m
        base = random_elements(dtype, span, rng)
        want = base.copy()
        orc.concatenate_copy(want, src, dtype, o2, i2, 0, 2, count)
        plan = t.plan_concatenate_copy(dtype, o2, span, i2, count, 0, 2)
        say("route concatenate_copy", dtype.name, m, n, plan.grid)
        d = to_device(base)
        hip.concatenate_copy(d, d_src, dtype, o2, i2, 0, 2, count, plan, stream())
        assert np.array_equal(to_host(d, span * dtype.size), want.view(np.uint8))
