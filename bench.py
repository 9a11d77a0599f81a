"""Benchmark: effective GB/s and HBM-roofline fraction of the movement and
single-axis reduction path on one MI355X.

`python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload all]` prints ONE
JSON line. The default workload, `all`, is every benchmark configuration once
per step, each operation launched through the C ABI on one stream:

  C1  tiled transpose f32 C-[1024,1024] (1,0), and its roofline twin at 8192^2;
  C2  f32 C-[8192,8192] sum and max over the inner and the outer axis, i64 sum
      over the inner axis (planned split reductions, t4a_hip_reduction);
  C3  strided_to_strided of f64 and of c32 C-[64,128,64,32], permutation
      (3,1,0,2), axis 1 reversed;
  C4  f32 C-[32,1048576,4] sum of squares and min over the middle axis, i32
      product over the last axis;
  C5  c64 C-[16]^6 permuted (5,2,0,4,1,3) into a compact tensor, then summed
      over C-axis 3 of the permuted tensor.

Inputs are the configurations' seeded values (t4a_cuda_kernels.configs: the
reference's SplitMix64 with uniform, Box-Muller normal and integer draws),
resident in HBM before timing. Every input has ROTATE device copies, and the
copy an operation reads advances with every launch of the step, so no operation
finds its input in the 256 MB Infinity Cache left by the operation before it
(C5's sum reads the permuted tensor the permute wrote one step earlier).

`value` = the step's effective bytes (each logical input element read once,
each logical output element written once; partials excluded; 1 GB = 1e9 B) over
the step's time, K steps timed with HIP events on the launch stream after W
warmup steps. Inside the timed region the library must issue exactly the
planned number of kernel launches (t4a_hip_launch_count) and nothing may
allocate, copy, fill or wait on the host (hipmem.COUNTS), as the reference's
benchmark asserts for its measured region (examples/bench_kernels.rs:283-306).

`roofline` is the dominant kernel (the longest launch of the step), its
algorithmic bytes per launch over its average launch time, measured here with
HIP events on its launch stream, against the 8 TB/s HBM peak; `traffic` is that
kernel's HBM bytes per launch from rocprofv3 counter passes (`--kernel-only`),
recorded in TRAFFIC below. `breakdown` gives every configuration's operations
with their own times and their dominant kernel's fraction of the peak.

`cpu_baseline` is the CPU oracle (the reference algorithm restated in C) running
whole steps of the same workload on the same inputs for about `--cpu-seconds`,
on all OpenMP threads (the loops over independent outputs split between them),
with the one-thread figure beside it. Its outputs then check the GPU's: every
operation's output of the timed step must equal the oracle's bytes (`parity`).

Other workloads (development and single-config lines): c1, c1big, c2, c3, c4,
c5, c1graph (C1's transposes replayed as one HIP graph), copy (the copy
ceiling), entries (the other movement entries), general (the rank-9 `_any`
twins), route1 (the reference-named kernel entries from the gfx950 code
objects under the reference planner's launch geometry).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import sys
import time
from ctypes import byref, c_int, c_longlong, c_void_p
from dataclasses import dataclass, field
from pathlib import Path
from typing import Callable

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "t4a-cuda-kernels_amd"))
sys.path.insert(0, str(REPO))

import numpy as np  # noqa: E402

import t4a_cuda_kernels as t  # noqa: E402
from t4a_cuda_kernels import _lib, configs, hip, hipmem  # noqa: E402

HBM_PEAK_GBPS = 8000.0
ROTATE = 3
METRIC = "effective GB/s + % HBM roofline: transpose, strided permute, axis reduce"

# HBM bytes per launch of an operation's dominant kernel, from one rocprofv3
# --pmc pass over `bench.py --workload W --kernel-only OP` counting the TCC's
# DRAM requests by size (TCC_EA0_RDREQ / _RDREQ_32B and TCC_EA0_WRREQ /
# _WRREQ_64B, summed over the 16 channels x 8 XCDs, averaged over the
# launches): reads are 128 bytes unless counted as 32-byte requests, writes 64
# bytes when counted as such and 32 otherwise -- no calibration factor: by this
# count copy_exact of 256 MiB (268,435,456 bytes a side) reads 268,465,792 and
# writes 268,673,003. A kernel change needs a new measurement; until then the
# entry is left out and traffic is null.
SRC = "profiles/traffic_default_workload_requests.md"
TRAFFIC: dict[str, dict] = {
    "transpose_f32_1024": {"bytes": 8473600, "source": SRC},
    "transpose_f32_8192": {"bytes": 537184661, "source": SRC},
    "sum_f32_inner": {"bytes": 269825557, "source": SRC},
    "max_f32_inner": {"bytes": 269906309, "source": SRC},
    "sum_f32_outer": {"bytes": 269590293, "source": SRC},
    "max_f32_outer": {"bytes": 269615637, "source": SRC},
    "sum_i64_inner": {"bytes": 539006283, "source": SRC},
    "permute4_F64": {"bytes": 268540693, "source": SRC},
    "permute4_C32": {"bytes": 268574571, "source": SRC},
    "sumsq_f32_middle": {"bytes": 539053083, "source": SRC},
    "min_f32_middle": {"bytes": 539098752, "source": SRC},
    "prod_i32_last": {"bytes": 671129643, "source": SRC},
    "permute6_c64": {"bytes": 537073323, "source": SRC},
    "sum_c64_axis3": {"bytes": 285289195, "source": SRC},
    "copy_f32_256MiB": {"bytes": 537138795, "source": SRC},
}

NUMPY_DTYPE = {t.DType.F32: np.float32, t.DType.F64: np.float64, t.DType.I32: np.int32,
               t.DType.I64: np.int64, t.DType.Bool: np.uint8, t.DType.C32: np.complex64,
               t.DType.C64: np.complex128}


def _oracle():
    """The CPU oracle, imported only by the cpu_baseline leg and its check."""
    from oracle import t4a_oracle as orc
    return orc


@dataclass
class Op:
    """One planned entry (or planned reduction) over rotating buffer sets."""

    name: str
    config: str                      # the benchmark configuration it belongs to
    kernel: str                      # dominant kernel's name, for the roofline
    algo_bytes: int                  # logical input + output bytes
    launch: Callable[[int], None]    # enqueue the op on buffer set r
    launches: int                    # kernel launches per call
    dominant: Callable[[int], None]  # enqueue only the dominant kernel
    dominant_bytes: int              # algorithmic bytes of the dominant kernel
    cpu: Callable[[], None] | None = None     # the same op through the CPU oracle
    # the buffers the op writes on set r, as (buffer, bytes)
    outputs: Callable[[int], list] | None = None
    # the oracle's bytes for outputs(r), once cpu() has run (same order)
    expected: Callable[[], list] | None = None


@dataclass
class Workload:
    name: str
    description: str
    dtype: str
    ops: list[Op] = field(default_factory=list)
    keep: list = field(default_factory=list)


_STREAM = None


def _stream() -> hipmem.Stream:
    global _STREAM
    if _STREAM is None:
        _STREAM = hipmem.Stream()
    return _STREAM


def _sets(host: np.ndarray) -> list:
    """ROTATE device copies of one host array (distinct addresses, same data)."""
    first = hipmem.DeviceBuffer.from_array(host)
    out = [first]
    for _ in range(ROTATE - 1):
        b = hipmem.DeviceBuffer(first.nbytes)
        b.copy_from(first)
        out.append(b)
    return out


def _empty(nbytes: int) -> list:
    return [hipmem.DeviceBuffer(nbytes) for _ in range(ROTATE)]


def _check(status: int) -> None:
    if status != 0:
        raise t.T4aError(status)


class Bound:
    """A library call with its ctypes arguments built once. Device buffers are
    passed as the buffer objects themselves: the call converts them to their
    addresses and keeps them, so a buffer lives as long as a call that uses it
    (a raw address alone would let the buffer be freed under the kernel)."""

    def __init__(self, fn_name: str, *args):
        self.fn = getattr(_lib.load(), fn_name)
        self.buffers = [a for a in args if isinstance(a, hipmem.DeviceBuffer)]
        self.args = tuple(c_void_p(a.ptr) if isinstance(a, hipmem.DeviceBuffer)
                          else c_void_p(0) if a is None else a for a in args)

    def __call__(self) -> None:
        _check(self.fn(*self.args))


# ---- operations --------------------------------------------------------------------

def reduction_op(name, config, dtype, op, in_ext, axis, sets, host, host_src=None) -> Op:
    """A planned reduction over compact `in_ext` (reference axis order) through
    t4a_hip_reduction; `host` is the input's host copy, which the CPU leg
    reduces with the same plan (`host_src()`, when given, returns it at run
    time: C5's sum reduces the CPU leg's permuted tensor)."""
    in_l = t.Layout.compact(in_ext)
    oe = list(in_ext)
    oe[axis] = 1
    out_l = t.Layout.compact(oe)
    n, on = in_l.element_count(), out_l.element_count()
    plan = t.plan_reduction(dtype, op, out_l, on, in_l, n, axis, 32)
    es = dtype.size
    outs = _empty(on * es)
    if plan.kind == "Split":
        pl = t.reduction_partials_layout(in_l, axis, plan.split.splits)
        parts = _empty(pl.element_count() * es)
    else:
        pl, parts = None, [None] * ROTATE
    joined = plan.kind == "Split" and hip.reduction_joins(plan, sets[0], dtype, op, out_l, in_l,
                                                          axis, on)
    plan_c, s = plan.to_c(), c_void_p(_stream().handle)
    calls = [Bound("t4a_hip_reduction", outs[r], sets[r], parts[r],
                    int(dtype), int(op), byref(out_l.c), byref(in_l.c), axis, on,
                    byref(plan_c), s) for r in range(ROTATE)]
    if joined or plan.kind == "Direct":
        dominant = calls
    else:
        p1 = plan.pass1.to_c()
        dominant = [Bound("t4a_hip_reduce_partials", parts[r], sets[r], int(dtype),
                           int(op), byref(pl.c), byref(in_l.c), axis, on, plan.split.splits,
                           plan.split.chunk_len, byref(p1), s) for r in range(ROTATE)]
    host_bufs = {}

    def cpu():
        orc = _oracle()
        src = host_src() if host_src is not None else host
        if not host_bufs:
            host_bufs["out"] = np.zeros(on, dtype=NUMPY_DTYPE[dtype])
            if pl is not None:
                host_bufs["part"] = np.zeros(pl.element_count(), dtype=NUMPY_DTYPE[dtype])
        h_out = host_bufs["out"]
        if plan.kind == "Split":
            h_part = host_bufs["part"]
            orc.reduce_partials(h_part, src, dtype, op, 32, pl, in_l, axis, on,
                                plan.split.splits, plan.split.chunk_len)
            width = (plan.pass2.block[0] if plan.combine_strategy == t.ReduceStrategy.Plane
                     else 32)
            orc.reduce(h_out, h_part, dtype, plan.combine_op, plan.combine_strategy, width,
                       out_l, pl, axis, on)
        else:
            width = plan.launch.block[0] if plan.strategy == t.ReduceStrategy.Plane else 32
            orc.reduce(h_out, src, dtype, op, plan.strategy, width, out_l, in_l, axis, on)

    if joined:  # pass 1 and the combine in one launch: input, partials and finals
        kernel, dom_bytes = "reduction_joined", (n + pl.element_count() + on) * es
        launches = 1
    elif plan.kind == "Split":
        kernel, dom_bytes = "reduce_partials", (n + pl.element_count()) * es
        launches = 2
    else:
        kernel, dom_bytes = "reduce", (n + on) * es
        launches = 1
    return Op(name, config, kernel, (n + on) * es, lambda r: calls[r](), launches,
              lambda r: dominant[r](), dom_bytes, cpu,
              lambda r: [(outs[r], on * es)],
              lambda: [host_bufs["out"].view(np.uint8)])


def transpose_op(name, config, dtype, m, n, sets, outs, host) -> Op:
    plan = t.plan_tiled_transpose(dtype, t.TransposeConfig.DEFAULT, 0, m * n, m, n, 1, m * n,
                                  m * n)
    cfg, plan_c, s = t.TransposeConfig.DEFAULT.c, plan.to_c(), c_void_p(_stream().handle)
    calls = [Bound("t4a_hip_tiled_transpose", outs[r], sets[r], int(dtype), 0,
                    m * n, m, n, cfg, byref(plan_c), s) for r in range(ROTATE)]
    h_dst = []

    def cpu():
        if not h_dst:
            h_dst.append(np.empty_like(host))
        _oracle().tiled_transpose(h_dst[0], host, dtype, 0, m * n, m, n, 1)

    nbytes = m * n * dtype.size
    return Op(name, config, "tiled_transpose", 2 * nbytes, lambda r: calls[r](), 1,
              lambda r: calls[r](), 2 * nbytes, cpu, lambda r: [(outs[r], nbytes)],
              lambda: [h_dst[0].view(np.uint8)])


def move_op(name, config, dtype, src_l, dst_l, sets, outs, host, h_dst=None) -> Op:
    """strided_to_strided over `src_l` -> `dst_l`; `h_dst` (a one-slot list)
    receives the CPU leg's destination, for an operation that reads it."""
    count = src_l.element_count()
    src_len = src_l.max_reachable_offset() + 1
    dst_len = dst_l.max_reachable_offset() + 1
    plan = t.plan_strided_to_strided(dtype, src_l, src_len, dst_l, dst_len)
    plan_c, s = plan.to_c(), c_void_p(_stream().handle)
    calls = [Bound("t4a_hip_strided_to_strided", outs[r], sets[r], int(dtype),
                    byref(src_l.c), byref(dst_l.c), count, byref(plan_c), s)
             for r in range(ROTATE)]
    h_dst = h_dst if h_dst is not None else []

    def cpu():
        if not h_dst:
            h_dst.append(np.empty(dst_len, dtype=NUMPY_DTYPE[dtype]))
        _oracle().strided_to_strided(h_dst[0], host, dtype, src_l, dst_l, count)

    return Op(name, config, "strided_to_strided", 2 * count * dtype.size, lambda r: calls[r](),
              1, lambda r: calls[r](), 2 * count * dtype.size, cpu,
              lambda r: [(outs[r], dst_len * dtype.size)], lambda: [h_dst[0].view(np.uint8)])


# ---- workloads ---------------------------------------------------------------------

def build_c1(m: int, config: str = "C1") -> Workload:
    w = Workload(f"c1-{m}", f"C1: tiled transpose f32 C-[{m},{m}] (1,0)", "f32")
    host = configs.c1_input(m)
    sets = _sets(host)
    outs = _empty(host.nbytes)
    w.ops.append(transpose_op(f"transpose_f32_{m}", config, t.DType.F32, m, m, sets, outs, host))
    return w


def build_c2() -> Workload:
    w = Workload("c2", "C2: f32 C-[8192,8192] sum+max over the inner and the outer axis, i64 "
                 "C-[8192,8192] sum over the inner axis (planned split reductions)", "f32,i64")
    ext = [8192, 8192]  # C-shape [8192, 8192]: reference axis 0 is the inner one
    hf, hi = configs.c2_inputs()
    f, i64 = _sets(hf), _sets(hi)
    F32, Sum, Max = t.DType.F32, t.ReduceOp.Sum, t.ReduceOp.Max
    w.ops.append(reduction_op("sum_f32_inner", "C2", F32, Sum, ext, 0, f, hf))
    w.ops.append(reduction_op("max_f32_inner", "C2", F32, Max, ext, 0, f, hf))
    w.ops.append(reduction_op("sum_f32_outer", "C2", F32, Sum, ext, 1, f, hf))
    w.ops.append(reduction_op("max_f32_outer", "C2", F32, Max, ext, 1, f, hf))
    w.ops.append(reduction_op("sum_i64_inner", "C2", t.DType.I64, Sum, ext, 0, i64, hi))
    return w


C3_SRC = t.Layout([64, 64, 128, 32], [32, 262144, -2048, 1], 260096)
C5_SRC = t.Layout([16] * 6, [256, 65536, 16, 1048576, 4096, 1], 0)


def build_c3() -> Workload:
    w = Workload("c3", "C3: strided_to_strided C-[64,128,64,32] perm (3,1,0,2), axis 1 "
                 "reversed, f64 and c32", "f64,c32")
    dst_l = t.Layout.compact([64, 64, 128, 32])
    for dt, npt in ((t.DType.F64, np.float64), (t.DType.C32, np.complex64)):
        host = configs.c3_input(npt)
        sets = _sets(host)
        outs = _empty(host.nbytes)
        w.ops.append(move_op(f"permute4_{dt.name}", "C3", dt, C3_SRC, dst_l, sets, outs, host))
    return w


def build_c4() -> Workload:
    w = Workload("c4", "C4: f32 C-[32,1048576,4] sumsq+min over the middle axis, i32 prod "
                 "over the last axis", "f32,i32")
    ext = [4, 1048576, 32]
    hf, hi = configs.c4_inputs()
    f, i32 = _sets(hf), _sets(hi)
    w.ops.append(reduction_op("sumsq_f32_middle", "C4", t.DType.F32, t.ReduceOp.SumSquares, ext,
                              1, f, hf))
    w.ops.append(reduction_op("min_f32_middle", "C4", t.DType.F32, t.ReduceOp.Min, ext, 1, f, hf))
    w.ops.append(reduction_op("prod_i32_last", "C4", t.DType.I32, t.ReduceOp.Prod, ext, 0, i32,
                              hi))
    return w


def build_c5() -> Workload:
    w = Workload("c5", "C5: c64 C-[16]^6 permute (5,2,0,4,1,3) into a compact tensor, then sum "
                 "over C-axis 3 of the permuted tensor", "c64")
    dst_l = t.Layout.compact([16] * 6)
    host = configs.c5_input()
    sets = _sets(host)
    outs = _empty(host.nbytes)
    permuted = []  # the CPU leg's permuted tensor, which its sum reads
    w.ops.append(move_op("permute6_c64", "C5", t.DType.C64, C5_SRC, dst_l, sets, outs, host,
                         permuted))
    w.ops.append(reduction_op("sum_c64_axis3", "C5", t.DType.C64, t.ReduceOp.Sum, [16] * 6, 2,
                              outs, None, lambda: permuted[0]))
    return w


def build_all() -> Workload:
    parts = [build_c1(1024), build_c1(8192, "C1-roofline"), build_c2(), build_c3(), build_c4(),
             build_c5()]
    w = Workload("all", "every benchmark config once per step: C1 transpose f32 C-[1024,1024] "
                 "and its 8192^2 roofline twin; C2 f32 C-[8192,8192] sum+max inner and outer, "
                 "i64 sum inner; C3 f64 and c32 C-[64,128,64,32] permute (3,1,0,2) with axis 1 "
                 "reversed; C4 f32 C-[32,1048576,4] sumsq+min over the middle axis, i32 prod "
                 "over the last; C5 c64 C-[16]^6 permute (5,2,0,4,1,3) then sum over C-axis 3",
                 "f32,i64,f64,c32,i32,c64")
    for p in parts:
        w.ops.extend(p.ops)
        w.keep.extend(p.keep)
    return w


def build_c1_graph(m: int, count: int = 100) -> Workload:
    """C1's transposes captured into one HIP graph: `count` launches over the
    rotating sets per replay, so the per-launch cost of a small transpose is
    the graph's, not one submission's."""
    w = Workload(f"c1graph-{m}", f"C1: {count} tiled transposes f32 C-[{m},{m}] (1,0) replayed "
                 "as one HIP graph", "f32")
    host = configs.c1_input(m)
    sets = _sets(host)
    outs = _empty(host.nbytes)
    dt = t.DType.F32
    cfg = t.TransposeConfig.DEFAULT
    plan = t.plan_tiled_transpose(dt, cfg, 0, m * m, m, m, 1, m * m, m * m)
    s = _stream()

    def record():
        for i in range(count):
            r = i % ROTATE
            hip.tiled_transpose(outs[r], sets[r], dt, 0, m * m, m, m, cfg, plan, s)

    graph = hipmem.Graph(s, record)
    w.keep = [graph, sets, outs]
    replay = lambda r: graph.launch(s)  # noqa: E731
    nbytes = 2 * m * m * dt.size * count
    w.ops.append(Op(f"transpose_f32_{m}_x{count}_graph", "C1", "tiled_transpose (graph)",
                    nbytes, replay, 0, replay, nbytes))
    return w


def build_copy() -> Workload:
    """The copy ceiling: copy_exact of 256 MiB (f32 [8192, 8192])."""
    w = Workload("copy", "copy_exact f32 [8192,8192] (the measured copy ceiling)", "f32")
    n = 8192 * 8192
    sets = _sets(configs.uniform(5, n, np.float32))
    outs = _empty(n * 4)
    plan = t.plan_copy_exact(t.DType.F32, n)

    def launch(r):
        hip.copy_exact(outs[r], sets[r], t.DType.F32, n, plan, _stream())

    w.ops.append(Op("copy_f32_256MiB", "copy", "copy_exact", 2 * n * 4, launch, 1, launch,
                    2 * n * 4))
    return w


def build_entries() -> Workload:
    """The other movement entries at 256 MiB of f32 each: fill_zero, fill_zero_view
    over every other 32 KiB row, contiguous_to_view into a transposed view,
    broadcast_in_dim of one row to [8192, 8192], and concatenate_copy of two
    halves along the inner and the outer axis."""
    w = Workload("entries", "fill_zero, fill_zero_view, contiguous_to_view, broadcast_in_dim, "
                 "concatenate_copy over f32 [8192,8192]", "f32")
    F32 = t.DType.F32
    n = 8192 * 8192
    host = configs.uniform(6, n, np.float32)
    sets = _sets(host)
    outs = _empty(n * 4)
    wide = _empty(2 * n * 4)
    orc_out = []

    def h_out(nbytes):
        if not orc_out or orc_out[0].nbytes < nbytes:
            orc_out[:] = [np.empty(nbytes, dtype=np.uint8)]
        return orc_out[0]

    plan = t.plan_fill_zero(F32, n)
    fill = lambda r: hip.fill_zero(outs[r], F32, n, plan, _stream())  # noqa: E731
    flat = t.Layout.compact([n])
    w.ops.append(Op("fill_zero_f32", "entries", "fill_zero", n * 4, fill, 1, fill, n * 4,
                    lambda: _oracle().fill_zero_view(h_out(n * 4).view(np.float32), F32, flat,
                                                     n)))

    rows = t.Layout([8192, 8192], [1, 16384], 0)
    vplan = t.plan_fill_zero_view(F32, rows, 2 * n)
    fview = lambda r: hip.fill_zero_view(wide[r], F32, rows, n, vplan, _stream())  # noqa: E731
    w.ops.append(Op("fill_zero_view_f32_rows", "entries", "fill_zero_view", n * 4, fview, 1,
                    fview, n * 4,
                    lambda: _oracle().fill_zero_view(h_out(2 * n * 4).view(np.float32), F32,
                                                     rows, n)))

    tr = t.Layout([8192, 8192], [8192, 1], 0)
    cplan = t.plan_contiguous_to_view(F32, tr, n)
    scat = lambda r: hip.contiguous_to_view(outs[r], sets[r], F32, tr, n, cplan,  # noqa: E731
                                            _stream())
    w.ops.append(Op("contiguous_to_view_f32_transposed", "entries", "contiguous_to_view",
                    2 * n * 4, scat, 1, scat, 2 * n * 4,
                    lambda: _oracle().contiguous_to_view(h_out(n * 4).view(np.float32), host,
                                                         F32, tr, n)))

    out_l = t.Layout.compact([8192, 8192])
    row = t.Layout.compact([8192])
    bplan = t.plan_broadcast_in_dim(F32, out_l, n, row, 8192, [0])
    bc = lambda r: hip.broadcast_in_dim(outs[r], sets[r], F32, out_l, row, [0], n,  # noqa: E731
                                        bplan, _stream())
    w.ops.append(Op("broadcast_in_dim_f32_rows", "entries", "broadcast_in_dim", (n + 8192) * 4,
                    bc, 1, bc, (n + 8192) * 4,
                    lambda: _oracle().broadcast_in_dim(h_out(n * 4).view(np.float32), host, F32,
                                                       out_l, row, [0], n)))

    for axis, ext, name in ((1, [8192, 4096], "outer"), (0, [4096, 8192], "inner")):
        half = t.Layout.compact(ext)
        m = n // 2
        offs = (0, ext[axis])
        plans = [t.plan_concatenate_copy(F32, out_l, n, half, m, axis, o) for o in offs]

        def cat(r, half=half, plans=plans, offs=offs, axis=axis, m=m):
            for o, p in zip(offs, plans):
                hip.concatenate_copy(outs[r], sets[r], F32, out_l, half, axis, o, m, p,
                                     _stream())

        def cat_cpu(half=half, offs=offs, axis=axis, m=m):
            for o in offs:
                _oracle().concatenate_copy(h_out(n * 4).view(np.float32), host, F32, out_l,
                                           half, axis, o, m)

        first = lambda r, half=half, p=plans[0], axis=axis, m=m: hip.concatenate_copy(  # noqa: E731
            outs[r], sets[r], F32, out_l, half, axis, 0, m, p, _stream())
        w.ops.append(Op(f"concatenate_copy_f32_{name}", "entries", "concatenate_copy",
                        2 * n * 4, cat, 2, first, 2 * m * 4, cat_cpu))
    return w


def build_general() -> Workload:
    """The general-rank twins at rank 9 (the benchmark layouts with extent-1 axes
    appended, so the plans are GENERAL and fuse back to the rank <= 8 ones):
    the C3 f64 and C5 c64 permutes, the 8192^2 f32 transpose, an f32 row copy,
    and pass 1 of the C2 f32 sums over the inner and the outer axis, all with
    their geometry in device memory."""
    w = Workload("general", "rank-9 _any twins: C3 f64 / C5 c64 permutes, 8192^2 f32 "
                 "transpose and row copy, C2 f32 inner / outer sum pass 1", "f64,c64,f32")
    keep = []  # device geometry arrays, alive for the workload's lifetime

    def geometry(layout):
        k = 9 - layout.rank
        wide = t.WideLayout(layout.extents + [1] * k, layout.strides + [3] * k, layout.offset)
        ext = hipmem.DeviceBuffer.from_array(np.array(wide.extents, dtype=np.int64))
        st = hipmem.DeviceBuffer.from_array(np.array(wide.strides, dtype=np.int64))
        keep.extend([ext, st])
        return wide, wide.device_c(ext.ptr, st.ptr)

    moves = [("permute4_F64", t.DType.F64, C3_SRC), ("permute6_c64", t.DType.C64, C5_SRC),
             ("transpose_f32_8192", t.DType.F32, t.Layout([8192, 8192], [8192, 1], 0)),
             ("rows_f32_8192", t.DType.F32, t.Layout([8192, 8192], [1, 16384], 0))]
    for seed, (name, dt, src_l) in enumerate(moves):
        n = src_l.element_count()
        span = src_l.max_reachable_offset() + 1
        dst_l = t.Layout.compact(src_l.extents)
        ws, cs = geometry(src_l)
        wd, cd = geometry(dst_l)
        plan = t.plan_strided_to_strided(dt, ws, span, wd, n)
        host = configs.integers(70 + seed, span * dt.size, 0, 255, np.uint8)
        sets = _sets(host)
        outs = _empty(n * dt.size)

        def move(r, dt=dt, cs=cs, cd=cd, n=n, plan=plan, sets=sets, outs=outs):
            hip.strided_to_strided_any(outs[r], sets[r], dt, cs, cd, n, plan, _stream())

        w.ops.append(Op(f"{name}_any", "general", "strided_to_strided_any", 2 * n * dt.size,
                        move, 1, move, 2 * n * dt.size))
    ext = [8192, 8192]
    f = _sets(configs.uniform(7, 8192 * 8192, np.float32))
    for name, axis in (("sum_f32_inner_pass1", 0), ("sum_f32_outer_pass1", 1)):
        in_l = t.Layout.compact(ext)
        oe = list(ext)
        oe[axis] = 1
        out_l = t.Layout.compact(oe)
        n, on = in_l.element_count(), out_l.element_count()
        rplan = t.plan_reduction(t.DType.F32, t.ReduceOp.Sum, out_l, on, in_l, n, axis, 32)
        wi, ci = geometry(in_l)
        wp = t.reduction_partials_layout(wi, axis, rplan.split.splits)
        pe = hipmem.DeviceBuffer.from_array(np.array(wp.extents, dtype=np.int64))
        ps = hipmem.DeviceBuffer.from_array(np.array(wp.strides, dtype=np.int64))
        keep.extend([pe, ps])
        cp = wp.device_c(pe.ptr, ps.ptr)
        pn = wp.element_count()
        p1 = t.plan_reduce_partials(t.DType.F32, t.ReduceOp.Sum, wp, pn, wi, n, axis,
                                    rplan.split, 32)
        part = hipmem.DeviceBuffer(pn * 4)

        def pass1(r, cp=cp, ci=ci, axis=axis, on=on, rplan=rplan, p1=p1, part=part):
            hip.reduce_partials_any(part, f[r], t.DType.F32, t.ReduceOp.Sum, cp, ci, axis, on,
                                    rplan.split.splits, rplan.split.chunk_len, p1, _stream())

        w.ops.append(Op(f"{name}_any", "general", "reduce_partials_any", (n + pn) * 4, pass1, 1,
                        pass1, (n + pn) * 4))
    w.keep = keep
    return w


# ---- route 1: the reference-named entries under the reference planner's geometry ----

def _ceil_div(a: int, b: int) -> int:
    return -(-a // b)


def _ref_flat(length: int):
    """Reference flat_launch (src/lib.rs:1465-1482): one thread per element."""
    return (_ceil_div(length, 256), 1, 1), (256, 1, 1)


def _ref_partials(cubes: int, chunk_len: int, width: int = 32):
    """Reference plan_reduce_partials (src/lib.rs:3412-3430)."""
    planes = 4 if width == 32 and cubes <= 8192 and chunk_len <= 1024 else 1
    return (_ceil_div(cubes, planes), 1, 1), (width * planes, 1, 1)


def _ref_reduce(strategy, output_len: int, width: int):
    """Reference launch_for (src/lib.rs:3242-3286)."""
    if strategy == t.ReduceStrategy.Unit:
        return (_ceil_div(output_len, width), 1, 1), (width, 1, 1)
    return (output_len, 1, 1), (width, 1, 1)


def build_route1() -> Workload:
    """C2's reductions, C3's permutes and C5 through the kernel entries loaded by
    name from t4a_movement / t4a_reduce .gfx950.hsaco with hipModuleLaunchKernel
    and the reference planner's geometry: a caller that keeps the reference
    crate's planning and swaps only the kernel module."""
    w = Workload("route1", "reference-named kernel entries (code objects, hipModuleLaunchKernel) "
                 "under the reference planner's geometry: C2 reductions, C3 permutes, C5",
                 "f32,i64,f64,c32,c64")
    pkg = Path(t.__file__).resolve().parent
    mods = {"movement": hipmem.Module(pkg / "t4a_movement.gfx950.hsaco"),
            "reduce": hipmem.Module(pkg / "t4a_reduce.gfx950.hsaco")}
    w.keep.append(mods)
    s = _stream()

    def reduction(name, config, dtype, op, ext, axis, sets):
        in_l = t.Layout.compact(ext)
        oe = list(ext)
        oe[axis] = 1
        out_l = t.Layout.compact(oe)
        n, on = in_l.element_count(), out_l.element_count()
        plan = t.plan_reduction(dtype, op, out_l, on, in_l, n, axis, 32)
        es = dtype.size
        outs = _empty(on * es)
        w.keep.extend([sets, outs])  # the bound launches hold only their addresses
        if plan.kind == "Direct":
            width = plan.launch.block[0] if plan.strategy == t.ReduceStrategy.Plane else 32
            geo = _ref_reduce(plan.strategy, on, width)
            calls = [mods["reduce"].bind(
                "t4a_cuda_reduce", *geo, 0, s,
                [c_void_p(outs[r].ptr), c_void_p(sets[r].ptr), c_int(dtype), c_int(op),
                 c_int(plan.strategy), out_l.c, in_l.c, c_int(axis), c_longlong(on)])
                for r in range(ROTATE)]
            w.ops.append(Op(name, config, "t4a_cuda_reduce", (n + on) * es,
                            lambda r, c=calls: c[r](), 1, lambda r, c=calls: c[r](),
                            (n + on) * es))
            return
        pl = t.reduction_partials_layout(in_l, axis, plan.split.splits)
        parts = _empty(pl.element_count() * es)
        w.keep.append(parts)
        g1 = _ref_partials(on * plan.split.splits, plan.split.chunk_len)
        width = plan.pass2.block[0] if plan.combine_strategy == t.ReduceStrategy.Plane else 32
        g2 = _ref_reduce(plan.combine_strategy, on, width)
        pass1 = [mods["reduce"].bind(
            "t4a_cuda_reduce_partials", *g1, 0, s,
            [c_void_p(parts[r].ptr), c_void_p(sets[r].ptr), c_int(dtype), c_int(op), pl.c,
             in_l.c, c_int(axis), c_longlong(on), c_longlong(plan.split.splits),
             c_longlong(plan.split.chunk_len)]) for r in range(ROTATE)]
        pass2 = [mods["reduce"].bind(
            "t4a_cuda_reduce", *g2, 0, s,
            [c_void_p(outs[r].ptr), c_void_p(parts[r].ptr), c_int(dtype),
             c_int(plan.combine_op), c_int(plan.combine_strategy), out_l.c, pl.c, c_int(axis),
             c_longlong(on)]) for r in range(ROTATE)]

        def both(r, p1=pass1, p2=pass2):
            p1[r]()
            p2[r]()

        w.ops.append(Op(name, config, "t4a_cuda_reduce_partials", (n + on) * es, both, 2,
                        lambda r, p1=pass1: p1[r](), (n + pl.element_count()) * es))

    def permute(name, config, dtype, src_l, sets, outs):
        w.keep.extend([sets, outs])
        dst_l = t.Layout.compact(src_l.extents)
        count = src_l.element_count()
        geo = _ref_flat(count)
        calls = [mods["movement"].bind(
            "t4a_cuda_strided_to_strided", *geo, 0, s,
            [c_void_p(outs[r].ptr), c_void_p(sets[r].ptr), c_int(dtype), src_l.c, dst_l.c,
             c_longlong(count)]) for r in range(ROTATE)]
        w.ops.append(Op(name, config, "t4a_cuda_strided_to_strided", 2 * count * dtype.size,
                        lambda r: calls[r](), 1, lambda r: calls[r](), 2 * count * dtype.size))

    ext = [8192, 8192]
    hf, hi = configs.c2_inputs()
    f, i64 = _sets(hf), _sets(hi)
    del hf, hi
    for name, dt, op, axis, sets in (("sum_f32_inner", t.DType.F32, t.ReduceOp.Sum, 0, f),
                                     ("max_f32_inner", t.DType.F32, t.ReduceOp.Max, 0, f),
                                     ("sum_f32_outer", t.DType.F32, t.ReduceOp.Sum, 1, f),
                                     ("max_f32_outer", t.DType.F32, t.ReduceOp.Max, 1, f),
                                     ("sum_i64_inner", t.DType.I64, t.ReduceOp.Sum, 0, i64)):
        reduction(name, "C2", dt, op, ext, axis, sets)
    for dt, npt in ((t.DType.F64, np.float64), (t.DType.C32, np.complex64)):
        host = configs.c3_input(npt)
        permute(f"permute4_{dt.name}", "C3", dt, C3_SRC, _sets(host), _empty(host.nbytes))
    host = configs.c5_input()
    c5_out = _empty(host.nbytes)
    permute("permute6_c64", "C5", t.DType.C64, C5_SRC, _sets(host), c5_out)
    reduction("sum_c64_axis3", "C5", t.DType.C64, t.ReduceOp.Sum, [16] * 6, 2, c5_out)
    return w


WORKLOADS = {
    "all": build_all,
    "general": build_general,
    "entries": build_entries,
    "copy": build_copy,
    "c2": build_c2,
    "c1": lambda: build_c1(1024),
    "c1big": lambda: build_c1(8192, "C1-roofline"),
    "c1graph": lambda: build_c1_graph(1024),
    "c3": build_c3,
    "c4": build_c4,
    "c5": build_c5,
    "route1": build_route1,
}


# ---- timing --------------------------------------------------------------------------

class Rotation:
    """The step: every operation once, each on the next buffer set (the set index
    advances with every launch, across steps)."""

    def __init__(self, ops: list[Op]):
        self.ops = ops
        self.count = 0

    def step(self) -> None:
        for op in self.ops:
            op.launch(self.count % ROTATE)
            self.count += 1


def time_calls(fn: Callable[[], None], count: int) -> float:
    """Average milliseconds per call of `fn` over `count` calls, HIP events on the
    launch stream."""
    s = _stream()
    start, stop = hipmem.Event(), hipmem.Event()
    s.synchronize()
    start.record(s)
    for _ in range(count):
        fn()
    stop.record(s)
    stop.synchronize()
    return start.elapsed_ms(stop) / count


def time_rotating(fn: Callable[[int], None], count: int) -> float:
    it = iter(range(1 << 62))
    return time_calls(lambda: fn(next(it) % ROTATE), count)


def cpu_leg(cpu_ops: list, seconds: float, threads: int) -> dict:
    """Whole CPU steps of the workload through the oracle on `threads` OpenMP
    threads, repeated until `seconds` have passed (at most 100 steps)."""
    orc = _oracle()
    orc.set_threads(threads)
    try:
        steps, t0 = 0, time.perf_counter()
        while True:
            for o in cpu_ops:
                o.cpu()
            steps += 1
            dt = time.perf_counter() - t0
            if dt >= seconds or steps >= 100:
                break
    finally:
        orc.set_threads(1)
    moved = steps * sum(o.algo_bytes for o in cpu_ops)
    return {"value": round(moved / dt / 1e9, 3), "seconds": round(dt, 2), "steps": steps}


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def parity(ops: list[Op]) -> dict:
    """Each operation's GPU output (every buffer set) against the oracle's bytes
    from the CPU leg."""
    hipmem.synchronize()
    checked, failed = 0, []
    for op in ops:
        if op.outputs is None or op.expected is None:
            continue
        want = op.expected()
        for r in range(ROTATE):
            for (buf, n), x in zip(op.outputs(r), want):
                if not np.array_equal(buf.download(n), x[:n]):
                    failed.append(f"{op.name}[set {r}]")
        checked += 1
    return {"ops_checked": checked, "bit_exact": not failed, "failed": failed,
            "against": "CPU oracle outputs of the cpu_baseline leg, same inputs"}


def captured_steps(w: Workload, rot: Rotation) -> list:
    """ROTATE HIP graphs, graph k holding the step that starts at rotation count
    k * len(ops), so replaying them in turn repeats the eager rotation."""
    s = _stream()
    graphs = []
    for k in range(ROTATE):
        rot.count = k * len(w.ops)
        graphs.append(hipmem.Graph(s, rot.step))
    rot.count = 0
    return graphs


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="all", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true",
                    help="skip the CPU baseline leg (and with it the parity check)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="repeat whole CPU steps until this much time has passed")
    ap.add_argument("--kernel-only", metavar="OP",
                    help="launch only OP's dominant kernel, warmup + steps times (for "
                         "rocprofv3 counter passes), and print one line")
    ap.add_argument("--graph", action="store_true",
                    help="time the step captured into HIP graphs and replayed")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build runs on a single MI355X and has no "
              f"multi-GPU path (asked for --gpus {args.gpus})", file=sys.stderr)
        sys.exit(2)
    if hipmem.device_count() < 1:
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)

    w = WORKLOADS[args.workload]()
    lib = _lib.load()
    if args.kernel_only:
        ops = {op.name: op for op in w.ops}
        if args.kernel_only not in ops:
            print(f"no op {args.kernel_only!r} in workload {w.name}: {sorted(ops)}",
                  file=sys.stderr)
            sys.exit(2)
        op = ops[args.kernel_only]
        for i in range(args.warmup + args.steps):
            op.dominant(i % ROTATE)
        _stream().synchronize()
        print(json.dumps({"kernel_only": op.name, "workload": w.name, "kernel": op.kernel,
                          "launches": args.warmup + args.steps,
                          "algorithmic_bytes": op.dominant_bytes}))
        return

    rot = Rotation(w.ops)
    for _ in range(max(args.warmup, 1)):
        rot.step()
    _stream().synchronize()
    step_bytes = sum(op.algo_bytes for op in w.ops)

    # The timed region: K steps between events on the launch stream, with the
    # launches counted and nothing allocated, copied, filled or waited for.
    before, launches0 = hipmem.counts(), lib.t4a_hip_launch_count()
    s = _stream()
    start, stop = hipmem.Event(), hipmem.Event()
    start.record(s)
    for _ in range(args.steps):
        rot.step()
    stop.record(s)
    after, launches1 = hipmem.counts(), lib.t4a_hip_launch_count()
    stop.synchronize()
    eager_ms = start.elapsed_ms(stop) / args.steps
    planned = sum(op.launches for op in w.ops) * args.steps
    issued = (launches1 - launches0) + (after["module_launches"] - before["module_launches"])
    region = {k: after[k] - before[k] for k in ("allocations", "transfer_bytes", "fills",
                                                 "host_waits")}
    if issued != planned or any(region.values()):
        sys.exit(f"bench.py: the timed region issued {issued} kernel launches (planned "
                 f"{planned}) and {region}; it must launch exactly the plan and allocate, "
                 f"copy, fill and wait for nothing")
    measured_region = {"kernel_launches": issued, "per_step": issued // args.steps, **region}

    launch_mode, ms_per_step = "eager", eager_ms
    if args.graph:
        graphs = captured_steps(w, rot)
        for i in range(args.warmup):
            graphs[i % ROTATE].launch(s)
        it = iter(range(1 << 62))
        ms_per_step = time_calls(lambda: graphs[next(it) % ROTATE].launch(s), args.steps)
        launch_mode = "hip_graph"
    value = step_bytes / (ms_per_step * 1e-3) / 1e9

    # Per-op and dominant-kernel timings (same stream, rotating sets).
    reps = max(args.steps, 20)
    breakdown: dict[str, dict] = {}
    dom = None
    for op in w.ops:
        op_ms = time_rotating(op.launch, reps)
        k_ms = time_rotating(op.dominant, reps)
        frac = op.dominant_bytes / (k_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS
        cfg = breakdown.setdefault(op.config, {"ops": {}})
        cfg["ops"][op.name] = {
            "ms": round(op_ms, 5), "GBps": round(op.algo_bytes / (op_ms * 1e-3) / 1e9, 1),
            "kernel": op.kernel, "kernel_ms": round(k_ms, 5),
            "kernel_GBps": round(op.dominant_bytes / (k_ms * 1e-3) / 1e9, 1),
            "kernel_frac": round(frac, 4)}
        if op.name in TRAFFIC:
            cfg["ops"][op.name]["kernel_traffic_ratio"] = round(
                TRAFFIC[op.name]["bytes"] / op.dominant_bytes, 4)
        if dom is None or k_ms > dom[1]:
            dom = (op, k_ms)
    for cfg in breakdown.values():
        ops = cfg["ops"].values()
        ms = sum(o["ms"] for o in ops)
        nbytes = sum(o["GBps"] * o["ms"] for o in ops)  # GB/s x ms = MB
        cfg["ms"] = round(ms, 5)
        cfg["GBps"] = round(nbytes / ms, 1)
        cfg["min_kernel_frac"] = min(o["kernel_frac"] for o in ops)
    op, k_ms = dom
    achieved = op.dominant_bytes / (k_ms * 1e-3) / 1e9
    measured = TRAFFIC.get(op.name)
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                "traffic": measured["bytes"] if measured else None,
                "algorithmic_bytes": op.dominant_bytes,
                "kernel": f"{op.kernel} ({op.config} {op.name})", "kernel_ms": round(k_ms, 5)}
    if measured:
        roofline["traffic_source"] = measured["source"]

    cpu, check = None, None
    cpu_ops = [o for o in w.ops if o.cpu is not None]
    if cpu_ops and not args.no_cpu:
        orc = _oracle()
        threads = orc.max_threads()
        one = cpu_leg(cpu_ops, args.cpu_seconds, 1)
        many = cpu_leg(cpu_ops, args.cpu_seconds, threads)
        cpu = {"value": many["value"], "unit": "GB/s", "cores": threads, "kind": "port",
               "sample": f"CPU oracle (the reference's algorithm and fold topology restated in "
                         f"C; OpenMP over independent outputs, each output folded serially), "
                         f"{many['steps']} whole step(s) of workload {w.name} "
                         f"({len(cpu_ops)} operations) on {threads} threads, on the same "
                         f"full-size inputs, same effective-byte count",
               "seconds": many["seconds"], "steps": many["steps"], "cpu_model": cpu_model(),
               "single_thread": dict(one, cores=1)}
        check = parity(cpu_ops)

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "launch": launch_mode,
        "eager": {"ms_per_step": round(eager_ms, 5),
                  "value": round(step_bytes / (eager_ms * 1e-3) / 1e9, 1)},
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": w.dtype,
        "data": "synthetic: the configs' seeded SplitMix64 inputs (uniform, Box-Muller normal, "
                "integers), resident in HBM",
        "config": {"workload": w.description, "step_bytes": step_bytes, "global_batch": 1,
                   "parallelism": "single GPU"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "parity": check,
        "measured_region": measured_region,
        "breakdown": breakdown,
    }
    print(json.dumps(line))
    if check is not None and not check["bit_exact"]:
        sys.exit(3)


if __name__ == "__main__":
    main()
