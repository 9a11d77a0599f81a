"""Benchmark: effective GB/s and HBM-roofline fraction of the movement and
single-axis reduction path on one MI355X.

`python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c2]` prints ONE
JSON line. The default workload is benchmark configuration C2: f32
[8192, 8192] sum and max over the inner (contiguous) and the outer axis, and an
i64 sum over the inner axis, each a planned reduction (pass 1 + combine)
launched through the C ABI. One step = those five reductions over one input
set. Inputs are resident in HBM before timing; three input sets rotate so a
step never finds its input in the 256 MB Infinity Cache left by the previous
step. The step is launched one call at a time (`"launch": "eager"`); with
`--graph` it is captured once per input set into a HIP graph and replayed
(`"launch": "hip_graph"`, each graph's output bytes checked against the eager
step's before timing), and `"eager"` keeps the eager figure beside it.

Effective bytes = logical input bytes read once + logical output bytes written
once (partials excluded), 1 GB = 1e9 B. `roofline` is the dominant kernel's
algorithmic bytes per launch over its average launch time, measured here with
HIP events on the launch stream, against the 8 TB/s HBM peak; `traffic` is that
kernel's HBM bytes per launch from rocprofv3 FETCH_SIZE and WRITE_SIZE passes
(`--kernel-only`), each scaled by what the counter reads for copy_exact of a
known size, recorded in TRAFFIC below. `cpu_baseline` is the CPU oracle (the
reference algorithm restated in C) running whole steps of the same workload on
the same inputs for about `--cpu-seconds`, on all OpenMP threads
(`omp_get_max_threads()`, the loops over independent outputs split between
them), with the one-thread figure beside it as `single_thread`.

Other workloads (--workload c1|c1big|c3|c4|c5) run the other benchmark configs
the same way, `c1graph` C1's transposes replayed as one HIP graph, `copy` the
copy ceiling, `entries` the other movement entries
(fill_zero, fill_zero_view, contiguous_to_view, broadcast_in_dim,
concatenate_copy) and `general` the rank-9 `_any` twins; they are for
development, the driver's line is c2.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from dataclasses import dataclass, field
from pathlib import Path
from typing import Callable

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "t4a-cuda-kernels_amd"))
sys.path.insert(0, str(REPO))

import numpy as np  # noqa: E402

import t4a_cuda_kernels as t  # noqa: E402
from t4a_cuda_kernels import hip, hipmem  # noqa: E402

HBM_PEAK_GBPS = 8000.0
ROTATE = 3

# HBM bytes per launch of a workload's dominant kernel, from two rocprofv3 --pmc
# passes over `bench.py --workload W --kernel-only OP` (FETCH_SIZE, then
# WRITE_SIZE, KiB per dispatch averaged over the launches), each multiplied by
# the copy calibration: copy_exact of 256 MiB reads and writes 268435456 bytes,
# and the factor is that over what the counter reports for it. A kernel change
# needs a new measurement; until then the entry is left out and traffic is null.
TRAFFIC: dict[tuple[str, str], dict] = {
    ("c2", "sum_i64_inner"): {"bytes": 538948628, "source": "profiles/traffic_c2_sum_i64_inner.md"},
    ("c2", "sum_f32_inner"): {"bytes": 269794476, "source": "profiles/traffic_c2_sum_f32_inner.md"},
    ("c2", "sum_f32_outer"): {"bytes": 269562792, "source": "profiles/traffic_c2_sum_f32_outer.md"},
    ("c1big", "transpose_f32_8192"): {"bytes": 536952925, "source": "profiles/traffic_c1big_transpose_f32_8192.md"},
    ("c3", "permute4_F64"): {"bytes": 268455680, "source": "profiles/traffic_c3_permute4_F64.md"},
    ("c4", "sumsq_f32_middle"): {"bytes": 539009101, "source": "profiles/traffic_c4_sumsq_f32_middle.md"},
    ("c4", "prod_i32_last"): {"bytes": 671012891, "source": "profiles/traffic_c4_prod_i32_last.md"},
    ("c5", "permute6_c64"): {"bytes": 537005613, "source": "profiles/traffic_c5_permute6_c64.md"},
    ("entries", "contiguous_to_view_f32_transposed"): {"bytes": 536883971, "source": "profiles/traffic_entries_contiguous_to_view_f32_transposed.md"},
    ("entries", "broadcast_in_dim_f32_rows"): {"bytes": 268405994, "source": "profiles/traffic_entries_broadcast_in_dim_f32_rows.md"},
    ("entries", "concatenate_copy_f32_inner"): {"bytes": 268421058, "source": "profiles/traffic_entries_concatenate_copy_f32_inner.md"},
    ("entries", "concatenate_copy_f32_outer"): {"bytes": 268472325, "source": "profiles/traffic_entries_concatenate_copy_f32_outer.md"},
    ("entries", "fill_zero_f32"): {"bytes": 268378148, "source": "profiles/traffic_entries_fill_zero_f32.md"},
    ("entries", "fill_zero_view_f32_rows"): {"bytes": 268247785, "source": "profiles/traffic_entries_fill_zero_view_f32_rows.md"},
}

NUMPY_DTYPE = {t.DType.F32: np.float32, t.DType.F64: np.float64, t.DType.I32: np.int32,
               t.DType.I64: np.int64, t.DType.Bool: np.uint8, t.DType.C32: np.complex64,
               t.DType.C64: np.complex128}


def _oracle():
    """The CPU oracle, imported only by the cpu_baseline leg."""
    from oracle import t4a_oracle as orc
    return orc


@dataclass
class Op:
    """One planned entry (or planned reduction) over rotating buffer sets."""

    name: str
    kernel: str                      # dominant kernel's name, for the roofline
    algo_bytes: int                  # logical input + output bytes
    launch: Callable[[int], None]    # enqueue the op on buffer set r
    dominant: Callable[[int], None]  # enqueue only the dominant kernel
    dominant_bytes: int              # algorithmic bytes of the dominant kernel
    cpu: Callable[[], None] | None = None  # the same op through the CPU oracle
    # the buffers the op writes on set r, as (buffer, bytes): lets a captured
    # step be checked against the eager one
    outputs: Callable[[int], list] | None = None


@dataclass
class Workload:
    name: str
    description: str
    dtype: str
    ops: list[Op] = field(default_factory=list)


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


def _empty_like(bufs) -> list:
    return [hipmem.DeviceBuffer(b.nbytes) for b in bufs]


def reduction_op(name, dtype, op, in_ext, axis, sets, host) -> Op:
    """A planned reduction over compact `in_ext` (reference axis order); `host`
    is the input's host copy, which the CPU leg reduces with the same plan."""
    in_l = t.Layout.compact(in_ext)
    oe = list(in_ext)
    oe[axis] = 1
    out_l = t.Layout.compact(oe)
    n, on = in_l.element_count(), out_l.element_count()
    plan = t.plan_reduction(dtype, op, out_l, on, in_l, n, axis, 32)
    es = dtype.size
    out = hipmem.DeviceBuffer(on * es)
    if plan.kind == "Split":
        pl = t.reduction_partials_layout(in_l, axis, plan.split.splits)
        part = hipmem.DeviceBuffer(pl.element_count() * es)
    else:
        pl, part = None, None
    # The whole plan through t4a_hip_reduction: one launch where a block can
    # hold all of an output's chunks and fold their partials itself.
    joined = plan.kind == "Split" and hip.reduction_joins(plan, sets[0], dtype, op, out_l, in_l,
                                                          axis, on)

    def launch(r):
        hip.reduction(plan, out, sets[r], part, dtype, op, out_l, in_l, axis, on, _stream())

    def dominant(r):
        if joined:
            launch(r)
        elif plan.kind == "Split":
            hip.reduce_partials(part, sets[r], dtype, op, pl, in_l, axis, on,
                                plan.split.splits, plan.split.chunk_len, plan.pass1, _stream())
        else:
            hip.reduce(out, sets[r], dtype, op, plan.strategy, out_l, in_l, axis, on,
                       plan.launch, _stream())

    host_bufs = {}

    def cpu():
        orc = _oracle()
        if not host_bufs:
            host_bufs["out"] = np.zeros(on, dtype=NUMPY_DTYPE[dtype])
            if pl is not None:
                host_bufs["part"] = np.zeros(pl.element_count(), dtype=NUMPY_DTYPE[dtype])
        h_out = host_bufs["out"]
        if plan.kind == "Split":
            h_part = host_bufs["part"]
            orc.reduce_partials(h_part, host, dtype, op, 32, pl, in_l, axis, on,
                                plan.split.splits, plan.split.chunk_len)
            width = (plan.pass2.block[0] if plan.combine_strategy == t.ReduceStrategy.Plane
                     else 32)
            orc.reduce(h_out, h_part, dtype, plan.combine_op, plan.combine_strategy, width,
                       out_l, pl, axis, on)
        else:
            width = plan.launch.block[0] if plan.strategy == t.ReduceStrategy.Plane else 32
            orc.reduce(h_out, host, dtype, op, plan.strategy, width, out_l, in_l, axis, on)

    if joined:  # pass 1 and the combine in one launch: input, partials and finals
        kernel, dom_bytes = "reduction_joined", (n + pl.element_count() + on) * es
    elif plan.kind == "Split":
        kernel, dom_bytes = "reduce_partials", (n + pl.element_count()) * es
    else:
        kernel, dom_bytes = "reduce", (n + on) * es
    written = [(out, on * es)] + ([(part, pl.element_count() * es)] if part is not None else [])
    return Op(name, kernel, (n + on) * es, launch, dominant, dom_bytes, cpu,
              lambda r: written)


def transpose_op(name, dtype, m, n, sets, outs, host) -> Op:
    plan = t.plan_tiled_transpose(dtype, t.TransposeConfig.DEFAULT, 0, m * n, m, n, 1, m * n,
                                  m * n)
    cfg = t.TransposeConfig.DEFAULT

    def launch(r):
        hip.tiled_transpose(outs[r], sets[r], dtype, 0, m * n, m, n, cfg, plan, _stream())

    h_dst = []

    def cpu():
        if not h_dst:
            h_dst.append(np.empty_like(host))
        _oracle().tiled_transpose(h_dst[0], host, dtype, 0, m * n, m, n, 1)

    return Op(name, "tiled_transpose", 2 * m * n * dtype.size, launch, launch,
              2 * m * n * dtype.size, cpu, lambda r: [(outs[r], m * n * dtype.size)])


def move_op(name, dtype, src_l, dst_l, sets, outs, host) -> Op:
    count = src_l.element_count()
    src_len = src_l.max_reachable_offset() + 1
    dst_len = dst_l.max_reachable_offset() + 1
    plan = t.plan_strided_to_strided(dtype, src_l, src_len, dst_l, dst_len)

    def launch(r):
        hip.strided_to_strided(outs[r], sets[r], dtype, src_l, dst_l, count, plan, _stream())

    h_dst = []

    def cpu():
        if not h_dst:
            h_dst.append(np.empty(dst_len * dtype.size, dtype=np.uint8))
        _oracle().strided_to_strided(h_dst[0], host, dtype, src_l, dst_l, count)

    return Op(name, "strided_to_strided", 2 * count * dtype.size, launch, launch,
              2 * count * dtype.size, cpu, lambda r: [(outs[r], dst_len * dtype.size)])


# ---- workloads ---------------------------------------------------------------------

def build_c2() -> Workload:
    w = Workload("c2", "C2: f32 [8192,8192] sum+max over inner and outer axis, i64 [8192,8192] "
                 "sum over the inner axis (planned split reductions)", "f32,i64")
    ext = [8192, 8192]  # C-shape [8192, 8192]: reference axis 0 is the inner one
    rng = np.random.default_rng(1)
    hf = rng.uniform(-1.0, 1.0, 8192 * 8192).astype(np.float32)
    hi = rng.integers(-1000, 1001, 8192 * 8192, dtype=np.int64)
    f, i64 = _sets(hf), _sets(hi)
    w.ops.append(reduction_op("sum_f32_inner", t.DType.F32, t.ReduceOp.Sum, ext, 0, f, hf))
    w.ops.append(reduction_op("max_f32_inner", t.DType.F32, t.ReduceOp.Max, ext, 0, f, hf))
    w.ops.append(reduction_op("sum_f32_outer", t.DType.F32, t.ReduceOp.Sum, ext, 1, f, hf))
    w.ops.append(reduction_op("max_f32_outer", t.DType.F32, t.ReduceOp.Max, ext, 1, f, hf))
    w.ops.append(reduction_op("sum_i64_inner", t.DType.I64, t.ReduceOp.Sum, ext, 0, i64, hi))
    return w


def build_c1(m: int) -> Workload:
    w = Workload(f"c1-{m}", f"C1: tiled transpose f32 [{m},{m}] (1,0)", "f32")
    host = np.random.default_rng(0).uniform(-1.0, 1.0, m * m).astype(np.float32)
    sets = _sets(host)
    outs = _empty_like(sets)
    w.ops.append(transpose_op(f"transpose_f32_{m}", t.DType.F32, m, m, sets, outs, host))
    return w


def build_c1_graph(m: int, count: int = 100) -> Workload:
    """C1's transposes captured into one HIP graph: `count` launches over the
    rotating sets per replay, so the per-launch cost of a small transpose is
    the graph's, not one submission's."""
    w = Workload(f"c1graph-{m}", f"C1: {count} tiled transposes f32 [{m},{m}] (1,0) replayed "
                 "as one HIP graph", "f32")
    host = np.random.default_rng(0).uniform(-1.0, 1.0, m * m).astype(np.float32)
    sets = _sets(host)
    outs = _empty_like(sets)
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
    w.ops.append(Op(f"transpose_f32_{m}_x{count}_graph", "tiled_transpose (graph)", nbytes,
                    replay, replay, nbytes))
    return w


def build_c3() -> Workload:
    w = Workload("c3", "C3: strided_to_strided C-[64,128,64,32] perm (3,1,0,2), reversed "
                 "axis, f64 and c32", "f64,c32")
    src_l = t.Layout([64, 64, 128, 32], [32, 262144, -2048, 1], 260096)
    dst_l = t.Layout.compact([64, 64, 128, 32])
    rng = np.random.default_rng(2)
    for dt in (t.DType.F64, t.DType.C32):
        host = rng.standard_normal(16777216 * dt.size // 8)
        sets = _sets(host)
        outs = _empty_like(sets)
        w.ops.append(move_op(f"permute4_{dt.name}", dt, src_l, dst_l, sets, outs, host))
    return w


def build_c4() -> Workload:
    w = Workload("c4", "C4: f32 C-[32,1048576,4] sumsq+min over the middle axis, i32 prod "
                 "over the last axis", "f32,i32")
    ext = [4, 1048576, 32]
    rng = np.random.default_rng(3)
    hf = rng.standard_normal(4 * 1048576 * 32).astype(np.float32)
    hi = rng.choice(np.array([-1, 1, 2], dtype=np.int32), 4 * 1048576 * 32)
    f, i32 = _sets(hf), _sets(hi)
    w.ops.append(reduction_op("sumsq_f32_middle", t.DType.F32, t.ReduceOp.SumSquares, ext, 1, f,
                              hf))
    w.ops.append(reduction_op("min_f32_middle", t.DType.F32, t.ReduceOp.Min, ext, 1, f, hf))
    w.ops.append(reduction_op("prod_i32_last", t.DType.I32, t.ReduceOp.Prod, ext, 0, i32, hi))
    return w


def build_c5() -> Workload:
    w = Workload("c5", "C5: c64 [16]^6 permute (5,2,0,4,1,3) then sum over C-axis 3", "c64")
    src_l = t.Layout([16] * 6, [256, 65536, 16, 1048576, 4096, 1], 0)
    dst_l = t.Layout.compact([16] * 6)
    host = np.random.default_rng(4).standard_normal(16 ** 6 * 2)
    sets = _sets(host)
    outs = _empty_like(sets)
    w.ops.append(move_op("permute6_c64", t.DType.C64, src_l, dst_l, sets, outs, host))
    # the sum reads the permuted (compact) tensor; the CPU leg reduces a tensor of
    # the same shape (the source), which is the same work
    w.ops.append(reduction_op("sum_c64_axis3", t.DType.C64, t.ReduceOp.Sum, [16] * 6, 2, outs,
                              host))
    return w


def build_copy() -> Workload:
    """The copy ceiling: copy_exact of 256 MiB (f32 [8192, 8192])."""
    w = Workload("copy", "copy_exact f32 [8192,8192] (the measured copy ceiling)", "f32")
    n = 8192 * 8192
    sets = _sets(np.random.default_rng(5).uniform(-1, 1, n).astype(np.float32))
    outs = _empty_like(sets)
    plan = t.plan_copy_exact(t.DType.F32, n)

    def launch(r):
        hip.copy_exact(outs[r], sets[r], t.DType.F32, n, plan, _stream())

    w.ops.append(Op("copy_f32_256MiB", "copy_exact", 2 * n * 4, launch, launch, 2 * n * 4))
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
    rng = np.random.default_rng(6)
    host = rng.uniform(-1.0, 1.0, n).astype(np.float32)
    sets = _sets(host)
    outs = _empty_like(sets)
    wide = [hipmem.DeviceBuffer(2 * n * 4) for _ in range(ROTATE)]
    orc_out = []

    def h_out(nbytes):
        if not orc_out or orc_out[0].nbytes < nbytes:
            orc_out[:] = [np.empty(nbytes, dtype=np.uint8)]
        return orc_out[0]

    plan = t.plan_fill_zero(F32, n)
    fill = lambda r: hip.fill_zero(outs[r], F32, n, plan, _stream())  # noqa: E731
    flat = t.Layout.compact([n])
    w.ops.append(Op("fill_zero_f32", "fill_zero", n * 4, fill, fill, n * 4,
                    lambda: _oracle().fill_zero_view(h_out(n * 4).view(np.float32), F32, flat,
                                                     n)))

    rows = t.Layout([8192, 8192], [1, 16384], 0)
    vplan = t.plan_fill_zero_view(F32, rows, 2 * n)
    fview = lambda r: hip.fill_zero_view(wide[r], F32, rows, n, vplan, _stream())  # noqa: E731
    w.ops.append(Op("fill_zero_view_f32_rows", "fill_zero_view", n * 4, fview, fview, n * 4,
                    lambda: _oracle().fill_zero_view(h_out(2 * n * 4).view(np.float32), F32,
                                                     rows, n)))

    tr = t.Layout([8192, 8192], [8192, 1], 0)
    cplan = t.plan_contiguous_to_view(F32, tr, n)
    scat = lambda r: hip.contiguous_to_view(outs[r], sets[r], F32, tr, n, cplan,  # noqa: E731
                                            _stream())
    w.ops.append(Op("contiguous_to_view_f32_transposed", "contiguous_to_view", 2 * n * 4, scat,
                    scat, 2 * n * 4,
                    lambda: _oracle().contiguous_to_view(h_out(n * 4).view(np.float32), host,
                                                         F32, tr, n)))

    out_l = t.Layout.compact([8192, 8192])
    row = t.Layout.compact([8192])
    bplan = t.plan_broadcast_in_dim(F32, out_l, n, row, 8192, [0])
    bc = lambda r: hip.broadcast_in_dim(outs[r], sets[r], F32, out_l, row, [0], n,  # noqa: E731
                                        bplan, _stream())
    w.ops.append(Op("broadcast_in_dim_f32_rows", "broadcast_in_dim", (n + 8192) * 4, bc, bc,
                    (n + 8192) * 4,
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
        w.ops.append(Op(f"concatenate_copy_f32_{name}", "concatenate_copy", 2 * n * 4, cat,
                        first, 2 * m * 4, cat_cpu))
    return w


def build_general() -> Workload:
    """The general-rank twins at rank 9 (the benchmark layouts with extent-1 axes
    appended, so the plans are GENERAL and fuse back to the rank <= 8 ones):
    the C3 f64 and C5 c64 permutes, the 8192^2 f32 transpose, an f32 row copy,
    and pass 1 of the C2 f32 sums over the inner and the outer axis, all with
    their geometry in device memory."""
    w = Workload("general", "rank-9 _any twins: C3 f64 / C5 c64 permutes, 8192^2 f32 "
                 "transpose and row copy, C2 f32 inner / outer sum pass 1", "f64,c64,f32")
    rng = np.random.default_rng(7)
    keep = []  # device geometry arrays, alive for the workload's lifetime

    def geometry(layout):
        k = 9 - layout.rank
        wide = t.WideLayout(layout.extents + [1] * k, layout.strides + [3] * k, layout.offset)
        ext = hipmem.DeviceBuffer.from_array(np.array(wide.extents, dtype=np.int64))
        st = hipmem.DeviceBuffer.from_array(np.array(wide.strides, dtype=np.int64))
        keep.extend([ext, st])
        return wide, wide.device_c(ext.ptr, st.ptr)

    moves = [("permute4_F64", t.DType.F64,
              t.Layout([64, 64, 128, 32], [32, 262144, -2048, 1], 260096)),
             ("permute6_c64", t.DType.C64,
              t.Layout([16] * 6, [256, 65536, 16, 1048576, 4096, 1], 0)),
             ("transpose_f32_8192", t.DType.F32, t.Layout([8192, 8192], [8192, 1], 0)),
             ("rows_f32_8192", t.DType.F32, t.Layout([8192, 8192], [1, 16384], 0))]
    for name, dt, src_l in moves:
        n = src_l.element_count()
        span = src_l.max_reachable_offset() + 1
        dst_l = t.Layout.compact(src_l.extents)
        ws, cs = geometry(src_l)
        wd, cd = geometry(dst_l)
        plan = t.plan_strided_to_strided(dt, ws, span, wd, n)
        host = rng.integers(0, 255, span * dt.size, dtype=np.uint8)
        sets = _sets(host)
        outs = [hipmem.DeviceBuffer(n * dt.size) for _ in range(ROTATE)]

        def move(r, dt=dt, cs=cs, cd=cd, n=n, plan=plan, sets=sets, outs=outs):
            hip.strided_to_strided_any(outs[r], sets[r], dt, cs, cd, n, plan, _stream())

        w.ops.append(Op(f"{name}_any", "strided_to_strided_any", 2 * n * dt.size, move, move,
                        2 * n * dt.size))
    ext = [8192, 8192]
    hf = rng.uniform(-1.0, 1.0, 8192 * 8192).astype(np.float32)
    f = _sets(hf)
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

        w.ops.append(Op(f"{name}_any", "reduce_partials_any", (n + pn) * 4, pass1, pass1,
                        (n + pn) * 4))
    w.keep = keep
    return w


WORKLOADS = {
    "general": build_general,
    "entries": build_entries,
    "copy": build_copy,
    "c2": build_c2,
    "c1": lambda: build_c1(1024),
    "c1big": lambda: build_c1(8192),
    "c1graph": lambda: build_c1_graph(1024),
    "c3": build_c3,
    "c4": build_c4,
    "c5": build_c5,
}


def time_ops(fn: Callable[[int], None], count: int) -> float:
    """Average milliseconds per call of `fn` over `count` calls, events on the
    launch stream."""
    s = _stream()
    start, stop = hipmem.Event(), hipmem.Event()
    s.synchronize()
    start.record(s)
    for i in range(count):
        fn(i % ROTATE)
    stop.record(s)
    stop.synchronize()
    return start.elapsed_ms(stop) / count


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


def captured_steps(w: Workload, step: Callable[[int], None]) -> list:
    """One HIP graph per buffer set holding the whole step's launches. Each is
    checked once before it is timed: the eager step's output bytes are kept,
    the outputs refilled with a sentinel, and one replay must write the same
    bytes (partials included)."""
    s = _stream()
    graphs = []
    for r in range(ROTATE):
        g = hipmem.Graph(s, lambda r=r: step(r))
        step(r)
        s.synchronize()
        bufs = [b for op in w.ops for b in op.outputs(r)]
        want = [buf.download(n) for buf, n in bufs]
        for buf, _ in bufs:
            buf.fill(0xCD)
        g.launch(s)
        s.synchronize()
        for (buf, n), x in zip(bufs, want):
            if not np.array_equal(buf.download(n), x):
                sys.exit(f"bench.py: the captured step of set {r} wrote other bytes than the "
                         f"eager step")
        graphs.append(g)
    return graphs


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="c2", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="repeat whole CPU steps until this much time has passed")
    ap.add_argument("--kernel-only", metavar="OP",
                    help="launch only OP's dominant kernel, warmup + steps times (for "
                         "rocprofv3 counter passes), and print one line")
    ap.add_argument("--graph", action="store_true",
                    help="time the step captured once per input set into a HIP graph and "
                         "replayed (checked against the eager step first)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build runs on a single MI355X and has no "
              f"multi-GPU path (asked for --gpus {args.gpus})", file=sys.stderr)
        sys.exit(2)
    if hipmem.device_count() < 1:
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)

    w = WORKLOADS[args.workload]()
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
    step = lambda r: [op.launch(r) for op in w.ops]  # noqa: E731
    for i in range(args.warmup):
        step(i % ROTATE)
    _stream().synchronize()
    step_bytes = sum(op.algo_bytes for op in w.ops)
    eager_ms = time_ops(step, args.steps)
    launch_mode, ms_per_step = "eager", eager_ms
    if args.graph and all(op.outputs is not None for op in w.ops):
        graphs = captured_steps(w, step)
        replay = lambda r: graphs[r].launch(_stream())  # noqa: E731
        for i in range(args.warmup):
            replay(i % ROTATE)
        _stream().synchronize()
        ms_per_step = time_ops(replay, args.steps)
        launch_mode = "hip_graph"
    value = step_bytes / (ms_per_step * 1e-3) / 1e9

    # Per-op and dominant-kernel timings (same stream, same rotation).
    breakdown = {}
    dom = None
    for op in w.ops:
        op_ms = time_ops(op.launch, max(args.steps, 10))
        k_ms = time_ops(op.dominant, max(args.steps, 10))
        breakdown[op.name] = {
            "ms": round(op_ms, 5), "GBps": round(op.algo_bytes / (op_ms * 1e-3) / 1e9, 1),
            "kernel": op.kernel, "kernel_ms": round(k_ms, 5),
            "kernel_GBps": round(op.dominant_bytes / (k_ms * 1e-3) / 1e9, 1)}
        if dom is None or k_ms > dom[1]:
            dom = (op, k_ms)
    op, k_ms = dom
    achieved = op.dominant_bytes / (k_ms * 1e-3) / 1e9
    measured = TRAFFIC.get((w.name, op.name))
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                "traffic": measured["bytes"] if measured else None,
                "algorithmic_bytes": op.dominant_bytes,
                "kernel": f"{op.kernel} ({op.name})", "kernel_ms": round(k_ms, 5)}
    if measured:
        roofline["traffic_source"] = measured["source"]

    cpu = None
    cpu_ops = [o for o in w.ops if o.cpu is not None]
    if cpu_ops and not args.no_cpu:
        orc = _oracle()
        threads = orc.max_threads()
        one = cpu_leg(cpu_ops, args.cpu_seconds, 1)
        many = cpu_leg(cpu_ops, args.cpu_seconds, threads)
        names = ", ".join(o.name for o in cpu_ops)
        cpu = {"value": many["value"], "unit": "GB/s", "cores": threads, "kind": "port",
               "sample": f"CPU oracle (the reference's algorithm and fold topology restated in "
                         f"C; OpenMP over independent outputs, each output folded serially), "
                         f"{many['steps']} whole step(s) of workload {w.name} ({names}) on "
                         f"{threads} threads, on the same full-size inputs, same effective-byte "
                         f"count",
               "seconds": many["seconds"], "steps": many["steps"], "cpu_model": cpu_model(),
               "single_thread": dict(one, cores=1)}

    print(json.dumps({
        "metric": "effective GB/s + % HBM roofline: transpose, strided permute, axis reduce",
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
        "data": "synthetic (uniform/normal/integer inputs of the config's shape, seeded)",
        "config": {"workload": w.description, "global_batch": 1, "parallelism": "single GPU"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "breakdown": breakdown,
    }))


if __name__ == "__main__":
    main()
