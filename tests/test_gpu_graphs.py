"""Launches captured into a HIP graph and replayed (hipmem.Graph): a tiled
transpose, a strided gather, a planned split reduction, a concatenation and a
broadcast, recorded once on a stream. Every replay, with the program's own
eager work and synchronizations between replays and the outputs refilled with
a sentinel before each, gives the eager run's bytes; the transpose and the
reduction are also checked against the oracle. No memset is recorded: the
launchers issue kernels only."""
import numpy as np
import pytest

import t4a_cuda_kernels as t
from t4a_cuda_kernels import DType, Layout, hip, hipmem
from gpu_util import SENTINEL, random_elements, say, sentinel, to_device, to_host
from oracle import t4a_oracle as orc

pytestmark = pytest.mark.gpu

F32 = DType.F32


def test_captured_launches_replay_the_eager_bytes():
    rng = np.random.default_rng(95)
    s = hipmem.Stream()
    m = n = 1024
    src = random_elements(F32, m * n, rng)
    d_src = to_device(src)
    outs = {}

    # the sequence, on stream s into the buffers in `outs`
    tplan = t.plan_tiled_transpose(F32, t.TransposeConfig.DEFAULT, 0, m * n, m, n, 1, m * n,
                                   m * n)
    # a reversed-axis permuted view inside the 1024 x 1024 source
    view = Layout([32, 32, 16, 32], [32, 32768, -1024, 1], 15 * 1024)
    assert view.min_reachable_offset() >= 0 and view.max_reachable_offset() < m * n
    vcount = view.element_count()
    mplan = t.plan_materialize_strided(F32, view, m * n)
    in_l, out_l = Layout.compact([4096, 64]), Layout.compact([1, 64])
    rplan = t.plan_reduction(F32, t.ReduceOp.Sum, out_l, 64, in_l, 4096 * 64, 0, 32)
    pl = t.reduction_partials_layout(in_l, 0, rplan.split.splits)
    part = hipmem.DeviceBuffer(pl.element_count() * 4)
    cat_out, half = Layout.compact([512, 2048]), Layout.compact([512, 1024])
    cplans = [t.plan_concatenate_copy(F32, cat_out, 512 * 2048, half, 512 * 1024, 1, o)
              for o in (0, 1024)]
    bout, row = Layout.compact([1024, 256]), Layout.compact([1024])
    bplan = t.plan_broadcast_in_dim(F32, bout, 1024 * 256, row, 1024, [0])
    sizes = {"t": m * n, "m": vcount, "r": 64, "c": 512 * 2048, "b": 1024 * 256}
    for k, v in sizes.items():
        outs[k] = sentinel(v * 4)

    def record():
        hip.tiled_transpose(outs["t"], d_src, F32, 0, m * n, m, n, t.TransposeConfig.DEFAULT,
                            tplan, s)
        hip.materialize_strided(outs["m"], d_src, F32, view, vcount, mplan, s)
        hip.reduction(rplan, outs["r"], d_src, part, F32, t.ReduceOp.Sum, out_l, in_l, 0, 64, s)
        for o, p in zip((0, 1024), cplans):
            hip.concatenate_copy(outs["c"], d_src, F32, cat_out, half, 1, o, 512 * 1024, p, s)
        hip.broadcast_in_dim(outs["b"], d_src, F32, bout, row, [0], 1024 * 256, bplan, s)

    say("graphs: eager run")
    record()
    s.synchronize()
    eager = {k: to_host(outs[k], sizes[k] * 4) for k in sizes}
    want_t = np.empty(m * n, np.float32)
    orc.tiled_transpose(want_t, src, F32, 0, m * n, m, n, 1)
    assert np.array_equal(eager["t"], want_t.view(np.uint8))
    want_p = np.zeros(pl.element_count(), np.float32)
    orc.reduce_partials(want_p, src, F32, t.ReduceOp.Sum, 32, pl, in_l, 0, 64,
                        rplan.split.splits, rplan.split.chunk_len)
    want_r = np.zeros(64, np.float32)
    width = rplan.pass2.block[0] if rplan.combine_strategy == t.ReduceStrategy.Plane else 32
    orc.reduce(want_r, want_p, F32, rplan.combine_op, rplan.combine_strategy, width, out_l, pl, 0,
               64)
    assert np.array_equal(eager["r"], want_r.view(np.uint8))

    say("graphs: capture")
    graph = hipmem.Graph(s, record)
    other_src, other_dst = to_device(src), sentinel(m * n * 4)
    for replay in range(5):
        for k in sizes:
            outs[k].fill(SENTINEL)
        # the program's own eager work between replays
        hip.tiled_transpose(other_dst, other_src, F32, 0, m * n, m, n, t.TransposeConfig.DEFAULT,
                            tplan, s)
        s.synchronize()
        say("graphs: replay", replay)
        graph.launch(s)
        s.synchronize()
        for k in sizes:
            assert np.array_equal(to_host(outs[k], sizes[k] * 4), eager[k]), (replay, k)
    assert np.array_equal(to_host(other_dst, m * n * 4), want_t.view(np.uint8))
    graph.destroy()


def test_captured_reduction_step_replays_the_eager_bytes():
    """A C2-shaped step of planned reductions (an inner-axis f32 Sum and Max that
    join into one launch, a strided-axis f32 Sum and Max on the column tiles plus
    a combine, an inner-axis i64 Sum on two launches) captured once and replayed
    five times between the program's own eager work: every replay gives the
    eager bytes, and those are the oracle's."""
    rng = np.random.default_rng(96)
    s = hipmem.Stream()
    I64 = DType.I64
    inner_ext, outer_ext = [8192, 512], [1024, 8192]  # reference axis 0 fastest
    hf_in = rng.uniform(-1.0, 1.0, 8192 * 512).astype(np.float32)
    hf_out = rng.uniform(-1.0, 1.0, 1024 * 8192).astype(np.float32)
    hi = rng.integers(-1000, 1001, 8192 * 512, dtype=np.int64)
    cases = [("sum_f32_inner", F32, t.ReduceOp.Sum, inner_ext, 0, hf_in),
             ("max_f32_inner", F32, t.ReduceOp.Max, inner_ext, 0, hf_in),
             ("sum_f32_outer", F32, t.ReduceOp.Sum, outer_ext, 1, hf_out),
             ("max_f32_outer", F32, t.ReduceOp.Max, outer_ext, 1, hf_out),
             ("sum_i64_inner", I64, t.ReduceOp.Sum, inner_ext, 0, hi)]
    inputs = {id(h): to_device(h) for h in (hf_in, hf_out, hi)}
    runs, joined = [], []
    for name, dt, op, ext, axis, host in cases:
        in_l = Layout.compact(ext)
        oe = list(ext)
        oe[axis] = 1
        out_l = Layout.compact(oe)
        on = out_l.element_count()
        plan = t.plan_reduction(dt, op, out_l, on, in_l, in_l.element_count(), axis, 32)
        assert plan.kind == "Split"
        pl = t.reduction_partials_layout(in_l, axis, plan.split.splits)
        part = hipmem.DeviceBuffer(pl.element_count() * dt.size)
        out = sentinel(on * dt.size)
        d_in = inputs[id(host)]
        joined.append(hip.reduction_joins(plan, d_in, dt, op, out_l, in_l, axis, on))
        runs.append((name, dt, op, axis, host, in_l, out_l, on, plan, pl, part, out, d_in))
    assert joined == [True, True, False, False, False]

    def record():
        for (_, dt, op, axis, _, in_l, out_l, on, plan, _, part, out, d_in) in runs:
            hip.reduction(plan, out, d_in, part, dt, op, out_l, in_l, axis, on, s)

    say("graphs: reduction step, eager run")
    record()
    s.synchronize()
    eager = []
    for (name, dt, op, axis, host, in_l, out_l, on, plan, pl, _, out, _) in runs:
        got = to_host(out, on * dt.size)
        np_t = host.dtype
        want_p = np.zeros(pl.element_count(), np_t)
        orc.reduce_partials(want_p, host, dt, op, 32, pl, in_l, axis, on, plan.split.splits,
                            plan.split.chunk_len)
        width = plan.pass2.block[0] if plan.combine_strategy == t.ReduceStrategy.Plane else 32
        want = np.zeros(on, np_t)
        orc.reduce(want, want_p, dt, plan.combine_op, plan.combine_strategy, width, out_l, pl,
                   axis, on)
        assert np.array_equal(got, want.view(np.uint8)), name
        eager.append(got)

    say("graphs: reduction step, capture")
    graph = hipmem.Graph(s, record)
    m = n = 1024
    src = random_elements(F32, m * n, rng)
    other_src, other_dst = to_device(src), sentinel(m * n * 4)
    tplan = t.plan_tiled_transpose(F32, t.TransposeConfig.DEFAULT, 0, m * n, m, n, 1, m * n,
                                   m * n)
    for replay in range(5):
        for r in runs:
            r[11].fill(SENTINEL)
        hip.tiled_transpose(other_dst, other_src, F32, 0, m * n, m, n, t.TransposeConfig.DEFAULT,
                            tplan, s)
        s.synchronize()
        say("graphs: reduction step, replay", replay)
        graph.launch(s)
        s.synchronize()
        for r, want in zip(runs, eager):
            assert np.array_equal(to_host(r[11], r[7] * r[1].size), want), (replay, r[0])
    graph.destroy()
