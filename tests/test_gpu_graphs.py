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
