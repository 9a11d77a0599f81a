"""The CPU oracle's OpenMP loops (bench.py's all-core CPU baseline): every
output is folded serially on one thread, so any thread count gives the
single-thread bytes. Checked on a split reduction (pass 1 and the combine), a
unit reduction over a strided axis, a strided permute and a tiled transpose."""
import numpy as np
import pytest

import t4a_cuda_kernels as t
from t4a_cuda_kernels import DType, Layout
from oracle import t4a_oracle as orc


@pytest.fixture
def threads():
    yield
    orc.set_threads(1)


def _both(fn):
    orc.set_threads(1)
    one = fn()
    orc.set_threads(4)
    many = fn()
    return one, many


def test_split_reduction_bytes_do_not_depend_on_threads(threads):
    rng = np.random.default_rng(7)
    ext = [2048, 96]
    x = rng.standard_normal(2048 * 96).astype(np.float32)
    in_l, out_l = Layout.compact(ext), Layout.compact([1, 96])
    plan = t.plan_reduction(DType.F32, t.ReduceOp.SumSquares, out_l, 96, in_l, x.size, 0, 32)
    assert plan.kind == "Split"
    pl = t.reduction_partials_layout(in_l, 0, plan.split.splits)

    def run():
        part = np.zeros(pl.element_count(), np.float32)
        orc.reduce_partials(part, x, DType.F32, t.ReduceOp.SumSquares, 32, pl, in_l, 0, 96,
                            plan.split.splits, plan.split.chunk_len)
        out = np.zeros(96, np.float32)
        width = plan.pass2.block[0] if plan.combine_strategy == t.ReduceStrategy.Plane else 32
        orc.reduce(out, part, DType.F32, plan.combine_op, plan.combine_strategy, width, out_l,
                   pl, 0, 96)
        assert np.count_nonzero(part) == part.size and np.count_nonzero(out) == out.size
        return part.tobytes() + out.tobytes()

    one, many = _both(run)
    assert one == many


def test_unit_reduction_and_movement_bytes_do_not_depend_on_threads(threads):
    rng = np.random.default_rng(8)
    x = rng.standard_normal(8 ** 5 * 2)  # c64 [8]^5
    src = Layout([8] * 5, [64, 4096, 8, 512, 1], 0)
    dst = Layout.compact([8] * 5)

    def move():
        out = np.zeros_like(x)
        orc.strided_to_strided(out, x, DType.C64, src, dst, 8 ** 5)
        red = np.zeros(8 ** 4 * 2)
        out_l = Layout.compact([8, 8, 1, 8, 8])
        orc.reduce(red, out, DType.C64, t.ReduceOp.Sum, t.ReduceStrategy.Unit, 32, out_l, dst, 2,
                   8 ** 4)
        y = x[:96 * 160]
        tr = np.zeros(96 * 160)
        orc.tiled_transpose(tr, y, DType.F64, 0, 96 * 160, 96, 160, 1)
        assert np.count_nonzero(out) == out.size and np.count_nonzero(red) == red.size
        assert np.count_nonzero(tr) == tr.size
        return out.tobytes() + red.tobytes() + tr.tobytes()

    one, many = _both(move)
    assert one == many
    assert orc.max_threads() >= 1
