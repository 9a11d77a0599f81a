"""bench.py's workloads keep every device buffer their launches use alive, CPU
only, with a stand-in device.

The benchmark binds each launch's arguments once (the ctypes call, or the
module launch's argument block) and then holds only what the binding holds. A
buffer that nothing references any more is freed by Python, and a later launch
on its address would touch freed device memory. Here DeviceBuffer, the stream
and the code-object module are replaced by stand-ins that allocate nothing and
record when a buffer is freed; every workload is built (its plans and routes
come from the real library, which needs no device for them) and, after a
garbage collection, no buffer may have been freed while the workload lives.
"""
import gc
import sys
import types
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(REPO))


class FakeBuffer:
    freed: list = []
    next_ptr = 1 << 32

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.ptr = FakeBuffer.next_ptr
        FakeBuffer.next_ptr += (self.nbytes + 4095) // 4096 * 4096 + 4096

    @classmethod
    def from_array(cls, arr, extra=0, fill=None):
        return cls(arr.nbytes + extra)

    def data_ptr(self):
        return self.ptr

    def copy_from(self, other):
        pass

    def upload(self, arr, offset=0):
        pass

    def fill(self, byte):
        pass

    def __del__(self):
        FakeBuffer.freed.append(self.ptr)


class FakeModule:
    def __init__(self, path):
        pass

    def bind(self, name, grid, block, shared, stream, args):
        return lambda: None


@pytest.fixture
def bench(monkeypatch):
    import bench as b
    from t4a_cuda_kernels import hipmem
    monkeypatch.setattr(hipmem, "DeviceBuffer", FakeBuffer)
    monkeypatch.setattr(hipmem, "Module", FakeModule)
    monkeypatch.setattr(b, "_STREAM", types.SimpleNamespace(handle=0))
    # Inputs of the configurations' sizes, without generating their values.
    cfg = b.configs
    monkeypatch.setattr(cfg, "c1_input", lambda m=1024: np.zeros(m * m, np.float32))
    monkeypatch.setattr(cfg, "c2_inputs", lambda: (np.zeros(1 << 26, np.float32),
                                                   np.zeros(1 << 26, np.int64)))
    monkeypatch.setattr(cfg, "c3_input", lambda d: np.zeros(1 << 24, d))
    monkeypatch.setattr(cfg, "c4_inputs", lambda: (np.zeros(1 << 27, np.float32),
                                                   np.zeros(1 << 27, np.int32)))
    monkeypatch.setattr(cfg, "c5_input", lambda: np.zeros(1 << 24, np.complex128))
    FakeBuffer.freed = []
    yield b
    FakeBuffer.freed = []


@pytest.mark.parametrize("name", ["all", "c1", "c2", "c3", "c4", "c5", "route1"])
def test_workload_keeps_its_buffers(bench, name):
    w = bench.WORKLOADS[name]()
    gc.collect()
    assert not FakeBuffer.freed, f"{name}: {len(FakeBuffer.freed)} buffer(s) freed while in use"
    assert w.ops
    assert all(op.launches >= 1 and op.algo_bytes > 0 and op.dominant_bytes > 0
               for op in w.ops)
    del w
    gc.collect()
    assert FakeBuffer.freed  # the stand-in does notice frees


def test_all_covers_every_configuration(bench):
    w = bench.build_all()
    assert {op.config for op in w.ops} == {"C1", "C1-roofline", "C2", "C3", "C4", "C5"}
    names = [op.name for op in w.ops]
    assert len(names) == len(set(names)) == 14
    # one timed step's planned launches: joined inner f32 C2 ops are one launch,
    # the other split plans two, direct plans and movements one
    assert sum(op.launches for op in w.ops) == 19
