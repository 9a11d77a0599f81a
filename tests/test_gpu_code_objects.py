"""The prepare step on the GPU: `Prepared` loads the code objects into the
current context and binds entries by name; launches through its handles match
the oracle; two preparations own separate modules, and closing one leaves the
other usable (reference docs/design/cubecl-kernel-port.md:88-109: loaded modules
stay private to their runtime)."""
import ctypes

import numpy as np
import pytest

import t4a_cuda_kernels as t
from t4a_cuda_kernels import hipmem
from t4a_cuda_kernels.code_objects import Prepared, code_objects
from gpu_util import random_elements, say, sentinel, to_device, to_host

pytestmark = pytest.mark.gpu


def copy_args(dst, src, dtype, n):
    return [ctypes.c_void_p(dst.ptr), ctypes.c_void_p(src.ptr), ctypes.c_int(int(dtype)),
            ctypes.c_longlong(n)]


def test_prepared_entries_launch_and_stay_private():
    rng = np.random.default_rng(80)
    n = 100003
    src = random_elements(t.DType.F64, n, rng)
    d_src = to_device(src)
    plan = t.plan_copy_exact(t.DType.F64, n)
    geo = (tuple(plan.grid), tuple(plan.block), plan.shared_bytes)
    say("prepare all entries")
    every = Prepared()
    assert every.entries == sorted(e for c in code_objects() for e in c.entries)
    say("prepare copy_exact twice")
    a = Prepared(["t4a_cuda_copy_exact"])
    b = Prepared(["t4a_cuda_copy_exact", "t4a_cuda_reduce"])
    assert a.function("t4a_cuda_copy_exact") != b.function("t4a_cuda_copy_exact")
    for p in (every, a, b):
        d = sentinel(n * 8)
        p.launch("t4a_cuda_copy_exact", *geo, None, copy_args(d, d_src, t.DType.F64, n))
        assert np.array_equal(to_host(d, n * 8), src.view(np.uint8))
    hipmem.synchronize()
    a.close()
    d = sentinel(n * 8)
    b.launch("t4a_cuda_copy_exact", *geo, None, copy_args(d, d_src, t.DType.F64, n))
    assert np.array_equal(to_host(d, n * 8), src.view(np.uint8))
    hipmem.synchronize()
    b.close()
    every.close()


def test_prepare_refuses_unknown_entries():
    with pytest.raises(KeyError):
        Prepared(["t4a_cuda_add"])
