"""Device buffers, streams and events over the HIP runtime libt4a_hip.so links.

The C ABI leaves device memory and streams to the caller. This module is the
Python caller's side of that: a thin ctypes layer over the same
`libamdhip64.so.7` the kernels' library is linked against, so pointers, streams
and launches all live in one runtime. (torch ships a separate HIP runtime of
its own; mixing its streams or allocations with this library's launches in one
process is not supported, so the tests and the benchmark use this module.)
"""
from __future__ import annotations

import ctypes
from ctypes import byref, c_float, c_int, c_size_t, c_void_p

import numpy as np

from . import _lib

H2D, D2H, D2D = 1, 2, 3
_HIP = None

# What this process has asked of the device through this module: device
# allocations, bytes copied (either direction, device to device included),
# memsets, host waits (device, stream and event synchronizations) and module
# kernel launches. A benchmark snapshots them around its timed region, as the
# reference benchmark does with its own counters (examples/bench_kernels.rs:
# 86-152); kernel launches of the library itself are t4a_hip_launch_count().
COUNTS = {"allocations": 0, "transfer_bytes": 0, "fills": 0, "host_waits": 0,
          "module_launches": 0}


def counts() -> dict:
    """A copy of COUNTS."""
    return dict(COUNTS)


def hip() -> ctypes.CDLL:
    """The HIP runtime already mapped by libt4a_hip.so (same soname, same handle)."""
    global _HIP
    if _HIP is None:
        _lib.load()
        lib = ctypes.CDLL("libamdhip64.so.7")
        lib.hipMalloc.argtypes = [ctypes.POINTER(c_void_p), c_size_t]
        lib.hipFree.argtypes = [c_void_p]
        lib.hipMemcpy.argtypes = [c_void_p, c_void_p, c_size_t, c_int]
        lib.hipMemcpyAsync.argtypes = [c_void_p, c_void_p, c_size_t, c_int, c_void_p]
        lib.hipMemset.argtypes = [c_void_p, c_int, c_size_t]
        lib.hipGetErrorString.restype = ctypes.c_char_p
        lib.hipGetErrorString.argtypes = [c_int]
        lib.hipGetDeviceCount.argtypes = [ctypes.POINTER(c_int)]
        lib.hipStreamCreate.argtypes = [ctypes.POINTER(c_void_p)]
        lib.hipStreamDestroy.argtypes = [c_void_p]
        lib.hipStreamSynchronize.argtypes = [c_void_p]
        lib.hipEventCreate.argtypes = [ctypes.POINTER(c_void_p)]
        lib.hipEventDestroy.argtypes = [c_void_p]
        lib.hipEventRecord.argtypes = [c_void_p, c_void_p]
        lib.hipEventSynchronize.argtypes = [c_void_p]
        lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(c_float), c_void_p, c_void_p]
        lib.hipDeviceGetName.argtypes = [ctypes.c_char_p, c_int, c_int]
        lib.hipModuleLoadData.argtypes = [ctypes.POINTER(c_void_p), c_void_p]
        lib.hipModuleUnload.argtypes = [c_void_p]
        lib.hipModuleGetFunction.argtypes = [ctypes.POINTER(c_void_p), c_void_p, ctypes.c_char_p]
        lib.hipModuleLaunchKernel.argtypes = [c_void_p, ctypes.c_uint, ctypes.c_uint,
                                              ctypes.c_uint, ctypes.c_uint, ctypes.c_uint,
                                              ctypes.c_uint, ctypes.c_uint, c_void_p,
                                              ctypes.POINTER(c_void_p), ctypes.POINTER(c_void_p)]
        lib.hipStreamBeginCapture.argtypes = [c_void_p, c_int]
        lib.hipStreamEndCapture.argtypes = [c_void_p, ctypes.POINTER(c_void_p)]
        lib.hipGraphInstantiate.argtypes = [ctypes.POINTER(c_void_p), c_void_p, c_void_p,
                                            ctypes.c_char_p, c_size_t]
        lib.hipGraphLaunch.argtypes = [c_void_p, c_void_p]
        lib.hipGraphExecDestroy.argtypes = [c_void_p]
        lib.hipGraphDestroy.argtypes = [c_void_p]
        _HIP = lib
    return _HIP


class HipError(RuntimeError):
    pass


def check(status: int, what: str) -> None:
    if status != 0:
        msg = hip().hipGetErrorString(status).decode()
        raise HipError(f"{what}: {msg} ({status})")


def device_count() -> int:
    n = c_int(0)
    status = hip().hipGetDeviceCount(byref(n))
    return n.value if status == 0 else 0


def device_name(device: int = 0) -> str:
    buf = ctypes.create_string_buffer(256)
    check(hip().hipDeviceGetName(buf, 256, device), "hipDeviceGetName")
    return buf.value.decode()


def synchronize() -> None:
    COUNTS["host_waits"] += 1
    check(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")


class DeviceBuffer:
    """`nbytes` of device memory, freed with the object."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = c_void_p()
        COUNTS["allocations"] += 1
        check(hip().hipMalloc(byref(p), max(self.nbytes, 1)), f"hipMalloc({self.nbytes})")
        self.ptr = p.value

    @classmethod
    def from_array(cls, arr: np.ndarray, extra: int = 0, fill: int | None = None):
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes + extra)
        if fill is not None:
            buf.fill(fill)
        buf.upload(arr)
        return buf

    def data_ptr(self) -> int:
        return self.ptr

    def upload(self, arr: np.ndarray, offset: int = 0) -> None:
        arr = np.ascontiguousarray(arr)
        assert offset + arr.nbytes <= self.nbytes
        COUNTS["transfer_bytes"] += arr.nbytes
        if arr.nbytes:
            check(hip().hipMemcpy(c_void_p(self.ptr + offset), c_void_p(arr.ctypes.data),
                                  arr.nbytes, H2D), "hipMemcpy H2D")

    def download(self, nbytes: int | None = None, offset: int = 0) -> np.ndarray:
        """`nbytes` (default: the rest of the buffer) from byte `offset`."""
        n = self.nbytes - offset if nbytes is None else int(nbytes)
        assert 0 <= offset and offset + n <= self.nbytes
        out = np.empty(n, dtype=np.uint8)
        COUNTS["transfer_bytes"] += n
        if n:
            check(hip().hipMemcpy(c_void_p(out.ctypes.data), c_void_p(self.ptr + offset), n,
                                  D2H), "hipMemcpy D2H")
        return out

    def copy_from(self, other: "DeviceBuffer") -> None:
        n = min(self.nbytes, other.nbytes)
        COUNTS["transfer_bytes"] += n
        check(hip().hipMemcpy(c_void_p(self.ptr), c_void_p(other.ptr), n, D2D), "hipMemcpy D2D")

    def fill(self, byte: int) -> None:
        COUNTS["fills"] += 1
        check(hip().hipMemset(c_void_p(self.ptr), int(byte), self.nbytes), "hipMemset")

    def free(self) -> None:
        if getattr(self, "ptr", None):
            hip().hipFree(c_void_p(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    """A HIP stream of default priority."""

    def __init__(self):
        s = c_void_p()
        check(hip().hipStreamCreate(byref(s)), "hipStreamCreate")
        self.handle = s.value

    @property
    def cuda_stream(self) -> int:
        return self.handle or 0

    def synchronize(self) -> None:
        COUNTS["host_waits"] += 1
        check(hip().hipStreamSynchronize(c_void_p(self.handle)), "hipStreamSynchronize")

    def __del__(self):
        try:
            if self.handle:
                hip().hipStreamDestroy(c_void_p(self.handle))
        except Exception:
            pass


class Graph:
    """The launches `record()` enqueues on `stream`, captured once into a HIP
    graph (hipStreamBeginCapture / hipStreamEndCapture, thread-local mode) and
    instantiated; `launch()` replays them with one submission. The library's
    launchers allocate nothing and record no memsets, so they capture as they
    run; a replay reads and writes the buffers the capture named."""

    _THREAD_LOCAL = 1  # hipStreamCaptureModeThreadLocal

    def __init__(self, stream: "Stream", record):
        lib = hip()
        check(lib.hipStreamBeginCapture(c_void_p(stream.handle), self._THREAD_LOCAL),
              "hipStreamBeginCapture")
        g = c_void_p()
        try:
            record()
        finally:
            status = lib.hipStreamEndCapture(c_void_p(stream.handle), byref(g))
        check(status, "hipStreamEndCapture")
        self._graph = g.value
        e = c_void_p()
        check(lib.hipGraphInstantiate(byref(e), c_void_p(self._graph), None, None, 0),
              "hipGraphInstantiate")
        self._exec = e.value

    def launch(self, stream: "Stream") -> None:
        check(hip().hipGraphLaunch(c_void_p(self._exec), c_void_p(stream.handle)),
              "hipGraphLaunch")

    def destroy(self) -> None:
        if getattr(self, "_exec", None):
            hip().hipGraphExecDestroy(c_void_p(self._exec))
            self._exec = None
        if getattr(self, "_graph", None):
            hip().hipGraphDestroy(c_void_p(self._graph))
            self._graph = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class Event:
    def __init__(self):
        e = c_void_p()
        check(hip().hipEventCreate(byref(e)), "hipEventCreate")
        self.handle = e.value

    def record(self, stream: Stream | None = None) -> None:
        s = c_void_p(stream.handle if stream is not None else 0)
        check(hip().hipEventRecord(c_void_p(self.handle), s), "hipEventRecord")

    def synchronize(self) -> None:
        COUNTS["host_waits"] += 1
        check(hip().hipEventSynchronize(c_void_p(self.handle)), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = c_float()
        check(hip().hipEventElapsedTime(byref(ms), c_void_p(self.handle), c_void_p(end.handle)),
              "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        try:
            if self.handle:
                hip().hipEventDestroy(c_void_p(self.handle))
        except Exception:
            pass


class Module:
    """A loaded gfx950 code object whose kernels are found by name, as the
    reference's callers load its cubins (reference tests/gpu/mod.rs:81-111)."""

    def __init__(self, path):
        self._image = ctypes.create_string_buffer(open(path, "rb").read())
        m = c_void_p()
        check(hip().hipModuleLoadData(byref(m), ctypes.cast(self._image, c_void_p)),
              f"hipModuleLoadData({path})")
        self.handle = m.value
        self._functions: dict[str, int] = {}

    def function(self, name: str) -> int:
        if name not in self._functions:
            f = c_void_p()
            check(hip().hipModuleGetFunction(byref(f), c_void_p(self.handle), name.encode()),
                  f"hipModuleGetFunction({name})")
            self._functions[name] = f.value
        return self._functions[name]

    def launch(self, name: str, grid, block, shared_bytes: int, stream, args) -> None:
        """Launch `name` with `kernelParams` pointing at each ctypes argument in
        `args` (by-value structs included); an empty grid launches nothing."""
        if 0 in tuple(grid):
            return
        COUNTS["module_launches"] += 1
        params = (c_void_p * len(args))(*[ctypes.cast(byref(a), c_void_p) for a in args])
        s = c_void_p(stream.handle if isinstance(stream, Stream) else (stream or 0))
        check(hip().hipModuleLaunchKernel(c_void_p(self.function(name)), *map(int, grid),
                                          *map(int, block), int(shared_bytes), s, params, None),
              f"hipModuleLaunchKernel({name})")

    def bind(self, name: str, grid, block, shared_bytes: int, stream, args):
        """`launch` with the argument block built once: returns a callable that
        launches `name` again with the same arguments (their ctypes objects are
        kept alive by the callable)."""
        if 0 in tuple(grid):
            return lambda: None
        params = (c_void_p * len(args))(*[ctypes.cast(byref(a), c_void_p) for a in args])
        s = c_void_p(stream.handle if isinstance(stream, Stream) else (stream or 0))
        fn = c_void_p(self.function(name))
        g, b = tuple(map(int, grid)), tuple(map(int, block))
        lib = hip()
        keep = (params, args)

        def go():
            COUNTS["module_launches"] += 1
            check(lib.hipModuleLaunchKernel(fn, *g, *b, int(shared_bytes), s, params, None),
                  f"hipModuleLaunchKernel({name})")
        go.keep = keep
        return go

    def unload(self) -> None:
        if getattr(self, "handle", None):
            hip().hipModuleUnload(c_void_p(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.unload()
        except Exception:
            pass
