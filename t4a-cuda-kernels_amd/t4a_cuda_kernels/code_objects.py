"""The gfx950 code objects that export the reference-named kernel entries, and
a prepare step that loads them.

The reference hands its CUDA text to the consumer (reference src/lib.rs:32-130,
`source::MODULES` and `source::module_of`) and its design compiles that text in
a prepare step before any numerical work, keeping loaded modules private to
each runtime (reference docs/design/cubecl-kernel-port.md:88-109). On this
target the code objects are built ahead of time next to libt4a_hip.so, so
prepare is: load each needed file into the current HIP context, bind the
entries by name, and fail there (not in the middle of a run) when a file is
missing or was built for another target. A `Prepared` owns its modules; two of
them never share handles, and closing one leaves the other's bindings valid.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from pathlib import Path
from typing import Iterable, Optional

from . import _lib


@dataclass(frozen=True)
class CodeObject:
    index: int
    name: str      # the translation unit, as the reference's module names
    file: str      # the file name next to libt4a_hip.so
    entries: tuple

    @property
    def path(self) -> Path:
        return path_of(self.index)


def target() -> str:
    """The architecture every code object is built for."""
    return _lib.load().t4a_code_object_target().decode()


def code_objects() -> list[CodeObject]:
    lib = _lib.load()
    out = []
    for i in range(lib.t4a_code_object_count()):
        entries = tuple(lib.t4a_code_object_entry(i, k).decode()
                        for k in range(lib.t4a_code_object_entry_count(i)))
        out.append(CodeObject(i, lib.t4a_code_object_name(i).decode(),
                              lib.t4a_code_object_file(i).decode(), entries))
    return out


def module_of(entry: str) -> Optional[CodeObject]:
    """The code object exporting `entry`, or None (reference source::module_of)."""
    i = _lib.load().t4a_code_object_of(entry.encode())
    return code_objects()[i] if i >= 0 else None


def path_of(index: int) -> Path:
    buf = ctypes.create_string_buffer(4096)
    status = _lib.load().t4a_code_object_path(index, buf, len(buf))
    if status != 0:
        from . import T4aError
        raise T4aError(status)
    return Path(buf.value.decode())


class Prepared:
    """Code objects loaded into the current HIP context with the named entries
    bound: the artifacts of a prepare step, owned by this object."""

    def __init__(self, entries: Optional[Iterable[str]] = None):
        from . import hipmem
        wanted = list(entries) if entries is not None else [
            e for c in code_objects() for e in c.entries]
        self._modules: dict[int, "hipmem.Module"] = {}
        self._functions: dict[str, tuple[int, int]] = {}
        try:
            for entry in wanted:
                c = module_of(entry)
                if c is None:
                    raise KeyError(f"no {target()} code object exports {entry!r}")
                if c.index not in self._modules:
                    path = c.path
                    if not path.exists():
                        raise FileNotFoundError(f"{path} is not built")
                    self._modules[c.index] = hipmem.Module(path)
                self._functions[entry] = (c.index, self._modules[c.index].function(entry))
        except BaseException:
            self.close()
            raise

    def function(self, entry: str) -> int:
        """The bound kernel handle (hipFunction_t) of a prepared entry."""
        return self._functions[entry][1]

    def launch(self, entry: str, grid, block, shared_bytes: int, stream, args) -> None:
        """hipModuleLaunchKernel of a prepared entry with by-value `args`."""
        self._modules[self._functions[entry][0]].launch(entry, grid, block, shared_bytes,
                                                        stream, args)

    @property
    def entries(self) -> list[str]:
        return sorted(self._functions)

    def close(self) -> None:
        """Unload this object's modules (the caller has finished its launches)."""
        for m in self._modules.values():
            m.unload()
        self._modules.clear()
        self._functions.clear()

    def __enter__(self) -> "Prepared":
        return self

    def __exit__(self, *exc) -> None:
        self.close()
