"""The code-object table (t4a_code_object_*), CPU only: it names exactly the
kernels each gfx950 code object exports (read from the files' ELF symbol
tables), maps every reference-named entry of this path to its file (reference
src/lib.rs:98-107, `source::module_of`) and finds the files next to the
library."""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

import t4a_cuda_kernels as t
from t4a_cuda_kernels import T4aError, _lib
from t4a_cuda_kernels import code_objects as co

READELF = Path("/opt/rocm/llvm/bin/llvm-readelf")


def exported_kernels(path: Path) -> set[str]:
    syms = subprocess.run([str(READELF), "--syms", "--wide", str(path)], capture_output=True,
                          text=True, check=True).stdout
    # the reference-named (extern "C") kernels; the launchers' own kernels are
    # C++-mangled
    return {k for k in re.findall(r"OBJECT\s+GLOBAL\s+\S+\s+\S+\s+(\S+)\.kd$", syms, re.M)
            if not k.startswith("_Z")}


def test_the_table_names_exactly_what_each_file_exports():
    objs = co.code_objects()
    assert [c.name for c in objs] == ["movement", "reduce"]
    assert co.target() == "gfx950"
    for c in objs:
        assert c.file == f"t4a_{c.name}.gfx950.hsaco"
        assert c.path.parent == Path(_lib.LIB_PATH).parent and c.path.exists()
        assert set(c.entries) == exported_kernels(c.path), c.name
        assert len(set(c.entries)) == len(c.entries)


def test_module_of_every_entry():
    for c in co.code_objects():
        for e in c.entries:
            assert co.module_of(e) == c
    assert co.module_of("t4a_cuda_reduce_partials").name == "reduce"
    assert co.module_of("t4a_cuda_tiled_transpose").name == "movement"
    # reference entries outside this path, and nonsense, map to nothing
    for e in ("t4a_cuda_add", "t4a_cuda_gather", "t4a_cuda_reduce_x", ""):
        assert co.module_of(e) is None
    assert _lib.load().t4a_code_object_of(None) == -1


def test_path_errors():
    lib = _lib.load()
    with pytest.raises(T4aError) as e:
        co.path_of(7)
    assert e.value.status == 102 and "NotFound" in str(e.value)
    small = ctypes.create_string_buffer(4)
    assert lib.t4a_code_object_path(0, small, len(small)) == 103
    assert lib.t4a_status_name(103).decode() == "TooSmall"
    assert lib.t4a_code_object_name(-1) is None and lib.t4a_code_object_file(2) is None
    assert lib.t4a_code_object_entry(0, 999) is None and lib.t4a_code_object_entry_count(9) == 0
