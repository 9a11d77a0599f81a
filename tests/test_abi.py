"""The C ABI, CPU only: the shared library loads without a GPU and exports every
function include/t4a/t4a.h declares plus the reference kernel entry names; the
headers compile as C11 and C++17 with their layout assertions; the revision and
the status numbering agree between the header, the library and the Python
mirror (reference tests/planning.rs:12-34 checks the same for its crate)."""
import ctypes
import re
import subprocess
from pathlib import Path

import t4a_cuda_kernels as t
from t4a_cuda_kernels import _lib

REPO = Path(__file__).resolve().parent.parent
HEADER = REPO / "include" / "t4a" / "t4a.h"
ABI_HEADER = REPO / "include" / "t4a" / "abi.h"

# The reference's kernel entries this library exports under the same names
# (reference cuda/src/movement.cu:514-685, cuda/src/reduce.cu:765-940), the
# general-rank `_any` twins included.
KERNEL_SYMBOLS = [
    "t4a_cuda_copy_exact",
    "t4a_cuda_materialize_strided",
    "t4a_cuda_strided_to_strided",
    "t4a_cuda_tiled_transpose",
    "t4a_cuda_reduce",
    "t4a_cuda_reduce_partials",
    "t4a_cuda_materialize_strided_any",
    "t4a_cuda_strided_to_strided_any",
    "t4a_cuda_reduce_any",
    "t4a_cuda_reduce_partials_any",
    "t4a_cuda_fill_zero",
    "t4a_cuda_fill_zero_view",
    "t4a_cuda_fill_zero_view_any",
    "t4a_cuda_contiguous_to_view",
    "t4a_cuda_contiguous_to_view_any",
    "t4a_cuda_broadcast_in_dim",
    "t4a_cuda_broadcast_in_dim_any",
    "t4a_cuda_concatenate_copy",
    "t4a_cuda_concatenate_copy_any",
]


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(t4a_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_function():
    lib = _lib.load()
    names = declared_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    # and the Python binding knows every one of them
    assert set(names) <= set(_lib.SIGNATURES), set(names) - set(_lib.SIGNATURES)


def test_library_exports_the_reference_kernel_entries():
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in KERNEL_SYMBOLS:
        assert hasattr(lib, name), name


def test_code_objects_export_the_reference_kernel_entries():
    """The gfx950 code objects a module-loading caller finds kernels in by name."""
    readelf = Path("/opt/rocm/llvm/bin/llvm-readelf")
    pkg = Path(_lib.LIB_PATH).parent
    wanted = {"t4a_movement.gfx950.hsaco": [n for n in KERNEL_SYMBOLS if "reduce" not in n],
              "t4a_reduce.gfx950.hsaco": [n for n in KERNEL_SYMBOLS if "reduce" in n]}
    for name, symbols in wanted.items():
        path = pkg / name
        assert path.exists(), f"{name} not built"
        syms = subprocess.run([str(readelf), "--syms", "--wide", str(path)], capture_output=True,
                              text=True, check=True).stdout
        for sym in symbols:
            assert re.search(rf"FUNC\s+GLOBAL\s+\S+\s+\S+\s+{sym}$", syms, re.M), (name, sym)
            assert re.search(rf"OBJECT\s+GLOBAL\s+\S+\s+\S+\s+{sym}\.kd$", syms, re.M), (name, sym)


def test_headers_compile_as_c_and_cxx(tmp_path):
    src = tmp_path / "probe.c"
    src.write_text('#include "t4a/abi.h"\n#include "t4a/t4a.h"\n'
                   "int main(void) { t4a_launch l; t4a_cuda_layout x; (void)l; (void)x;"
                   " return T4A_CUDA_ABI_REVISION == 14 ? 0 : 1; }\n")
    for compiler, std, name in (("gcc", "-std=c11", "probe.c"), ("g++", "-std=c++17", "probe.cc")):
        path = tmp_path / name
        path.write_text(src.read_text())
        out = tmp_path / (name + ".bin")
        proc = subprocess.run([compiler, std, "-Wall", "-Werror", f"-I{REPO / 'include'}",
                               str(path), "-o", str(out)], capture_output=True, text=True)
        assert proc.returncode == 0, proc.stderr
        assert subprocess.run([str(out)]).returncode == 0


def test_revision_agrees_everywhere():
    declared = re.search(r"#define T4A_CUDA_ABI_REVISION (\d+)", ABI_HEADER.read_text())
    assert int(declared.group(1)) == t.ABI_REVISION == t.abi_revision() == 14


def test_status_numbering_is_the_reference_error_plus_one():
    lib = _lib.load()
    for e in t.Error:
        assert lib.t4a_status_name(int(e) + 1).decode() == e.name
    assert lib.t4a_status_name(0).decode() == "Ok"
    text = HEADER.read_text()
    assert "T4A_ERR_OFFSET_OUT_OF_SPAN = 7" in text and "T4A_ERR_UNSUPPORTED_OP = 25" in text


def test_struct_layouts_match_the_header():
    assert ctypes.sizeof(_lib.CLayout) == 144
    assert _lib.CLayout.extents.offset == 16 and _lib.CLayout.strides.offset == 80
    assert ctypes.sizeof(_lib.CTransposeConfig) == 16
    d = _lib.load().t4a_transpose_config_default()
    assert (d.tile, d.block_rows, d.padding, d.vector_width) == (16, 8, 1, 1)


def test_dtype_sizes():
    lib = _lib.load()
    for d in t.DType:
        assert lib.t4a_dtype_size(int(d)) == d.size
    assert lib.t4a_dtype_size(7) == 0
