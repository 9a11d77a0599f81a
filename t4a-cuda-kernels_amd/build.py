"""Build libt4a_hip.so: the gfx950 kernels, their launchers and the host planner.

Run `python t4a-cuda-kernels_amd/build.py` (or `__graft_entry__.build()`). The
shared library is written next to the Python package
(`t4a_cuda_kernels/libt4a_hip.so`) so that it travels with the source tree.

Each HIP source is also built as a standalone gfx950 code object
(`t4a_cuda_kernels/t4a_movement.gfx950.hsaco`, `t4a_reduce.gfx950.hsaco`) that
exports the reference's kernel entry names, for callers that load kernels by
name from a module (`hipModuleLoadData` + `hipModuleGetFunction`), as the
reference's callers do with its cubins.

HIP sources are compiled for gfx950 only, with:
  -ffp-contract=off      every floating-point rounding is the one written
                         (the fold topology and the complex product spell
                         out their fused multiply-adds);
  -packed-fp32-ops off   no packed FP32 instructions are generated.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
REPO = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
OUT_DIR = PKG_ROOT / "t4a_cuda_kernels"
LIB_NAME = "libt4a_hip.so"
ARCH = "gfx950"

HIP_SOURCES = ["movement.hip", "reduce.hip"]
CXX_SOURCES = ["planner.cpp", "code_objects.cpp"]


def code_object_name(source: str) -> str:
    return f"t4a_{Path(source).stem}.{ARCH}.hsaco"


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}")


def build(verbose: bool = False) -> Path:
    """Compile every source and link the shared library; returns its path."""
    hipcc = _hipcc()
    obj_dir = PKG_ROOT / "_build"
    obj_dir.mkdir(exist_ok=True)
    includes = [f"-I{REPO / 'include'}", f"-I{CSRC}"]
    objects = []
    for src in CXX_SOURCES:
        obj = obj_dir / (Path(src).stem + ".o")
        cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", *includes,
               "-c", str(CSRC / src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd))
        _run(cmd)
        objects.append(obj)
    hip_flags = [
        f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
        "-ffp-contract=off",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-command-line-argument",
    ]
    OUT_DIR.mkdir(exist_ok=True)
    hip_cmds = []
    for src in HIP_SOURCES:
        obj = obj_dir / (Path(src).stem + ".o")
        hip_cmds.append([hipcc, *hip_flags, *includes, "-c", str(CSRC / src), "-o", str(obj)])
        objects.append(obj)
        hip_cmds.append([hipcc, "--genco", "--no-gpu-bundle-output", *hip_flags, *includes,
                         str(CSRC / src), "-o", str(OUT_DIR / code_object_name(src))])
    # The translation units are independent: compile them side by side.
    with ThreadPoolExecutor(max_workers=len(hip_cmds)) as pool:
        for cmd in hip_cmds:
            if verbose:
                print(" ".join(cmd))
        list(pool.map(_run, hip_cmds))
    out = OUT_DIR / LIB_NAME
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects),
           "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd))
    _run(cmd)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
