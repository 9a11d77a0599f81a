"""The reference's split-reduction golden cases: inputs and expected outputs.

`tests/golden/reduce-golden.tsv` (copied from the reference's
tests/data/reduce-golden.tsv, MIT OR Apache-2.0, see tests/golden/NOTICE) holds
1332 A100 captures of planned two-pass reductions: the split plan, the FNV-1a
hash of the whole pass-1 partials buffer, and the bytes of every final output.
The inputs are not stored: they are regenerated here from the reference
generator's definition (reference tests/gpu_reduce_golden.rs:49-315):

  * SplitMix64 seeded with FNV-1a of "{shape}|{dtype}|{op}|{class}";
  * one `unit()` draw per component (two for the Overflow class);
  * class transforms, then NaN payloads / infinities / zeros placed at the axis
    positions where pass 1 and the combine meet them.

This module is shared by the CPU oracle test and the GPU test.
"""
from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path

import numpy as np

from t4a_cuda_kernels import configs

GOLDEN = Path(__file__).resolve().parent / "golden" / "reduce-golden.tsv"

# (name, extents in reference axis-0-fastest order, axis)
SHAPES = [
    ("n1048576", (1_048_576,), 0),
    ("n1000003", (1_000_003,), 0),
    ("n4194304", (4_194_304,), 0),
    ("n65541", (65_541,), 0),
    ("n8195", (8_195,), 0),
    ("3x100003-axis1", (3, 100_003), 1),
    ("131075x3-axis0", (131_075, 3), 0),
]
SHAPE_BY_NAME = {name: (ext, axis) for name, ext, axis in SHAPES}

DTYPES = {"F32": (0, 4, 1), "F64": (1, 8, 1), "C32": (5, 4, 2), "C64": (6, 8, 2)}
OPS = {"Sum": 0, "Prod": 1, "SumSquares": 2, "Max": 3, "Min": 4}
CLASSES = ["Random", "NanPayloads", "Infs", "SignedZeros", "NegZeros", "Overflow"]

# The config generator: SplitMix64 and unit() (t4a_cuda_kernels.configs). The
# golden inputs are regenerated with it, so these vectors pin the generator the
# benchmark and the config tests use.
unit = configs.unit


def splitmix_draws(seed: int, n: int) -> np.ndarray:
    """The first n outputs of SplitMix64(seed): state += gamma, then mix."""
    return configs.draws(seed, n)


def fnv1a64_text(text: str) -> int:
    h = 0xCBF29CE484222325
    for b in text.encode():
        h ^= b
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def compact_strides(extents) -> list[int]:
    out, s = [], 1
    for e in extents:
        out.append(s)
        s *= e
    return out


def line_base(extents, axis: int, o: int) -> int:
    strides = compact_strides(extents)
    base = 0
    for d, e in enumerate(extents):
        if d == axis:
            continue
        base += (o % e) * strides[d]
        o //= e
    return base


def nan_positions(axis_len: int, splits: int, chunk: int) -> list[int]:
    out = [0, 1, 33] + [32 * k for k in range(1, 32)]
    out += [k * chunk + 7 for k in (5, 37, 69, 133, 517, 1029) if k < splits]
    out.append(axis_len - 1)
    return sorted({p for p in out if p < axis_len})


def _nan_bits(width: int, k: int) -> int:
    if width == 4:
        sign = 0x80000000 if k % 2 == 1 else 0
        return sign | 0x7FC00000 | (0x100 + k * 0x11)
    sign = 1 << 63 if k % 2 == 1 else 0
    return sign | 0x7FF8000000000000 | (0x1000 + k * 0x111)


def input_array(shape: str, dtype: str, op: str, cls: str, splits: int) -> np.ndarray:
    """The reference input bytes as a numpy array of components
    (float32/float64, complex interleaved re, im)."""
    extents, axis = SHAPE_BY_NAME[shape]
    _, width, comps = DTYPES[dtype]
    count = int(np.prod(extents))
    seed = fnv1a64_text(f"{shape}|{dtype}|{op}|{cls}")
    prod = op == "Prod"
    per = 2 if cls == "Overflow" else 1
    draws = unit(splitmix_draws(seed, count * comps * per)).reshape(count, comps, per)
    u = draws[:, :, 0]
    if cls == "SignedZeros":
        vals = np.where(u < 0.0, -0.0, 0.0)
    elif cls == "NegZeros":
        vals = np.full_like(u, -0.0)
    elif cls == "Overflow":
        mag = 2.0 + 0.5 * draws[:, :, 1]
        vals = np.where(u < 0.0, -mag, mag)
    elif prod:
        vals = u * (1.0 / 512.0)
        vals[:, 0] = 1.0 + u[:, 0] * (1.0 / 512.0)
    else:
        vals = u
    ftype = np.float32 if width == 4 else np.float64
    itype = np.uint32 if width == 4 else np.uint64
    arr = vals.astype(ftype).reshape(-1)
    bits = arr.view(itype)
    axis_len = extents[axis]
    axis_stride = compact_strides(extents)[axis]
    outputs = count // axis_len
    chunk = axis_len // max(splits, 1)
    lines = [0] + ([outputs - 1] if outputs > 1 else [])
    k = 0
    for line in lines:
        base = line_base(extents, axis, line)

        def put(position, comp, value=None, nan=None):
            at = (base + position * axis_stride) * comps + comp
            if nan is not None:
                bits[at] = itype(nan)
            else:
                arr[at] = ftype(value)

        if cls == "NanPayloads":
            for position in nan_positions(axis_len, splits, chunk):
                put(position, k % comps, nan=_nan_bits(width, k))
                k += 1
        elif cls == "Infs":
            late = 41 * chunk + 2 if 41 < splits else min(40, axis_len - 1)
            put(min(9 * chunk + 2, axis_len - 1), 0, np.inf)
            put(late, 0, -np.inf)
            if prod:
                put(min(3 * chunk + 1, axis_len - 1), 0, 0.0)
        elif cls == "Overflow":
            put(min(3 * chunk + 1, axis_len - 1), 0, 0.0)
    return arr


@dataclass(frozen=True)
class GoldenCase:
    key: str
    shape: str
    width: int
    dtype: str
    op: str
    cls: str
    plan: str
    partials_bytes: int
    partials_fnv: int
    finals: bytes


def load_cases(path: Path = GOLDEN, path_kind: str = "fast") -> list[GoldenCase]:
    """The golden rows of one launch path ("fast": the by-value entries)."""
    out = []
    for line in path.read_text().splitlines():
        if line.startswith("#") or not line:
            continue
        key, plan, nbytes, fnv, finals = line.split("\t")
        shape, w, dtype, op, cls, kind = key.split("|")
        if kind != path_kind:
            continue
        out.append(GoldenCase(key, shape, int(w[1:]), dtype, op, cls, plan, int(nbytes),
                              int(fnv, 16), bytes.fromhex(finals)))
    return out


def parse_plan(plan: str) -> tuple[int, int, str, int]:
    """'splits=512 chunk=256 combine=Plane/32' -> (512, 256, 'Plane', 32)."""
    fields = dict(item.split("=") for item in plan.split())
    strategy, width = fields["combine"].split("/")
    return int(fields["splits"]), int(fields["chunk"]), strategy, int(width)


def components_equal(dtype: str, golden: bytes, got: bytes, payload_free: bool) -> bool:
    """Bytes equal; or, when `payload_free`, equal except NaN components whose
    payloads differ (the contract promises "is NaN" only,
    reference docs/abi/c-kernel-abi.md:364-366)."""
    if golden == got:
        return True
    if not payload_free or len(golden) != len(got):
        return False
    _, width, _ = DTYPES[dtype]
    ft = np.float32 if width == 4 else np.float64
    a = np.frombuffer(golden, dtype=ft)
    b = np.frombuffer(got, dtype=ft)
    ai = np.frombuffer(golden, dtype=np.uint32 if width == 4 else np.uint64)
    bi = np.frombuffer(got, dtype=np.uint32 if width == 4 else np.uint64)
    same = (ai == bi) | (np.isnan(a) & np.isnan(b))
    return bool(same.all())


def payloads_decided_by_arithmetic(case: GoldenCase) -> bool:
    """Whether a NaN in this case's outputs comes out of an add or multiply,
    whose NaN payload is the hardware's choice; max/min select an operand and
    keep its payload everywhere."""
    return case.op in ("Sum", "Prod", "SumSquares") and case.cls in (
        "NanPayloads", "Infs", "Overflow")
