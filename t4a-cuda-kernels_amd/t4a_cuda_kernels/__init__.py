"""Host-side mirror of the reference crate `t4a_cuda_kernels` (reference src/lib.rs)
for the movement and single-axis reduction path, over the MI355X C ABI.

Names, argument order and error behaviour follow the reference: a planner
returns a `Launch` (or `ReductionPlan`) or raises `T4aError` carrying the
reference `Error` variant for the same bad input. Geometry is this library's
MI355X geometry. Launching lives in `t4a_cuda_kernels.hip` (raw device
pointers and a HIP stream, the caller owning both).
"""
from __future__ import annotations

import ctypes
import enum
from ctypes import byref, c_int, c_longlong
from dataclasses import dataclass
from typing import Optional, Sequence

from . import _lib
from ._lib import (CAxisValues, CAxisValuesAny, CLaunch, CLayout, CLayoutAny, CReductionPlan,
                   CSplit, CTransposeConfig)

MAX_RANK = 8
ABI_REVISION = 14
FLAT_BLOCK = 256
PLANE_BLOCK = 32
PLANE_WIDTHS = (8, 16, 32)
MIN_CHUNK_PLANES = 8
MAX_SPLITS = 4096
MAX_GRID_X = 2**31 - 1
MAX_GRID_YZ = 65535
DEFAULT_SHARED_BYTES = 48 * 1024


class DType(enum.IntEnum):
    """Element type tags (reference src/lib.rs:151-215)."""

    F32 = 0
    F64 = 1
    I32 = 2
    I64 = 3
    Bool = 4
    C32 = 5
    C64 = 6

    @property
    def tag(self) -> int:
        return int(self)

    @property
    def size(self) -> int:
        return {0: 4, 1: 8, 2: 4, 3: 8, 4: 1, 5: 8, 6: 16}[int(self)]


class ReduceOp(enum.IntEnum):
    """Reduction operation tags (reference src/lib.rs:3065-3127)."""

    Sum = 0
    Prod = 1
    SumSquares = 2
    Max = 3
    Min = 4

    @property
    def tag(self) -> int:
        return int(self)

    def combine(self) -> "ReduceOp":
        """Operation of the combine pass: squared partials combine by a sum."""
        return ReduceOp.Sum if self is ReduceOp.SumSquares else self

    def supports(self, dtype: DType) -> bool:
        if self in (ReduceOp.Sum, ReduceOp.Prod):
            return dtype in (DType.F32, DType.F64, DType.I32, DType.I64, DType.C32, DType.C64)
        if self is ReduceOp.SumSquares:
            return dtype in (DType.F32, DType.F64)
        return dtype in (DType.F32, DType.F64, DType.I32, DType.I64)


class ReduceStrategy(enum.IntEnum):
    Unit = 0
    Plane = 1

    @property
    def tag(self) -> int:
        return int(self)


class Error(enum.IntEnum):
    """The reference `Error` enum (src/lib.rs:217-274); the C status is value + 1."""

    RankOutOfRange = 0
    RankLength = 1
    NegativeExtent = 2
    NegativeCount = 3
    Overflow = 4
    CountMismatch = 5
    OffsetOutOfSpan = 6
    BroadcastDestination = 7
    UnsupportedDType = 8
    NotElementwise = 9
    LaunchLimit = 10
    InvalidTransposeConfig = 11
    InvalidAxis = 12
    DuplicateAxis = 13
    NotCompact = 14
    ShapeMismatch = 15
    InvalidStep = 16
    InvalidPadding = 17
    DomainTooLarge = 18
    InvalidStride = 19
    StrategyMismatch = 20
    InvalidPlaneWidth = 21
    InvalidSplit = 22
    IndexVectorMismatch = 23
    UnsupportedOp = 24


class T4aError(Exception):
    """A planner refusal (`error` is the reference variant) or a launch failure."""

    def __init__(self, status: int):
        self.status = status
        self.error: Optional[Error] = Error(status - 1) if 1 <= status <= 25 else None
        lib = _lib.load()
        name = lib.t4a_status_name(status).decode()
        detail = ""
        if status == 100:  # T4A_HIP_ERR_LAUNCH: name the runtime's error
            code = lib.t4a_hip_last_error()
            from . import hipmem
            detail = f": {hipmem.hip().hipGetErrorString(code).decode()} (hipError {code})"
        super().__init__(f"{name} (status {status}){detail}")


def _check(status: int) -> None:
    if status != 0:
        raise T4aError(status)


class Layout:
    """Logical strided layout, axis 0 fastest (reference src/lib.rs:322-450)."""

    __slots__ = ("_c",)

    def __init__(self, extents: Sequence[int], strides: Sequence[int], offset: int = 0):
        if len(extents) != len(strides):
            raise T4aError(Error.RankLength + 1)
        rank = len(extents)
        c = CLayout()
        ext = (c_longlong * max(rank, 1))(*extents)
        st = (c_longlong * max(rank, 1))(*strides)
        _check(_lib.load().t4a_layout_new(byref(c), rank, ext, st, offset))
        self._c = c

    @classmethod
    def compact(cls, extents: Sequence[int]) -> "Layout":
        strides, stride = [], 1
        for e in extents:
            strides.append(stride)
            stride *= e
        if len(extents) > MAX_RANK:
            raise T4aError(Error.RankOutOfRange + 1)
        if stride >= 2**63:
            raise T4aError(Error.Overflow + 1)
        return cls(extents, strides, 0)

    @classmethod
    def from_c(cls, c: CLayout) -> "Layout":
        out = cls.__new__(cls)
        out._c = c
        return out

    @property
    def c(self) -> CLayout:
        return self._c

    @property
    def rank(self) -> int:
        return self._c.rank

    @property
    def offset(self) -> int:
        return self._c.offset

    @property
    def extents(self) -> list[int]:
        return list(self._c.extents[: self.rank])

    @property
    def strides(self) -> list[int]:
        return list(self._c.strides[: self.rank])

    def element_count(self) -> int:
        n = c_longlong()
        _check(_lib.load().t4a_layout_element_count(byref(self._c), byref(n)))
        return n.value

    def _reach(self, maximum: bool) -> int:
        total = self.offset
        for e, s in zip(self.extents, self.strides):
            step = (e - 1) * s
            total += max(step, 0) if maximum else min(step, 0)
        return total

    def min_reachable_offset(self) -> int:
        return self._reach(False)

    def max_reachable_offset(self) -> int:
        return self._reach(True)

    def is_compact(self) -> bool:
        if self.offset != 0:
            return False
        stride = 1
        for e, s in zip(self.extents, self.strides):
            if s != stride:
                return False
            stride *= e
        return True

    def __eq__(self, other: object) -> bool:
        return (isinstance(other, Layout) and self.extents == other.extents
                and self.strides == other.strides and self.offset == other.offset)

    def __repr__(self) -> str:
        return f"Layout(extents={self.extents}, strides={self.strides}, offset={self.offset})"


class WideLayout:
    """Strided layout of any rank, axis 0 fastest (reference WideLayout,
    src/lib.rs:1066-1110, validated as LayoutRef::new, 908-928): the geometry of
    the general-rank `_any` twins. The planners read it from host memory
    (`host_c`); the launchers take a `t4a_cuda_layout_any` whose arrays the
    caller has copied to the device (`device_c`, `pack`)."""

    __slots__ = ("_ext", "_str", "_offset")

    def __init__(self, extents: Sequence[int], strides: Sequence[int], offset: int = 0):
        if len(extents) != len(strides):
            raise T4aError(Error.RankLength + 1)
        if any(e < 0 for e in extents):
            raise T4aError(Error.NegativeExtent + 1)
        self._ext = [int(e) for e in extents]
        self._str = [int(x) for x in strides]
        self._offset = int(offset)

    @classmethod
    def compact(cls, extents: Sequence[int]) -> "WideLayout":
        strides, stride = [], 1
        for e in extents:
            strides.append(stride)
            stride *= e
            if stride >= 2**63:
                raise T4aError(Error.Overflow + 1)
        return cls(extents, strides, 0)

    @classmethod
    def of(cls, layout: "Layout") -> "WideLayout":
        return cls(layout.extents, layout.strides, layout.offset)

    @property
    def rank(self) -> int:
        return len(self._ext)

    @property
    def offset(self) -> int:
        return self._offset

    @property
    def extents(self) -> list[int]:
        return list(self._ext)

    @property
    def strides(self) -> list[int]:
        return list(self._str)

    def element_count(self) -> int:
        n = 1
        for e in self._ext:
            n *= e
            if n >= 2**63:
                raise T4aError(Error.Overflow + 1)
        return n

    def max_reachable_offset(self) -> int:
        return self._offset + sum(max((e - 1) * s, 0) for e, s in zip(self._ext, self._str))

    def min_reachable_offset(self) -> int:
        return self._offset + sum(min((e - 1) * s, 0) for e, s in zip(self._ext, self._str))

    def pack(self) -> list[int]:
        """The extents, then the strides (reference LayoutRef::pack, src/lib.rs:1029-1038)."""
        return self._ext + self._str

    def host_c(self) -> CLayoutAny:
        """A t4a_cuda_layout_any over host copies of the arrays (kept alive by
        the returned struct), for the t4a_plan_*_any planners."""
        n = max(self.rank, 1)
        ext = (c_longlong * n)(*self._ext)
        st = (c_longlong * n)(*self._str)
        c = CLayoutAny()
        c.rank = self.rank
        c.offset = self._offset
        c.extents = ctypes.addressof(ext)
        c.strides = ctypes.addressof(st)
        c._keep = (ext, st)  # the arrays live as long as the struct
        return c

    def device_c(self, extents_ptr: int, strides_ptr: int) -> CLayoutAny:
        """The launchers' t4a_cuda_layout_any: the arrays at `extents_ptr` and
        `strides_ptr`, device copies the caller made of `extents` / `strides`."""
        c = CLayoutAny()
        c.rank = self.rank
        c.offset = self._offset
        c.extents = extents_ptr
        c.strides = strides_ptr
        return c

    def __eq__(self, other: object) -> bool:
        return (isinstance(other, WideLayout) and self._ext == other._ext
                and self._str == other._str and self._offset == other._offset)

    def __repr__(self) -> str:
        return f"WideLayout(extents={self._ext}, strides={self._str}, offset={self._offset})"


@dataclass(frozen=True)
class TransposeConfig:
    """Tiled-transpose configuration (reference src/lib.rs:452-517)."""

    tile: int
    block_rows: int
    padding: int
    vector_width: int

    def __post_init__(self):
        c = CTransposeConfig()
        _check(_lib.load().t4a_transpose_config_new(
            self.tile, self.block_rows, self.padding, self.vector_width, byref(c)))

    @property
    def c(self) -> CTransposeConfig:
        return CTransposeConfig(self.tile, self.block_rows, self.padding, self.vector_width)

    def shared_bytes(self, element_size: int) -> int:
        return self.tile * (self.tile + self.padding) * element_size


TransposeConfig.DEFAULT = TransposeConfig(16, 8, 1, 1)


class RankVariant(enum.IntEnum):
    Fast = 0
    General = 1


class MoveRoute(enum.IntEnum):
    """The kernel the movement launchers run for a layout pair (t4a_move_route)."""

    Empty = 0
    Linear = 1     # one run contiguous on both sides: the copy kernel
    Rows = 2       # a dim contiguous on both sides: 16-byte row units
    Transpose = 3  # one compact 2-D transpose: the tiled transpose's kernel
    TileOnce = 4   # LDS tiles of one of the tile walk's shapes
    Tiles = 5      # persistent blocks walking LDS tiles
    Elements = 6   # one decode per element


@dataclass(frozen=True)
class Launch:
    """Planned geometry (reference src/lib.rs:840-873)."""

    grid: tuple
    block: tuple
    shared_bytes: int
    variant: RankVariant = RankVariant.Fast

    @classmethod
    def from_c(cls, c: CLaunch) -> "Launch":
        return cls(tuple(c.grid), tuple(c.block), c.shared_bytes, RankVariant(c.variant))

    def to_c(self) -> CLaunch:
        c = CLaunch()
        c.grid[:] = list(self.grid)
        c.block[:] = list(self.block)
        c.shared_bytes = self.shared_bytes
        c.variant = int(self.variant)
        return c

    def is_empty(self) -> bool:
        return 0 in self.grid


@dataclass(frozen=True)
class Split:
    splits: int
    chunk_len: int

    def to_c(self) -> CSplit:
        return CSplit(self.splits, self.chunk_len)


@dataclass(frozen=True)
class ReductionPlan:
    """`Direct` fills strategy/launch; `Split` fills split/pass1/combine_*/pass2."""

    kind: str
    strategy: Optional[ReduceStrategy] = None
    launch: Optional[Launch] = None
    split: Optional[Split] = None
    pass1: Optional[Launch] = None
    combine_strategy: Optional[ReduceStrategy] = None
    combine_op: Optional[ReduceOp] = None
    pass2: Optional[Launch] = None

    def to_c(self) -> CReductionPlan:
        c = CReductionPlan()
        if self.kind == "Direct":
            c.kind = 0
            c.strategy = int(self.strategy)
            c.launch = self.launch.to_c()
        else:
            c.kind = 1
            c.split = self.split.to_c()
            c.pass1 = self.pass1.to_c()
            c.combine_strategy = int(self.combine_strategy)
            c.combine_op = int(self.combine_op)
            c.pass2 = self.pass2.to_c()
        return c


def _layout(x) -> CLayout:
    return x.c if isinstance(x, Layout) else x


def plan_copy_exact(dtype: DType, length: int) -> Launch:
    out = CLaunch()
    _check(_lib.load().t4a_plan_copy_exact(int(dtype), length, byref(out)))
    return Launch.from_c(out)


def _wide(*layouts) -> bool:
    """Whether a call takes the general-rank planners: any WideLayout operand."""
    return any(isinstance(x, WideLayout) for x in layouts)


def _any(x) -> CLayoutAny:
    return (x if isinstance(x, WideLayout) else WideLayout.of(x)).host_c()


def plan_materialize_strided(dtype: DType, src, src_len: int) -> Launch:
    out = CLaunch()
    if _wide(src):
        _check(_lib.load().t4a_plan_materialize_strided_any(int(dtype), byref(_any(src)),
                                                            src_len, byref(out)))
    else:
        _check(_lib.load().t4a_plan_materialize_strided(int(dtype), byref(_layout(src)),
                                                        src_len, byref(out)))
    return Launch.from_c(out)


def plan_strided_to_strided(dtype: DType, src, src_len: int, dst, dst_len: int) -> Launch:
    out = CLaunch()
    if _wide(src, dst):
        _check(_lib.load().t4a_plan_strided_to_strided_any(int(dtype), byref(_any(src)), src_len,
                                                           byref(_any(dst)), dst_len,
                                                           byref(out)))
    else:
        _check(_lib.load().t4a_plan_strided_to_strided(int(dtype), byref(_layout(src)), src_len,
                                                       byref(_layout(dst)), dst_len,
                                                       byref(out)))
    return Launch.from_c(out)


def move_route(dtype: DType, src: Layout, dst: Optional[Layout] = None) -> MoveRoute:
    """The route of strided_to_strided(src -> dst), or of materialize_strided
    when `dst` is None, validated as those planners validate (spans of exactly
    the layouts' reach). No reference counterpart: route selection is the
    consumer's there."""
    out = c_int()
    _check(_lib.load().t4a_plan_move_route(int(dtype), byref(_layout(src)),
                                           byref(_layout(dst)) if dst is not None else None,
                                           byref(out)))
    return MoveRoute(out.value)


def plan_fill_zero(dtype: DType, length: int) -> Launch:
    """Reference plan_fill_zero (src/lib.rs:1601-1603)."""
    out = CLaunch()
    _check(_lib.load().t4a_plan_fill_zero(int(dtype), length, byref(out)))
    return Launch.from_c(out)


def plan_fill_zero_view(dtype: DType, dst, dst_len: int) -> Launch:
    """Reference plan_fill_zero_view (src/lib.rs:1605-1622)."""
    out = CLaunch()
    if _wide(dst):
        _check(_lib.load().t4a_plan_fill_zero_view_any(int(dtype), byref(_any(dst)), dst_len,
                                                       byref(out)))
    else:
        _check(_lib.load().t4a_plan_fill_zero_view(int(dtype), byref(_layout(dst)), dst_len,
                                                   byref(out)))
    return Launch.from_c(out)


def plan_contiguous_to_view(dtype: DType, dst, dst_len: int) -> Launch:
    """Reference plan_contiguous_to_view (src/lib.rs:1641-1658)."""
    out = CLaunch()
    if _wide(dst):
        _check(_lib.load().t4a_plan_contiguous_to_view_any(int(dtype), byref(_any(dst)), dst_len,
                                                           byref(out)))
    else:
        _check(_lib.load().t4a_plan_contiguous_to_view(int(dtype), byref(_layout(dst)), dst_len,
                                                       byref(out)))
    return Launch.from_c(out)


def axis_values(values: Sequence[int]) -> CAxisValues:
    """t4a_cuda_axis_values over at most eight values (RankLength beyond)."""
    if len(values) > MAX_RANK:
        raise T4aError(Error.RankLength + 1)
    c = CAxisValues()
    c.rank = len(values)
    for i, v in enumerate(values):
        c.values[i] = int(v)
    return c


def axis_values_any(values: Sequence[int], pointer: Optional[int] = None) -> CAxisValuesAny:
    """t4a_cuda_axis_values_any: over a host copy of `values` (the planners),
    or over `pointer`, a device copy the caller made (the launchers)."""
    c = CAxisValuesAny()
    c.rank = len(values)
    if pointer is None:
        arr = (c_longlong * max(len(values), 1))(*values)
        c.values = ctypes.addressof(arr)
        c._keep = arr
    else:
        c.values = pointer
    return c


def plan_broadcast_in_dim(dtype: DType, out, out_len: int, input, in_len: int,
                          dims: Sequence[int]) -> Launch:
    """Reference plan_broadcast_in_dim (src/lib.rs:1484-1533): dims[i] is the
    destination axis of input axis i."""
    out_c = CLaunch()
    if _wide(out, input) or len(dims) > MAX_RANK:
        _check(_lib.load().t4a_plan_broadcast_in_dim_any(
            int(dtype), byref(_any(out)), out_len, byref(_any(input)), in_len,
            byref(axis_values_any(dims)), byref(out_c)))
    else:
        _check(_lib.load().t4a_plan_broadcast_in_dim(
            int(dtype), byref(_layout(out)), out_len, byref(_layout(input)), in_len,
            byref(axis_values(dims)), byref(out_c)))
    return Launch.from_c(out_c)


def plan_concatenate_copy(dtype: DType, out, out_len: int, input, in_len: int, axis: int,
                          axis_offset: int) -> Launch:
    """Reference plan_concatenate_copy (src/lib.rs:1535-1589)."""
    out_c = CLaunch()
    if _wide(out, input):
        _check(_lib.load().t4a_plan_concatenate_copy_any(
            int(dtype), byref(_any(out)), out_len, byref(_any(input)), in_len, axis, axis_offset,
            byref(out_c)))
    else:
        _check(_lib.load().t4a_plan_concatenate_copy(
            int(dtype), byref(_layout(out)), out_len, byref(_layout(input)), in_len, axis,
            axis_offset, byref(out_c)))
    return Launch.from_c(out_c)


def plan_tiled_transpose(dtype: DType, config: TransposeConfig, src_offset: int,
                         batch_stride: int, dst_fast_extent: int, src_fast_extent: int,
                         batches: int, src_len: int, dst_len: int) -> Launch:
    out = CLaunch()
    _check(_lib.load().t4a_plan_tiled_transpose(
        int(dtype), config.c, src_offset, batch_stride, dst_fast_extent, src_fast_extent,
        batches, src_len, dst_len, byref(out)))
    return Launch.from_c(out)


def split_policy(reduce_len: int, plane_width: int) -> Optional[Split]:
    has = c_int()
    out = CSplit()
    _check(_lib.load().t4a_split_policy(reduce_len, plane_width, byref(has), byref(out)))
    return Split(out.splits, out.chunk_len) if has.value else None


def plan_reduce(dtype: DType, op: ReduceOp, strategy: ReduceStrategy, out_layout: Layout,
                out_len: int, in_layout: Layout, in_len: int, axis: int,
                plane_width: int) -> Launch:
    out = CLaunch()
    if _wide(out_layout, in_layout):
        _check(_lib.load().t4a_plan_reduce_any(int(dtype), int(op), int(strategy),
                                               byref(_any(out_layout)), out_len,
                                               byref(_any(in_layout)), in_len, axis, plane_width,
                                               byref(out)))
    else:
        _check(_lib.load().t4a_plan_reduce(int(dtype), int(op), int(strategy),
                                           byref(_layout(out_layout)), out_len,
                                           byref(_layout(in_layout)), in_len, axis, plane_width,
                                           byref(out)))
    return Launch.from_c(out)


def plan_reduce_partials(dtype: DType, op: ReduceOp, partials_layout: Layout,
                         partials_len: int, in_layout: Layout, in_len: int, axis: int,
                         split: Split, plane_width: int) -> Launch:
    out = CLaunch()
    if _wide(partials_layout, in_layout):
        _check(_lib.load().t4a_plan_reduce_partials_any(int(dtype), int(op),
                                                        byref(_any(partials_layout)),
                                                        partials_len, byref(_any(in_layout)),
                                                        in_len, axis, split.to_c(), plane_width,
                                                        byref(out)))
    else:
        _check(_lib.load().t4a_plan_reduce_partials(int(dtype), int(op),
                                                    byref(_layout(partials_layout)),
                                                    partials_len, byref(_layout(in_layout)),
                                                    in_len, axis, split.to_c(), plane_width,
                                                    byref(out)))
    return Launch.from_c(out)


def plan_reduction(dtype: DType, op: ReduceOp, out_layout: Layout, out_len: int,
                   in_layout: Layout, in_len: int, axis: int,
                   plane_width: int) -> ReductionPlan:
    p = CReductionPlan()
    if _wide(out_layout, in_layout):
        _check(_lib.load().t4a_plan_reduction_any(int(dtype), int(op), byref(_any(out_layout)),
                                                  out_len, byref(_any(in_layout)), in_len, axis,
                                                  plane_width, byref(p)))
    else:
        _check(_lib.load().t4a_plan_reduction(int(dtype), int(op), byref(_layout(out_layout)),
                                              out_len, byref(_layout(in_layout)), in_len, axis,
                                              plane_width, byref(p)))
    if p.kind == 0:
        return ReductionPlan("Direct", strategy=ReduceStrategy(p.strategy),
                             launch=Launch.from_c(p.launch))
    return ReductionPlan("Split", split=Split(p.split.splits, p.split.chunk_len),
                         pass1=Launch.from_c(p.pass1),
                         combine_strategy=ReduceStrategy(p.combine_strategy),
                         combine_op=ReduceOp(p.combine_op), pass2=Launch.from_c(p.pass2))


def reduction_partials_layout(in_layout, axis: int, splits: int):
    """The compact partials layout; a WideLayout for a WideLayout input."""
    if _wide(in_layout):
        n = max(in_layout.rank, 1)
        ext, st = (c_longlong * n)(), (c_longlong * n)()
        _check(_lib.load().t4a_reduction_partials_layout_any(byref(_any(in_layout)), axis, splits,
                                                             ext, st))
        return WideLayout(list(ext[: in_layout.rank]), list(st[: in_layout.rank]), 0)
    out = CLayout()
    _check(_lib.load().t4a_reduction_partials_layout(byref(_layout(in_layout)), axis, splits,
                                                     byref(out)))
    return Layout.from_c(out)


def abi_revision() -> int:
    return _lib.load().t4a_abi_revision()


__all__ = [
    "ABI_REVISION", "DEFAULT_SHARED_BYTES", "DType", "Error", "FLAT_BLOCK", "Launch", "Layout",
    "MAX_GRID_X", "MAX_GRID_YZ", "MAX_RANK", "MAX_SPLITS", "MIN_CHUNK_PLANES", "PLANE_BLOCK",
    "PLANE_WIDTHS", "RankVariant", "ReduceOp", "ReduceStrategy", "ReductionPlan", "Split",
    "T4aError", "TransposeConfig", "abi_revision", "plan_copy_exact", "plan_materialize_strided",
    "plan_reduce", "plan_reduce_partials", "plan_reduction", "plan_strided_to_strided",
    "plan_tiled_transpose", "reduction_partials_layout", "split_policy",
    "MoveRoute", "WideLayout", "axis_values", "axis_values_any", "move_route",
    "plan_broadcast_in_dim", "plan_concatenate_copy", "plan_contiguous_to_view",
    "plan_fill_zero", "plan_fill_zero_view",
]
