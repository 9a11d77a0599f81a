// Checked host planning of the movement and reduction entries.
//
// Validation restates the reference planner (src/lib.rs) step for step, so the
// same bad input is refused with the same Error; each function cites the
// reference function it follows. The returned geometry is this library's own
// (MI355X wavefront-sized blocks, work decomposed by geometry.h), except where
// the geometry carries the fold topology: a PLANE reduction's block width is its
// plane width, and a pass-1 block of at most 32 threads is one plane of that
// width, exactly as in the reference (docs/abi/c-kernel-abi.md:291-312).
#include <climits>
#include <cstdint>
#include <cstring>
#include <vector>

#include "geometry.h"
#include "t4a/t4a.h"

namespace {

using t4a::kBlock;

// Reference constants (src/lib.rs:139-150, 3031-3063).
constexpr unsigned kFlatBlock = 256;
constexpr unsigned kMaxGridYZ = 65535;
constexpr unsigned kMaxGridX = INT32_MAX;
constexpr uint64_t kDefaultSharedBytes = 48 * 1024;
constexpr long long kMinChunkPlanes = 8;
constexpr long long kMaxSplits = 4096;
// Blocks of the packed plane launch (256 threads, 8 to 32 planes each): about
// two rounds of the blocks the device holds at once.
constexpr long long kPlaneMultiBlocks = 4096;
constexpr unsigned kMaxBlockWidth = 512;
constexpr long long kWideCombineMinSplits = 64;
constexpr long long kCombineTargetFoldsPerLane = 8;
// Grid-stride kernels stop growing the grid here: 1024 blocks per CU.
constexpr long long kMaxBlocks = 262144;

int ok() { return T4A_OK; }

bool checked_mul(long long a, long long b, long long* out) {
  return !__builtin_mul_overflow(a, b, out);
}
bool checked_add(long long a, long long b, long long* out) {
  return !__builtin_add_overflow(a, b, out);
}

// A layout as the planners read it, of any rank: the by-value t4a_cuda_layout
// (rank <= 8) or the general-rank t4a_cuda_layout_any pointing at host memory
// (the reference planners take LayoutRef slices of any rank).
struct View {
  int rank;
  long long offset;
  const long long* extents;
  const long long* strides;
};

View V(const t4a_cuda_layout* l) { return View{l->rank, l->offset, l->extents, l->strides}; }
View V(const t4a_cuda_layout_any* l) {
  return View{l->rank, l->offset, l->extents, l->strides};
}

// Reference LayoutRef::new / Layout::new validation (src/lib.rs:342-360, 908-928):
// rank at most `max_rank` (8 for the by-value layout, unbounded for the
// general-rank one, reference WideLayout), no negative extent.
int check_view(const View& l, int max_rank) {
  if (l.rank < 0 || l.rank > max_rank) return T4A_ERR_RANK_OUT_OF_RANGE;
  if (l.rank > 0 && (l.extents == nullptr || l.strides == nullptr))
    return T4A_HIP_ERR_NULL_ARGUMENT;
  for (int k = 0; k < l.rank; ++k) {
    if (l.extents[k] < 0) return T4A_ERR_NEGATIVE_EXTENT;
  }
  return T4A_OK;
}

int check_layout(const t4a_cuda_layout* l) {
  if (l == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  return check_view(V(l), T4A_CUDA_MAX_RANK);
}

int check_any(const t4a_cuda_layout_any* l) {
  if (l == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  return check_view(V(l), INT_MAX);
}

// Reference element_count (src/lib.rs:392-397).
int element_count(const View& l, long long* count) {
  long long acc = 1;
  for (int k = 0; k < l.rank; ++k) {
    if (!checked_mul(acc, l.extents[k], &acc)) return T4A_ERR_OVERFLOW;
  }
  *count = acc;
  return T4A_OK;
}

// Reference reachable_offset (src/lib.rs:409-422).
int reachable_offset(const View& l, bool maximum, long long* out) {
  long long total = l.offset;
  for (int k = 0; k < l.rank; ++k) {
    long long step;
    if (!checked_mul(l.extents[k] - 1, l.strides[k], &step)) return T4A_ERR_OVERFLOW;
    step = maximum ? (step > 0 ? step : 0) : (step < 0 ? step : 0);
    if (!checked_add(total, step, &total)) return T4A_ERR_OVERFLOW;
  }
  *out = total;
  return T4A_OK;
}

// Reference LayoutRef::check_span (src/lib.rs:1011-1027).
int check_span(const View& l, long long len, int esize) {
  if (len < 0) return T4A_ERR_NEGATIVE_COUNT;
  long long count;
  if (int s = element_count(l, &count)) return s;
  if (count == 0) return ok();
  long long lo, hi, bytes;
  if (int s = reachable_offset(l, false, &lo)) return s;
  if (int s = reachable_offset(l, true, &hi)) return s;
  if (lo < 0 || hi >= len) return T4A_ERR_OFFSET_OUT_OF_SPAN;
  if (!checked_mul(hi, esize, &bytes)) return T4A_ERR_OVERFLOW;
  return ok();
}

// Reference require_destination / rejects_broadcast_axis (src/lib.rs:4057-4065, 444-449).
int require_destination(const View& l) {
  for (int k = 0; k < l.rank; ++k) {
    if (l.extents[k] > 1 && l.strides[k] == 0) return T4A_ERR_BROADCAST_DESTINATION;
  }
  return ok();
}

// Reference is_compact (src/lib.rs:424-439).
bool is_compact(const View& l) {
  if (l.offset != 0) return false;
  long long stride = 1;
  for (int k = 0; k < l.rank; ++k) {
    if (l.strides[k] != stride) return false;
    if (!checked_mul(stride, l.extents[k], &stride)) return false;
  }
  return true;
}

bool dtype_known(int dtype) { return t4a::dtype_size(dtype) != 0; }

void set_launch(t4a_launch* out, long long grid, unsigned block, unsigned shared) {
  out->grid[0] = static_cast<unsigned>(grid);
  out->grid[1] = grid > 0 ? 1u : 0u;
  out->grid[2] = grid > 0 ? 1u : 0u;
  out->block[0] = block;
  out->block[1] = 1;
  out->block[2] = 1;
  out->shared_bytes = shared;
  out->variant = T4A_VARIANT_FAST;
}

long long blocks_for(long long items, long long per_block) {
  long long blocks = (items + per_block - 1) / per_block;
  return blocks < kMaxBlocks ? blocks : kMaxBlocks;
}

// Reference flat_launch (src/lib.rs:1465-1482): its refusals are kept; the
// geometry is this library's.
int flat_launch_check(long long len) {
  if (len < 0) return T4A_ERR_NEGATIVE_COUNT;
  if (len == 0) return ok();
  const unsigned long long blocks = (static_cast<unsigned long long>(len) + kFlatBlock - 1) /
                                    kFlatBlock;
  if (blocks > kMaxGridX) return T4A_ERR_LAUNCH_LIMIT;
  return ok();
}

void movement_launch(const t4a::MovePlan& plan, int esize, t4a_launch* out) {
  long long blocks = 0;
  switch (plan.mode) {
    // Tiled blocks are persistent: four per CU on 256 CUs, each walking its
    // run of tiles (the launchers walk TilePlan shapes with a grid of their
    // own; this one is what the entries run under, every block working).
    case t4a::kMoveTiled:
      blocks = plan.tiles < 1024 ? plan.tiles : 1024;
      break;
    // One run: copy_exact's geometry (a 16-byte vector per thread). Rows as
    // 16-byte units, one per thread, when the row plan applies.
    case t4a::kMoveContig: {
      t4a::RowPlan rp;
      if (t4a::linear_route(plan))
        blocks = blocks_for(plan.len * esize, kBlock * 16);
      else
        blocks = t4a::row_plan(&rp, plan, esize, true) ? blocks_for(rp.units, kBlock)
                                                         : blocks_for(plan.len, kBlock * 4);
      break;
    }
    case t4a::kMoveGeneric: blocks = blocks_for(plan.len, kBlock * 4); break;
    default: blocks = 0; break;
  }
  set_launch(out, blocks, kBlock, 0);
}

// ---- reductions ----

bool op_supports(int op, int dtype) {
  switch (op) {
    case T4A_CUDA_REDUCE_SUM:
    case T4A_CUDA_REDUCE_PROD:
      return dtype == T4A_CUDA_F32 || dtype == T4A_CUDA_F64 || dtype == T4A_CUDA_I32 ||
             dtype == T4A_CUDA_I64 || dtype == T4A_CUDA_C32 || dtype == T4A_CUDA_C64;
    case T4A_CUDA_REDUCE_SUM_SQUARES:
      return dtype == T4A_CUDA_F32 || dtype == T4A_CUDA_F64;
    case T4A_CUDA_REDUCE_MAX:
    case T4A_CUDA_REDUCE_MIN:
      return dtype == T4A_CUDA_F32 || dtype == T4A_CUDA_F64 || dtype == T4A_CUDA_I32 ||
             dtype == T4A_CUDA_I64;
    default:
      return false;
  }
}

bool plane_width_ok(unsigned w) { return w == 8 || w == 16 || w == 32; }
bool combine_width_ok(unsigned w) { return w == 64 || w == 128 || w == 256 || w == 512; }

// Reference reduce_problem (src/lib.rs:3193-3233).
int reduce_problem(int dtype, int op, const View& out, long long out_len, const View& in,
                   long long in_len, unsigned axis, long long* reduce_len,
                   long long* output_len) {
  if (!op_supports(op, dtype)) return T4A_ERR_UNSUPPORTED_DTYPE;
  if (axis >= static_cast<unsigned>(in.rank)) return T4A_ERR_INVALID_AXIS;
  if (out.rank != in.rank) return T4A_ERR_RANK_LENGTH;
  for (int k = 0; k < in.rank; ++k) {
    if (static_cast<unsigned>(k) == axis) continue;
    if (out.extents[k] != in.extents[k]) return T4A_ERR_SHAPE_MISMATCH;
  }
  if (out.extents[axis] != 1) return T4A_ERR_SHAPE_MISMATCH;
  *reduce_len = in.extents[axis];
  if (*reduce_len < 1) return T4A_ERR_NEGATIVE_COUNT;
  if (int s = element_count(out, output_len)) return s;
  if (int s = require_destination(out)) return s;
  const int es = t4a::dtype_size(dtype);
  if (int s = check_span(in, in_len, es)) return s;
  if (int s = check_span(out, out_len, es)) return s;
  return ok();
}

int strategy_for(long long reduce_len, unsigned w) {
  return reduce_len <= static_cast<long long>(w) ? T4A_CUDA_REDUCE_UNIT : T4A_CUDA_REDUCE_PLANE;
}

// Reference launch_for (src/lib.rs:3243-3286), with this library's UNIT geometry:
// a unit reduction's fold does not depend on the block, so it runs 256-thread
// blocks, or 64-thread ones when that still leaves fewer than 1024 blocks (a
// combine pass over a few thousand outputs then spreads over more CUs); a
// PLANE block is the plane.
int launch_for(int strategy, long long output_len, unsigned w, t4a_launch* out) {
  if (strategy == T4A_CUDA_REDUCE_UNIT) {
    if (output_len < 0) return T4A_ERR_NEGATIVE_COUNT;
    const unsigned long long blocks =
        (static_cast<unsigned long long>(output_len) + w - 1) / w;
    if (blocks > UINT32_MAX) return T4A_ERR_LAUNCH_LIMIT;
    if (blocks > kMaxGridX) return T4A_ERR_LAUNCH_LIMIT;
    const long long bs = output_len < 1024LL * kBlock ? t4a::kUnitSmallBlock : kBlock;
    set_launch(out, output_len == 0 ? 0 : blocks_for(output_len, bs), static_cast<unsigned>(bs),
               0);
    return ok();
  }
  if (output_len < 0 || output_len > static_cast<long long>(UINT32_MAX))
    return T4A_ERR_LAUNCH_LIMIT;
  if (static_cast<unsigned long long>(output_len) > kMaxGridX) return T4A_ERR_LAUNCH_LIMIT;
  set_launch(out, output_len, w, 0);
  if (output_len == 0) out->grid[1] = out->grid[2] = 1;
  return ok();
}

int combine_block_width(long long splits) {
  const long long target = splits / kCombineTargetFoldsPerLane;
  unsigned width = static_cast<unsigned>(kWideCombineMinSplits);
  while (static_cast<long long>(width) < target && width < kMaxBlockWidth) width *= 2;
  return width < kMaxBlockWidth ? width : kMaxBlockWidth;
}

// Reference RankVariant::select (src/lib.rs:817-838): the general symbol when
// any participating rank exceeds T4A_CUDA_MAX_RANK.
void set_variant(t4a_launch* launch, int rank) {
  launch->variant = rank > T4A_CUDA_MAX_RANK ? T4A_VARIANT_GENERAL : T4A_VARIANT_FAST;
}

// Movement geometry of any rank: fused first (fuse_move, the fusion move_plan
// itself applies), then move_plan on the fused axes when at most eight remain;
// wider geometries are decoded per element by the general twins.
void movement_geometry(const View& src, const long long* dst_strides, long long dst_offset,
                       long long len, int es, t4a_launch* launch) {
  long long fe[t4a::kMaxFusedDims], fs[t4a::kMaxFusedDims], fd[t4a::kMaxFusedDims];
  const int n = len > 0 ? t4a::fuse_move(src.rank, src.extents, src.strides, dst_strides, fe,
                                         fs, fd, t4a::kMaxFusedDims)
                        : 0;
  if (n >= 0 && n <= t4a::kMaxDims) {
    t4a::MovePlan plan;
    t4a::move_plan_view(&plan, n, src.offset, fe, fs, fd, dst_offset, len, es);
    movement_launch(plan, es, launch);
  } else {
    set_launch(launch, blocks_for(len, kBlock * 4), kBlock, 0);
  }
  set_variant(launch, src.rank);
}

// The launchers' route for a planned move (their choices in launch_move, in
// the same order, under the planner's own geometry).
int move_route(const View& src, const long long* dst_strides, long long dst_offset,
               long long len, int es) {
  if (len <= 0) return T4A_MOVE_ROUTE_EMPTY;
  long long fe[t4a::kMaxFusedDims], fs[t4a::kMaxFusedDims], fd[t4a::kMaxFusedDims];
  const int n =
      t4a::fuse_move(src.rank, src.extents, src.strides, dst_strides, fe, fs, fd,
                     t4a::kMaxFusedDims);
  if (n < 0 || n > t4a::kMaxDims) return T4A_MOVE_ROUTE_ELEMENTS;
  t4a::MovePlan plan;
  t4a::move_plan_view(&plan, n, src.offset, fe, fs, fd, dst_offset, len, es);
  t4a_launch launch;
  movement_launch(plan, es, &launch);
  t4a::RowPlan rp;
  t4a::TransposeRoute tr;
  t4a::TilePlan tp;
  switch (plan.mode) {
    case t4a::kMoveEmpty: return T4A_MOVE_ROUTE_EMPTY;
    case t4a::kMoveGeneric: return T4A_MOVE_ROUTE_ELEMENTS;
    case t4a::kMoveContig:
      if (t4a::linear_route(plan)) return T4A_MOVE_ROUTE_LINEAR;
      return t4a::row_plan(&rp, plan, es, true) && launch.grid[0] <= (1u << 23)
                 ? T4A_MOVE_ROUTE_ROWS
                 : T4A_MOVE_ROUTE_ELEMENTS;
    case t4a::kMoveTiled:
      if (t4a::transpose_route(plan, &tr)) return T4A_MOVE_ROUTE_TRANSPOSE;
      if (es >= 4 && t4a::tile_plan(&tp, plan, es) && t4a::tile_walk_applies(plan, tp, es))
        return T4A_MOVE_ROUTE_TILE_ONCE;
      return T4A_MOVE_ROUTE_TILES;
    default: return T4A_MOVE_ROUTE_ELEMENTS;
  }
}

// Reference plan_materialize_strided (src/lib.rs:1628-1641) after the layout
// checks.
int plan_materialize(int dtype, const View& src, long long src_len, t4a_launch* launch) {
  if (!dtype_known(dtype)) return T4A_ERR_UNSUPPORTED_DTYPE;
  long long len;
  if (int s = element_count(src, &len)) return s;
  const int es = t4a::dtype_size(dtype);
  if (int s = check_span(src, src_len, es)) return s;
  if (int s = flat_launch_check(len)) return s;
  movement_geometry(src, nullptr, 0, len, es, launch);
  return ok();
}

// Reference plan_strided_to_strided (src/lib.rs:1660-1679) after the layout
// checks.
int plan_strided(int dtype, const View& src, long long src_len, const View& dst,
                 long long dst_len, t4a_launch* launch) {
  if (!dtype_known(dtype)) return T4A_ERR_UNSUPPORTED_DTYPE;
  bool same = src.rank == dst.rank;
  for (int k = 0; same && k < src.rank; ++k) same = src.extents[k] == dst.extents[k];
  if (!same) return T4A_ERR_COUNT_MISMATCH;
  long long len;
  if (int s = element_count(src, &len)) return s;
  if (int s = require_destination(dst)) return s;
  const int es = t4a::dtype_size(dtype);
  if (int s = check_span(src, src_len, es)) return s;
  if (int s = check_span(dst, dst_len, es)) return s;
  if (int s = flat_launch_check(len)) return s;
  movement_geometry(src, dst.strides, dst.offset, len, es, launch);
  return ok();
}

// A reduction's layouts as a rank <= 8 pair with the same fused dims: the
// by-value layouts themselves, or for a wider rank the non-axis dims fused
// (reduce_dims_view) with the axis appended last -- reduce_dims of the pair
// reproduces those dims. False when more than 7 non-axis dims remain.
bool reduction_pair(const View& out, const View& in, unsigned axis, t4a_cuda_layout* o8,
                    t4a_cuda_layout* i8, int* axis8) {
  t4a::ReduceDimsN<t4a::kMaxDims - 1> work;
  return t4a::reduction_pair_view(in.rank, out.offset, out.extents, out.strides, in.offset,
                                  in.extents, in.strides, static_cast<int>(axis), o8, i8, axis8,
                                  &work);
}

// Reference plan_reduce (src/lib.rs:3318-3338) with check_reduce_width and
// check_strategy (3288-3316), after the layout checks.
int plan_reduce(int dtype, int op, int strategy, const View& out, long long out_len,
                const View& in, long long in_len, unsigned axis, unsigned plane_width,
                t4a_launch* launch) {
  if (strategy != T4A_CUDA_REDUCE_UNIT && strategy != T4A_CUDA_REDUCE_PLANE)
    return T4A_ERR_UNSUPPORTED_OP;
  if (strategy == T4A_CUDA_REDUCE_UNIT) {
    if (!plane_width_ok(plane_width)) return T4A_ERR_INVALID_PLANE_WIDTH;
  } else if (!combine_width_ok(plane_width) && !plane_width_ok(plane_width)) {
    return T4A_ERR_INVALID_PLANE_WIDTH;
  }
  long long reduce_len, output_len;
  if (int s = reduce_problem(dtype, op, out, out_len, in, in_len, axis, &reduce_len,
                             &output_len))
    return s;
  if (strategy == T4A_CUDA_REDUCE_UNIT && reduce_len > static_cast<long long>(plane_width))
    return T4A_ERR_STRATEGY_MISMATCH;
  if (strategy == T4A_CUDA_REDUCE_PLANE && reduce_len < static_cast<long long>(plane_width))
    return T4A_ERR_STRATEGY_MISMATCH;
  if (int s = launch_for(strategy, output_len, plane_width, launch)) return s;
  // A one-group axis in kBlock-thread blocks: threads take several outputs.
  t4a_cuda_layout o8, i8;
  int axis8;
  // PLANE with planes of at most 32 lanes: 256 / W planes a block (block.y),
  // a grid of at most kPlaneMultiBlocks blocks striding over the outputs, when
  // the launchers' compact plan takes the outputs (at most three fused dims).
  if (strategy == T4A_CUDA_REDUCE_PLANE && plane_width <= static_cast<unsigned>(t4a::kWarp) &&
      output_len > 0 && in.rank <= T4A_CUDA_MAX_RANK &&
      reduction_pair(out, in, axis, &o8, &i8, &axis8)) {
    t4a::ReduceDims rd;
    t4a::reduce_dims(&rd, o8, i8, axis8);
    const long long planes = kBlock / static_cast<long long>(plane_width);
    long long blocks = (output_len + planes - 1) / planes;
    if (blocks > kPlaneMultiBlocks) blocks = kPlaneMultiBlocks;
    if (t4a::unit_plan_fits(rd, output_len) &&
        t4a::grid_stride_fits(output_len, static_cast<unsigned int>(blocks),
                              4ull * static_cast<unsigned long long>(planes))) {
      launch->grid[0] = static_cast<unsigned int>(blocks);
      launch->grid[1] = launch->grid[2] = 1;
      launch->block[0] = plane_width;
      launch->block[1] = static_cast<unsigned int>(planes);
      launch->block[2] = 1;
      launch->shared_bytes = 0;
    }
  }
  if (strategy == T4A_CUDA_REDUCE_UNIT && output_len > 0 &&
      launch->block[0] == static_cast<unsigned>(kBlock) &&
      reduction_pair(out, in, axis, &o8, &i8, &axis8)) {
    t4a::ReduceDims rd;
    t4a::reduce_dims(&rd, o8, i8, axis8);
    if (t4a::unit_one_group(rd, dtype))
      set_launch(launch, blocks_for(output_len, kBlock * t4a::kUnitOutputsPerThread), kBlock,
                 0);
  }
  set_variant(launch, in.rank);
  return ok();
}

// Reference plan_reduce_partials (src/lib.rs:3340-3431) after the layout checks.
int plan_reduce_partials(int dtype, int op, const View& partials, long long partials_len,
                         const View& in, long long in_len, unsigned axis, t4a_split split,
                         unsigned plane_width, t4a_launch* launch) {
  if (!plane_width_ok(plane_width)) return T4A_ERR_INVALID_PLANE_WIDTH;
  if (!op_supports(op, dtype)) return T4A_ERR_UNSUPPORTED_DTYPE;
  if (axis >= static_cast<unsigned>(in.rank)) return T4A_ERR_INVALID_AXIS;
  if (partials.rank != in.rank) return T4A_ERR_RANK_LENGTH;
  for (int k = 0; k < in.rank; ++k) {
    if (static_cast<unsigned>(k) == axis) continue;
    if (partials.extents[k] != in.extents[k]) return T4A_ERR_SHAPE_MISMATCH;
  }
  const long long reduce_len = in.extents[axis];
  if (reduce_len < 1) return T4A_ERR_NEGATIVE_COUNT;
  if (split.splits < 2 || split.chunk_len < static_cast<long long>(plane_width) ||
      split.chunk_len != reduce_len / split.splits || split.splits > kMaxSplits)
    return T4A_ERR_INVALID_SPLIT;
  if (partials.extents[axis] != split.splits) return T4A_ERR_SHAPE_MISMATCH;
  if (int s = require_destination(partials)) return s;
  const int es = t4a::dtype_size(dtype);
  if (int s = check_span(in, in_len, es)) return s;
  if (int s = check_span(partials, partials_len, es)) return s;
  long long output_len = 1;
  for (int k = 0; k < partials.rank; ++k) {
    if (static_cast<unsigned>(k) == axis) continue;
    if (!checked_mul(output_len, partials.extents[k], &output_len)) return T4A_ERR_OVERFLOW;
  }
  if (output_len < 0) return T4A_ERR_NEGATIVE_COUNT;
  long long cubes;
  if (!checked_mul(output_len, split.splits, &cubes)) return T4A_ERR_OVERFLOW;
  if (cubes > static_cast<long long>(UINT32_MAX)) return T4A_ERR_LAUNCH_LIMIT;
  if (cubes > static_cast<long long>(kMaxGridX)) return T4A_ERR_LAUNCH_LIMIT;
  if (plane_width != static_cast<unsigned>(t4a::kWarp)) {
    set_launch(launch, cubes, plane_width, 0);
    if (cubes == 0) launch->grid[1] = launch->grid[2] = 1;
    set_variant(launch, in.rank);
    return ok();
  }
  t4a_cuda_layout p8, i8;
  int axis8;
  if (!reduction_pair(partials, in, axis, &p8, &i8, &axis8)) {
    // Too many dims for a mapping: the general twin's plane walk, eight
    // planes per block.
    set_launch(launch, cubes == 0 ? 0 : blocks_for(cubes, kBlock / t4a::kWarp), kBlock, 0);
    set_variant(launch, in.rank);
    return ok();
  }
  t4a::PartialsPlan plan;
  t4a::partials_plan(&plan, p8, i8, axis8, output_len, split.splits, t4a::kWarp,
                     t4a::sideways_dtype(dtype), es, 16);
  // Units per block: one (TILES), a plane per 32 lanes (PLANE, VECROWS), a
  // wavefront per 64 (ROWS).
  long long per_block = kBlock / t4a::kWave;
  if (plan.mode == t4a::kPartialsTiles) per_block = 1;
  if (plan.mode == t4a::kPartialsPlane || plan.mode == t4a::kPartialsVecRows)
    per_block = kBlock / t4a::kWarp;
  // Lean planes take one cube each; streaming planes take runs of cubes.
  if (!t4a::lean_slots(plan, dtype, op, split.splits, split.chunk_len, t4a::kWarp) &&
      t4a::stream_applies(plan, dtype, op, split.chunk_len, t4a::kWarp))
    per_block *= t4a::stream_cubes_per_plane(cubes);
  set_launch(launch, plan.units == 0 ? 0 : blocks_for(plan.units, per_block), kBlock, 0);
  set_variant(launch, in.rank);
  return ok();
}

// Reference plan_reduction (src/lib.rs:3457-3528) with combine_geometry and
// combine_block_width (3433-3452), after the layout checks. The partials
// layout is the compact one over the input's extents with the axis replaced by
// the split count (reference partials_layout_for, src/lib.rs:3530-3557).
int plan_reduction(int dtype, int op, const View& out, long long out_len, const View& in,
                   long long in_len, unsigned axis, unsigned plane_width,
                   t4a_reduction_plan* plan) {
  if (!plane_width_ok(plane_width)) return T4A_ERR_INVALID_PLANE_WIDTH;
  long long reduce_len, output_len;
  if (int s = reduce_problem(dtype, op, out, out_len, in, in_len, axis, &reduce_len,
                             &output_len))
    return s;
  const int strategy = strategy_for(reduce_len, plane_width);
  int has_split;
  t4a_split split;
  if (int s = t4a_split_policy(reduce_len, plane_width, &has_split, &split)) return s;
  if (!has_split) {
    plan->kind = T4A_PLAN_DIRECT;
    plan->strategy = strategy;
    return plan_reduce(dtype, op, strategy, out, out_len, in, in_len, axis, plane_width,
                       &plan->launch);
  }
  std::vector<long long> pe(static_cast<size_t>(in.rank)), ps(static_cast<size_t>(in.rank));
  long long stride = 1;
  for (int k = 0; k < in.rank; ++k) {
    pe[k] = static_cast<unsigned>(k) == axis ? split.splits : in.extents[k];
    ps[k] = stride;
    if (!checked_mul(stride, pe[k], &stride)) return T4A_ERR_OVERFLOW;
  }
  const View partials{in.rank, 0, pe.data(), ps.data()};
  long long partials_len;
  if (int s = element_count(partials, &partials_len)) return s;
  plan->kind = T4A_PLAN_SPLIT;
  plan->split = split;
  if (int s = plan_reduce_partials(dtype, op, partials, partials_len, in, in_len, axis, split,
                                   plane_width, &plan->pass1))
    return s;
  const int combine_op = op == T4A_CUDA_REDUCE_SUM_SQUARES ? T4A_CUDA_REDUCE_SUM : op;
  int combine_strategy;
  unsigned combine_width;
  if (combine_op == T4A_CUDA_REDUCE_PROD || split.splits < kWideCombineMinSplits) {
    combine_strategy = strategy_for(split.splits, plane_width);
    combine_width = plane_width;
  } else {
    combine_strategy = T4A_CUDA_REDUCE_PLANE;
    combine_width = static_cast<unsigned>(combine_block_width(split.splits));
  }
  plan->combine_strategy = combine_strategy;
  plan->combine_op = combine_op;
  return plan_reduce(dtype, combine_op, combine_strategy, out, out_len, partials, partials_len,
                     axis, combine_width, &plan->pass2);
}

// Geometry of a move over derived geometry (contiguous_to_view,
// broadcast_in_dim, concatenate_copy): the launchers' plan when at most eight
// fused axes remain, else the general twins' flat walk.
template <typename SrcStride, typename DstStride>
void derived_geometry(int rank, const long long* ext, SrcStride src, long long src_offset,
                      DstStride dst, long long dst_offset, long long len, int es,
                      t4a_launch* launch) {
  t4a::MovePlan plan;
  if (len > 0 && t4a::move_plan_by(&plan, rank, ext, src, src_offset, dst, dst_offset, len, es))
    movement_launch(plan, es, launch);
  else
    set_launch(launch, len == 0 ? 0 : blocks_for(len, kBlock * 4), kBlock, 0);
}

// Reference plan_fill_zero_view / plan_contiguous_to_view (src/lib.rs:1606-1622,
// 1641-1658) after the layout checks: the same checks for both.
int plan_view_entry(int dtype, const View& dst, long long dst_len, long long* len) {
  if (!dtype_known(dtype)) return T4A_ERR_UNSUPPORTED_DTYPE;
  if (int s = element_count(dst, len)) return s;
  if (int s = require_destination(dst)) return s;
  if (int s = check_span(dst, dst_len, t4a::dtype_size(dtype))) return s;
  return flat_launch_check(*len);
}

int plan_fill_view(int dtype, const View& dst, long long dst_len, t4a_launch* launch) {
  long long len;
  if (int s = plan_view_entry(dtype, dst, dst_len, &len)) return s;
  // A thread per 16-byte vector where the view allows one (the pointer's
  // alignment is checked at launch; the kernel strides over what is left).
  const int es = t4a::dtype_size(dtype);
  const int v = es >= 4 && es <= 8 ? 16 / es : 1;
  long long fe[t4a::kMaxFusedDims], fs[t4a::kMaxFusedDims], fd[t4a::kMaxFusedDims];
  const int n = len > 0 ? t4a::fuse_move(dst.rank, dst.extents, dst.strides, dst.strides, fe, fs,
                                         fd, t4a::kMaxFusedDims)
                        : 0;
  t4a::FillPlan fp;
  const bool vec = t4a::fill_plan(&fp, n, fe, fs, dst.offset, len) && t4a::fill_vectorizable(fp, v);
  set_launch(launch, len == 0 ? 0 : blocks_for(vec ? len / v : len, kBlock), kBlock, 0);
  set_variant(launch, dst.rank);
  return ok();
}

int plan_contiguous(int dtype, const View& dst, long long dst_len, t4a_launch* launch) {
  long long len;
  if (int s = plan_view_entry(dtype, dst, dst_len, &len)) return s;
  derived_geometry(dst.rank, dst.extents, t4a::strides_of(nullptr, dst.extents), 0,
                   t4a::strides_of(dst.strides, dst.extents), dst.offset, len,
                   t4a::dtype_size(dtype), launch);
  set_variant(launch, dst.rank);
  return ok();
}

// Reference plan_broadcast_in_dim (src/lib.rs:1484-1533) after the layout
// checks; `dims` has `dims_rank` values.
int plan_broadcast(int dtype, const View& out, long long out_len, const View& in,
                   long long in_len, const long long* dims, int dims_rank, t4a_launch* launch) {
  if (!dtype_known(dtype)) return T4A_ERR_UNSUPPORTED_DTYPE;
  if (!is_compact(out)) return T4A_ERR_NOT_COMPACT;
  if (int s = require_destination(out)) return s;
  if (dims_rank != in.rank) return T4A_ERR_RANK_LENGTH;
  if (dims_rank > 0 && dims == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  for (int i = 0; i < dims_rank; ++i) {
    const long long d = dims[i];
    if (d < 0 || d >= out.rank) return T4A_ERR_INVALID_AXIS;
    for (int j = 0; j < i; ++j) {
      if (dims[j] == d) return T4A_ERR_DUPLICATE_AXIS;
    }
    const long long ie = in.extents[i];
    if (ie != out.extents[d] && ie != 1) return T4A_ERR_SHAPE_MISMATCH;
  }
  long long len;
  if (int s = element_count(out, &len)) return s;
  const int es = t4a::dtype_size(dtype);
  if (int s = check_span(in, in_len, es)) return s;
  if (int s = check_span(out, out_len, es)) return s;
  if (int s = flat_launch_check(len)) return s;
  derived_geometry(out.rank, out.extents, t4a::BroadcastStrides{dims, dims_rank, in.extents,
                                                                  in.strides},
                   in.offset, t4a::strides_of(nullptr, out.extents), 0, len, es, launch);
  const int widest = out.rank > in.rank ? out.rank : in.rank;
  set_variant(launch, widest > dims_rank ? widest : dims_rank);
  return ok();
}

// Reference plan_concatenate_copy (src/lib.rs:1535-1589) after the layout
// checks.
int plan_concatenate(int dtype, const View& out, long long out_len, const View& in,
                     long long in_len, unsigned axis, long long axis_offset,
                     t4a_launch* launch) {
  if (!dtype_known(dtype)) return T4A_ERR_UNSUPPORTED_DTYPE;
  if (!is_compact(in)) return T4A_ERR_NOT_COMPACT;
  if (out.rank != in.rank) return T4A_ERR_RANK_LENGTH;
  if (axis >= static_cast<unsigned>(out.rank)) return T4A_ERR_INVALID_AXIS;
  if (axis_offset < 0) return T4A_ERR_NEGATIVE_COUNT;
  if (int s = require_destination(out)) return s;
  for (int k = 0; k < out.rank; ++k) {
    if (static_cast<unsigned>(k) != axis && out.extents[k] != in.extents[k])
      return T4A_ERR_SHAPE_MISMATCH;
  }
  long long end;
  if (!checked_add(axis_offset, in.extents[axis], &end)) return T4A_ERR_OVERFLOW;
  if (end > out.extents[axis]) return T4A_ERR_SHAPE_MISMATCH;
  long long len;
  if (int s = element_count(in, &len)) return s;
  const int es = t4a::dtype_size(dtype);
  if (int s = check_span(in, in_len, es)) return s;
  if (int s = check_span(out, out_len, es)) return s;
  if (int s = flat_launch_check(len)) return s;
  derived_geometry(in.rank, in.extents, t4a::strides_of(nullptr, in.extents), 0,
                   t4a::strides_of(out.strides, in.extents),
                   out.offset + axis_offset * out.strides[axis], len, es, launch);
  set_variant(launch, out.rank);
  return ok();
}

// A GENERAL movement plan is for the `_any` kernels, which plan inside the
// kernel (thread 0 fuses the device-resident geometry into LDS and builds the
// move plan): at most kAnyMoveBlocks persistent blocks, so that each block
// plans once and then strides over many tiles, rows or elements (one block
// per tile measured 3-4x slower, every block paying the serial planning).
// Rank-9 versions of the benchmark movements measured best at 512 blocks (two
// per CU): 4.1-5.0 TB/s, against 3.0-4.2 at 256, 3.6-4.7 at 1024 and 2.7-4.2
// at 2048.
constexpr unsigned kAnyMoveBlocks = 512;
// Moves on the row route (a dim contiguous on both sides, or one run) keep
// 1024: the rank-9 8192^2 f32 row copy took 97 us there against 114 at 512,
// while the tiled ones were slower at 1024 (C3 64 against 60 us, the 8192^2
// transpose 112 against 105).
constexpr unsigned kAnyRowBlocks = 1024;

int general_movement(int status, t4a_launch* launch, unsigned cap = kAnyMoveBlocks) {
  if (status == T4A_OK && launch->variant == T4A_VARIANT_GENERAL && launch->grid[0] > cap)
    launch->grid[0] = cap;
  return status;
}

// The block cap of a GENERAL move of `src` into dst_strides / dst_offset
// (nullptr: the compact destination), by the route its fused plan takes.
unsigned any_move_cap(int dtype, const View& src, const long long* dst_strides,
                      long long dst_offset) {
  long long len;
  if (element_count(src, &len) != T4A_OK) return kAnyMoveBlocks;
  const int r = move_route(src, dst_strides, dst_offset, len, t4a::dtype_size(dtype));
  return r == T4A_MOVE_ROUTE_ROWS || r == T4A_MOVE_ROUTE_LINEAR ? kAnyRowBlocks
                                                                : kAnyMoveBlocks;
}

// The same for the reduction twins (thread 0 fuses the geometry per block;
// their loops stride over outputs and cubes). Pass 1 over a strided axis, where
// a block may take the column tiles, measured best at 512 blocks (rank-9 f32:
// 4.8 TB/s, against 4.5 at 1024 and 3.8 at 2048); over a contiguous axis, the
// plane mapping over short cubes, at 1024 (4.0 TB/s, against 2.5 at 512 and
// 3.9 at 2048). Direct reductions and the combine keep 1024.
constexpr unsigned kAnyReduceBlocks = 1024;
constexpr unsigned kAnyPass1StridedBlocks = 512;

void general_reduction(t4a_launch* launch, unsigned cap = kAnyReduceBlocks) {
  if (launch->variant == T4A_VARIANT_GENERAL && launch->grid[0] > cap) launch->grid[0] = cap;
}

// The pass-1 cap for reducing `axis` of `in` (a checked layout, axis < rank).
unsigned pass1_blocks(const t4a_cuda_layout_any* in, unsigned int axis) {
  const long long stride = V(in).strides[axis];
  return stride == 1 || stride == -1 ? kAnyReduceBlocks : kAnyPass1StridedBlocks;
}

}  // namespace

extern "C" {

int t4a_abi_revision(void) { return T4A_CUDA_ABI_REVISION; }

int t4a_dtype_size(int dtype) { return t4a::dtype_size(dtype); }

const char* t4a_status_name(int status) {
  static const char* const names[] = {
      "Ok",                 "RankOutOfRange",    "RankLength",
      "NegativeExtent",     "NegativeCount",     "Overflow",
      "CountMismatch",      "OffsetOutOfSpan",   "BroadcastDestination",
      "UnsupportedDType",   "NotElementwise",    "LaunchLimit",
      "InvalidTransposeConfig", "InvalidAxis",   "DuplicateAxis",
      "NotCompact",         "ShapeMismatch",     "InvalidStep",
      "InvalidPadding",     "DomainTooLarge",    "InvalidStride",
      "StrategyMismatch",   "InvalidPlaneWidth", "InvalidSplit",
      "IndexVectorMismatch", "UnsupportedOp"};
  if (status >= 0 && status < static_cast<int>(sizeof(names) / sizeof(names[0])))
    return names[status];
  if (status == T4A_HIP_ERR_LAUNCH) return "HipLaunch";
  if (status == T4A_HIP_ERR_NULL_ARGUMENT) return "NullArgument";
  if (status == T4A_HIP_ERR_NOT_FOUND) return "NotFound";
  if (status == T4A_HIP_ERR_TOO_SMALL) return "TooSmall";
  if (status == T4A_HIP_ERR_SCRATCH_LIMIT) return "ScratchLimit";
  return "Unknown";
}

int t4a_layout_new(t4a_cuda_layout* out, int rank, const long long* extents,
                   const long long* strides, long long offset) {
  if (out == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (rank < 0 || rank > T4A_CUDA_MAX_RANK) return T4A_ERR_RANK_OUT_OF_RANGE;
  if (rank > 0 && (extents == nullptr || strides == nullptr)) return T4A_HIP_ERR_NULL_ARGUMENT;
  for (int k = 0; k < rank; ++k) {
    if (extents[k] < 0) return T4A_ERR_NEGATIVE_EXTENT;
  }
  std::memset(out, 0, sizeof(*out));
  out->rank = rank;
  out->offset = offset;
  for (int k = 0; k < rank; ++k) {
    out->extents[k] = extents[k];
    out->strides[k] = strides[k];
  }
  return ok();
}

// Reference Layout::compact (src/lib.rs:362-374).
int t4a_layout_compact(t4a_cuda_layout* out, int rank, const long long* extents) {
  if (out == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (rank < 0 || rank > T4A_CUDA_MAX_RANK) return T4A_ERR_RANK_OUT_OF_RANGE;
  long long strides[T4A_CUDA_MAX_RANK] = {0};
  long long stride = 1;
  for (int k = 0; k < rank; ++k) {
    strides[k] = stride;
    if (!checked_mul(stride, extents[k], &stride)) return T4A_ERR_OVERFLOW;
  }
  return t4a_layout_new(out, rank, extents, strides, 0);
}

int t4a_layout_element_count(const t4a_cuda_layout* layout, long long* count) {
  if (count == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (int s = check_layout(layout)) return s;
  return element_count(V(layout), count);
}

// Reference plan_copy_exact -> plan_elementwise (src/lib.rs:1592-1599, 1624-1626): every
// dtype, flat_launch's refusals; each thread copies one 16-byte vector.
int t4a_plan_copy_exact(int dtype, long long len, t4a_launch* launch) {
  if (launch == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (!dtype_known(dtype)) return T4A_ERR_UNSUPPORTED_DTYPE;
  if (int s = flat_launch_check(len)) return s;
  long long bytes;
  if (!checked_mul(len, t4a::dtype_size(dtype), &bytes)) return T4A_ERR_OVERFLOW;
  set_launch(launch, len == 0 ? 0 : blocks_for(bytes, kBlock * 16), kBlock, 0);
  return ok();
}

// Reference plan_materialize_strided (src/lib.rs:1628-1641).
int t4a_plan_materialize_strided(int dtype, const t4a_cuda_layout* src, long long src_len,
                                 t4a_launch* launch) {
  if (launch == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (int s = check_layout(src)) return s;
  return plan_materialize(dtype, V(src), src_len, launch);
}

int t4a_plan_materialize_strided_any(int dtype, const t4a_cuda_layout_any* src,
                                     long long src_len, t4a_launch* launch) {
  if (launch == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (int s = check_any(src)) return s;
  const int status = plan_materialize(dtype, V(src), src_len, launch);
  return general_movement(status, launch,
                          status == T4A_OK ? any_move_cap(dtype, V(src), nullptr, 0)
                                           : kAnyMoveBlocks);
}

// Reference plan_strided_to_strided (src/lib.rs:1660-1679).
int t4a_plan_strided_to_strided(int dtype, const t4a_cuda_layout* src, long long src_len,
                                const t4a_cuda_layout* dst, long long dst_len,
                                t4a_launch* launch) {
  if (launch == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (int s = check_layout(src)) return s;
  if (int s = check_layout(dst)) return s;
  return plan_strided(dtype, V(src), src_len, V(dst), dst_len, launch);
}

int t4a_plan_move_route(int dtype, const t4a_cuda_layout* src, const t4a_cuda_layout* dst,
                        int* route) {
  if (route == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (int s = check_layout(src)) return s;
  if (dst != nullptr) {
    if (int s = check_layout(dst)) return s;
  }
  const View sv = V(src);
  long long src_reach;
  if (int s = reachable_offset(sv, true, &src_reach)) return s;
  t4a_launch launch;
  long long len;
  if (dst == nullptr) {
    if (int s = plan_materialize(dtype, sv, src_reach + 1, &launch)) return s;
    if (int s = element_count(sv, &len)) return s;
    *route = move_route(sv, nullptr, 0, len, t4a::dtype_size(dtype));
    return ok();
  }
  const View dv = V(dst);
  long long dst_reach;
  if (int s = reachable_offset(dv, true, &dst_reach)) return s;
  if (int s = plan_strided(dtype, sv, src_reach + 1, dv, dst_reach + 1, &launch)) return s;
  if (int s = element_count(sv, &len)) return s;
  *route = move_route(sv, dv.strides, dv.offset, len, t4a::dtype_size(dtype));
  return ok();
}

int t4a_plan_strided_to_strided_any(int dtype, const t4a_cuda_layout_any* src,
                                    long long src_len, const t4a_cuda_layout_any* dst,
                                    long long dst_len, t4a_launch* launch) {
  if (launch == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (int s = check_any(src)) return s;
  if (int s = check_any(dst)) return s;
  const int status = plan_strided(dtype, V(src), src_len, V(dst), dst_len, launch);
  return general_movement(status, launch,
                          status == T4A_OK ? any_move_cap(dtype, V(src), V(dst).strides,
                                                          V(dst).offset)
                                           : kAnyMoveBlocks);
}

// Reference TransposeConfig::new (src/lib.rs:471-491).
int t4a_transpose_config_new(int tile, int block_rows, int padding, int vector_width,
                             t4a_cuda_transpose_config* config) {
  if (config == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  const bool ok_tile = tile == 8 || tile == 16 || tile == 32;
  const bool ok_rows = block_rows == 4 || block_rows == 8 || block_rows == 16;
  const bool ok_pad = padding == 0 || padding == 1;
  const bool ok_vw = vector_width == 1 || vector_width == 2 || vector_width == 4;
  if (!ok_tile || !ok_rows || !ok_pad || !ok_vw || tile % vector_width != 0)
    return T4A_ERR_INVALID_TRANSPOSE_CONFIG;
  config->tile = tile;
  config->block_rows = block_rows;
  config->padding = padding;
  config->vector_width = vector_width;
  return ok();
}

t4a_cuda_transpose_config t4a_transpose_config_default(void) {
  t4a_cuda_transpose_config c = {16, 8, 1, 1};
  return c;
}

// Reference plan_tiled_transpose (src/lib.rs:1681-1737). The config is validated
// and its shared-memory demand checked exactly as the reference does; the
// MI355X kernel stages its own 64-element-wide tiles in static LDS, so the
// returned launch is a 1-D grid of tiles with no dynamic shared memory.
int t4a_plan_tiled_transpose(int dtype, t4a_cuda_transpose_config config, long long src_offset,
                             long long batch_stride, long long dst_fast_extent,
                             long long src_fast_extent, long long batches, long long src_len,
                             long long dst_len, t4a_launch* launch) {
  if (launch == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  t4a_cuda_transpose_config checked;
  if (int s = t4a_transpose_config_new(config.tile, config.block_rows, config.padding,
                                       config.vector_width, &checked))
    return s;
  if (!dtype_known(dtype)) return T4A_ERR_UNSUPPORTED_DTYPE;
  if (dst_fast_extent < 0 || src_fast_extent < 0 || batches < 0 || src_offset < 0)
    return T4A_ERR_NEGATIVE_COUNT;
  long long matrix, span, end;
  if (!checked_mul(dst_fast_extent, src_fast_extent, &matrix)) return T4A_ERR_OVERFLOW;
  if (batch_stride != matrix) return T4A_ERR_INVALID_TRANSPOSE_CONFIG;
  if (!checked_mul(matrix, batches, &span)) return T4A_ERR_OVERFLOW;
  if (!checked_add(src_offset, span, &end)) return T4A_ERR_OVERFLOW;
  if (end > src_len || span > dst_len) return T4A_ERR_OFFSET_OUT_OF_SPAN;
  const int es = t4a::dtype_size(dtype);
  const uint64_t shared = static_cast<uint64_t>(config.tile) *
                          static_cast<uint64_t>(config.tile + config.padding) *
                          static_cast<uint64_t>(es);
  if (shared > kDefaultSharedBytes) return T4A_ERR_LAUNCH_LIMIT;
  const unsigned long long gx = (static_cast<unsigned long long>(dst_fast_extent) + config.tile - 1) /
                                static_cast<unsigned long long>(config.tile);
  const unsigned long long gy = (static_cast<unsigned long long>(src_fast_extent) + config.tile - 1) /
                                static_cast<unsigned long long>(config.tile);
  if (gx > UINT32_MAX || gy > UINT32_MAX) return T4A_ERR_LAUNCH_LIMIT;
  if (static_cast<unsigned long long>(batches) > UINT32_MAX) return T4A_ERR_LAUNCH_LIMIT;
  if (gx > kMaxGridX || gy > kMaxGridYZ || static_cast<unsigned long long>(batches) > kMaxGridYZ)
    return T4A_ERR_LAUNCH_LIMIT;
  if (gx == 0 || gy == 0 || batches == 0) {
    set_launch(launch, 0, t4a::kTransposeBlock, 0);
    return ok();
  }
  // One matrix's tiles stride over x; the batch is the z coordinate, as in the
  // reference grid (the kernel reads the batch count from nowhere else).
  const t4a::TransposeTiling tiling = t4a::transpose_tiling(dst_fast_extent, src_fast_extent, 1, es);
  set_launch(launch, blocks_for(tiling.total, 1), t4a::kTransposeBlock, 0);
  launch->grid[2] = static_cast<unsigned>(batches);
  return ok();
}

// Reference split_policy (src/lib.rs:3152-3166).
int t4a_split_policy(long long reduce_len, unsigned int plane_width, int* has_split,
                     t4a_split* split) {
  if (has_split == nullptr || split == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  *has_split = 0;
  split->splits = 0;
  split->chunk_len = 0;
  if (!plane_width_ok(plane_width)) return T4A_ERR_INVALID_PLANE_WIDTH;
  if (reduce_len < 1) return ok();
  const long long min_chunk = static_cast<long long>(plane_width) * kMinChunkPlanes;
  long long splits = reduce_len / min_chunk;
  if (splits < 1) splits = 1;
  if (splits > kMaxSplits) splits = kMaxSplits;
  if (splits <= 1) return ok();
  *has_split = 1;
  split->splits = splits;
  split->chunk_len = reduce_len / splits;
  return ok();
}

// Reference plan_reduce (src/lib.rs:3318-3338) with check_reduce_width and
// check_strategy (3288-3316).
int t4a_plan_reduce(int dtype, int op, int strategy, const t4a_cuda_layout* out_layout,
                    long long out_len, const t4a_cuda_layout* in_layout, long long in_len,
                    unsigned int axis, unsigned int plane_width, t4a_launch* launch) {
  if (launch == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (int s = check_layout(out_layout)) return s;
  if (int s = check_layout(in_layout)) return s;
  return plan_reduce(dtype, op, strategy, V(out_layout), out_len, V(in_layout), in_len, axis,
                     plane_width, launch);
}

int t4a_plan_reduce_any(int dtype, int op, int strategy, const t4a_cuda_layout_any* out_layout,
                        long long out_len, const t4a_cuda_layout_any* in_layout,
                        long long in_len, unsigned int axis, unsigned int plane_width,
                        t4a_launch* launch) {
  if (launch == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (int s = check_any(out_layout)) return s;
  if (int s = check_any(in_layout)) return s;
  const int status = plan_reduce(dtype, op, strategy, V(out_layout), out_len, V(in_layout),
                                 in_len, axis, plane_width, launch);
  if (status == T4A_OK) general_reduction(launch);
  return status;
}

// Reference plan_reduce_partials (src/lib.rs:3340-3431). A 32-lane plan runs
// 256-thread blocks (eight planes, or four wavefronts of the COLUMNS/ROWS
// mappings); an 8- or 16-lane plan keeps one plane per block.
int t4a_plan_reduce_partials(int dtype, int op, const t4a_cuda_layout* partials_layout,
                             long long partials_len, const t4a_cuda_layout* in_layout,
                             long long in_len, unsigned int axis, t4a_split split,
                             unsigned int plane_width, t4a_launch* launch) {
  if (launch == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (int s = check_layout(partials_layout)) return s;
  if (int s = check_layout(in_layout)) return s;
  return plan_reduce_partials(dtype, op, V(partials_layout), partials_len, V(in_layout), in_len,
                              axis, split, plane_width, launch);
}

int t4a_plan_reduce_partials_any(int dtype, int op, const t4a_cuda_layout_any* partials_layout,
                                 long long partials_len, const t4a_cuda_layout_any* in_layout,
                                 long long in_len, unsigned int axis, t4a_split split,
                                 unsigned int plane_width, t4a_launch* launch) {
  if (launch == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (int s = check_any(partials_layout)) return s;
  if (int s = check_any(in_layout)) return s;
  const int status = plan_reduce_partials(dtype, op, V(partials_layout), partials_len,
                                          V(in_layout), in_len, axis, split, plane_width, launch);
  if (status == T4A_OK) general_reduction(launch, pass1_blocks(in_layout, axis));
  return status;
}

// Reference plan_reduction (src/lib.rs:3457-3528) with combine_geometry and
// combine_block_width (3433-3452).
int t4a_plan_reduction(int dtype, int op, const t4a_cuda_layout* out_layout, long long out_len,
                       const t4a_cuda_layout* in_layout, long long in_len, unsigned int axis,
                       unsigned int plane_width, t4a_reduction_plan* plan) {
  if (plan == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  std::memset(plan, 0, sizeof(*plan));
  if (int s = check_layout(out_layout)) return s;
  if (int s = check_layout(in_layout)) return s;
  return plan_reduction(dtype, op, V(out_layout), out_len, V(in_layout), in_len, axis,
                        plane_width, plan);
}

int t4a_plan_reduction_any(int dtype, int op, const t4a_cuda_layout_any* out_layout,
                           long long out_len, const t4a_cuda_layout_any* in_layout,
                           long long in_len, unsigned int axis, unsigned int plane_width,
                           t4a_reduction_plan* plan) {
  if (plan == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  std::memset(plan, 0, sizeof(*plan));
  if (int s = check_any(out_layout)) return s;
  if (int s = check_any(in_layout)) return s;
  const int status = plan_reduction(dtype, op, V(out_layout), out_len, V(in_layout), in_len,
                                    axis, plane_width, plan);
  if (status == T4A_OK) {
    general_reduction(&plan->launch);
    general_reduction(&plan->pass1, pass1_blocks(in_layout, axis));
    general_reduction(&plan->pass2);
  }
  return status;
}

// Reference reduction_partials_layout / partials_layout_for (src/lib.rs:3530-3557).
int t4a_reduction_partials_layout(const t4a_cuda_layout* in_layout, unsigned int axis,
                                  long long splits, t4a_cuda_layout* partials_layout) {
  if (partials_layout == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (int s = check_layout(in_layout)) return s;
  if (axis >= static_cast<unsigned>(in_layout->rank)) return T4A_ERR_INVALID_AXIS;
  long long extents[T4A_CUDA_MAX_RANK];
  for (int k = 0; k < in_layout->rank; ++k) extents[k] = in_layout->extents[k];
  extents[axis] = splits;
  return t4a_layout_compact(partials_layout, in_layout->rank, extents);
}

// The same for any rank: the compact partials layout's `rank` extents and
// strides into the caller's arrays (its offset is 0).
int t4a_reduction_partials_layout_any(const t4a_cuda_layout_any* in_layout, unsigned int axis,
                                      long long splits, long long* extents,
                                      long long* strides) {
  if (int s = check_any(in_layout)) return s;
  if (axis >= static_cast<unsigned>(in_layout->rank)) return T4A_ERR_INVALID_AXIS;
  if (extents == nullptr || strides == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  // As t4a_layout_compact: the strides (overflow) first, then the extents.
  long long stride = 1;
  for (int k = 0; k < in_layout->rank; ++k) {
    const long long e = static_cast<unsigned>(k) == axis ? splits : in_layout->extents[k];
    extents[k] = e;
    strides[k] = stride;
    if (!checked_mul(stride, e, &stride)) return T4A_ERR_OVERFLOW;
  }
  for (int k = 0; k < in_layout->rank; ++k) {
    if (extents[k] < 0) return T4A_ERR_NEGATIVE_EXTENT;
  }
  return ok();
}

// Reference plan_fill_zero -> plan_elementwise (src/lib.rs:1591-1603): every
// dtype, flat_launch's refusals; one 16-byte vector per thread.
int t4a_plan_fill_zero(int dtype, long long len, t4a_launch* launch) {
  return t4a_plan_copy_exact(dtype, len, launch);
}

// Reference plan_fill_zero_view (src/lib.rs:1605-1622).
int t4a_plan_fill_zero_view(int dtype, const t4a_cuda_layout* dst, long long dst_len,
                            t4a_launch* launch) {
  if (launch == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (int s = check_layout(dst)) return s;
  return plan_fill_view(dtype, V(dst), dst_len, launch);
}

int t4a_plan_fill_zero_view_any(int dtype, const t4a_cuda_layout_any* dst, long long dst_len,
                                t4a_launch* launch) {
  if (launch == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (int s = check_any(dst)) return s;
  return general_movement(plan_fill_view(dtype, V(dst), dst_len, launch), launch);
}

// Reference plan_contiguous_to_view (src/lib.rs:1641-1658).
int t4a_plan_contiguous_to_view(int dtype, const t4a_cuda_layout* dst, long long dst_len,
                                t4a_launch* launch) {
  if (launch == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (int s = check_layout(dst)) return s;
  return plan_contiguous(dtype, V(dst), dst_len, launch);
}

int t4a_plan_contiguous_to_view_any(int dtype, const t4a_cuda_layout_any* dst,
                                    long long dst_len, t4a_launch* launch) {
  if (launch == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (int s = check_any(dst)) return s;
  return general_movement(plan_contiguous(dtype, V(dst), dst_len, launch), launch);
}

// Reference plan_broadcast_in_dim (src/lib.rs:1484-1533).
int t4a_plan_broadcast_in_dim(int dtype, const t4a_cuda_layout* out, long long out_len,
                              const t4a_cuda_layout* in, long long in_len,
                              const t4a_cuda_axis_values* dims, t4a_launch* launch) {
  if (launch == nullptr || dims == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (int s = check_layout(out)) return s;
  if (int s = check_layout(in)) return s;
  if (dims->rank < 0 || dims->rank > T4A_CUDA_MAX_RANK) return T4A_ERR_RANK_LENGTH;
  return plan_broadcast(dtype, V(out), out_len, V(in), in_len, dims->values, dims->rank,
                        launch);
}

int t4a_plan_broadcast_in_dim_any(int dtype, const t4a_cuda_layout_any* out, long long out_len,
                                  const t4a_cuda_layout_any* in, long long in_len,
                                  const t4a_cuda_axis_values_any* dims, t4a_launch* launch) {
  if (launch == nullptr || dims == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (int s = check_any(out)) return s;
  if (int s = check_any(in)) return s;
  if (dims->rank < 0) return T4A_ERR_RANK_LENGTH;
  return general_movement(
      plan_broadcast(dtype, V(out), out_len, V(in), in_len, dims->values, dims->rank, launch),
      launch);
}

// Reference plan_concatenate_copy (src/lib.rs:1535-1589).
int t4a_plan_concatenate_copy(int dtype, const t4a_cuda_layout* out, long long out_len,
                              const t4a_cuda_layout* in, long long in_len, unsigned int axis,
                              long long axis_offset, t4a_launch* launch) {
  if (launch == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (int s = check_layout(out)) return s;
  if (int s = check_layout(in)) return s;
  return plan_concatenate(dtype, V(out), out_len, V(in), in_len, axis, axis_offset, launch);
}

int t4a_plan_concatenate_copy_any(int dtype, const t4a_cuda_layout_any* out, long long out_len,
                                  const t4a_cuda_layout_any* in, long long in_len,
                                  unsigned int axis, long long axis_offset, t4a_launch* launch) {
  if (launch == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (int s = check_any(out)) return s;
  if (int s = check_any(in)) return s;
  return general_movement(
      plan_concatenate(dtype, V(out), out_len, V(in), in_len, axis, axis_offset, launch), launch);
}

}  // extern "C"
