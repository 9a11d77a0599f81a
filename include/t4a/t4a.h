/*
 * t4a MI355X host C ABI: checked launch planning and the HIP launchers of the
 * movement and single-axis reduction entries.
 *
 * The reference splits its boundary in two: a Rust host planner
 * (reference src/lib.rs) that validates metadata and returns launch geometry,
 * and `extern "C" __global__` kernels (reference cuda/src/movement.cu,
 * cuda/src/reduce.cu) that the caller launches on its own stream with that
 * geometry. This library keeps both halves behind plain C functions:
 *
 *   t4a_plan_*     restate the reference planners (same validation order, same
 *                  error for the same bad input) and return MI355X geometry;
 *   t4a_hip_*      launch the gfx950 kernel of the same name on the caller's
 *                  stream with a planned geometry (the reference caller's
 *                  cuLaunchKernel, tests/gpu/mod.rs:297-324).
 *
 * Ownership is the reference's (docs/abi/c-kernel-abi.md:3-14): the caller owns
 * the device, stream, every buffer and the partials workspace, and decides when
 * to synchronize. Nothing here allocates device memory or synchronizes.
 *
 * Status values: 0 is success; otherwise the reference `Error` discriminant
 * plus one (reference src/lib.rs:217-274), or one of the T4A_HIP_* launch
 * statuses below. The by-value planners and launchers take rank <= 8
 * (T4A_CUDA_MAX_RANK, the reference's fast path `Layout`/`CLayout`); their
 * `_any` twins take t4a_cuda_layout_any of any rank (the reference's general
 * path, docs/abi/c-kernel-abi.md "Dynamic rank"): the planners read its arrays
 * from host memory, the launchers pass arrays in device memory to the kernels.
 */
#ifndef T4A_T4A_H_
#define T4A_T4A_H_

#include "t4a/abi.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  T4A_OK = 0,
  T4A_ERR_RANK_OUT_OF_RANGE = 1,
  T4A_ERR_RANK_LENGTH = 2,
  T4A_ERR_NEGATIVE_EXTENT = 3,
  T4A_ERR_NEGATIVE_COUNT = 4,
  T4A_ERR_OVERFLOW = 5,
  T4A_ERR_COUNT_MISMATCH = 6,
  T4A_ERR_OFFSET_OUT_OF_SPAN = 7,
  T4A_ERR_BROADCAST_DESTINATION = 8,
  T4A_ERR_UNSUPPORTED_DTYPE = 9,
  T4A_ERR_NOT_ELEMENTWISE = 10,
  T4A_ERR_LAUNCH_LIMIT = 11,
  T4A_ERR_INVALID_TRANSPOSE_CONFIG = 12,
  T4A_ERR_INVALID_AXIS = 13,
  T4A_ERR_DUPLICATE_AXIS = 14,
  T4A_ERR_NOT_COMPACT = 15,
  T4A_ERR_SHAPE_MISMATCH = 16,
  T4A_ERR_INVALID_STEP = 17,
  T4A_ERR_INVALID_PADDING = 18,
  T4A_ERR_DOMAIN_TOO_LARGE = 19,
  T4A_ERR_INVALID_STRIDE = 20,
  T4A_ERR_STRATEGY_MISMATCH = 21,
  T4A_ERR_INVALID_PLANE_WIDTH = 22,
  T4A_ERR_INVALID_SPLIT = 23,
  T4A_ERR_INDEX_VECTOR_MISMATCH = 24,
  T4A_ERR_UNSUPPORTED_OP = 25,
  /* Launch-side statuses of the t4a_hip_* functions (no reference counterpart:
   * the reference returns nothing from a raw launch). */
  T4A_HIP_ERR_LAUNCH = 100,        /* the HIP runtime refused the launch */
  T4A_HIP_ERR_NULL_ARGUMENT = 101, /* a required pointer argument is NULL */
  T4A_HIP_ERR_NOT_FOUND = 102,     /* no such code object, or the library's path is unknown */
  T4A_HIP_ERR_TOO_SMALL = 103,     /* a caller's buffer cannot hold the result */
  T4A_HIP_ERR_SCRATCH_LIMIT = 104  /* the partials exceed T4A_HIP_SCRATCH_BYTES */
} t4a_status;

/* Reference RankVariant (src/lib.rs:800-838): FAST selects the by-value symbol. */
typedef enum { T4A_VARIANT_FAST = 0, T4A_VARIANT_GENERAL = 1 } t4a_rank_variant;

/* Reference Launch (src/lib.rs:840-873). Any zero grid dimension means "no
 * work": the caller (and every t4a_hip_* launcher) skips the launch. */
typedef struct {
  unsigned int grid[3];
  unsigned int block[3];
  unsigned int shared_bytes;
  int variant;
} t4a_launch;

/* Reference Split (src/lib.rs:3146-3150). */
typedef struct {
  long long splits;
  long long chunk_len;
} t4a_split;

typedef enum { T4A_PLAN_DIRECT = 0, T4A_PLAN_SPLIT = 1 } t4a_reduction_plan_kind;

/* Reference ReductionPlan (src/lib.rs:3168-3182). DIRECT fills `strategy` and
 * `launch`; SPLIT fills `split`, `pass1`, `combine_strategy`, `combine_op` and
 * `pass2`. */
typedef struct {
  int kind;
  int strategy;
  t4a_launch launch;
  t4a_split split;
  t4a_launch pass1;
  int combine_strategy;
  int combine_op;
  t4a_launch pass2;
} t4a_reduction_plan;

/* ---- library facts ---------------------------------------------------------- */

int t4a_abi_revision(void);                 /* T4A_CUDA_ABI_REVISION */
const char* t4a_status_name(int status);    /* "OffsetOutOfSpan", ..., "Ok" */
int t4a_dtype_size(int dtype);              /* reference DType::size; 0 if unknown */

/* ---- layouts (reference Layout, src/lib.rs:322-450) -------------------------- */

/* Build a layout of `rank` axes; the unused slots are zeroed.
 * Errors: RankOutOfRange (rank > 8 or < 0), NegativeExtent. */
int t4a_layout_new(t4a_cuda_layout* out, int rank, const long long* extents,
                   const long long* strides, long long offset);
/* Compact layout over `extents`, axis 0 fastest. Errors: as above, Overflow. */
int t4a_layout_compact(t4a_cuda_layout* out, int rank, const long long* extents);
/* Checked extent product (reference Layout::element_count). */
int t4a_layout_element_count(const t4a_cuda_layout* layout, long long* count);

/* ---- movement planners (reference src/lib.rs:1592-1737) ---------------------- */

/* Reference plan_copy_exact (src/lib.rs:1624-1626). */
int t4a_plan_copy_exact(int dtype, long long len, t4a_launch* launch);

int t4a_plan_materialize_strided(int dtype, const t4a_cuda_layout* src, long long src_len,
                                 t4a_launch* launch);
int t4a_plan_strided_to_strided(int dtype, const t4a_cuda_layout* src, long long src_len,
                                const t4a_cuda_layout* dst, long long dst_len,
                                t4a_launch* launch);
/* The kernel the t4a_hip_* movement launchers run for a source/destination
 * pair under its planned geometry (no reference counterpart: the reference
 * leaves route selection to its consumer, which fuses axes and then picks the
 * tiled transpose or a strided copy). materialize_strided is the pair with
 * `dst` NULL (the compact destination); contiguous_to_view, broadcast_in_dim
 * and concatenate_copy are moves over the pairs their geometry implies.
 * Alignment only decides between 16-byte and element accesses inside a route. */
typedef enum {
  T4A_MOVE_ROUTE_EMPTY = 0,     /* nothing to move */
  T4A_MOVE_ROUTE_LINEAR = 1,    /* one run contiguous on both sides: the copy kernel */
  T4A_MOVE_ROUTE_ROWS = 2,      /* a dim contiguous on both sides: 16-byte row units */
  T4A_MOVE_ROUTE_TRANSPOSE = 3, /* one compact 2-D transpose: the tiled transpose's kernel */
  T4A_MOVE_ROUTE_TILE_ONCE = 4, /* LDS tiles of one of the tile walk's shapes */
  T4A_MOVE_ROUTE_TILES = 5,     /* persistent blocks walking LDS tiles */
  T4A_MOVE_ROUTE_ELEMENTS = 6   /* one decode per element */
} t4a_move_route;

/* Validates as t4a_plan_strided_to_strided (or t4a_plan_materialize_strided
 * when dst is NULL) with spans of exactly the layouts' reach, then writes the
 * route to *route. */
int t4a_plan_move_route(int dtype, const t4a_cuda_layout* src, const t4a_cuda_layout* dst,
                        int* route);

/* Reference plan_fill_zero (src/lib.rs:1601-1603). */
int t4a_plan_fill_zero(int dtype, long long len, t4a_launch* launch);
/* Reference plan_fill_zero_view (src/lib.rs:1605-1622). */
int t4a_plan_fill_zero_view(int dtype, const t4a_cuda_layout* dst, long long dst_len,
                            t4a_launch* launch);
/* Reference plan_contiguous_to_view (src/lib.rs:1641-1658). */
int t4a_plan_contiguous_to_view(int dtype, const t4a_cuda_layout* dst, long long dst_len,
                                t4a_launch* launch);
/* Reference plan_broadcast_in_dim (src/lib.rs:1484-1533): dims->values[i] is
 * the destination axis of input axis i; dims->rank must be the input rank. */
int t4a_plan_broadcast_in_dim(int dtype, const t4a_cuda_layout* out, long long out_len,
                              const t4a_cuda_layout* in, long long in_len,
                              const t4a_cuda_axis_values* dims, t4a_launch* launch);
/* Reference plan_concatenate_copy (src/lib.rs:1535-1589). */
int t4a_plan_concatenate_copy(int dtype, const t4a_cuda_layout* out, long long out_len,
                              const t4a_cuda_layout* in, long long in_len, unsigned int axis,
                              long long axis_offset, t4a_launch* launch);
/* Reference TransposeConfig::new (src/lib.rs:471-491). */
int t4a_transpose_config_new(int tile, int block_rows, int padding, int vector_width,
                             t4a_cuda_transpose_config* config);
/* The reference default configuration {16, 8, 1, 1} (src/lib.rs:463-468). */
t4a_cuda_transpose_config t4a_transpose_config_default(void);
int t4a_plan_tiled_transpose(int dtype, t4a_cuda_transpose_config config, long long src_offset,
                             long long batch_stride, long long dst_fast_extent,
                             long long src_fast_extent, long long batches, long long src_len,
                             long long dst_len, t4a_launch* launch);

/* ---- reduction planners (reference src/lib.rs:3031-3557) ---------------------- */

/* `*has_split` is 0 when the axis takes one pass (reference Ok(None)). */
int t4a_split_policy(long long reduce_len, unsigned int plane_width, int* has_split,
                     t4a_split* split);
int t4a_plan_reduce(int dtype, int op, int strategy, const t4a_cuda_layout* out_layout,
                    long long out_len, const t4a_cuda_layout* in_layout, long long in_len,
                    unsigned int axis, unsigned int plane_width, t4a_launch* launch);
int t4a_plan_reduce_partials(int dtype, int op, const t4a_cuda_layout* partials_layout,
                             long long partials_len, const t4a_cuda_layout* in_layout,
                             long long in_len, unsigned int axis, t4a_split split,
                             unsigned int plane_width, t4a_launch* launch);
int t4a_plan_reduction(int dtype, int op, const t4a_cuda_layout* out_layout, long long out_len,
                       const t4a_cuda_layout* in_layout, long long in_len, unsigned int axis,
                       unsigned int plane_width, t4a_reduction_plan* plan);
/* Compact partials layout: the input's extents with the axis set to `splits`
 * (reference reduction_partials_layout, src/lib.rs:3530-3557). */
int t4a_reduction_partials_layout(const t4a_cuda_layout* in_layout, unsigned int axis,
                                  long long splits, t4a_cuda_layout* partials_layout);

/* ---- general-rank planners ------------------------------------------------------
 * The same validation, errors and geometry for layouts of any rank (reference
 * planners over LayoutRef / WideLayout, whose rank is not bounded), with the
 * layouts' arrays in HOST memory. `launch->variant` is T4A_VARIANT_GENERAL when
 * a rank exceeds 8 (reference RankVariant::select, src/lib.rs:817-838): launch
 * the `_any` twin then; at rank <= 8 either twin runs the geometry. */
int t4a_plan_materialize_strided_any(int dtype, const t4a_cuda_layout_any* src,
                                     long long src_len, t4a_launch* launch);
int t4a_plan_strided_to_strided_any(int dtype, const t4a_cuda_layout_any* src,
                                    long long src_len, const t4a_cuda_layout_any* dst,
                                    long long dst_len, t4a_launch* launch);
int t4a_plan_reduce_any(int dtype, int op, int strategy, const t4a_cuda_layout_any* out_layout,
                        long long out_len, const t4a_cuda_layout_any* in_layout,
                        long long in_len, unsigned int axis, unsigned int plane_width,
                        t4a_launch* launch);
int t4a_plan_reduce_partials_any(int dtype, int op, const t4a_cuda_layout_any* partials_layout,
                                 long long partials_len, const t4a_cuda_layout_any* in_layout,
                                 long long in_len, unsigned int axis, t4a_split split,
                                 unsigned int plane_width, t4a_launch* launch);
int t4a_plan_fill_zero_view_any(int dtype, const t4a_cuda_layout_any* dst, long long dst_len,
                                t4a_launch* launch);
int t4a_plan_contiguous_to_view_any(int dtype, const t4a_cuda_layout_any* dst,
                                    long long dst_len, t4a_launch* launch);
int t4a_plan_broadcast_in_dim_any(int dtype, const t4a_cuda_layout_any* out, long long out_len,
                                  const t4a_cuda_layout_any* in, long long in_len,
                                  const t4a_cuda_axis_values_any* dims, t4a_launch* launch);
int t4a_plan_concatenate_copy_any(int dtype, const t4a_cuda_layout_any* out, long long out_len,
                                  const t4a_cuda_layout_any* in, long long in_len,
                                  unsigned int axis, long long axis_offset, t4a_launch* launch);
/* Writes pass1 / pass2 variants as above. */
int t4a_plan_reduction_any(int dtype, int op, const t4a_cuda_layout_any* out_layout,
                           long long out_len, const t4a_cuda_layout_any* in_layout,
                           long long in_len, unsigned int axis, unsigned int plane_width,
                           t4a_reduction_plan* plan);
/* The compact partials layout of any rank: `in_layout->rank` extents and
 * strides into the caller's arrays (offset 0). */
int t4a_reduction_partials_layout_any(const t4a_cuda_layout_any* in_layout, unsigned int axis,
                                      long long splits, long long* extents,
                                      long long* strides);

/* ---- HIP launchers ------------------------------------------------------------
 * Each launches the gfx950 kernel of the reference entry's name with the
 * arguments of that entry, on `stream` (a hipStream_t; NULL is the null stream),
 * using `launch` as returned by the matching planner. An empty launch returns
 * T4A_OK without touching the device. Metadata is not re-validated here (the
 * reference raw entry is caller UB past its planner, c-kernel-abi.md:9-14).
 */

/* Reference t4a_cuda_tiled_transpose, cuda/src/movement.cu:571-573. */
int t4a_hip_tiled_transpose(void* dst, const void* src, int dtype, long long src_offset,
                            long long batch_stride, long long dst_fast_extent,
                            long long src_fast_extent, t4a_cuda_transpose_config config,
                            const t4a_launch* launch, void* stream);
/* Reference t4a_cuda_copy_exact, cuda/src/movement.cu:528-533. */
int t4a_hip_copy_exact(void* dst, const void* src, int dtype, long long len,
                       const t4a_launch* launch, void* stream);
/* Reference t4a_cuda_materialize_strided, cuda/src/movement.cu:535-537. */
int t4a_hip_materialize_strided(void* dst, const void* src, int dtype,
                                const t4a_cuda_layout* src_layout, long long len,
                                const t4a_launch* launch, void* stream);
/* Reference t4a_cuda_strided_to_strided, cuda/src/movement.cu:553-556. */
int t4a_hip_strided_to_strided(void* dst, const void* src, int dtype,
                               const t4a_cuda_layout* src_layout,
                               const t4a_cuda_layout* dst_layout, long long len,
                               const t4a_launch* launch, void* stream);
/* Reference t4a_cuda_fill_zero, cuda/src/movement.cu:514-518. */
int t4a_hip_fill_zero(void* out, int dtype, long long len, const t4a_launch* launch,
                      void* stream);
/* Reference t4a_cuda_fill_zero_view, cuda/src/movement.cu:520-526. */
int t4a_hip_fill_zero_view(void* out, int dtype, const t4a_cuda_layout* layout, long long len,
                           const t4a_launch* launch, void* stream);
/* Reference t4a_cuda_contiguous_to_view, cuda/src/movement.cu:544-551. */
int t4a_hip_contiguous_to_view(void* dst, const void* src, int dtype,
                               const t4a_cuda_layout* dst_layout, long long len,
                               const t4a_launch* launch, void* stream);
/* Reference t4a_cuda_broadcast_in_dim, cuda/src/movement.cu:648-656. */
int t4a_hip_broadcast_in_dim(void* out, const void* in, int dtype,
                             const t4a_cuda_layout* out_layout, const t4a_cuda_layout* in_layout,
                             const t4a_cuda_axis_values* dims, long long out_len,
                             const t4a_launch* launch, void* stream);
/* Reference t4a_cuda_concatenate_copy, cuda/src/movement.cu:668-676. */
int t4a_hip_concatenate_copy(void* out, const void* in, int dtype,
                             const t4a_cuda_layout* out_layout, const t4a_cuda_layout* in_layout,
                             int axis, long long axis_offset, long long in_len,
                             const t4a_launch* launch, void* stream);
/* Reference t4a_cuda_reduce, cuda/src/reduce.cu:765-768. */
int t4a_hip_reduce(void* out, const void* in, int dtype, int op, int strategy,
                   const t4a_cuda_layout* out_layout, const t4a_cuda_layout* in_layout,
                   int axis, long long output_len, const t4a_launch* launch, void* stream);
/* Reference t4a_cuda_reduce_partials, cuda/src/reduce.cu:813-817. */
int t4a_hip_reduce_partials(void* partials, const void* in, int dtype, int op,
                            const t4a_cuda_layout* partials_layout,
                            const t4a_cuda_layout* in_layout, int axis, long long output_len,
                            long long splits, long long chunk_len, const t4a_launch* launch,
                            void* stream);

/* The general-rank twins (reference cuda/src/movement.cu:620-646,
 * cuda/src/reduce.cu:854-940): the layouts' arrays in device memory, ordered
 * before the launch on `stream` and unchanged until it completes; any geometry
 * from the matching t4a_plan_*_any (or by-value) planner. The kernels fuse the
 * geometry themselves and return the by-value twins' bits. */
int t4a_hip_materialize_strided_any(void* dst, const void* src, int dtype,
                                    const t4a_cuda_layout_any* src_layout, long long len,
                                    const t4a_launch* launch, void* stream);
int t4a_hip_strided_to_strided_any(void* dst, const void* src, int dtype,
                                   const t4a_cuda_layout_any* src_layout,
                                   const t4a_cuda_layout_any* dst_layout, long long len,
                                   const t4a_launch* launch, void* stream);
int t4a_hip_fill_zero_view_any(void* out, int dtype, const t4a_cuda_layout_any* layout,
                               long long len, const t4a_launch* launch, void* stream);
int t4a_hip_contiguous_to_view_any(void* dst, const void* src, int dtype,
                                   const t4a_cuda_layout_any* dst_layout, long long len,
                                   const t4a_launch* launch, void* stream);
int t4a_hip_broadcast_in_dim_any(void* out, const void* in, int dtype,
                                 const t4a_cuda_layout_any* out_layout,
                                 const t4a_cuda_layout_any* in_layout,
                                 const t4a_cuda_axis_values_any* dims, long long out_len,
                                 const t4a_launch* launch, void* stream);
int t4a_hip_concatenate_copy_any(void* out, const void* in, int dtype,
                                 const t4a_cuda_layout_any* out_layout,
                                 const t4a_cuda_layout_any* in_layout, int axis,
                                 long long axis_offset, long long in_len,
                                 const t4a_launch* launch, void* stream);
int t4a_hip_reduce_any(void* out, const void* in, int dtype, int op, int strategy,
                       const t4a_cuda_layout_any* out_layout,
                       const t4a_cuda_layout_any* in_layout, int axis, long long output_len,
                       const t4a_launch* launch, void* stream);
int t4a_hip_reduce_partials_any(void* partials, const void* in, int dtype, int op,
                                const t4a_cuda_layout_any* partials_layout,
                                const t4a_cuda_layout_any* in_layout, int axis,
                                long long output_len, long long splits, long long chunk_len,
                                const t4a_launch* launch, void* stream);

/* A whole reduction_plan (reference src/lib.rs:3457-3528 plans it; its caller
 * then launches pass 1 and the combine, reduce.cu:813-852 and 765-811): Direct
 * runs t4a_hip_reduce; Split runs pass 1 into `partials` (the
 * t4a_reduction_partials_layout of the plan) and the combine into `out`, on
 * `stream`. A Split plan whose combine is a unit fold over at most 32 partials
 * of a contiguous, end-to-end chunk layout runs as ONE launch: each block holds
 * all of an output's chunks and folds their partials in the unit order, so
 * finals and partials are the two launches' bits. */
int t4a_hip_reduction(void* out, const void* in, void* partials, int dtype, int op,
                      const t4a_cuda_layout* out_layout, const t4a_cuda_layout* in_layout,
                      int axis, long long output_len, const t4a_reduction_plan* plan,
                      void* stream);

/* t4a_hip_reduction without a caller's partials workspace, allocating nothing.
 * No counterpart in the reference (its caller always owns the workspace); it is
 * for callers that cannot allocate device memory: code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc. A Split plan's partials
 * live in a library-owned device array of T4A_HIP_SCRATCH_BYTES per GPU (held
 * until the process ends; its address is looked up on a device's first call);
 * a plan whose partials layout needs more returns T4A_HIP_ERR_SCRATCH_LIMIT
 * before touching the device. A Direct plan needs no workspace. Pass 1 writes
 * every partial the combine reads, so nothing need start at zero. Every call on
 * one GPU shares that GPU's array: calls on the same stream are ordered, calls
 * that overlap on one GPU (other streams, other host threads) race. Same
 * outputs, bit for bit, as t4a_hip_reduction with a workspace of its own. */
#define T4A_HIP_SCRATCH_BYTES (8u * 1024u * 1024u)
int t4a_hip_reduction_scratch(void* out, const void* in, int dtype, int op,
                              const t4a_cuda_layout* out_layout,
                              const t4a_cuda_layout* in_layout, int axis, long long output_len,
                              const t4a_reduction_plan* plan, void* stream);

/* 1 if t4a_hip_reduction runs `plan` over an input at `in` as one launch, else
 * 0 (no reference counterpart: it tells a caller which kernels a profile will
 * show). */
int t4a_hip_reduction_joins(const void* in, int dtype, int op, const t4a_cuda_layout* out_layout,
                            const t4a_cuda_layout* in_layout, int axis, long long output_len,
                            const t4a_reduction_plan* plan);

/* The hipError_t of the most recent launch on this thread that returned
 * T4A_HIP_ERR_LAUNCH (0 if none). */
int t4a_hip_last_error(void);

/* Kernel launches the t4a_hip_* launchers have issued in this process, all
 * threads (no reference counterpart: the reference benchmark counts the
 * launches in its measured region through its own launch wrapper,
 * examples/bench_kernels.rs:283-306; this is that count for this library). */
unsigned long long t4a_hip_launch_count(void);

/* ---- code objects (the prepare step's artifacts) -------------------------- */

/* The gfx950 code objects exporting the reference-named kernel entries, built
 * ahead of time next to libt4a_hip.so. The reference hands its CUDA text to the
 * consumer's NVRTC (src/lib.rs:32-130, `source::MODULES` / `module_of`) inside a
 * prepare step that loads modules privately per runtime
 * (docs/design/cubecl-kernel-port.md:88-109); here prepare is loading these
 * files (hipModuleLoadData) and binding entries by name (hipModuleGetFunction).
 * Names and files are static strings; nothing here loads or allocates. */
int t4a_code_object_count(void);
const char* t4a_code_object_name(int index);     /* "movement", "reduce"; NULL past the end */
const char* t4a_code_object_file(int index);     /* "t4a_movement.gfx950.hsaco", ... */
const char* t4a_code_object_target(void);        /* "gfx950" */
int t4a_code_object_entry_count(int index);
const char* t4a_code_object_entry(int index, int entry);
/* Index of the code object exporting `entry`, -1 for an entry none exports
 * (reference source::module_of). */
int t4a_code_object_of(const char* entry);
/* The code object's absolute path (the library's directory + its file) into
 * `path` of `capacity` bytes: T4A_HIP_ERR_NOT_FOUND for a bad index,
 * T4A_HIP_ERR_TOO_SMALL when it does not fit. */
int t4a_code_object_path(int index, char* path, unsigned long capacity);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif /* T4A_T4A_H_ */
