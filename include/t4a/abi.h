/*
 * t4a MI355X kernel ABI: the plain-data types and tags shared by the host
 * planner, the HIP kernels and any foreign caller (C, C++, Rust `extern "C"`).
 *
 * This header is C11 and C++17 clean and includes only <stddef.h>. It restates
 * the by-value structs and tags of the reference ABI so that a caller built
 * against the reference passes byte-identical arguments:
 *
 *   t4a_cuda_layout            reference cuda/include/t4a/abi.cuh:47-57
 *   t4a_cuda_layout_any        reference cuda/include/t4a/abi.cuh:109-121
 *   t4a_cuda_axis_values(_any) reference cuda/include/t4a/abi.cuh:74-79, 122-126
 *   t4a_cuda_transpose_config  reference cuda/include/t4a/abi.cuh:239-245
 *   t4a_cuda_dtype tags        reference cuda/include/t4a/abi.cuh:25-33
 *   reduce op / strategy tags  reference cuda/include/t4a/abi.cuh:59-71
 *   c32 / c64 element types    reference cuda/include/t4a/abi.cuh:35-45
 *
 * Axis 0 is the fastest-varying logical axis. A flat logical index f decodes as
 * coordinate = f % extent, f /= extent from axis 0 upward; the element address
 * is offset + sum(coordinate * stride). Strides and offsets are signed element
 * counts; stride zero is a broadcast axis. Unused array slots must be zero.
 */
#ifndef T4A_ABI_H_
#define T4A_ABI_H_

#include <stddef.h>

#define T4A_CUDA_MAX_RANK 8
/* Numerical topology and struct layouts of reference revision 14
 * (docs/abi/c-kernel-abi.md "Revision"). */
#define T4A_CUDA_ABI_REVISION 14

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  T4A_CUDA_F32 = 0,
  T4A_CUDA_F64 = 1,
  T4A_CUDA_I32 = 2,
  T4A_CUDA_I64 = 3,
  T4A_CUDA_BOOL = 4,
  T4A_CUDA_C32 = 5,
  T4A_CUDA_C64 = 6
} t4a_cuda_dtype;

/* Interleaved complex with the component's alignment (not float2/double2). */
typedef struct {
  float re;
  float im;
} t4a_cuda_c32;

typedef struct {
  double re;
  double im;
} t4a_cuda_c64;

/* 144 bytes, alignment 8: rank 0, reserved 4, offset 8, extents 16, strides 80. */
typedef struct {
  int rank;
  int reserved;
  long long offset;
  long long extents[T4A_CUDA_MAX_RANK];
  long long strides[T4A_CUDA_MAX_RANK];
} t4a_cuda_layout;

/* The general-rank layout of the `_any` entries (reference revision 9,
 * docs/abi/c-kernel-abi.md "Dynamic rank"): the same fields with `rank` values
 * of extents and of strides in caller-owned device memory (8-byte aligned,
 * unchanged until the launch completes; may be NULL when rank is 0). 32 bytes,
 * alignment 8: rank 0, reserved 4, offset 8, extents 16, strides 24. The
 * t4a_plan_*_any planners take the same struct pointing at host memory. */
typedef struct {
  int rank;
  int reserved;
  long long offset;
  const long long* extents;
  const long long* strides;
} t4a_cuda_layout_any;

/* A per-axis value map (broadcast_in_dim's `dims`: values[src_axis] is the
 * destination axis of input axis src_axis). 72 bytes, alignment 8: rank 0,
 * reserved 4, values 8; unused slots zero. */
typedef struct {
  int rank;
  int reserved;
  long long values[T4A_CUDA_MAX_RANK];
} t4a_cuda_axis_values;

/* Its general-rank form: `rank` values by pointer (device memory for the
 * kernels, host memory for the planners). 16 bytes, alignment 8. */
typedef struct {
  int rank;
  int reserved;
  const long long* values;
} t4a_cuda_axis_values_any;

typedef enum {
  T4A_CUDA_REDUCE_SUM = 0,
  T4A_CUDA_REDUCE_PROD = 1,
  T4A_CUDA_REDUCE_SUM_SQUARES = 2,
  T4A_CUDA_REDUCE_MAX = 3,
  T4A_CUDA_REDUCE_MIN = 4
} t4a_cuda_reduce_op;

typedef enum {
  T4A_CUDA_REDUCE_UNIT = 0,
  T4A_CUDA_REDUCE_PLANE = 1
} t4a_cuda_reduce_strategy;

/* 16 bytes, alignment 4. tile 8|16|32, block_rows 4|8|16, padding 0|1,
 * vector_width 1|2|4 with tile % vector_width == 0. */
typedef struct {
  int tile;
  int block_rows;
  int padding;
  int vector_width;
} t4a_cuda_transpose_config;

#ifdef __cplusplus
}  /* extern "C" */
#define T4A_STATIC_ASSERT(cond, msg) static_assert(cond, msg)
#define T4A_ALIGNOF(type) alignof(type)
#else
#define T4A_STATIC_ASSERT(cond, msg) _Static_assert(cond, msg)
#define T4A_ALIGNOF(type) _Alignof(type)
#endif

T4A_STATIC_ASSERT(sizeof(int) == 4, "the C ABI requires 32-bit int");
T4A_STATIC_ASSERT(sizeof(long long) == 8, "the C ABI requires 64-bit long long");
T4A_STATIC_ASSERT(sizeof(t4a_cuda_layout) == 144, "t4a_cuda_layout size");
T4A_STATIC_ASSERT(T4A_ALIGNOF(t4a_cuda_layout) == 8, "t4a_cuda_layout alignment");
T4A_STATIC_ASSERT(offsetof(t4a_cuda_layout, offset) == 8, "t4a_cuda_layout.offset");
T4A_STATIC_ASSERT(offsetof(t4a_cuda_layout, extents) == 16, "t4a_cuda_layout.extents");
T4A_STATIC_ASSERT(offsetof(t4a_cuda_layout, strides) == 80, "t4a_cuda_layout.strides");
T4A_STATIC_ASSERT(sizeof(void*) == 8, "the C ABI requires 64-bit pointers");
T4A_STATIC_ASSERT(sizeof(t4a_cuda_layout_any) == 32, "t4a_cuda_layout_any size");
T4A_STATIC_ASSERT(T4A_ALIGNOF(t4a_cuda_layout_any) == 8, "t4a_cuda_layout_any alignment");
T4A_STATIC_ASSERT(offsetof(t4a_cuda_layout_any, offset) == 8, "t4a_cuda_layout_any.offset");
T4A_STATIC_ASSERT(offsetof(t4a_cuda_layout_any, extents) == 16, "t4a_cuda_layout_any.extents");
T4A_STATIC_ASSERT(offsetof(t4a_cuda_layout_any, strides) == 24, "t4a_cuda_layout_any.strides");
T4A_STATIC_ASSERT(sizeof(t4a_cuda_axis_values) == 72, "t4a_cuda_axis_values size");
T4A_STATIC_ASSERT(offsetof(t4a_cuda_axis_values, values) == 8, "t4a_cuda_axis_values.values");
T4A_STATIC_ASSERT(sizeof(t4a_cuda_axis_values_any) == 16, "t4a_cuda_axis_values_any size");
T4A_STATIC_ASSERT(offsetof(t4a_cuda_axis_values_any, values) == 8,
                  "t4a_cuda_axis_values_any.values");
T4A_STATIC_ASSERT(sizeof(t4a_cuda_transpose_config) == 16, "t4a_cuda_transpose_config size");
T4A_STATIC_ASSERT(T4A_ALIGNOF(t4a_cuda_transpose_config) == 4,
                  "t4a_cuda_transpose_config alignment");
T4A_STATIC_ASSERT(sizeof(t4a_cuda_c32) == 8 && T4A_ALIGNOF(t4a_cuda_c32) == 4, "t4a_cuda_c32");
T4A_STATIC_ASSERT(sizeof(t4a_cuda_c64) == 16 && T4A_ALIGNOF(t4a_cuda_c64) == 8, "t4a_cuda_c64");

#endif /* T4A_ABI_H_ */
