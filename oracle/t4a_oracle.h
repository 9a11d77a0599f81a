/*
 * t4a CPU oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of what the reference kernels compute, used as the
 * checker for the HIP kernels and as the reported CPU baseline. Nothing in the
 * product path links or calls this library: only tests/, the smoke check and
 * bench.py's cpu_baseline leg load it.
 *
 * Every function cites the reference file:line it restates. Movement is byte
 * copies (bit-exact by construction); reductions reproduce the reference's
 * numerical topology element for element (which lane folds which element, in
 * which order, and how lanes are combined), so float results are bit-identical
 * to the reference kernels wherever IEEE rounding alone decides them.
 *
 * Parity pins (tests/test_oracle_*.py): the reference's A100 golden vectors
 * (tests/golden/reduce-golden.tsv, 1332 cases), closed-form index maps, brute
 * force on tiny inputs, and order-independent folds (integers, max/min). See
 * the test files for which check pins which function.
 */
#ifndef T4A_ORACLE_H_
#define T4A_ORACLE_H_

#include "t4a/abi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* dst[f] = src[decode(f, src_layout)] for f < len.
 * Reference: cuda/src/movement.cu:98-110, tests/gpu_kernels.rs:36-51. */
void t4a_oracle_materialize_strided(void* dst, const void* src, int dtype,
                                    const t4a_cuda_layout* src_layout, long long len);

/* dst[decode(f, dst_layout)] = src[decode(f, src_layout)], shared extents (the
 * source's). Reference: cuda/src/movement.cu:127-145. */
void t4a_oracle_strided_to_strided(void* dst, const void* src, int dtype,
                                   const t4a_cuda_layout* src_layout,
                                   const t4a_cuda_layout* dst_layout, long long len);

/* out[decode(f, layout)] = zero (all-zero bits) for f < len.
 * Reference: cuda/src/movement.cu:79-96, abi.cuh:520-538 (t4a_cuda_zero). */
void t4a_oracle_fill_zero_view(void* out, int dtype, const t4a_cuda_layout* layout,
                               long long len);

/* dst[decode(f, dst_layout)] = src[f]. Reference: cuda/src/movement.cu:113-125. */
void t4a_oracle_contiguous_to_view(void* dst, const void* src, int dtype,
                                   const t4a_cuda_layout* dst_layout, long long len);

/* out[f] = in[in.offset + sum_i (in.extents[i] == 1 ? 0 : coord(f, dims[i])) *
 * in.strides[i]], coordinates over the (compact) destination's extents.
 * Reference: cuda/src/movement.cu:397-437. */
void t4a_oracle_broadcast_in_dim(void* out, const void* in, int dtype,
                                 const t4a_cuda_layout* out_layout,
                                 const t4a_cuda_layout* in_layout, const long long* dims,
                                 int dims_rank, long long out_len);

/* out[out.offset + sum_k (coord(f, in) + (k == axis ? axis_offset : 0)) *
 * out.strides[k]] = in[f] for the compact input. Reference:
 * cuda/src/movement.cu:441-466. */
void t4a_oracle_concatenate_copy(void* out, const void* in, int dtype,
                                 const t4a_cuda_layout* out_layout,
                                 const t4a_cuda_layout* in_layout, int axis,
                                 long long axis_offset, long long in_len);

/* dst[b*S + i + j*M] = src[src_offset + b*S + i*N + j], S = M*N.
 * Reference: docs/abi/c-kernel-abi.md:151-159, tests/gpu_kernels.rs:330-339. */
void t4a_oracle_tiled_transpose(void* dst, const void* src, int dtype, long long src_offset,
                                long long batch_stride, long long dst_fast_extent,
                                long long src_fast_extent, long long batches);

/* t4a_cuda_reduce: strategy UNIT (serial fold per output) or PLANE with block
 * width `block_width` (8/16/32 narrow xor tree; 64..512 wide combine through
 * per-warp results). Reference: cuda/src/reduce.cu:110-340, 765-811. */
void t4a_oracle_reduce(void* out, const void* in, int dtype, int op, int strategy,
                       int block_width, const t4a_cuda_layout* out_layout,
                       const t4a_cuda_layout* in_layout, int axis, long long output_len);

/* t4a_cuda_reduce_partials with plane width `plane_width` (8/16/32): one plane
 * per (output, split), vector group walk or serial lane walk, xor tree.
 * Reference: cuda/src/reduce.cu:343-633, 813-852; docs/abi/c-kernel-abi.md:313-359. */
void t4a_oracle_reduce_partials(void* partials, const void* in, int dtype, int op,
                                int plane_width, const t4a_cuda_layout* partials_layout,
                                const t4a_cuda_layout* in_layout, int axis,
                                long long output_len, long long splits, long long chunk_len);

/* The reference tests' sequential CPU reduction, accumulated in double (complex:
 * componentwise double for SUM, double complex product for PROD); writes doubles,
 * two per complex element. Reference: tests/gpu_reduce.rs:79-130. */
void t4a_oracle_reduce_f64(double* out, const void* in, int dtype, int op,
                           const t4a_cuda_layout* in_layout, int axis, long long output_len);

/* FNV-1a 64 digest of a byte buffer (reference tests/gpu_reduce_golden.rs:66-73). */
unsigned long long t4a_oracle_fnv1a64(const void* bytes, unsigned long long len);

/* Bytes per element of a dtype tag, 0 for an unknown tag. */
int t4a_oracle_dtype_size(int dtype);

/* Threads for the movement and reduction loops (OpenMP over independent
 * outputs; results do not depend on it). Default 1. */
void t4a_oracle_set_threads(int n);
int t4a_oracle_max_threads(void);

#ifdef __cplusplus
}
#endif

#endif /* T4A_ORACLE_H_ */
