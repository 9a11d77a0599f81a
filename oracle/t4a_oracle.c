/*
 * t4a CPU oracle -- TEST INFRASTRUCTURE ONLY (see t4a_oracle.h).
 *
 * Built with -ffp-contract=off: every rounding below is the one written.
 */
#include "t4a_oracle.h"

#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* Threads for the loops over independent outputs (the all-core CPU baseline);
 * 1 unless set. Every output's fold stays one serial loop on one thread, so
 * no result depends on the count. */
static int g_threads = 1;

void t4a_oracle_set_threads(int n) { g_threads = n > 0 ? n : 1; }

int t4a_oracle_max_threads(void) { return omp_get_max_threads(); }

int t4a_oracle_dtype_size(int dtype) {
  switch (dtype) {
    case T4A_CUDA_F32: return 4;
    case T4A_CUDA_F64: return 8;
    case T4A_CUDA_I32: return 4;
    case T4A_CUDA_I64: return 8;
    case T4A_CUDA_BOOL: return 1;
    case T4A_CUDA_C32: return 8;
    case T4A_CUDA_C64: return 16;
    default: return 0;
  }
}

/* Element address of logical index `flat`: coordinate = flat % extent,
 * flat /= extent from axis 0 up (reference cuda/include/t4a/abi.cuh:422-438). */
static long long decode(long long flat, int rank, const long long* extents,
                        const long long* strides, long long offset) {
  for (int axis = 0; axis < rank; ++axis) {
    const long long extent = extents[axis];
    const long long coordinate = flat % extent;
    flat /= extent;
    offset += coordinate * strides[axis];
  }
  return offset;
}

/* ---- movement ------------------------------------------------------------ */

void t4a_oracle_materialize_strided(void* dst, const void* src, int dtype,
                                    const t4a_cuda_layout* l, long long len) {
  const int es = t4a_oracle_dtype_size(dtype);
  if (es == 0) return; /* unknown tag: no work (c-kernel-abi.md:107-108) */
  unsigned char* d = (unsigned char*)dst;
  const unsigned char* s = (const unsigned char*)src;
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (long long f = 0; f < len; ++f) {
    const long long index = decode(f, l->rank, l->extents, l->strides, l->offset);
    memcpy(d + f * es, s + index * es, (size_t)es);
  }
}

void t4a_oracle_strided_to_strided(void* dst, const void* src, int dtype,
                                   const t4a_cuda_layout* sl, const t4a_cuda_layout* dl,
                                   long long len) {
  const int es = t4a_oracle_dtype_size(dtype);
  if (es == 0) return;
  unsigned char* d = (unsigned char*)dst;
  const unsigned char* s = (const unsigned char*)src;
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (long long f = 0; f < len; ++f) {
    const long long si = decode(f, sl->rank, sl->extents, sl->strides, sl->offset);
    /* Both layouts share the source's extents (movement.cu:139-141). */
    const long long di = decode(f, sl->rank, sl->extents, dl->strides, dl->offset);
    memcpy(d + di * es, s + si * es, (size_t)es);
  }
}

void t4a_oracle_fill_zero_view(void* out, int dtype, const t4a_cuda_layout* l, long long len) {
  const int es = t4a_oracle_dtype_size(dtype);
  if (es == 0) return;
  unsigned char* o = (unsigned char*)out;
  for (long long f = 0; f < len; ++f) {
    const long long index = decode(f, l->rank, l->extents, l->strides, l->offset);
    memset(o + index * es, 0, (size_t)es); /* every dtype's zero is all-zero bits */
  }
}

void t4a_oracle_contiguous_to_view(void* dst, const void* src, int dtype,
                                   const t4a_cuda_layout* l, long long len) {
  const int es = t4a_oracle_dtype_size(dtype);
  if (es == 0) return;
  unsigned char* d = (unsigned char*)dst;
  const unsigned char* s = (const unsigned char*)src;
  for (long long f = 0; f < len; ++f) {
    const long long index = decode(f, l->rank, l->extents, l->strides, l->offset);
    memcpy(d + index * es, s + f * es, (size_t)es);
  }
}

/* Coordinates of flat index `f` over a layout's extents, axis 0 first
 * (reference cuda/src/movement.cu:397-408). */
static void coords_of(long long f, const t4a_cuda_layout* l, long long* c) {
  for (int axis = 0; axis < T4A_CUDA_MAX_RANK; ++axis) {
    c[axis] = 0;
    if (axis < l->rank) {
      c[axis] = f % l->extents[axis];
      f /= l->extents[axis];
    }
  }
}

void t4a_oracle_broadcast_in_dim(void* out, const void* in, int dtype,
                                 const t4a_cuda_layout* ol, const t4a_cuda_layout* il,
                                 const long long* dims, int dims_rank, long long out_len) {
  const int es = t4a_oracle_dtype_size(dtype);
  if (es == 0) return;
  unsigned char* o = (unsigned char*)out;
  const unsigned char* s = (const unsigned char*)in;
  long long c[T4A_CUDA_MAX_RANK];
  for (long long f = 0; f < out_len; ++f) {
    coords_of(f, ol, c);
    long long index = il->offset;
    for (int i = 0; i < dims_rank; ++i) {
      const long long coordinate = il->extents[i] == 1 ? 0 : c[dims[i]];
      index += coordinate * il->strides[i];
    }
    memcpy(o + f * es, s + index * es, (size_t)es); /* the destination is compact */
  }
}

void t4a_oracle_concatenate_copy(void* out, const void* in, int dtype,
                                 const t4a_cuda_layout* ol, const t4a_cuda_layout* il, int axis,
                                 long long axis_offset, long long in_len) {
  const int es = t4a_oracle_dtype_size(dtype);
  if (es == 0) return;
  unsigned char* o = (unsigned char*)out;
  const unsigned char* s = (const unsigned char*)in;
  long long c[T4A_CUDA_MAX_RANK];
  for (long long f = 0; f < in_len; ++f) {
    coords_of(f, il, c);
    long long index = ol->offset;
    for (int k = 0; k < ol->rank; ++k) {
      const long long coordinate = k == axis ? c[k] + axis_offset : c[k];
      index += coordinate * ol->strides[k];
    }
    memcpy(o + index * es, s + f * es, (size_t)es); /* the source is compact */
  }
}

void t4a_oracle_tiled_transpose(void* dst, const void* src, int dtype, long long src_offset,
                                long long batch_stride, long long m, long long n,
                                long long batches) {
  const int es = t4a_oracle_dtype_size(dtype);
  if (es == 0) return;
  unsigned char* d = (unsigned char*)dst;
  const unsigned char* s = (const unsigned char*)src;
#pragma omp parallel for collapse(2) num_threads(g_threads) schedule(static)
  for (long long b = 0; b < batches; ++b) {
    for (long long i = 0; i < m; ++i) {
      for (long long j = 0; j < n; ++j) {
        const long long from = src_offset + b * batch_stride + i * n + j;
        const long long to = b * batch_stride + i + j * m;
        memcpy(d + to * es, s + from * es, (size_t)es);
      }
    }
  }
}

/* ---- element arithmetic (reference cuda/include/t4a/abi.cuh:590-818) ------- */

static inline uint32_t f32_bits(float v) { uint32_t u; memcpy(&u, &v, 4); return u; }
static inline float f32_from(uint32_t u) { float v; memcpy(&v, &u, 4); return v; }
static inline uint64_t f64_bits(double v) { uint64_t u; memcpy(&u, &v, 8); return u; }
static inline double f64_from(uint64_t u) { double v; memcpy(&v, &u, 8); return v; }

/* NaN-propagating extrema (abi.cuh:743-801): a NaN lhs wins, then a NaN rhs,
 * else the ordered extremum with -0 < +0 (tests/gpu_reduce.rs:2754-2776). Equal
 * operands differ at most in the sign of zero: max keeps +0 (AND of the bits),
 * min keeps -0 (OR of the bits). */
static inline float f32_max(float l, float r) {
  if (l != l) return l;
  if (r != r) return r;
  if (l == r) return f32_from(f32_bits(l) & f32_bits(r));
  return r > l ? r : l;
}
static inline float f32_min(float l, float r) {
  if (l != l) return l;
  if (r != r) return r;
  if (l == r) return f32_from(f32_bits(l) | f32_bits(r));
  return r < l ? r : l;
}
static inline double f64_max(double l, double r) {
  if (l != l) return l;
  if (r != r) return r;
  if (l == r) return f64_from(f64_bits(l) & f64_bits(r));
  return r > l ? r : l;
}
static inline double f64_min(double l, double r) {
  if (l != l) return l;
  if (r != r) return r;
  if (l == r) return f64_from(f64_bits(l) | f64_bits(r));
  return r < l ? r : l;
}

/* Complex product, componentwise form of abi.cuh:672-685, with the FMA
 * contraction the reference build applies to it (its device code is compiled
 * with contraction on; c-kernel-abi.md "Arithmetic semantics"):
 *   re = fma(a.re, b.re, -(a.im*b.im)),  im = fma(a.im, b.re, a.re*b.im).
 * The reference's golden vectors select this form: of the five candidates
 * (no contraction, or either product fused in each component) it is the only
 * one that reproduces all 18 complex PROD Random cases bit for bit. */
#define CMUL_BODY(FMA, T, a, b, out)                   \
  do {                                                 \
    const T p_ii = (a).im * (b).im;                    \
    const T p_ri = (a).re * (b).im;                    \
    (out).re = FMA((a).re, (b).re, -p_ii);             \
    (out).im = FMA((a).im, (b).re, p_ri);              \
  } while (0)

typedef t4a_cuda_c32 c32;
typedef t4a_cuda_c64 c64;

static inline c32 c32_mul(c32 a, c32 b) { c32 o; CMUL_BODY(fmaf, float, a, b, o); return o; }
static inline c64 c64_mul(c64 a, c64 b) { c64 o; CMUL_BODY(fma, double, a, b, o); return o; }
static inline c32 c32_add(c32 a, c32 b) { c32 o = {a.re + b.re, a.im + b.im}; return o; }
static inline c64 c64_add(c64 a, c64 b) { c64 o = {a.re + b.re, a.im + b.im}; return o; }

/* Wrapping integer arithmetic (abi.cuh:596-605, 654-663). */
static inline int32_t i32_add(int32_t a, int32_t b) { return (int32_t)((uint32_t)a + (uint32_t)b); }
static inline int32_t i32_mul(int32_t a, int32_t b) { return (int32_t)((uint32_t)a * (uint32_t)b); }
static inline int64_t i64_add(int64_t a, int64_t b) { return (int64_t)((uint64_t)a + (uint64_t)b); }
static inline int64_t i64_mul(int64_t a, int64_t b) { return (int64_t)((uint64_t)a * (uint64_t)b); }
static inline int32_t i32_max(int32_t a, int32_t b) { return a > b ? a : b; }
static inline int32_t i32_min(int32_t a, int32_t b) { return a < b ? a : b; }
static inline int64_t i64_max(int64_t a, int64_t b) { return a > b ? a : b; }
static inline int64_t i64_min(int64_t a, int64_t b) { return a < b ? a : b; }

static inline float f32_add(float a, float b) { return a + b; }
static inline float f32_mul(float a, float b) { return a * b; }
static inline double f64_add(double a, double b) { return a + b; }
static inline double f64_mul(double a, double b) { return a * b; }
/* Square rounded once, before any addition (abi.cuh:803-818). */
static inline float f32_sq(float v) { return fmaf(v, v, 0.0f); }
static inline double f64_sq(double v) { return fma(v, v, 0.0); }

/* Ops a type does not serve are refused before dispatch; these keep the
 * per-type templates total. */
#define NO_OP2(T, name) static inline T name(T a, T b) { (void)b; return a; }
#define NO_OP1(T, name) static inline T name(T a) { return a; }
NO_OP1(int32_t, i32_sq)
NO_OP1(int64_t, i64_sq)
NO_OP1(c32, c32_sq)
NO_OP1(c64, c64_sq)
NO_OP2(c32, c32_max)
NO_OP2(c32, c32_min)
NO_OP2(c64, c64_max)
NO_OP2(c64, c64_min)

/* ---- per-type fold objects and walks (reference cuda/src/reduce.cu) ------- */
/*
 * seed(v)       : v, or v*v for SUM_SQUARES                  (reduce.cu:25-108)
 * fold(acc, v)  : acc (+) v, or acc + v*v for SUM_SQUARES
 * combine(a, b) : a (+) b, a plain sum for SUM_SQUARES
 */
#define DEFINE_TYPE(T, P)                                                                  \
  static inline T P##_seed(int op, T v) {                                                  \
    return op == T4A_CUDA_REDUCE_SUM_SQUARES ? P##_sq(v) : v;                              \
  }                                                                                        \
  static inline T P##_fold(int op, T a, T v) {                                             \
    switch (op) {                                                                          \
      case T4A_CUDA_REDUCE_SUM: return P##_add(a, v);                                      \
      case T4A_CUDA_REDUCE_PROD: return P##_mul(a, v);                                     \
      case T4A_CUDA_REDUCE_SUM_SQUARES: return P##_add(a, P##_sq(v));                      \
      case T4A_CUDA_REDUCE_MAX: return P##_max(a, v);                                      \
      default: return P##_min(a, v);                                                       \
    }                                                                                      \
  }                                                                                        \
  static inline T P##_combine(int op, T a, T b) {                                          \
    return op == T4A_CUDA_REDUCE_SUM_SQUARES ? P##_add(a, b) : P##_fold(op, a, b);         \
  }                                                                                        \
  /* Lane 0 of the xor tree over `n` lanes (offsets 1, 2, 4, ... < n): each lane */        \
  /* combines its own value (left) with its partner's, so lane 0 holds the own-left */    \
  /* pairwise tree. Reference reduce.cu:148-157. */                                        \
  static T P##_tree(int op, const T* v, int n) {                                           \
    if (n == 1) return v[0];                                                               \
    const int h = n / 2;                                                                   \
    return P##_combine(op, P##_tree(op, v, h), P##_tree(op, v + h, h));                    \
  }                                                                                        \
  /* Plane fold of `width` lane values: the narrow xor tree, or for a block wider */       \
  /* than 32 the per-warp tree, then warp 0 folding the warp results with the xor */       \
  /* tree over `warps` lanes (reduce.cu:160-194). */                                       \
  static T P##_plane_fold(int op, const T* lanes, int width) {                             \
    if (width <= 32) return P##_tree(op, lanes, width);                                    \
    T warp_results[16];                                                                    \
    const int warps = width / 32;                                                          \
    for (int w = 0; w < warps; ++w) warp_results[w] = P##_tree(op, lanes + 32 * w, 32);    \
    return P##_tree(op, warp_results, warps);                                              \
  }                                                                                        \
  /* Unit body (reduce.cu:196-224): serial fold seeded from element 0. */                  \
  static T P##_unit(int op, const T* in, long long base, long long stride, long long len) {\
    T acc = P##_seed(op, in[base]);                                                        \
    for (long long i = 1; i < len; ++i) acc = P##_fold(op, acc, in[base + i * stride]);    \
    return acc;                                                                            \
  }                                                                                        \
  /* Plane body (reduce.cu:226-340): lane t seeds element t and folds t + kW in */         \
  /* order (the load-ahead batching moves loads only), then the plane fold. */             \
  static T P##_plane(int op, const T* in, long long base, long long stride, long long len, \
                     int width) {                                                          \
    T lanes[512];                                                                          \
    for (int t = 0; t < width; ++t) {                                                      \
      T acc = P##_seed(op, in[base + (long long)t * stride]);                              \
      for (long long i = t + width; i < len; i += width)                                   \
        acc = P##_fold(op, acc, in[base + i * stride]);                                    \
      lanes[t] = acc;                                                                      \
    }                                                                                      \
    return P##_plane_fold(op, lanes, width);                                               \
  }                                                                                        \
  /* Scalar pass-1 walk (reduce.cu:349-365). */                                            \
  static T P##_walk_scalar(int op, const T* in, long long base, long long stride,          \
                           long long start, long long end, int w, int lane) {              \
    long long r = start + lane;                                                            \
    T acc = P##_seed(op, in[base + r * stride]);                                           \
    for (r += w; r < end; r += w) acc = P##_fold(op, acc, in[base + r * stride]);          \
    return acc;                                                                            \
  }                                                                                        \
  /* Value of group g of the chunk: pairwise tree of its seeded elements */                \
  /* (reduce.cu:437-447). */                                                               \
  static inline T P##_group(int op, const T* chunk, long long g, int v) {                  \
    const T* x = chunk + g * v;                                                            \
    if (v == 4)                                                                            \
      return P##_combine(op, P##_combine(op, P##_seed(op, x[0]), P##_seed(op, x[1])),      \
                         P##_combine(op, P##_seed(op, x[2]), P##_seed(op, x[3])));         \
    return P##_combine(op, P##_seed(op, x[0]), P##_seed(op, x[1]));                        \
  }                                                                                        \
  /* Vector pass-1 walk (reduce.cu:449-525; c-kernel-abi.md:313-359). */                   \
  static T P##_walk_vector(int op, const T* chunk, long long len, int w, int lane, int v) {\
    const long long groups = len / v;                                                      \
    T acc = P##_group(op, chunk, lane, v);                                                 \
    for (int b = 1; b < 4; ++b)                                                            \
      if (lane + (long long)b * w < groups)                                                \
        acc = P##_combine(op, acc, P##_group(op, chunk, lane + (long long)b * w, v));      \
    long long index = lane + 4LL * w;                                                      \
    for (; index + 3LL * w < groups; index += 4LL * w) {                                   \
      const T lo = P##_combine(op, P##_group(op, chunk, index, v),                         \
                               P##_group(op, chunk, index + w, v));                        \
      const T hi = P##_combine(op, P##_group(op, chunk, index + 2LL * w, v),               \
                               P##_group(op, chunk, index + 3LL * w, v));                  \
      acc = P##_combine(op, acc, P##_combine(op, lo, hi));                                 \
    }                                                                                      \
    for (int b = 0; b < 3; ++b)                                                            \
      if (index + (long long)b * w < groups)                                               \
        acc = P##_combine(op, acc, P##_group(op, chunk, index + (long long)b * w, v));     \
    const long long tail_start = groups * v;                                               \
    if (lane < len - tail_start) acc = P##_fold(op, acc, chunk[tail_start + lane]);        \
    return acc;                                                                            \
  }

DEFINE_TYPE(float, f32)
DEFINE_TYPE(double, f64)
DEFINE_TYPE(int32_t, i32)
DEFINE_TYPE(int64_t, i64)
DEFINE_TYPE(c32, c32)
DEFINE_TYPE(c64, c64)

/* Whether an op serves a dtype (reference src/lib.rs:3096-3109). */
static int op_supports(int op, int dtype) {
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
      return 0;
  }
}

/* Input base and output offset of one keepdims output (reduce.cu:110-130). */
static void reduce_offsets(const t4a_cuda_layout* out, const t4a_cuda_layout* in, long long o,
                           long long* in_base, long long* out_offset) {
  long long rest = o, base = in->offset, offset = out->offset;
  for (int d = 0; d < out->rank; ++d) {
    const long long c = rest % out->extents[d];
    rest /= out->extents[d];
    base += c * in->strides[d];
    offset += c * out->strides[d];
  }
  *in_base = base;
  *out_offset = offset;
}

#define REDUCE_CASE(T, P)                                                                  \
  do {                                                                                     \
    const T* src = (const T*)in;                                                           \
    T* dst = (T*)out;                                                                      \
    _Pragma("omp parallel for num_threads(g_threads) schedule(static)")                    \
    for (long long o = 0; o < output_len; ++o) {                                           \
      long long base, off;                                                                 \
      reduce_offsets(out_layout, in_layout, o, &base, &off);                               \
      dst[off] = strategy == T4A_CUDA_REDUCE_PLANE                                         \
                     ? P##_plane(op, src, base, stride, len, block_width)                  \
                     : P##_unit(op, src, base, stride, len);                               \
    }                                                                                      \
  } while (0)

void t4a_oracle_reduce(void* out, const void* in, int dtype, int op, int strategy,
                       int block_width, const t4a_cuda_layout* out_layout,
                       const t4a_cuda_layout* in_layout, int axis, long long output_len) {
  if (!op_supports(op, dtype)) return;
  if (strategy == T4A_CUDA_REDUCE_PLANE && (block_width < 1 || block_width > 512)) return;
  const long long stride = in_layout->strides[axis];
  const long long len = in_layout->extents[axis];
  switch (dtype) {
    case T4A_CUDA_F32: REDUCE_CASE(float, f32); break;
    case T4A_CUDA_F64: REDUCE_CASE(double, f64); break;
    case T4A_CUDA_I32: REDUCE_CASE(int32_t, i32); break;
    case T4A_CUDA_I64: REDUCE_CASE(int64_t, i64); break;
    case T4A_CUDA_C32: REDUCE_CASE(c32, c32); break;
    case T4A_CUDA_C64: REDUCE_CASE(c64, c64); break;
    default: break;
  }
}

/* Pass 1 (reduce.cu:583-633): cube = output * splits + split; the output index
 * decodes over the non-axis dims of the partials layout; the chunk is
 * [split*chunk_len, end) with the last split absorbing the remainder. */
#define PARTIALS_CASE(T, P, VEC)                                                           \
  do {                                                                                     \
    const T* src = (const T*)in;                                                           \
    T* dst = (T*)partials;                                                                 \
    _Pragma("omp parallel for num_threads(g_threads) schedule(static)")                    \
    for (long long cube = 0; cube < output_len * splits; ++cube) {                         \
      T lanes[32];                                                                         \
      const long long o = cube / splits, split = cube % splits;                            \
      long long base = in_layout->offset, poff = partials_layout->offset, rest = o;        \
      for (int d = 0; d < partials_layout->rank; ++d) {                                    \
        if (d == axis) {                                                                   \
          poff += split * partials_layout->strides[d];                                     \
        } else {                                                                           \
          const long long c = rest % partials_layout->extents[d];                          \
          rest /= partials_layout->extents[d];                                             \
          base += c * in_layout->strides[d];                                               \
          poff += c * partials_layout->strides[d];                                         \
        }                                                                                  \
      }                                                                                    \
      const long long start = split * chunk_len;                                           \
      const long long end = split + 1 == splits ? axis_len : start + chunk_len;            \
      const int vector = (VEC) > 0 && op != T4A_CUDA_REDUCE_PROD && stride == 1 &&         \
                         (end - start) / ((VEC) > 0 ? (VEC) : 1) >= w;                     \
      for (int t = 0; t < w; ++t)                                                          \
        lanes[t] = vector ? P##_walk_vector(op, src + base + start, end - start, w, t, VEC)\
                          : P##_walk_scalar(op, src, base, stride, start, end, w, t);      \
      dst[poff] = P##_tree(op, lanes, w);                                                  \
    }                                                                                      \
  } while (0)

void t4a_oracle_reduce_partials(void* partials, const void* in, int dtype, int op,
                                int plane_width, const t4a_cuda_layout* partials_layout,
                                const t4a_cuda_layout* in_layout, int axis,
                                long long output_len, long long splits, long long chunk_len) {
  if (!op_supports(op, dtype)) return;
  if (plane_width != 8 && plane_width != 16 && plane_width != 32) return;
  const int w = plane_width;
  const long long stride = in_layout->strides[axis];
  const long long axis_len = in_layout->extents[axis];
  /* The vector walk serves 4- and 8-byte real and integer types with V = 16 /
   * element size; complex types keep the scalar walk (reduce.cu:367-390). */
  switch (dtype) {
    case T4A_CUDA_F32: PARTIALS_CASE(float, f32, 4); break;
    case T4A_CUDA_F64: PARTIALS_CASE(double, f64, 2); break;
    case T4A_CUDA_I32: PARTIALS_CASE(int32_t, i32, 4); break;
    case T4A_CUDA_I64: PARTIALS_CASE(int64_t, i64, 2); break;
    case T4A_CUDA_C32: PARTIALS_CASE(c32, c32, 0); break;
    case T4A_CUDA_C64: PARTIALS_CASE(c64, c64, 0); break;
    default: break;
  }
}

/* ---- f64 sequential reference (tests/gpu_reduce.rs:79-130) ---------------- */

static inline double d_max(double c, double v) {
  if (c != c) return c;
  if (v != v) return v;
  return f64_max(c, v);
}
static inline double d_min(double c, double v) {
  if (c != c) return c;
  if (v != v) return v;
  return f64_min(c, v);
}

static void load_f64(const void* in, int dtype, long long index, double* re, double* im) {
  *im = 0.0;
  switch (dtype) {
    case T4A_CUDA_F32: *re = ((const float*)in)[index]; break;
    case T4A_CUDA_F64: *re = ((const double*)in)[index]; break;
    case T4A_CUDA_I32: *re = (double)((const int32_t*)in)[index]; break;
    case T4A_CUDA_I64: *re = (double)((const int64_t*)in)[index]; break;
    case T4A_CUDA_C32:
      *re = ((const c32*)in)[index].re;
      *im = ((const c32*)in)[index].im;
      break;
    case T4A_CUDA_C64:
      *re = ((const c64*)in)[index].re;
      *im = ((const c64*)in)[index].im;
      break;
    default: *re = 0.0; break;
  }
}

void t4a_oracle_reduce_f64(double* out, const void* in, int dtype, int op,
                           const t4a_cuda_layout* in_layout, int axis, long long output_len) {
  const int complex = dtype == T4A_CUDA_C32 || dtype == T4A_CUDA_C64;
  const long long stride = in_layout->strides[axis];
  const long long len = in_layout->extents[axis];
  for (long long o = 0; o < output_len; ++o) {
    long long rest = o, base = in_layout->offset;
    for (int d = 0; d < in_layout->rank; ++d) {
      if (d == axis) continue;
      base += (rest % in_layout->extents[d]) * in_layout->strides[d];
      rest /= in_layout->extents[d];
    }
    double are = 0.0, aim = 0.0;
    for (long long i = 0; i < len; ++i) {
      double re, im;
      load_f64(in, dtype, base + i * stride, &re, &im);
      if (i == 0) {
        are = op == T4A_CUDA_REDUCE_SUM_SQUARES ? re * re : re;
        aim = im;
        continue;
      }
      switch (op) {
        case T4A_CUDA_REDUCE_SUM: are += re; aim += im; break;
        case T4A_CUDA_REDUCE_PROD: {
          const double r = are * re - aim * im, m = are * im + aim * re;
          are = r;
          aim = m;
          break;
        }
        case T4A_CUDA_REDUCE_SUM_SQUARES: are += re * re; break;
        case T4A_CUDA_REDUCE_MAX: are = d_max(are, re); break;
        default: are = d_min(are, re); break;
      }
    }
    if (complex) {
      out[2 * o] = are;
      out[2 * o + 1] = aim;
    } else {
      out[o] = are;
    }
  }
}

/* ---- digest (tests/gpu_reduce_golden.rs:66-73) ---------------------------- */

unsigned long long t4a_oracle_fnv1a64(const void* bytes, unsigned long long len) {
  const unsigned char* p = (const unsigned char*)bytes;
  unsigned long long hash = 0xcbf29ce484222325ULL;
  for (unsigned long long i = 0; i < len; ++i) {
    hash ^= p[i];
    hash *= 0x00000100000001b3ULL;
  }
  return hash;
}
