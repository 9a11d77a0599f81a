// gfx950 single-axis reductions, exported under the reference entry names and
// argument lists: t4a_cuda_reduce (unit and plane strategies, narrow and wide
// plane folds) and t4a_cuda_reduce_partials (pass 1 of a split reduction).
// Reference: cuda/src/reduce.cu:110-633, 765-852.
//
// Every kernel keeps the reference's numerical topology: a unit output folds
// its axis serially from element 0; a plane lane t seeds element t and folds
// t + W, t + 2W, ... in order, then the lanes meet in the own-left xor tree; a
// pass-1 plane takes the grouped 16-byte walk on a contiguous axis and the
// serial lane walk elsewhere (reference docs/abi/c-kernel-abi.md:313-359). So
// float results equal the reference kernels' bit for bit wherever IEEE rounding
// alone decides them.
//
// What is MI355X-specific is where the plane lanes live:
//   - a 32-lane plane is half of a 64-lane wavefront (two cubes per wavefront),
//     its xor tree a width-32 lane exchange;
//   - on a strided axis, pass 1 turns the plane sideways: a wavefront lane holds
//     one output column and all (COLUMNS) or a residue class (ROWS) of its
//     plane's 32 lanes in registers, so each wavefront load reads 64 adjacent
//     elements of one or more rows instead of 32 elements a row apart.
#include <hip/hip_runtime.h>

#include <mutex>
#include <type_traits>

#include "device.h"
#include "geometry.h"
#include "t4a/t4a.h"

namespace t4a {
// Launch status of the last kernel launch on this thread, and the status of a
// HIP runtime call's error (both record it for t4a_hip_last_error; movement.hip).
int status_of_last_launch();
int status_of_hip(int error);

namespace {

template <typename T>
struct VecLanes {
  static constexpr int value = 0;
};
template <>
struct VecLanes<float> {
  static constexpr int value = 4;
};
template <>
struct VecLanes<double> {
  static constexpr int value = 2;
};
template <>
struct VecLanes<int> {
  static constexpr int value = 4;
};
template <>
struct VecLanes<long long> {
  static constexpr int value = 2;
};

template <typename T, int V>
struct alignas(16) Group {
  T x[V];
};

// Input base and output offset of output `o` over the fused non-axis dims
// (reference reduce.cu:110-130); `o` < output_len, so the last dim needs no
// division.
// The loop runs over the fixed maximum rank so every field index is a
// compile-time constant: a runtime subscript would copy the by-value plan into
// per-lane scratch memory.
template <typename RD>
__device__ __forceinline__ void decode_output(const RD& rd, long long o, long long* in_base,
                                              long long* out_off) {
  long long ib = rd.in_offset;
  long long ob = rd.out_offset;
  // Quotients in 32 bits when every output index fits (rd.narrow: the extent
  // product is below 2^32); AMD GPUs have no integer divide, and a 64-bit one
  // costs several times a 32-bit one.
  const bool narrow = rd.narrow;
  unsigned int o32 = static_cast<unsigned int>(o);
  auto digit = [&](int k) {
    long long c;
    if (k + 1 == rd.n) {
      c = narrow ? static_cast<long long>(o32) : o;
    } else if (narrow) {
      const unsigned int e = static_cast<unsigned int>(rd.ext[k]);
      c = o32 % e;
      o32 /= e;
    } else {
      const long long e = rd.ext[k];
      c = o % e;
      o /= e;
    }
    ib += c * rd.is[k];
    ob += c * rd.os[k];
  };
  if constexpr (RD::kDims <= kMaxDims) {
#pragma unroll
    for (int k = 0; k < RD::kDims; ++k) {
      if (k >= rd.n) break;
      digit(k);
    }
  } else {
    // The general-rank dims live in LDS: a runtime subscript is an LDS read.
    for (int k = 0; k < rd.n; ++k) digit(k);
  }
  *in_base = ib;
  *out_off = ob;
}

// ---- t4a_cuda_reduce: UNIT ---------------------------------------------------------
// One thread per output, serial fold from element 0 (reference reduce.cu:196-224).
// On a contiguous axis whose every output starts 16-byte aligned, the elements
// arrive as 16-byte groups; the fold order is unchanged.
template <typename Fold, typename T, bool Vector, int BS, typename RD>
__device__ __forceinline__ void unit_outputs(T* __restrict__ out, const T* __restrict__ in,
                                             const RD& rd, long long output_len,
                                             Fold f, unsigned int blocks) {
  const long long len = rd.axis_len;
  const long long stride = rd.axis_stride;
  const int bs = block_threads<BS>();
  const long long gstride = static_cast<long long>(blocks) * bs;
  for (long long o = static_cast<long long>(blockIdx.x) * bs + threadIdx.x; o < output_len;
       o += gstride) {
    long long ib, ob;
    decode_output(rd, o, &ib, &ob);
    const T* x = in + ib;
    T acc;
    if constexpr (Vector) {
      constexpr int V = VecLanes<T>::value;
      // Short axes keep every load in registers: only in the small-output
      // instance (combine passes), whose occupancy does not matter; the
      // registers would cost a many-output reduction its occupancy.
      constexpr int kShort = 16;  // groups held at once on a short axis
      if (BS == kUnitSmallBlock && len <= kShort * V) {
        // A short axis (a combine pass over a few dozen partials): every load
        // is issued before the first fold, then the fold runs in order.
        const int groups = static_cast<int>(len / V);
        Group<T, V> g[kShort];
#pragma unroll
        for (int k = 0; k < kShort; ++k) {
          if (k < groups) g[k] = reinterpret_cast<const Group<T, V>*>(x)[k];
        }
        acc = f.seed(g[0].x[0]);
#pragma unroll
        for (int c = 1; c < V; ++c) acc = f.fold(acc, g[0].x[c]);
#pragma unroll
        for (int k = 1; k < kShort; ++k) {
          if (k < groups) {
#pragma unroll
            for (int c = 0; c < V; ++c) acc = f.fold(acc, g[k].x[c]);
          }
        }
        for (long long i = static_cast<long long>(groups) * V; i < len; ++i) acc = f.fold(acc, x[i]);
        out[ob] = acc;
        continue;
      }
      const Group<T, V> g0 = *reinterpret_cast<const Group<T, V>*>(x);
      acc = f.seed(g0.x[0]);
#pragma unroll
      for (int c = 1; c < V; ++c) acc = f.fold(acc, g0.x[c]);
      long long i = V;
      for (; i + V <= len; i += V) {
        const Group<T, V> g = *reinterpret_cast<const Group<T, V>*>(x + i);
#pragma unroll
        for (int c = 0; c < V; ++c) acc = f.fold(acc, g.x[c]);
      }
      for (; i < len; ++i) acc = f.fold(acc, x[i]);
    } else {
      constexpr int kShort = 32;  // elements held at once on a short axis
      if (BS == kUnitSmallBlock && len <= kShort) {
        T v[kShort];
#pragma unroll
        for (int k = 0; k < kShort; ++k) {
          if (k < len) v[k] = x[k * stride];
        }
        acc = f.seed(v[0]);
#pragma unroll
        for (int k = 1; k < kShort; ++k) {
          if (k < len) acc = f.fold(acc, v[k]);
        }
      } else {
        acc = f.seed(x[0]);
#pragma unroll 4
        for (long long i = 1; i < len; ++i) acc = f.fold(acc, x[i * stride]);
      }
    }
    out[ob] = acc;
  }
}

// UNIT over a one-group axis (unit_one_group) in kBlock blocks: each wavefront
// takes runs of 64 * U consecutive outputs (U = kUnitOutputsPerThread), lane l
// the outputs run + l + 64u, issues their 16-byte loads together, then folds
// each output serially from element 0.
template <typename Fold, typename T, typename RD>
__device__ __forceinline__ void unit_outputs_grouped(T* __restrict__ out,
                                                     const T* __restrict__ in,
                                                     const RD& rd, long long output_len,
                                                     Fold f, unsigned int blocks) {
  constexpr int V = VecLanes<T>::value;
  constexpr int U = kUnitOutputsPerThread;
  constexpr long long kRun = static_cast<long long>(kWave) * U;
  const long long len = rd.axis_len;
  const int lane = threadIdx.x % kWave;
  const long long wave = (static_cast<long long>(blockIdx.x) * kBlock + threadIdx.x) / kWave;
  const long long run_stride = static_cast<long long>(blocks) * (kBlock / kWave) * kRun;
  for (long long run = wave * kRun; run < output_len; run += run_stride) {
    Group<T, V> g[U];
    long long ob[U];
    const T* xs[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long o = run + lane + static_cast<long long>(kWave) * u;
      long long ib;
      decode_output(rd, o < output_len ? o : run, &ib, &ob[u]);  // past the end: the run's first
      xs[u] = in + ib;
      const Vec<T, V> x = nt_load<T, V>(xs[u]);
      __builtin_memcpy(&g[u], &x, sizeof(g[u]));
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (run + lane + static_cast<long long>(kWave) * u < output_len) {
        T acc = f.seed(g[u].x[0]);
#pragma unroll
        for (int c = 1; c < V; ++c) acc = f.fold(acc, g[u].x[c]);
        for (long long i = V; i < len; ++i) acc = f.fold(acc, xs[u][i]);
        nt_store<T, 1>(out + ob[u], Vec<T, 1>{{acc}});
      }
    }
  }
}

template <typename Fold, typename T, int BS, typename RD>
__device__ __forceinline__ void unit_body(void* out, const void* in, const RD& rd,
                                          long long output_len, Fold f, unsigned int blocks) {
  T* o = static_cast<T*>(out);
  const T* x = static_cast<const T*>(in);
  if constexpr (VecLanes<T>::value > 0) {
    constexpr int V = VecLanes<T>::value;
    bool vector = rd.axis_stride == 1 && rd.axis_len >= V && rd.in_offset % V == 0 &&
                  (reinterpret_cast<uintptr_t>(in) & 15) == 0;
    // Compile-time subscripts for a by-value plan (a runtime one would copy the
    // plan into per-lane scratch memory); the wide plans live in LDS.
    if constexpr (RD::kDims <= kMaxDims) {
#pragma unroll
      for (int k = 0; k < RD::kDims; ++k) {
        if (k < rd.n) vector = vector && rd.is[k] % V == 0;
      }
    } else {
      for (int k = 0; k < rd.n; ++k) vector = vector && rd.is[k] % V == 0;
    }
    if (vector) {
      if constexpr (BS == kBlock) {
        if (rd.axis_len < 2 * V) {
          unit_outputs_grouped<Fold, T>(o, x, rd, output_len, f, blocks);
          return;
        }
      }
      unit_outputs<Fold, T, true, BS>(o, x, rd, output_len, f, blocks);
      return;
    }
  }
  unit_outputs<Fold, T, false, BS>(o, x, rd, output_len, f, blocks);
}

// ---- t4a_cuda_reduce: UNIT on a compact plan ----------------------------------------
// The same folds as unit_outputs / unit_outputs_grouped with the output decode
// on a UnitPlan (32-bit quotients by precomputed divisors) and the fold fixed
// at compile time: the general ReduceDims decode over eight dims keeps too many
// scalar registers live for a kernel whose wavefronts are short-lived.
__device__ __forceinline__ void unit_decode(const UnitPlan& up, unsigned int o, long long* ib,
                                            long long* ob) {
  long long i = up.in_offset;
  long long w = up.out_offset;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    if (k < up.n) {
      unsigned int c = o;
      if (k + 1 < up.n) {
        const unsigned int q = div_by(o, up.ext[k]);
        c = o - q * up.ext[k].d;
        o = q;
      }
      i += static_cast<long long>(c) * up.is[k];
      w += static_cast<long long>(c) * up.os[k];
    }
  }
  *ib = i;
  *ob = w;
}

// The plane body's decode on a compact plan (output indices below 2^31).
__device__ __forceinline__ void decode_output(const UnitPlan& up, long long o, long long* ib,
                                              long long* ob) {
  unit_decode(up, static_cast<unsigned int>(o), ib, ob);
}

// UNIT over a one-group axis on a compact plan (kBlock threads a block): runs
// of 64 * U consecutive outputs a wavefront, lane l the outputs run + l + 64u
// (unit_outputs_grouped's walk with 32-bit indices; `blocks`, the grid's block
// count, is needed only past the first run).
// `Linear`: at most one fused output dim (output o at in_offset + o is[0] and
// out_offset + o os[0]), decoded with one multiply instead of the general
// decode's uniform branches, which otherwise stand between the wavefront's
// start and each of its loads (i32 product over a last axis of 4, 2^25 outputs:
// 110 us with the general decode, 106 us with this one).
template <typename Fold, typename T, bool Linear = false>
__device__ __forceinline__ void unit_group_lean(T* __restrict__ out, const T* __restrict__ in,
                                                const UnitPlan& up, unsigned int output_len,
                                                Fold f, unsigned int blocks) {
  constexpr int V = VecLanes<T>::value;
  constexpr int U = kUnitOutputsPerThread;
  constexpr unsigned int kRun = kWave * U;
  const int len = up.axis_len;
  const unsigned int lane = threadIdx.x % kWave;
  const unsigned int wave = (blockIdx.x * kBlock + threadIdx.x) / kWave;
  for (unsigned int run = wave * kRun; run < output_len;
       run += blocks * (kBlock / kWave) * kRun) {
    Group<T, V> g[U];
    long long ob[U];
    const T* xs[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const unsigned int o = run + lane + kWave * u;
      long long ib;
      if constexpr (Linear) {
        const long long oc = o < output_len ? o : run;
        ib = up.in_offset + (up.n > 0 ? oc * up.is[0] : 0);
        ob[u] = up.out_offset + (up.n > 0 ? oc * up.os[0] : 0);
      } else {
        unit_decode(up, o < output_len ? o : run, &ib, &ob[u]);
      }
      xs[u] = in + ib;
      const Vec<T, V> x = nt_load<T, V>(xs[u]);
      __builtin_memcpy(&g[u], &x, sizeof(g[u]));
    }
    // Both loads issue before the first fold waits on one.
    __builtin_amdgcn_sched_barrier(0);
    // Every fold (a lane past the end folds output `run`'s elements) before
    // any store: a store issued between two folds' loads would be waited on
    // with them, since the load counter counts stores too.
    T acc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      acc[u] = f.seed(g[u].x[0]);
#pragma unroll
      for (int c = 1; c < V; ++c) acc[u] = f.fold(acc[u], g[u].x[c]);
      for (int i = V; i < len; ++i) acc[u] = f.fold(acc[u], xs[u][i]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (run + lane + kWave * u < output_len) nt_store<T, 1>(out + ob[u], Vec<T, 1>{{acc[u]}});
  }
}

template <typename Fold, typename T, int BS>
__device__ __forceinline__ void unit_lean(T* __restrict__ out, const T* __restrict__ in,
                                          const UnitPlan& up, unsigned int output_len, Fold f) {
  const int len = up.axis_len;
  const unsigned int gstride = gridDim.x * BS;
  if constexpr (VecLanes<T>::value > 0) {
    constexpr int V = VecLanes<T>::value;
    if (up.vector) {
      if constexpr (BS == kBlock) {
        if (len < 2 * V) {
          unit_group_lean<Fold, T>(out, in, up, output_len, f, gridDim.x);
          return;
        }
      }
      for (unsigned int o = blockIdx.x * BS + threadIdx.x; o < output_len; o += gstride) {
        long long ib, ob;
        unit_decode(up, o, &ib, &ob);
        const T* x = in + ib;
        const Group<T, V>* g = reinterpret_cast<const Group<T, V>*>(x);
        const int groups = len / V;
        T acc;
        // A short axis: every load before the first fold (combine passes: up
        // to 16 groups; the large grids up to 8, e.g. 2^22 outputs over a
        // 16-element f32 axis, whose lanes otherwise wait on each group in
        // turn).
        constexpr int kShort = BS != kBlock ? 16 : 8;
        if (groups <= kShort) {
          Group<T, V> v[kShort];
#pragma unroll
          for (int k = 0; k < kShort; ++k) {
            if (k < groups) v[k] = g[k];
          }
          acc = f.seed(v[0].x[0]);
#pragma unroll
          for (int c = 1; c < V; ++c) acc = f.fold(acc, v[0].x[c]);
#pragma unroll
          for (int k = 1; k < kShort; ++k) {
            if (k < groups) {
#pragma unroll
              for (int c = 0; c < V; ++c) acc = f.fold(acc, v[k].x[c]);
            }
          }
        } else {
          const Group<T, V> g0 = g[0];
          acc = f.seed(g0.x[0]);
#pragma unroll
          for (int c = 1; c < V; ++c) acc = f.fold(acc, g0.x[c]);
          for (int k = 1; k < groups; ++k) {
            const Group<T, V> gk = g[k];
#pragma unroll
            for (int c = 0; c < V; ++c) acc = f.fold(acc, gk.x[c]);
          }
        }
        for (int i = groups * V; i < len; ++i) acc = f.fold(acc, x[i]);
        out[ob] = acc;
      }
      return;
    }
  }
  const long long stride = up.axis_stride;
  for (unsigned int o = blockIdx.x * BS + threadIdx.x; o < output_len; o += gstride) {
    long long ib, ob;
    unit_decode(up, o, &ib, &ob);
    const T* x = in + ib;
    T acc;
    // A short axis takes every load before the first fold: the combine passes
    // (up to 32 partials), and in the large grids up to 16 elements (the c64
    // [16]^6 sum over a stride-256 axis), whose wavefronts otherwise wait on
    // each group of four loads in turn.
    constexpr int kShort = BS != kBlock ? 32 : 16;
    if (len <= kShort) {
      T v[kShort];
#pragma unroll
      for (int k = 0; k < kShort; ++k) {
        // the large grids read their input once: streaming loads
        if (k < len) v[k] = BS == kBlock ? nt_load<T, 1>(x + k * stride).v[0] : x[k * stride];
      }
      acc = f.seed(v[0]);
#pragma unroll
      for (int k = 1; k < kShort; ++k) {
        if (k < len) acc = f.fold(acc, v[k]);
      }
    } else {
      acc = f.seed(x[0]);
#pragma unroll 4
      for (int i = 1; i < len; ++i) acc = f.fold(acc, x[i * stride]);
    }
    if constexpr (BS == kBlock)
      nt_store<T, 1>(out + ob, Vec<T, 1>{{acc}});
    else
      out[ob] = acc;
  }
}

// ---- t4a_cuda_reduce: PLANE --------------------------------------------------------
// One plane of W = blockDim.x lanes per output (reference reduce.cu:226-340).
// W <= 32: the xor tree. W = 64..512: the xor tree inside each 32-lane warp,
// warp results through LDS, then warp 0 folds them with the xor tree over the
// first W / 32 lanes (reference reduce.cu:170-194).
template <typename Fold, typename T, typename RD>
__device__ __forceinline__ void plane_body(void* out_ptr, const void* in_ptr, const RD& rd,
                                           long long output_len, Fold f, unsigned char* lds,
                                           unsigned int blocks) {
  T* out = static_cast<T*>(out_ptr);
  const T* in = static_cast<const T*>(in_ptr);
  T* warp_results = reinterpret_cast<T*>(lds);
  const int w = blockDim.x;
  const int lane = threadIdx.x;
  const long long len = rd.axis_len;
  const long long stride = rd.axis_stride;
  for (long long o = blockIdx.x; o < output_len; o += blocks) {
    long long ib, ob;
    decode_output(rd, o, &ib, &ob);
    const T* x = in + ib;
    T acc;
    // A plane holds len >= w elements. When a lane walks at most kAhead of them
    // (the combine passes: 8 partials a lane for 4096 splits at W = 512), every
    // load is issued before the first fold, one memory round trip per output.
    // kAhead holds 64 bytes of elements (16 f32, 8 f64 or c32, 4 c64): more
    // would set the register budget of every kernel that carries this body.
    constexpr int kAhead = sizeof(T) >= 16 ? 4 : sizeof(T) >= 8 ? 8 : 16;
    if (len <= static_cast<long long>(w) * kAhead) {
      T v[kAhead];
#pragma unroll
      for (int k = 0; k < kAhead; ++k) {
        const long long i = lane + static_cast<long long>(k) * w;
        if (i < len) v[k] = x[i * stride];
      }
      acc = f.seed(v[0]);
#pragma unroll
      for (int k = 1; k < kAhead; ++k) {
        if (lane + static_cast<long long>(k) * w < len) acc = f.fold(acc, v[k]);
      }
    } else {
      acc = f.seed(x[lane * stride]);
#pragma unroll 4
      for (long long i = lane + w; i < len; i += w) acc = f.fold(acc, x[i * stride]);
    }
    T reduced;
    if (w <= kWarp) {
      reduced = plane_tree(acc, w, f);
    } else {
      acc = plane_tree(acc, kWarp, f);
      const int warps = w / kWarp;
      const int wl = lane & (kWarp - 1);
      const int warp = lane / kWarp;
      if (wl == 0) warp_results[warp] = acc;
      __syncthreads();
      reduced = acc;
      if (warp == 0) {
        const T c = wl < warps ? warp_results[wl] : acc;
        reduced = plane_tree(c, warps, f);
      }
      __syncthreads();  // warp_results is reused by the next output
    }
    if (lane == 0) out[ob] = reduced;
  }
}

// PLANE with planes of W <= 32 lanes packed into 256-thread blocks (threadIdx.x
// the lane, threadIdx.y the plane; W-aligned lane groups, so the xor tree
// stays inside each plane): the launchers' geometry for the direct plane
// reductions of 33..511-element axes, where the reference geometry (one W-lane
// block per output, which the module entry keeps) leaves half of every
// wavefront idle and pays one block dispatch per output (2^20 outputs of a
// 64-element f32 axis: 687 us). When a lane holds at most kAhead / 4 elements
// of an output, plane q (= b * planes + p) takes runs of four consecutive
// outputs 4q + 4jS (S = gridDim.x * planes), every load of the four issued
// before the first fold; otherwise outputs q + jS one at a time. Each output is
// folded exactly as plane_body folds it: lane l seeds element l, folds l + W,
// l + 2W, ..., then the xor tree.
template <typename Fold, typename T>
__device__ __forceinline__ void plane_multi(T* __restrict__ out, const T* __restrict__ in,
                                            const UnitPlan& up, unsigned int output_len,
                                            Fold f) {
  const int w = blockDim.x;
  const int lane = threadIdx.x;
  const unsigned int span = gridDim.x * blockDim.y;
  const int len = up.axis_len;
  const long long stride = up.axis_stride;
  constexpr int kAhead = sizeof(T) >= 16 ? 4 : sizeof(T) >= 8 ? 8 : 16;
  constexpr int kQuarter = kAhead / 4;
  unsigned int o0 = blockIdx.x * blockDim.y + threadIdx.y;
  if (len <= w * kQuarter) {
    // Four consecutive outputs a plane at a time (neighbours in memory on a
    // contiguous axis), runs of four outputs S * 4 apart.
    for (unsigned int r = o0 * 4; r < output_len; r += 4 * span) {
      T v[4][kQuarter];
      long long ob[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const unsigned int o = r + u;
        long long ib;
        unit_decode(up, o < output_len ? o : r, &ib, &ob[u]);
        const T* x = in + ib;
#pragma unroll
        for (int k = 0; k < kQuarter; ++k) {
          const int i = lane + k * w;
          if (i < len) v[u][k] = x[i * stride];
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        T acc = f.seed(v[u][0]);
#pragma unroll
        for (int k = 1; k < kQuarter; ++k) {
          if (lane + k * w < len) acc = f.fold(acc, v[u][k]);
        }
        const T reduced = plane_tree(acc, w, f);
        if (lane == 0 && r + u < output_len) out[ob[u]] = reduced;
      }
    }
    return;
  }
  for (; o0 < output_len; o0 += span) {
    long long ib, ob;
    unit_decode(up, o0, &ib, &ob);
    const T* x = in + ib;
    T acc;
    if (len <= w * kAhead) {
      T v[kAhead];
#pragma unroll
      for (int k = 0; k < kAhead; ++k) {
        const int i = lane + k * w;
        if (i < len) v[k] = x[i * stride];
      }
      acc = f.seed(v[0]);
#pragma unroll
      for (int k = 1; k < kAhead; ++k) {
        if (lane + k * w < len) acc = f.fold(acc, v[k]);
      }
    } else {
      acc = f.seed(x[lane * stride]);
#pragma unroll 4
      for (long long i = lane + w; i < len; i += w) acc = f.fold(acc, x[i * stride]);
    }
    const T reduced = plane_tree(acc, w, f);
    if (lane == 0) out[ob] = reduced;
  }
}

// PLANE of W lanes computed by one thread per output: what lane 0 of that
// output's plane computes, bit for bit. Lane l folds elements l, l + W, l + 2W,
// ... (part[l]); the xor tree then leaves in lane 0 the balanced tree of
// part[0..W) in order (level s combines part[l] with part[l + s], lane 0's own
// value first: its partner lane l + s holds the same tree of its half). Threads
// take consecutive outputs, so on a strided axis every load instruction covers
// neighbouring elements (the planes' loads of one output each touch W lines).
template <typename Fold, typename T, int W>
__device__ __forceinline__ void plane_per_thread(T* __restrict__ out, const T* __restrict__ in,
                                                 const UnitPlan& up, unsigned int output_len,
                                                 Fold f) {
  const int len = up.axis_len;
  const long long stride = up.axis_stride;
  const unsigned int step = gridDim.x * blockDim.x;
  for (unsigned int o = blockIdx.x * blockDim.x + threadIdx.x; o < output_len; o += step) {
    long long ib, ob;
    unit_decode(up, o, &ib, &ob);
    const T* x = in + ib;
    T part[W];
#pragma unroll
    for (int l = 0; l < W; ++l) part[l] = f.seed(x[l * stride]);  // len >= W
    for (int base = W; base < len; base += W) {
#pragma unroll
      for (int l = 0; l < W; ++l) {
        if (base + l < len) part[l] = f.fold(part[l], x[(base + l) * stride]);
      }
    }
#pragma unroll
    for (int s = 1; s < W; s <<= 1) {
#pragma unroll
      for (int l = 0; l < W; l += 2 * s) part[l] = f.combine(part[l], part[l + s]);
    }
    out[ob] = part[0];
  }
}

// ---- t4a_cuda_reduce_partials -----------------------------------------------------

// Serial lane walk: lane t seeds start + t and folds start + t + kW (reference
// reduce.cu:349-365).
template <typename Fold, typename T>
__device__ __forceinline__ T walk_scalar(const T* __restrict__ in, long long ib,
                                         long long stride, long long start, long long end,
                                         int w, int lane, Fold f) {
  long long r = start + lane;
  T acc = f.seed(in[ib + r * stride]);
#pragma unroll 4
  for (r += w; r < end; r += w) acc = f.fold(acc, in[ib + r * stride]);
  return acc;
}

template <typename Fold, typename T, int V>
__device__ __forceinline__ T group_value(const Group<T, V>& g, Fold f) {
  if constexpr (V == 4) {
    return f.combine(f.combine(f.seed(g.x[0]), f.seed(g.x[1])),
                     f.combine(f.seed(g.x[2]), f.seed(g.x[3])));
  } else {
    return f.combine(f.seed(g.x[0]), f.seed(g.x[1]));
  }
}

template <typename T, int V, bool Aligned>
__device__ __forceinline__ Group<T, V> load_group(const T* chunk, long long g) {
  if constexpr (Aligned) {
    return reinterpret_cast<const Group<T, V>*>(chunk)[g];
  } else {
    Group<T, V> r;
#pragma unroll
    for (int c = 0; c < V; ++c) r.x[c] = chunk[g * V + c];
    return r;
  }
}

// Grouped walk of a contiguous chunk (reference reduce.cu:449-525, topology of
// c-kernel-abi.md:313-359): groups of V elements; lane t takes groups t, t+W,
// t+2W, ... in batches of four -- the first group seeds, the next three join one
// at a time, each later whole batch joins as (g0+g1)+(g2+g3), at most three
// leftovers join one at a time -- then lane t < len mod V folds tail element
// groups*V + t.
template <typename Fold, typename T, bool Aligned>
__device__ __forceinline__ T walk_vector(const T* __restrict__ chunk, long long len, int w,
                                         int lane, Fold f) {
  constexpr int V = VecLanes<T>::value;
  const long long groups = len / V;
  Group<T, V> b[4];
  b[0] = load_group<T, V, Aligned>(chunk, lane);
#pragma unroll
  for (int k = 1; k < 4; ++k) {
    if (lane + static_cast<long long>(k) * w < groups)
      b[k] = load_group<T, V, Aligned>(chunk, lane + static_cast<long long>(k) * w);
  }
  T acc = group_value<Fold, T, V>(b[0], f);
#pragma unroll
  for (int k = 1; k < 4; ++k) {
    if (lane + static_cast<long long>(k) * w < groups)
      acc = f.combine(acc, group_value<Fold, T, V>(b[k], f));
  }
  long long idx = lane + 4LL * w;
  for (; idx + 3LL * w < groups; idx += 4LL * w) {
#pragma unroll
    for (int k = 0; k < 4; ++k)
      b[k] = load_group<T, V, Aligned>(chunk, idx + static_cast<long long>(k) * w);
    const T lo = f.combine(group_value<Fold, T, V>(b[0], f), group_value<Fold, T, V>(b[1], f));
    const T hi = f.combine(group_value<Fold, T, V>(b[2], f), group_value<Fold, T, V>(b[3], f));
    acc = f.combine(acc, f.combine(lo, hi));
  }
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    if (idx + static_cast<long long>(k) * w < groups)
      b[k] = load_group<T, V, Aligned>(chunk, idx + static_cast<long long>(k) * w);
  }
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    if (idx + static_cast<long long>(k) * w < groups)
      acc = f.combine(acc, group_value<Fold, T, V>(b[k], f));
  }
  const long long tail = groups * V;
  if (lane < len - tail) acc = f.fold(acc, chunk[tail + lane]);
  return acc;
}

template <typename Fold, typename T>
__device__ __forceinline__ T pass1_walk(const T* __restrict__ in, long long ib, long long stride,
                                        long long start, long long end, int w, int lane,
                                        Fold f) {
  if constexpr (Fold::kRegroup && VecLanes<T>::value > 0) {
    constexpr int V = VecLanes<T>::value;
    // The stride is tested before a chunk pointer is formed: only a contiguous
    // axis makes in + ib + start an address inside the input.
    if (stride == 1 && (end - start) / V >= w) {
      const T* chunk = in + ib + start;
      if ((reinterpret_cast<uintptr_t>(chunk) & 15) == 0)
        return walk_vector<Fold, T, true>(chunk, end - start, w, lane, f);
      return walk_vector<Fold, T, false>(chunk, end - start, w, lane, f);
    }
  }
  return walk_scalar<Fold, T>(in, ib, stride, start, end, w, lane, f);
}

// Streaming PLANE mapping for a contiguous axis whose every chunk is 16-byte
// aligned and holds at least W groups (the host checks both): each 32-lane plane
// takes a run of consecutive cubes -- consecutive splits of one output, so
// consecutive memory -- and loads the next cube's first batch of groups before
// it folds the current one, so two cubes' loads are in flight per lane. Each
// cube's fold is exactly the grouped walk above; only load issue order changes.
template <typename Fold, typename T>
__device__ __forceinline__ void partials_stream(void* partials_ptr, const void* in_ptr,
                                                const PartialsPlan& pp, long long output_len,
                                                long long splits, long long chunk_len,
                                                long long per_plane, Fold f) {
  constexpr int V = VecLanes<T>::value;
  constexpr int W = kWarp;
  using G = Group<T, V>;
  T* partials = static_cast<T*>(partials_ptr);
  const T* in = static_cast<const T*>(in_ptr);
  const ReduceDims& rd = pp.dims;
  const int lane = threadIdx.x % W;
  const long long plane = (static_cast<long long>(blockIdx.x) * kBlock + threadIdx.x) / W;
  const long long cubes = output_len * splits;
  long long cube = plane * per_plane;
  const long long stop = cube + per_plane < cubes ? cube + per_plane : cubes;
  if (cube >= stop) return;
  // Incremental (output, split) walk: one division per run.
  long long o = cube / splits;
  long long split = cube - o * splits;
  long long ib, pb;
  decode_output(rd, o, &ib, &pb);
  const long long last_len = rd.axis_len - (splits - 1) * chunk_len;

  // First batch of a cube: groups lane + kW, k < 4, those below `groups`.
  auto first_batch = [&](const T* chunk, long long groups, G* b) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (k == 0 || lane + k * W < groups)
        b[k] = reinterpret_cast<const G*>(chunk)[lane + k * W];
    }
  };
  G cur[4];
  const T* chunk = in + ib + split * chunk_len;
  long long len = split + 1 == splits ? last_len : chunk_len;
  first_batch(chunk, len / V, cur);
  for (;;) {
    // Next cube's coordinates and first batch.
    long long n_split = split + 1, n_o = o, n_ib = ib, n_pb = pb;
    const bool more = cube + 1 < stop;
    G nxt[4];
    const T* n_chunk = chunk;
    long long n_len = 0;
    if (more) {
      if (n_split == splits) {
        n_split = 0;
        ++n_o;
        decode_output(rd, n_o, &n_ib, &n_pb);
      }
      n_chunk = in + n_ib + n_split * chunk_len;
      n_len = n_split + 1 == splits ? last_len : chunk_len;
      first_batch(n_chunk, n_len / V, nxt);
    }
    // Fold the current cube (reference reduce.cu:449-525 order).
    const long long groups = len / V;
    T acc = group_value<Fold, T, V>(cur[0], f);
#pragma unroll
    for (int k = 1; k < 4; ++k) {
      if (lane + k * W < groups) acc = f.combine(acc, group_value<Fold, T, V>(cur[k], f));
    }
    if (groups > 4 * W) {  // longer chunks: whole batches, then the partial batch
      long long idx = lane + 4LL * W;
      G b[4];
      for (; idx + 3LL * W < groups; idx += 4LL * W) {
#pragma unroll
        for (int k = 0; k < 4; ++k) b[k] = reinterpret_cast<const G*>(chunk)[idx + k * W];
        const T lo = f.combine(group_value<Fold, T, V>(b[0], f), group_value<Fold, T, V>(b[1], f));
        const T hi = f.combine(group_value<Fold, T, V>(b[2], f), group_value<Fold, T, V>(b[3], f));
        acc = f.combine(acc, f.combine(lo, hi));
      }
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        if (idx + k * W < groups) b[k] = reinterpret_cast<const G*>(chunk)[idx + k * W];
      }
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        if (idx + k * W < groups) acc = f.combine(acc, group_value<Fold, T, V>(b[k], f));
      }
    }
    const long long tail = groups * V;
    if (lane < len - tail) acc = f.fold(acc, chunk[tail + lane]);
    const T reduced = plane_tree(acc, W, f);
    if (lane == 0) partials[pb + split * rd.out_axis_stride] = reduced;
    if (!more) break;
    ++cube;
    split = n_split;
    o = n_o;
    ib = n_ib;
    pb = n_pb;
    chunk = n_chunk;
    len = n_len;
#pragma unroll
    for (int k = 0; k < 4; ++k) cur[k] = nxt[k];
  }
}

// One 32-lane plane's fold of its chunk (`len` elements from `chunk`; this
// thread is lane `lane`), for the LEAN mapping below: all K 16-byte groups of
// a lane loaded at once, non-temporally; the fold is the grouped walk's first
// batch -- the first group seeds, the others join one at a time -- then the
// tail element and the xor tree. A float Max / Min first folds in any order
// with the IEEE maximum / minimum and takes the exact order only when the
// plane's result is a NaN.
template <typename T, int K>
struct LeanShare {
  Group<T, VecLanes<T>::value> b[K];
  T t;  // the lane's tail element, if any (loaded with the groups)
};

// Every group load is unconditional -- a group past the chunk reloads group
// `lane` -- so no branch separates them and all are in flight before the first
// wait; the fold skips the stand-ins. The tail (len mod V elements, lanes below
// it) is loaded here only by planes whose chunk has one, usually none. With
// DeferTail the fold loads it instead: a plane holding several chunks would
// otherwise wait for each chunk's first group (the tail's default) before
// issuing the next chunk's loads.
template <typename T, int K, bool DeferTail = false>
__device__ __forceinline__ void lean_load(LeanShare<T, K>& s, const T* chunk, int len, int lane) {
  constexpr int V = VecLanes<T>::value;
  constexpr int W = kWarp;
  const int groups = len / V;
  const int tail = groups * V;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int g = k == 0 || lane + k * W < groups ? lane + k * W : lane;
    const Vec<T, V> x = nt_load<T, V>(chunk + g * V);
    __builtin_memcpy(&s.b[k], &x, sizeof(s.b[k]));
  }
  if constexpr (!DeferTail) {
    s.t = s.b[0].x[0];
    if (len != tail && lane < len - tail) s.t = chunk[tail + lane];
  }
}

template <typename Fold, typename T, int K, bool DeferTail = false>
__device__ __forceinline__ T lean_fold(LeanShare<T, K>& s, const T* chunk, int len, int lane,
                                       Fold f) {
  constexpr int V = VecLanes<T>::value;
  constexpr int W = kWarp;
  const int groups = len / V;
  const bool has_tail = lane < len - groups * V;
  if constexpr (DeferTail) {
    s.t = s.b[0].x[0];
    if (has_tail) s.t = chunk[groups * V + lane];
  }
  auto exact = [&]() {
    T acc = group_value<Fold, T, V>(s.b[0], f);
#pragma unroll
    for (int k = 1; k < K; ++k) {
      if (lane + k * W < groups) acc = f.combine(acc, group_value<Fold, T, V>(s.b[k], f));
    }
    if (has_tail) acc = f.fold(acc, s.t);
    return plane_tree32(acc, f);
  };
  using Fast = typename AnyOrder<Fold, T>::type;
  if constexpr (!std::is_void_v<Fast>) {
    // Without a NaN any order gives the exact result. The stand-in loads
    // repeat group `lane` and element 0 of the chunk (already among the lane's
    // elements or the plane's), which an extremum ignores.
    const Fast g;
    T acc = s.t;
#pragma unroll
    for (int k = 0; k < K; ++k) {
#pragma unroll
      for (int c = 0; c < V; ++c) acc = g.combine(acc, s.b[k].x[c]);
    }
    const T reduced = plane_tree32(acc, g);
    return reduced != reduced ? exact() : reduced;
  } else {
    return exact();
  }
}

template <typename Fold, typename T, int K>
__device__ __forceinline__ T lean_chunk(const T* chunk, int len, int lane, Fold f) {
  LeanShare<T, K> s;
  lean_load(s, chunk, len, lane);
  return lean_fold<Fold, T, K>(s, chunk, len, lane, f);
}

// LEAN plane mapping for a contiguous axis whose every chunk (the longer last
// one included) holds at most K * 32 groups, so each lane's whole share is the
// walk's first batch: one cube per 32-lane plane, consecutive planes on
// consecutive cubes (consecutive memory on an inner axis). Few registers keep
// eight wavefronts per SIMD in flight, which is what feeds HBM on this part.
template <typename Fold, typename T, int K, bool Linear>
__device__ __forceinline__ void partials_lean(void* partials_ptr, const void* in_ptr,
                                              const LeanPlan& lp, Fold f) {
  const unsigned int cubes = lp.cubes;
  constexpr int W = kWarp;
  // The block size is the launcher's constant kBlock: reading blockDim would
  // cost every wavefront a memory round trip (it is an implicit kernel argument
  // fetched by a vector load) before its first data load is issued.
  constexpr int kPlanes = kBlock / W;
  T* partials = static_cast<T*>(partials_ptr);
  const T* in = static_cast<const T*>(in_ptr);
  const int lane = threadIdx.x % W;
  // 32-bit cube indices: the planner bounds the cube count below 2^31. The
  // planned grid gives each plane one cube; the stride over the grid (which
  // reads gridDim) comes only after it.
  unsigned int cube = blockIdx.x * kPlanes + threadIdx.x / W;
  // The plan's fields are made operands of an empty asm statement ahead of the
  // exit test: otherwise the compiler sinks their loads past the branch on the
  // cube count, a second scalar round trip before the first data load.
  asm volatile("" ::"s"(lp.in_offset), "s"(lp.chunk_len), "s"(lp.out_offset),
               "s"(lp.out_axis_stride), "s"(in), "s"(partials));
  if (cube >= cubes) return;
  for (;; cube += gridDim.x * kPlanes) {
    if (cube >= cubes) break;
    const T* chunk;
    long long pidx;
    int len;
    unsigned int split = 0;
    if constexpr (Linear) {
      chunk = in + lp.in_offset + static_cast<long long>(cube) * lp.chunk_len;
      pidx = lp.out_offset + static_cast<long long>(cube) * lp.out_axis_stride;
      len = static_cast<int>(lp.chunk_len);
    } else {
      // cube = o * splits + split; o over the fused dims, first dim fastest.
      unsigned int o = div_by(cube, lp.splits);
      split = cube - o * lp.splits.d;
      long long ib = lp.in_offset;
      long long pb = lp.out_offset;
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        if (k < lp.n) {
          unsigned int c = o;
          if (k + 1 < lp.n) {
            const unsigned int q = div_by(o, lp.ext[k]);
            c = o - q * lp.ext[k].d;
            o = q;
          }
          ib += static_cast<long long>(c) * lp.is[k];
          pb += static_cast<long long>(c) * lp.os[k];
        }
      }
      chunk = in + ib + static_cast<long long>(split) * lp.chunk_len;
      pidx = pb + static_cast<long long>(split) * lp.out_axis_stride;
      len = split + 1 == lp.splits.d ? lp.last_len : static_cast<int>(lp.chunk_len);
    }
    const T reduced = lean_chunk<Fold, T, K>(chunk, len, lane, f);
    if (lane == 0) partials[pidx] = reduced;
  }
}

// Cube `cube` of a LeanPlan: its chunk, its partial's offset and its length
// (cube = o * splits + split, o over the fused dims, first dim fastest).
template <typename T>
__device__ __forceinline__ void lean_cube(const LeanPlan& lp, const T* in, unsigned int cube,
                                          const T** chunk, long long* pidx, int* len) {
  unsigned int o = div_by(cube, lp.splits);
  const unsigned int split = cube - o * lp.splits.d;
  long long ib = lp.in_offset;
  long long pb = lp.out_offset;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    if (k < lp.n) {
      unsigned int c = o;
      if (k + 1 < lp.n) {
        const unsigned int q = div_by(o, lp.ext[k]);
        c = o - q * lp.ext[k].d;
        o = q;
      }
      ib += static_cast<long long>(c) * lp.is[k];
      pb += static_cast<long long>(c) * lp.os[k];
    }
  }
  *chunk = in + ib + static_cast<long long>(split) * lp.chunk_len;
  *pidx = pb + static_cast<long long>(split) * lp.out_axis_stride;
  *len = split + 1 == lp.splits.d ? lp.last_len : static_cast<int>(lp.chunk_len);
}

// LEAN inside the reduce_partials entry, for the caller's block shape: a
// block of 32-lane planes (blockDim.x / 32 of them), the working blocks'
// planes striding over the cubes. Under the reference's geometry a block is
// often one 32-lane plane, and few blocks work (the rest return): each plane
// issues the loads of C cubes before it folds the first, so that it keeps
// C chunks in flight instead of one. Each cube folds as partials_lean folds it.
template <typename Fold, typename T, int K, int C>
__device__ __forceinline__ void partials_lean_entry(void* partials_ptr, const void* in_ptr,
                                                    const LeanPlan& lp, Fold f,
                                                    unsigned int blocks) {
  constexpr int W = kWarp;
  T* partials = static_cast<T*>(partials_ptr);
  const T* in = static_cast<const T*>(in_ptr);
  const unsigned int planes = blockDim.x / W;
  const int lane = threadIdx.x % W;
  const unsigned int stride = blocks * planes;
  const unsigned int cubes = lp.cubes;
  // Below 2^31 cubes (the lean plan's bound) and at most 2^24 planes, base +
  // C * stride stays below 2^32.
  for (unsigned int base = blockIdx.x * planes + threadIdx.x / W; base < cubes;
       base += C * stride) {
    LeanShare<T, K> sh[C];
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const unsigned int cube = base + c * stride < cubes ? base + c * stride : base;
      const T* chunk;
      long long pidx;
      int len;
      lean_cube(lp, in, cube, &chunk, &pidx, &len);
      lean_load<T, K, true>(sh[c], chunk, len, lane);
    }
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const unsigned int cube = base + c * stride;
      if (cube < cubes) {
        const T* chunk;
        long long pidx;
        int len;
        lean_cube(lp, in, cube, &chunk, &pidx, &len);
        const T reduced = lean_fold<Fold, T, K, true>(sh[c], chunk, len, lane, f);
        if (lane == 0) partials[pidx] = reduced;
      }
    }
  }
}

// Where a joined reduction writes its finals: output o at offset + o * stride
// of `out`; each block holds `outputs` whole outputs (their splits' chunks).
struct JoinedOut {
  void* out;
  long long offset;
  long long stride;
  unsigned int outputs;
};

// Pass 1 and the unit combine in one launch, for a linear LEAN plan of at most
// 8 * C splits: a block's eight 32-lane planes fold the chunks of its outputs,
// plane p the block's chunks p, p + 8, ... (up to C of them, every load issued
// before the first fold), each chunk as partials_lean folds it, and write the
// partials; then one thread per output folds that output's partials from LDS
// serially from split 0, the reference's unit walk (reduce.cu:196-224) -- the
// two launches' bits, with no memory traffic or ordering between blocks.
template <typename Fold, typename CFold, typename T, int K, int C>
__device__ __forceinline__ void reduction_joined(void* partials_ptr, const void* in_ptr,
                                                 const LeanPlan& lp, const JoinedOut& jo,
                                                 Fold f) {
  constexpr int W = kWarp;
  constexpr int kPlanes = kBlock / W;
  __shared__ T joined[kPlanes * C];
  T* partials = static_cast<T*>(partials_ptr);
  const T* in = static_cast<const T*>(in_ptr);
  const int lane = threadIdx.x % W;
  const unsigned int plane = threadIdx.x / W;
  const unsigned int splits = lp.splits.d;
  const unsigned int per_block = jo.outputs * splits;
  // The launcher's grid holds no block without an output: `first` is a chunk.
  const unsigned int first = blockIdx.x * per_block;
  const int len = static_cast<int>(lp.chunk_len);
  asm volatile("" ::"s"(lp.in_offset), "s"(lp.chunk_len), "s"(in));
  LeanShare<T, K> s[C];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const unsigned int q = plane + c * kPlanes;
    // A slot without a chunk reloads the block's first chunk (a stand-in).
    const unsigned int cube = q < per_block && first + q < lp.cubes ? first + q : first;
    lean_load<T, K, true>(s[c], in + lp.in_offset + static_cast<long long>(cube) * lp.chunk_len,
                          len, lane);
  }
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const unsigned int q = plane + c * kPlanes;
    const unsigned int cube = q < per_block && first + q < lp.cubes ? first + q : first;
    const T reduced = lean_fold<Fold, T, K, true>(
        s[c], in + lp.in_offset + static_cast<long long>(cube) * lp.chunk_len, len, lane, f);
    if (lane == 0 && q < per_block && first + q < lp.cubes) {
      partials[lp.out_offset + static_cast<long long>(first + q) * lp.out_axis_stride] = reduced;
      joined[q] = reduced;
    }
  }
  __syncthreads();
  const unsigned int o = blockIdx.x * jo.outputs + threadIdx.x;
  if (threadIdx.x < jo.outputs && o * splits < lp.cubes) {
    const T* p = joined + threadIdx.x * splits;
    const CFold cf{};
    T acc = cf.seed(p[0]);
    for (unsigned int k = 1; k < splits; ++k) acc = cf.fold(acc, p[k]);
    static_cast<T*>(jo.out)[jo.offset + static_cast<long long>(o) * jo.stride] = acc;
  }
}

// PLANE mapping: plane = W lanes (W = blockDim.x when blockDim.x <= 32, else 32
// with blockDim.x / 32 planes per block, reference reduce.cu:557-581); planes
// stride over the cubes.
template <typename Fold, typename T, typename RD>
__device__ __forceinline__ void partials_planes_dims(void* partials_ptr, const void* in_ptr,
                                                     const RD& rd, long long output_len,
                                                     long long splits, long long chunk_len,
                                                     Fold f, unsigned int blocks) {
  T* partials = static_cast<T*>(partials_ptr);
  const T* in = static_cast<const T*>(in_ptr);
  const int w = blockDim.x <= static_cast<unsigned>(kWarp) ? static_cast<int>(blockDim.x) : kWarp;
  const int planes = static_cast<int>(blockDim.x) / w;
  const int lane = static_cast<int>(threadIdx.x) % w;
  const long long cubes = output_len * splits;
  // Which cube a plane takes (never what it computes): on a contiguous axis
  // neighbouring planes take neighbouring chunks of one output, which stream
  // one run; on a strided axis they take neighbouring outputs of one split,
  // so a block's planes read neighbouring columns of the same rows.
  const bool split_major = rd.axis_stride != 1;
  for (long long idx = static_cast<long long>(blockIdx.x) * planes + threadIdx.x / w;
       idx < cubes; idx += static_cast<long long>(blocks) * planes) {
    // In the entries the dims live in LDS: without this, their loads are
    // hoisted out of the loop and held in vector registers for all of it
    // (about 50 of them, enough to cost the entry kernel an occupancy step).
    asm volatile("" ::: "memory");
    long long o, split;
    if (split_major) {
      split = idx / output_len;
      o = idx - split * output_len;
    } else {
      o = idx / splits;
      split = idx - o * splits;
    }
    long long ib, pb;
    decode_output(rd, o, &ib, &pb);
    pb += split * rd.out_axis_stride;
    const long long start = split * chunk_len;
    const long long end = split + 1 == splits ? rd.axis_len : start + chunk_len;
    const T acc = pass1_walk<Fold, T>(in, ib, rd.axis_stride, start, end, w, lane, f);
    const T reduced = plane_tree(acc, w, f);
    if (lane == 0) partials[pb] = reduced;
  }
}

template <typename Fold, typename T>
__device__ __forceinline__ void partials_planes(void* partials_ptr, const void* in_ptr,
                                                const PartialsPlan& pp, long long output_len,
                                                long long splits, long long chunk_len, Fold f,
                                                unsigned int blocks) {
  partials_planes_dims<Fold, T>(partials_ptr, in_ptr, pp.dims, output_len, splits, chunk_len,
                                f, blocks);
}

// Unit `u` of the COLUMNS/ROWS mappings: column block fastest, then the split,
// then the other non-axis coordinates -- neighbouring wavefronts read
// neighbouring columns of the same rows, or the next chunk of the same columns.
__device__ __forceinline__ void decode_unit(const PartialsPlan& pp, long long u, long long col,
                                            long long* ib, long long* pb, long long* split,
                                            long long splits) {
  const ReduceDims& rd = pp.dims;
  // Every quantity here is below the unit count, which the planner keeps
  // below 2^31: 32-bit quotients.
  const unsigned int rest = static_cast<unsigned int>(u) / static_cast<unsigned int>(pp.col_blocks);
  *split = rest % static_cast<unsigned int>(splits);
  unsigned int other = rest / static_cast<unsigned int>(splits);
  long long in_base = rd.in_offset;
  long long p_base = rd.out_offset + *split * rd.out_axis_stride;
#pragma unroll
  for (int k = 0; k < kMaxDims; ++k) {
    if (k >= rd.n) break;
    long long c;
    if (k == pp.col_dim) {
      c = col;
    } else {
      const unsigned int e = static_cast<unsigned int>(rd.ext[k]);
      c = other % e;
      other /= e;
    }
    in_base += c * rd.is[k];
    p_base += c * rd.os[k];
  }
  *ib = in_base;
  *pb = p_base;
}

// Load `N` adjacent elements (N = 1, 2 or 4; aligned to N elements) as one
// non-temporal access.
template <typename T, int N>
__device__ __forceinline__ Vec<T, N> load_n(const T* p) {
  return nt_load<T, N>(p);
}

// One plane lane's serial walk over rows q0, q0 + 32, ... below `len` of its
// chunk (q0 < len), each row N adjacent elements, folded in that order into
// `acc` (seeded from row q0); eight loads are issued per step. Row q0 of this
// lane sits at `base + lane_off` bytes and row q0 + 32k `k * step` bytes on;
// where the caller makes `base` and `step` the same for the whole wavefront,
// every load takes the scalar-base addressing form.
template <int N, typename Fold, typename T>
__device__ __forceinline__ void fold_lane_rows(const char* base, long long step,
                                               long long lane_off, int q0, int len, Fold f,
                                               T* acc) {
  constexpr int kStep = 8;
  auto at = [&](int k) {
    return reinterpret_cast<const T*>(base + k * step + lane_off);
  };
  // Unconditional loads (a row past the chunk reloads row q0) keep every
  // load of a step in flight before the first wait.
  Vec<T, N> v[kStep];
#pragma unroll
  for (int k = 0; k < kStep; ++k) v[k] = load_n<T, N>(at(k == 0 || q0 + k * kWarp < len ? k : 0));
#pragma unroll
  for (int c = 0; c < N; ++c) acc[c] = f.seed(v[0].v[c]);
#pragma unroll
  for (int k = 1; k < kStep; ++k) {
    if (q0 + k * kWarp < len) {
#pragma unroll
      for (int c = 0; c < N; ++c) acc[c] = f.fold(acc[c], v[k].v[c]);
    }
  }
  for (int b = kStep; q0 + b * kWarp < len; b += kStep) {
#pragma unroll
    for (int k = 0; k < kStep; ++k) v[k] = load_n<T, N>(at(q0 + (b + k) * kWarp < len ? b + k : 0));
#pragma unroll
    for (int k = 0; k < kStep; ++k) {
      if (q0 + (b + k) * kWarp < len) {
#pragma unroll
        for (int c = 0; c < N; ++c) acc[c] = f.fold(acc[c], v[k].v[c]);
      }
    }
  }
}

// Unit u = (column block, split, other) of a SidePlan: input element offset of
// the block's first column at the split's first row, partials offset of that
// column's partial, and the split's length.
__device__ __forceinline__ void side_unit(const SidePlan& sp, unsigned int u,
                                          unsigned int* block, long long* ib, long long* pb,
                                          int* len) {
  const unsigned int rest = div_by(u, sp.col_blocks);
  *block = u - rest * sp.col_blocks.d;
  unsigned int other = div_by(rest, sp.splits);
  const unsigned int split = rest - other * sp.splits.d;
  long long in_base = sp.in_offset + static_cast<long long>(split) * sp.chunk_len * sp.axis_stride;
  long long p_base = sp.out_offset + static_cast<long long>(split) * sp.out_axis_stride;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    if (k < sp.n_other) {
      unsigned int c = other;
      if (k + 1 < sp.n_other) {
        const unsigned int q = div_by(other, sp.ext[k]);
        c = other - q * sp.ext[k].d;
        other = q;
      }
      in_base += static_cast<long long>(c) * sp.is[k];
      p_base += static_cast<long long>(c) * sp.os[k];
    }
  }
  *ib = in_base;
  *pb = p_base;
  *len = split + 1 == sp.splits.d ? sp.last_len : sp.chunk_len;
}

// TILES: a block of NW wavefronts of WL lanes per unit (column block, split,
// other): four of 64 in the launchers; one, two or four in the entries, whose
// geometry the caller sets (one wavefront of 32 lanes for the reference's
// 32-thread blocks). Lane t holds columns col0 .. col0 + CPL - 1 and wavefront
// w the plane lanes l = (32 / NW) w .. (32 / NW)(w + 1) - 1 of those columns'
// cubes; plane lane l folds rows start + l + 32k in k order. A wavefront joins
// its plane lanes with the pairwise tree as they finish (a binary counter over
// l), and the NW subtree values meet through LDS as ((w0 + w1) + (w2 + w3)):
// together, the plane's own-left xor tree.
template <typename Fold, typename T, int CPL, int NW = kBlock / kWave, int WL = kWave>
__device__ __forceinline__ void partials_tiles(void* partials_ptr, const void* in_ptr,
                                               const SidePlan& sp, Fold f, T* lds, int* redo,
                                               unsigned int blocks) {
  static_assert(NW == 1 || NW == 2 || NW == 4, "one, two or four wavefronts");
  static_assert(WL == kWave || (WL == kWarp && NW == 1), "64-lane wavefronts or one of 32");
  constexpr int kLanesPerWave = kWarp / NW;  // plane lanes per wavefront: 32, 16 or 8
  constexpr int kLevels = NW == 1 ? 5 : NW == 2 ? 4 : 3;
  constexpr int BC = WL * CPL;  // columns per block
  T* partials = static_cast<T*>(partials_ptr);
  const char* in = static_cast<const char*>(in_ptr);
  // The wavefront index, explicitly uniform: the compiler cannot tell that
  // threadIdx.x / 64 is, and would otherwise turn every row test below into a
  // divergent branch.
  const int w = NW == 1 ? 0 : __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int t = threadIdx.x % WL;
  const long long row_bytes = sp.axis_stride * static_cast<long long>(sizeof(T));
  const long long lane_off = static_cast<long long>(t) * CPL * static_cast<long long>(sizeof(T));
  for (long long u = blockIdx.x; u < sp.units; u += blocks) {
    unsigned int block;
    long long ib, pb;
    int len;
    side_unit(sp, static_cast<unsigned int>(u), &block, &ib, &pb, &len);
    const long long block_col = static_cast<long long>(block) * BC;
    const bool active = block_col + t * CPL < sp.columns;  // CPL divides the column count
    // the block's first column at row 0 of the split, uniform across the block
    const char* rows = in + (ib + block_col) * static_cast<long long>(sizeof(T));
    // One pass of the unit under fold g: each wavefront's subtree (into LDS
    // when there are several), then wavefront 0's columns meet in r.
    auto pass = [&](auto g, T* r) {
      T level[kLevels][CPL];
      T sub[CPL];
      // Two plane lanes per step keep two lanes' loads in flight; the tree's
      // climb is a uniform branch on the lane index.
#pragma unroll 2
      for (int a = 0; a < kLanesPerWave; ++a) {
        T acc[CPL];
        const int q0 = w * kLanesPerWave + a;
        if (active) {
          fold_lane_rows<CPL>(rows + q0 * row_bytes, kWarp * row_bytes, lane_off, q0, len, g,
                              acc);
        } else {
#pragma unroll
          for (int c = 0; c < CPL; ++c) acc[c] = T{};
        }
        // Binary counter: lane a's value climbs while a ends in ones; the
        // last lane (all ones) carries the wavefront's whole subtree.
        bool parked = false;
#pragma unroll
        for (int lv = 0; lv < kLevels; ++lv) {
          if (!parked) {
            if (((a >> lv) & 1) == 0) {
#pragma unroll
              for (int c = 0; c < CPL; ++c) level[lv][c] = acc[c];
              parked = true;
            } else {
#pragma unroll
              for (int c = 0; c < CPL; ++c) acc[c] = g.combine(level[lv][c], acc[c]);
            }
          }
        }
        if (!parked) {
#pragma unroll
          for (int c = 0; c < CPL; ++c) sub[c] = acc[c];
        }
      }
      if constexpr (NW == 1) {
#pragma unroll
        for (int c = 0; c < CPL; ++c) r[c] = sub[c];
      } else {
#pragma unroll
        for (int c = 0; c < CPL; ++c) lds[w * BC + t * CPL + c] = sub[c];
        __syncthreads();
        if (w == 0 && active) {
#pragma unroll
          for (int c = 0; c < CPL; ++c) {
            const int i = t * CPL + c;
            if constexpr (NW == 2)
              r[c] = g.combine(lds[i], lds[BC + i]);
            else
              r[c] = g.combine(g.combine(lds[i], lds[BC + i]),
                               g.combine(lds[2 * BC + i], lds[3 * BC + i]));
          }
        }
      }
    };
    T r[CPL];
    using Fast = typename AnyOrder<Fold, T>::type;
    if constexpr (!std::is_void_v<Fast> && sizeof(T) == 4) {
      // An f32 Max / Min folds in any order with the IEEE maximum / minimum;
      // when a column's result is a NaN the block redoes the unit in the
      // exact order (wavefront 0 raises the flag, the whole block sees it).
      // Not for f64: the second pass's registers cost the kernel occupancy.
      pass(Fast{}, r);
      bool nan = false;
      if (w == 0 && active) {
#pragma unroll
        for (int c = 0; c < CPL; ++c) nan = nan || r[c] != r[c];
      }
      if (threadIdx.x == 0) *redo = 0;
      __syncthreads();
      if (nan) *redo = 1;
      __syncthreads();
      if (*redo) {
        pass(f, r);
      }
    } else {
      pass(f, r);
    }
    if (w == 0 && active) {
#pragma unroll
      for (int c = 0; c < CPL; ++c) partials[pb + (block_col + t * CPL + c) * sp.col_os] = r[c];
    }
    __syncthreads();  // the LDS tile is reused by the block's next unit
  }
}

// VECROWS: rows of C contiguous elements (8 or 16 bytes). A 32-lane plane takes
// unit u = (split, other), i.e. the cubes of all C columns; plane lane l loads
// whole rows start + l + 32k and folds each column in k order, then one xor tree
// per column.
template <typename Fold, typename T, int C>
__device__ __forceinline__ void partials_vecrows(void* partials_ptr, const void* in_ptr,
                                                 const SidePlan& sp, Fold f) {
  constexpr int W = kWarp;
  constexpr int kPlanes = kBlock / W;
  T* partials = static_cast<T*>(partials_ptr);
  const char* in = static_cast<const char*>(in_ptr);
  const int lane = threadIdx.x % W;
  const long long row_bytes = sp.axis_stride * static_cast<long long>(sizeof(T));
  const long long planes = static_cast<long long>(gridDim.x) * kPlanes;
  for (long long u = static_cast<long long>(blockIdx.x) * kPlanes + threadIdx.x / W;
       u < sp.units; u += planes) {
    unsigned int block;
    long long ib, pb;
    int len;
    side_unit(sp, static_cast<unsigned int>(u), &block, &ib, &pb, &len);
    T acc[C];
    fold_lane_rows<C>(in + ib * static_cast<long long>(sizeof(T)), kWarp * row_bytes,
                      lane * row_bytes, lane, len, f, acc);
#pragma unroll
    for (int c = 0; c < C; ++c) acc[c] = plane_tree(acc[c], W, f);
    if (lane == 0) {
#pragma unroll
      for (int c = 0; c < C; ++c) partials[pb + c * sp.col_os] = acc[c];
    }
  }
}

// ROWS: C = 64 / P columns; wavefront lane t = ro*C + c holds column c and the
// plane lanes ro + P*a (a < A = 32 / P) of its cube, so one load reads P
// consecutive rows of all C columns. Xor offsets below P cross lanes (a
// wavefront exchange at lane distance off*C), the rest combine registers.
template <int A, typename Fold, typename T>
__device__ __forceinline__ void partials_rows(void* partials_ptr, const void* in_ptr,
                                              const PartialsPlan& pp, long long chunk_len,
                                              long long splits, Fold f) {
  constexpr int P = kWarp / A;
  constexpr int C = kWave / P;
  T* partials = static_cast<T*>(partials_ptr);
  const T* in = static_cast<const T*>(in_ptr);
  const ReduceDims& rd = pp.dims;
  const long long stride = rd.axis_stride;
  const int t = threadIdx.x % kWave;
  const int c = t % C;
  const int ro = t / C;
  const long long nwaves = static_cast<long long>(gridDim.x) * (kBlock / kWave);
  for (long long u = (static_cast<long long>(blockIdx.x) * kBlock + threadIdx.x) / kWave;
       u < pp.units; u += nwaves) {
    long long ib, pb, split;
    decode_unit(pp, u, c, &ib, &pb, &split, splits);
    const long long start = split * chunk_len;
    const long long len = (split + 1 == splits ? rd.axis_len : start + chunk_len) - start;
    const T* x = in + ib + start * stride;
    // U row-steps of loads (16 per lane) are issued before they are folded;
    // each plane lane still folds its rows in increasing order, the first
    // step seeding (chunks hold at least 32 rows, so step 0 is whole).
    constexpr int U = A >= 16 ? 1 : 16 / A;
    T acc[A];
    {
      T v[U][A];
#pragma unroll
      for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int a = 0; a < A; ++a) {
          const long long q = u * kWarp + ro + P * a;
          if (u == 0 || q < len) v[u][a] = x[q * stride];
        }
      }
#pragma unroll
      for (int a = 0; a < A; ++a) acc[a] = f.seed(v[0][a]);
#pragma unroll
      for (int u = 1; u < U; ++u) {
#pragma unroll
        for (int a = 0; a < A; ++a) {
          if (u * kWarp + ro + P * a < len) acc[a] = f.fold(acc[a], v[u][a]);
        }
      }
    }
    long long q0 = U * kWarp;
    for (; q0 + U * kWarp <= len; q0 += U * kWarp) {
      T v[U][A];
#pragma unroll
      for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int a = 0; a < A; ++a) v[u][a] = x[(q0 + u * kWarp + ro + P * a) * stride];
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int a = 0; a < A; ++a) acc[a] = f.fold(acc[a], v[u][a]);
      }
    }
    for (; q0 + kWarp <= len; q0 += kWarp) {
      T v[A];
#pragma unroll
      for (int a = 0; a < A; ++a) v[a] = x[(q0 + ro + P * a) * stride];
#pragma unroll
      for (int a = 0; a < A; ++a) acc[a] = f.fold(acc[a], v[a]);
    }
#pragma unroll
    for (int a = 0; a < A; ++a) {
      if (q0 + ro + P * a < len) acc[a] = f.fold(acc[a], x[(q0 + ro + P * a) * stride]);
    }
#pragma unroll
    for (int off = 1; off < kWarp; off <<= 1) {
      if (off < P) {
#pragma unroll
        for (int a = 0; a < A; ++a) acc[a] = f.combine(acc[a], shfl_xor(acc[a], off * C, kWave));
      } else {
        const int s = off / P;
#pragma unroll
        for (int a = 0; a < A; a += 2 * s) acc[a] = f.combine(acc[a], acc[a + s]);
      }
    }
    if (ro == 0) partials[pb] = acc[0];
  }
}

// Fold dispatch for element type T over the reference's supported pairs
// (reduce.cu:765-852): SUM/PROD numeric, SUM_SQUARES float, MAX/MIN ordered;
// an unsupported op performs no work.
template <typename T, typename Fn>
__device__ __forceinline__ void dispatch_fold(int op, Fn&& fn) {
  constexpr bool kFloat = std::is_same_v<T, float> || std::is_same_v<T, double>;
  constexpr bool kOrdered = kFloat || std::is_same_v<T, int> || std::is_same_v<T, long long>;
  switch (op) {
    case T4A_CUDA_REDUCE_SUM: fn(SumFold{}); break;
    case T4A_CUDA_REDUCE_PROD: fn(ProdFold{}); break;
    case T4A_CUDA_REDUCE_SUM_SQUARES:
      if constexpr (kFloat) fn(SumSquaresFold{});
      break;
    case T4A_CUDA_REDUCE_MAX:
      if constexpr (kOrdered) fn(MaxFold{});
      break;
    case T4A_CUDA_REDUCE_MIN:
      if constexpr (kOrdered) fn(MinFold{});
      break;
    default: break;
  }
}

template <typename Fn>
__device__ __forceinline__ void dispatch_dtype(int dtype, Fn&& fn) {
  switch (dtype) {
    case T4A_CUDA_F32: fn(static_cast<float*>(nullptr)); break;
    case T4A_CUDA_F64: fn(static_cast<double*>(nullptr)); break;
    case T4A_CUDA_I32: fn(static_cast<int*>(nullptr)); break;
    case T4A_CUDA_I64: fn(static_cast<long long*>(nullptr)); break;
    case T4A_CUDA_C32: fn(static_cast<c32*>(nullptr)); break;
    case T4A_CUDA_C64: fn(static_cast<c64*>(nullptr)); break;
    default: break;
  }
}

template <typename T, typename RD>
__device__ __forceinline__ void reduce_run(void* out, const void* in, int op, bool plane,
                                           const RD& rd, long long output_len,
                                           unsigned char* warp_lds, unsigned int blocks) {
  dispatch_fold<T>(op, [&](auto fold) {
    if (plane) {
      plane_body<decltype(fold), T>(out, in, rd, output_len, fold, warp_lds, blocks);
    } else {
      unit_body<decltype(fold), T, 0>(out, in, rd, output_len, fold, blocks);
    }
  });
}

// ---- kernels the launchers use: one per element type (and pass-1 mapping), the
// plan computed on the host and passed by value. ----

template <typename T>
__global__ void __launch_bounds__(512)
    reduce_kernel(void* out, const void* in, int op, int strategy, ReduceDims rd,
                  long long output_len) {
  __shared__ alignas(16) unsigned char warp_lds[16 * sizeof(T)];
  reduce_run<T>(out, in, op, strategy == T4A_CUDA_REDUCE_PLANE, rd, output_len, warp_lds,
                gridDim.x);
}

// UNIT on a compact plan, one kernel per (element type, fold, block size).
template <typename T, typename Fold, int BS>
__global__ void __launch_bounds__(BS)
    reduce_unit_lean_kernel(void* out, const void* in, UnitPlan up, unsigned int output_len) {
  unit_lean<Fold, T, BS>(static_cast<T*>(out), static_cast<const T*>(in), up, output_len,
                         Fold{});
}

// UNIT over a one-group axis (C4's i32 product), a kernel of its own: its
// wavefronts live for two loads, and in the kernel that carries every unit
// walk the prologue computed the other walks' invariants (and spilled scalar
// registers) before the first load. The block count is an argument.
template <typename T, typename Fold, bool Linear>
__global__ void __launch_bounds__(kBlock)
    reduce_unit_group_kernel(void* out, const void* in, UnitPlan up, unsigned int output_len,
                             unsigned int blocks) {
  unit_group_lean<Fold, T, Linear>(static_cast<T*>(out), static_cast<const T*>(in), up,
                                   output_len, Fold{}, blocks);
}

// PLANE on a compact plan (the combine over thousands of partials): the plane
// body with the UnitPlan decode and the fold fixed at compile time. The general
// kernel's by-value eight-dim geometry takes a private segment, which every
// dispatch pays for (C4's combine: 12-14 us there).
template <typename T, typename Fold>
__global__ void __launch_bounds__(512)
    reduce_plane_lean_kernel(void* out, const void* in, UnitPlan up, unsigned int output_len) {
  __shared__ alignas(16) unsigned char warp_lds[16 * sizeof(T)];
  plane_body<Fold, T>(out, in, up, static_cast<long long>(output_len), Fold{}, warp_lds,
                      gridDim.x);
}

template <typename T, typename Fold>
__global__ void __launch_bounds__(256)
    reduce_plane_multi_kernel(void* out, const void* in, UnitPlan up, unsigned int output_len) {
  plane_multi<Fold, T>(static_cast<T*>(out), static_cast<const T*>(in), up, output_len, Fold{});
}

template <typename T, typename Fold>
__global__ void __launch_bounds__(256)
    reduce_plane_thread_kernel(void* out, const void* in, UnitPlan up, unsigned int output_len) {
  plane_per_thread<Fold, T, kWarp>(static_cast<T*>(out), static_cast<const T*>(in), up,
                                   output_len, Fold{});
}

// UNIT with the planner's blocks of BS threads.
template <typename T, int BS>
__global__ void __launch_bounds__(BS)
    reduce_unit_kernel(void* out, const void* in, int op, ReduceDims rd, long long output_len) {
  dispatch_fold<T>(op, [&](auto fold) {
    unit_body<decltype(fold), T, BS>(out, in, rd, output_len, fold, gridDim.x);
  });
}

template <typename T>
__global__ void __launch_bounds__(256)
    partials_plane_kernel(void* partials, const void* in, int op, PartialsPlan pp,
                          long long output_len, long long splits, long long chunk_len) {
  dispatch_fold<T>(op, [&](auto fold) {
    partials_planes<decltype(fold), T>(partials, in, pp, output_len, splits, chunk_len, fold,
                                       gridDim.x);
  });
}

template <typename T>
__global__ void __launch_bounds__(256)
    partials_stream_kernel(void* partials, const void* in, int op, PartialsPlan pp,
                           long long output_len, long long splits, long long chunk_len,
                           long long per_plane) {
  if constexpr (VecLanes<T>::value > 0) {
    dispatch_fold<T>(op, [&](auto fold) {
      if constexpr (decltype(fold)::kRegroup)
        partials_stream<decltype(fold), T>(partials, in, pp, output_len, splits, chunk_len,
                                           per_plane, fold);
    });
  }
}

// Pass 1 and the unit combine in one launch, up to C chunks per plane (linear
// LEAN plans): CFold is the combine pass's fold (Sum after SumSquares, else the
// same).
template <typename T, int K, typename Fold, typename CFold, int C>
__global__ void __launch_bounds__(kBlock)
    reduction_joined_kernel(void* partials, const void* in, LeanPlan lp, JoinedOut jo) {
  reduction_joined<Fold, CFold, T, K, C>(partials, in, lp, jo, Fold{});
}

// One kernel per (element type, batch slots, fold, linear walk): the fold is
// chosen on the host, so each kernel carries one fold's code only.
template <typename T, int K, typename Fold, bool Linear>
__global__ void __launch_bounds__(kBlock)
    partials_lean_kernel(void* partials, const void* in, LeanPlan lp) {
  partials_lean<Fold, T, K, Linear>(partials, in, lp, Fold{});
}

template <typename T, int CPL>
__global__ void __launch_bounds__(kBlock)
    partials_tiles_kernel(void* partials, const void* in, int op, SidePlan sp) {
  __shared__ T lds[(kBlock / kWave) * kWave * CPL];
  __shared__ int redo;
  dispatch_fold<T>(op, [&](auto fold) {
    partials_tiles<decltype(fold), T, CPL>(partials, in, sp, fold, lds, &redo, gridDim.x);
  });
}

template <typename T, int C>
__global__ void __launch_bounds__(kBlock)
    partials_vecrows_kernel(void* partials, const void* in, int op, SidePlan sp) {
  dispatch_fold<T>(op, [&](auto fold) {
    partials_vecrows<decltype(fold), T, C>(partials, in, sp, fold);
  });
}

template <typename T, int A>
__global__ void __launch_bounds__(kBlock)
    partials_rows_kernel(void* partials, const void* in, int op, PartialsPlan pp,
                         long long splits, long long chunk_len) {
  dispatch_fold<T>(op, [&](auto fold) {
    partials_rows<A, decltype(fold), T>(partials, in, pp, chunk_len, splits, fold);
  });
}

}  // namespace
}  // namespace t4a

// ---- the reference entry symbols -----------------------------------------------------
// Complete kernels for callers that load the code object and launch by name
// (reference docs/abi/c-kernel-abi.md:3-7): the plan is derived in the kernel
// from the entry's own arguments, and pass 1 keeps the plane mapping (any
// geometry that planes the cubes computes the same partials).

extern "C" __global__ void __launch_bounds__(512)
    t4a_cuda_reduce(void* out, const void* in, int dtype, int op, int strategy,
                    t4a_cuda_layout out_layout, t4a_cuda_layout in_layout, int axis,
                    long long output_len) {
  if (t4a::entry_block_idle(t4a::kReduceEntryWaves)) return;
  const unsigned int blocks = t4a::entry_blocks(t4a::kReduceEntryWaves);
  __shared__ t4a::ReduceDims rd;
  __shared__ alignas(16) unsigned char warp_lds[16 * sizeof(t4a::c64)];
  if (threadIdx.x == 0) t4a::reduce_dims(&rd, out_layout, in_layout, axis);
  __syncthreads();
  const bool plane = strategy == T4A_CUDA_REDUCE_PLANE;
  t4a::dispatch_dtype(dtype, [&](auto* tag) {
    using T = std::remove_pointer_t<decltype(tag)>;
    t4a::reduce_run<T>(out, in, op, plane, rd, output_len, warp_lds, blocks);
  });
}

// Pass 1 under the caller's geometry: thread 0 plans as the launchers do for
// this block shape. A strided axis with neighbouring output columns takes the
// TILES mapping when the block is one to four whole wavefronts or one 32-lane
// plane (the reference's shapes); a contiguous axis whose chunks fit the LEAN
// mapping takes it with the block's planes; anything else walks planes.
extern "C" __global__ void __launch_bounds__(256)
    t4a_cuda_reduce_partials(void* partials, const void* in, int dtype, int op,
                             t4a_cuda_layout partials_layout, t4a_cuda_layout in_layout,
                             int axis, long long output_len, long long splits,
                             long long chunk_len) {
  if (t4a::entry_block_idle(t4a::partials_entry_waves())) return;
  const unsigned int blocks = t4a::entry_blocks(t4a::partials_entry_waves());
  __shared__ t4a::PartialsPlan pp;
  __shared__ t4a::SidePlan side;
  __shared__ t4a::LeanPlan lean;
  // 0: planes; 1 or 2: TILES with that many columns per lane; -K: LEAN, K slots
  __shared__ int route;
  __shared__ alignas(16) unsigned char tiles_lds[t4a::kBlock * 2 * 8];
  __shared__ int redo;
  const unsigned int bs = blockDim.x;
  const bool flat = blockDim.y == 1 && blockDim.z == 1;
  if (threadIdx.x == 0) {
    const int w = bs <= 32u ? static_cast<int>(bs) : t4a::kWarp;
    const bool tile_shape = flat && (bs == 32 || bs == 64 || bs == 128 || bs == 256);
    const uintptr_t address = reinterpret_cast<uintptr_t>(in);
    const int align =
        (address & 15) == 0 ? 16 : (address & 7) == 0 ? 8 : (address & 3) == 0 ? 4 : 1;
    t4a::partials_plan(&pp, partials_layout, in_layout, axis, output_len, splits, w,
                       tile_shape && t4a::sideways_dtype(dtype) ? 1 : 0, t4a::dtype_size(dtype),
                       align);
    route = 0;
    if (pp.mode == t4a::kPartialsTiles) {
      // The launchers' plan counts 64-lane column blocks; a 32-lane block
      // covers half as many columns.
      const long long bc = static_cast<long long>(bs == 32 ? t4a::kWarp : t4a::kWave) * pp.cpl;
      const long long col_blocks = (pp.columns + bc - 1) / bc;
      const long long units = col_blocks * pp.others * splits;
      if (units < (1ll << 31)) {
        t4a::side_plan_into(&side, pp, splits, chunk_len);
        side.col_blocks = t4a::fast_div(static_cast<unsigned int>(col_blocks));
        side.units = units;
        route = pp.cpl;
      }
    } else if (pp.mode == t4a::kPartialsPlane && flat && bs % 32 == 0 && align == 16 &&
               static_cast<unsigned long long>(blocks) * (bs / 32) <= (1ull << 24)) {
      const int k = t4a::lean_slots(pp, dtype, op, splits, chunk_len, w);
      if (k > 0) {
        lean = t4a::lean_plan(pp, splits, chunk_len);
        route = -k;
      }
    }
  }
  __syncthreads();
  const int r = route;
  t4a::dispatch_dtype(dtype, [&](auto* tag) {
    using T = std::remove_pointer_t<decltype(tag)>;
    t4a::dispatch_fold<T>(op, [&](auto fold) {
      using F = decltype(fold);
      if constexpr (t4a::VecLanes<T>::value > 0) {
        if (r > 0) {
          // From LDS: copied to scalar registers the plan would spill.
          const t4a::SidePlan& sp = side;
          T* lds = reinterpret_cast<T*>(tiles_lds);
          auto tiles = [&](auto cpl_tag) {
            constexpr int CPL = decltype(cpl_tag)::value;
            if (bs == 32)
              t4a::partials_tiles<F, T, CPL, 1, t4a::kWarp>(partials, in, sp, fold, lds, &redo,
                                                            blocks);
            else if (bs == 64)
              t4a::partials_tiles<F, T, CPL, 1>(partials, in, sp, fold, lds, &redo, blocks);
            else if (bs == 128)
              t4a::partials_tiles<F, T, CPL, 2>(partials, in, sp, fold, lds, &redo, blocks);
            else
              t4a::partials_tiles<F, T, CPL, 4>(partials, in, sp, fold, lds, &redo, blocks);
          };
          if (r == 2)
            tiles(std::integral_constant<int, 2>{});
          else
            tiles(std::integral_constant<int, 1>{});
          return;
        }
        if (r < 0) {
          const t4a::LeanPlan& lp = lean;
          switch (-r) {
            case 1: t4a::partials_lean_entry<F, T, 1, 4>(partials, in, lp, fold, blocks); break;
            case 2: t4a::partials_lean_entry<F, T, 2, 4>(partials, in, lp, fold, blocks); break;
            case 3: t4a::partials_lean_entry<F, T, 3, 2>(partials, in, lp, fold, blocks); break;
            default: t4a::partials_lean_entry<F, T, 4, 2>(partials, in, lp, fold, blocks); break;
          }
          return;
        }
      }
      t4a::partials_planes<F, T>(partials, in, pp, output_len, splits, chunk_len, fold, blocks);
    });
  });
}

// General-rank twins (reference reduce.cu:854-940, docs/abi/c-kernel-abi.md
// "Dynamic rank"): the geometry arrays live in caller-owned device memory.
// Thread 0 fuses them into LDS dims (at most 62 remain for any layout of fewer
// than 2^63 elements) and the block runs the by-value entries' bodies on them,
// so the results are the fast twins' bits. An axis outside the rank, or ranks
// that differ, do no work.
__device__ __forceinline__ void any_dims(t4a::ReduceDimsWide* rd, const t4a_cuda_layout_any& out,
                                         const t4a_cuda_layout_any& in, int axis) {
  if (axis < 0 || axis >= in.rank || out.rank != in.rank) {
    rd->n = -1;
    return;
  }
  t4a::reduce_dims_view(rd, in.rank, axis, out.offset, out.extents, out.strides, in.offset,
                        in.extents, in.strides);
}

extern "C" __global__ void __launch_bounds__(512)
    t4a_cuda_reduce_any(void* out, const void* in, int dtype, int op, int strategy,
                        t4a_cuda_layout_any out_layout, t4a_cuda_layout_any in_layout, int axis,
                        long long output_len) {
  if (t4a::entry_block_idle(t4a::kReduceEntryWaves)) return;
  const unsigned int blocks = t4a::entry_blocks(t4a::kReduceEntryWaves);
  __shared__ t4a::ReduceDimsWide rd;
  __shared__ alignas(16) unsigned char warp_lds[16 * sizeof(t4a::c64)];
  if (threadIdx.x == 0) any_dims(&rd, out_layout, in_layout, axis);
  __syncthreads();
  if (rd.n < 0) return;
  const bool plane = strategy == T4A_CUDA_REDUCE_PLANE;
  t4a::dispatch_dtype(dtype, [&](auto* tag) {
    using T = std::remove_pointer_t<decltype(tag)>;
    t4a::reduce_run<T>(out, in, op, plane, rd, output_len, warp_lds, blocks);
  });
}

// The launchers' column mapping for a general-rank pass 1 (a strided axis
// with neighbouring output columns): thread 0 rebuilds the rank <= 8 layout
// pair the host planner plans with (reduction_pair_view), plans pass 1 as the
// by-value launcher does, and keeps the SidePlan when that plan is TILES
// (returning its columns per lane, 0 otherwise).
// Thread 0's planning temporaries of the general-rank pass 1, in LDS: as
// locals, their runtime-subscripted arrays would take per-lane scratch memory,
// which every dispatch of the kernel would pay for.
struct AnySideScratch {
  t4a_cuda_layout p8, i8;
  t4a::PartialsPlan pp;
  t4a::ReduceDimsN<t4a::kMaxDims - 1> fused;
  int axis8;
};

// On a contiguous axis the same plan may instead be the lean mapping's: then
// the LeanPlan goes to `lean` and the result is minus its slot count.
__device__ __forceinline__ int any_side_plan(t4a::SidePlan* side, t4a::LeanPlan* lean,
                                             AnySideScratch* tmp, int dtype, int op,
                                             const void* in,
                                             const t4a_cuda_layout_any& partials,
                                             const t4a_cuda_layout_any& input, int axis,
                                             long long output_len, long long splits,
                                             long long chunk_len, bool whole_waves) {
  if (!t4a::sideways_dtype(dtype) || axis < 0 || axis >= input.rank ||
      partials.rank != input.rank)
    return 0;
  if (!t4a::reduction_pair_view(input.rank, partials.offset, partials.extents, partials.strides,
                                input.offset, input.extents, input.strides, axis, &tmp->p8,
                                &tmp->i8, &tmp->axis8, &tmp->fused))
    return 0;
  const int axis8 = tmp->axis8;
  const uintptr_t address = reinterpret_cast<uintptr_t>(in);
  const int align = (address & 15) == 0 ? 16 : (address & 7) == 0 ? 8 : (address & 3) == 0 ? 4 : 1;
  t4a::partials_plan(&tmp->pp, tmp->p8, tmp->i8, axis8, output_len, splits, t4a::kWarp,
                     whole_waves ? 1 : 0, t4a::dtype_size(dtype), align);
  if (tmp->pp.mode == t4a::kPartialsTiles) {
    t4a::side_plan_into(side, tmp->pp, splits, chunk_len);
    return tmp->pp.cpl;
  }
  if (tmp->pp.mode == t4a::kPartialsPlane && align == 16) {
    const int k = t4a::lean_slots(tmp->pp, dtype, op, splits, chunk_len, t4a::kWarp);
    if (k > 0) {
      *lean = t4a::lean_plan(tmp->pp, splits, chunk_len);
      return -k;
    }
  }
  return 0;
}

extern "C" __global__ void __launch_bounds__(256)
    t4a_cuda_reduce_partials_any(void* partials, const void* in, int dtype, int op,
                                 t4a_cuda_layout_any partials_layout,
                                 t4a_cuda_layout_any in_layout, int axis, long long output_len,
                                 long long splits, long long chunk_len) {
  __shared__ t4a::ReduceDimsWide rd;
  __shared__ t4a::SidePlan side;
  __shared__ t4a::LeanPlan lean;
  __shared__ AnySideScratch side_tmp;
  // > 0: TILES with that many columns per lane; < 0: LEAN with minus that
  // many slots; 0: planes
  __shared__ int side_cpl;
  __shared__ alignas(16) unsigned char tiles_lds[(t4a::kBlock / t4a::kWave) * t4a::kWave * 2 * 8];
  __shared__ int redo;
  if (t4a::entry_block_idle(t4a::partials_entry_waves())) return;
  const unsigned int blocks = t4a::entry_blocks(t4a::partials_entry_waves());
  const bool whole_waves = blockDim.x == static_cast<unsigned>(t4a::kBlock) &&
                           blockDim.y == 1 && blockDim.z == 1;
  // The lean walk's planes: 32-lane planes filling 1-D blocks, a stride of
  // at most 2^24 planes (its 32-bit cube indices).
  const bool plane_blocks = blockDim.x % 32u == 0 && blockDim.y == 1 && blockDim.z == 1 &&
                            static_cast<unsigned long long>(blocks) * (blockDim.x / 32u) <=
                                (1ull << 24);
  if (threadIdx.x == 0) {
    any_dims(&rd, partials_layout, in_layout, axis);
    // A strided axis can take the column mapping (whole wavefronts), a
    // contiguous one the lean mapping.
    const bool strided = rd.axis_stride != 1;
    side_cpl = rd.n >= 0 && (strided ? whole_waves : plane_blocks)
                   ? any_side_plan(&side, &lean, &side_tmp, dtype, op, in, partials_layout,
                                   in_layout, axis, output_len, splits, chunk_len,
                                   strided && whole_waves)
                   : 0;
  }
  __syncthreads();
  if (rd.n < 0) return;
  if (side_cpl < 0) {
    const t4a::LeanPlan& lp = lean;  // from LDS
    const int k = -side_cpl;
    t4a::dispatch_dtype(dtype, [&](auto* tag) {
      using T = std::remove_pointer_t<decltype(tag)>;
      if constexpr (t4a::VecLanes<T>::value > 0) {
        t4a::dispatch_fold<T>(op, [&](auto fold) {
          using F = decltype(fold);
          switch (k) {
            case 1: t4a::partials_lean_entry<F, T, 1, 4>(partials, in, lp, fold, blocks); break;
            case 2: t4a::partials_lean_entry<F, T, 2, 4>(partials, in, lp, fold, blocks); break;
            case 3: t4a::partials_lean_entry<F, T, 3, 2>(partials, in, lp, fold, blocks); break;
            default: t4a::partials_lean_entry<F, T, 4, 2>(partials, in, lp, fold, blocks); break;
          }
        });
      }
    });
    return;
  }
  if (side_cpl > 0) {
    const t4a::SidePlan& sp = side;  // from LDS (copied to scalar registers it spills)
    const int cpl = side_cpl;
    t4a::dispatch_dtype(dtype, [&](auto* tag) {
      using T = std::remove_pointer_t<decltype(tag)>;
      if constexpr (t4a::VecLanes<T>::value > 0) {
        T* lds = reinterpret_cast<T*>(tiles_lds);
        t4a::dispatch_fold<T>(op, [&](auto fold) {
          if (cpl == 2)
            t4a::partials_tiles<decltype(fold), T, 2>(partials, in, sp, fold, lds, &redo, blocks);
          else
            t4a::partials_tiles<decltype(fold), T, 1>(partials, in, sp, fold, lds, &redo, blocks);
        });
      }
    });
    return;
  }
  t4a::dispatch_dtype(dtype, [&](auto* tag) {
    using T = std::remove_pointer_t<decltype(tag)>;
    t4a::dispatch_fold<T>(op, [&](auto fold) {
      t4a::partials_planes_dims<decltype(fold), T>(partials, in, rd, output_len, splits,
                                                   chunk_len, fold, blocks);
    });
  });
}

// ---- launchers -----------------------------------------------------------------------

namespace {

bool launch_empty(const t4a_launch* l) {
  return l->grid[0] == 0 || l->grid[1] == 0 || l->grid[2] == 0;
}

template <typename Fn>
int with_dtype(int dtype, Fn&& fn) {
  switch (dtype) {
    case T4A_CUDA_F32: return fn(static_cast<float*>(nullptr));
    case T4A_CUDA_F64: return fn(static_cast<double*>(nullptr));
    case T4A_CUDA_I32: return fn(static_cast<int*>(nullptr));
    case T4A_CUDA_I64: return fn(static_cast<long long*>(nullptr));
    case T4A_CUDA_C32: return fn(static_cast<t4a::c32*>(nullptr));
    case T4A_CUDA_C64: return fn(static_cast<t4a::c64*>(nullptr));
    default: return T4A_OK;  // unknown tag: no work, as the reference entry
  }
}

using t4a::status_of_last_launch;

}  // namespace

namespace {

// The unit kernel for (fold, block size), both chosen on the host, over the
// reference's op matrix for T.
template <typename T, typename Fold>
void launch_unit_fold(unsigned threads, dim3 grid, dim3 block, hipStream_t s, void* out,
                      const void* in, const t4a::UnitPlan& up, unsigned int output_len) {
  if constexpr (t4a::VecLanes<T>::value > 0) {
    if (threads == static_cast<unsigned>(t4a::kBlock) && up.vector &&
        up.axis_len < 2 * t4a::VecLanes<T>::value) {
      if (up.n <= 1)
        hipLaunchKernelGGL((t4a::reduce_unit_group_kernel<T, Fold, true>), grid, block, 0, s,
                           out, in, up, output_len, grid.x);
      else
        hipLaunchKernelGGL((t4a::reduce_unit_group_kernel<T, Fold, false>), grid, block, 0, s,
                           out, in, up, output_len, grid.x);
      return;
    }
  }
  if (threads == static_cast<unsigned>(t4a::kBlock))
    hipLaunchKernelGGL((t4a::reduce_unit_lean_kernel<T, Fold, t4a::kBlock>), grid, block, 0, s,
                       out, in, up, output_len);
  else
    hipLaunchKernelGGL((t4a::reduce_unit_lean_kernel<T, Fold, t4a::kUnitSmallBlock>), grid,
                       block, 0, s, out, in, up, output_len);
}

template <typename T>
void launch_unit_lean(int op, unsigned threads, dim3 grid, dim3 block, hipStream_t s, void* out,
                      const void* in, const t4a::UnitPlan& up, unsigned int output_len) {
  constexpr bool kFloat = std::is_same_v<T, float> || std::is_same_v<T, double>;
  constexpr bool kOrdered = kFloat || std::is_same_v<T, int> || std::is_same_v<T, long long>;
  switch (op) {
    case T4A_CUDA_REDUCE_SUM:
      launch_unit_fold<T, t4a::SumFold>(threads, grid, block, s, out, in, up, output_len);
      break;
    case T4A_CUDA_REDUCE_PROD:
      launch_unit_fold<T, t4a::ProdFold>(threads, grid, block, s, out, in, up, output_len);
      break;
    case T4A_CUDA_REDUCE_SUM_SQUARES:
      if constexpr (kFloat)
        launch_unit_fold<T, t4a::SumSquaresFold>(threads, grid, block, s, out, in, up,
                                                 output_len);
      break;
    case T4A_CUDA_REDUCE_MAX:
      if constexpr (kOrdered)
        launch_unit_fold<T, t4a::MaxFold>(threads, grid, block, s, out, in, up, output_len);
      break;
    case T4A_CUDA_REDUCE_MIN:
      if constexpr (kOrdered)
        launch_unit_fold<T, t4a::MinFold>(threads, grid, block, s, out, in, up, output_len);
      break;
    default: break;
  }
}

// The lean plane kernel for `op` over the reference's op matrix for T.
template <typename T>
void launch_plane_lean(int op, dim3 grid, dim3 block, hipStream_t s, void* out, const void* in,
                       const t4a::UnitPlan& up, unsigned int output_len) {
  constexpr bool kFloat = std::is_same_v<T, float> || std::is_same_v<T, double>;
  constexpr bool kOrdered = kFloat || std::is_same_v<T, int> || std::is_same_v<T, long long>;
  // Several planes a block (block.y > 1): 32-lane planes of at most 8-byte
  // elements over a strided axis one thread per output (neighbouring outputs'
  // loads coalesce: 2^20 outputs over a 64-element axis 4 MiB apart, 88 us
  // against 370 with packed planes); else the packed planes (a contiguous
  // 64-element axis: 114 us against 375 one thread per output).
  const bool multi = block.y > 1;
  const bool per_thread = multi && block.x == static_cast<unsigned>(t4a::kWarp) &&
                          sizeof(T) <= 8 && up.axis_stride != 1;
  auto go = [&](auto fold) {
    using Fold = decltype(fold);
    if (per_thread)
      hipLaunchKernelGGL((t4a::reduce_plane_thread_kernel<T, Fold>),
                         dim3((output_len + t4a::kBlock - 1) / t4a::kBlock < grid.x * block.y
                                  ? (output_len + t4a::kBlock - 1) / t4a::kBlock
                                  : grid.x * block.y),
                         dim3(t4a::kBlock), 0, s, out, in, up, output_len);
    else if (multi)
      hipLaunchKernelGGL((t4a::reduce_plane_multi_kernel<T, Fold>), grid, block, 0, s, out, in,
                         up, output_len);
    else
      hipLaunchKernelGGL((t4a::reduce_plane_lean_kernel<T, Fold>), grid, block, 0, s, out, in,
                         up, output_len);
  };
  switch (op) {
    case T4A_CUDA_REDUCE_SUM: go(t4a::SumFold{}); break;
    case T4A_CUDA_REDUCE_PROD: go(t4a::ProdFold{}); break;
    case T4A_CUDA_REDUCE_SUM_SQUARES:
      if constexpr (kFloat) go(t4a::SumSquaresFold{});
      break;
    case T4A_CUDA_REDUCE_MAX:
      if constexpr (kOrdered) go(t4a::MaxFold{});
      break;
    case T4A_CUDA_REDUCE_MIN:
      if constexpr (kOrdered) go(t4a::MinFold{});
      break;
    default: break;
  }
}

}  // namespace

extern "C" int t4a_hip_reduce(void* out, const void* in, int dtype, int op, int strategy,
                              const t4a_cuda_layout* out_layout,
                              const t4a_cuda_layout* in_layout, int axis, long long output_len,
                              const t4a_launch* launch, void* stream) {
  if (launch == nullptr || out_layout == nullptr || in_layout == nullptr)
    return T4A_HIP_ERR_NULL_ARGUMENT;
  if (launch_empty(launch)) return T4A_OK;
  if (out == nullptr || in == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  t4a::ReduceDims rd;
  t4a::reduce_dims(&rd, *out_layout, *in_layout, axis);
  const dim3 grid(launch->grid[0], launch->grid[1], launch->grid[2]);
  const dim3 block(launch->block[0], launch->block[1], launch->block[2]);
  return with_dtype(dtype, [&](auto* tag) {
    using T = std::remove_pointer_t<decltype(tag)>;
    const unsigned threads = block.x * block.y * block.z;
    // The block-size-specialised kernels number threads by x alone.
    const bool flat_blocks = block.y == 1 && block.z == 1;
    if (strategy == T4A_CUDA_REDUCE_UNIT && t4a::unit_plan_fits(rd, output_len) && flat_blocks &&
        (threads == static_cast<unsigned>(t4a::kBlock) ||
         threads == static_cast<unsigned>(t4a::kUnitSmallBlock)) &&
        t4a::unit_lean_fits(output_len, grid.x, threads)) {
      const bool aligned = (reinterpret_cast<uintptr_t>(in) & 15) == 0;
      const t4a::UnitPlan up = t4a::unit_plan(rd, t4a::VecLanes<T>::value, aligned);
      launch_unit_lean<T>(op, threads, grid, block, static_cast<hipStream_t>(stream), out, in,
                          up, static_cast<unsigned int>(output_len));
    } else if (strategy == T4A_CUDA_REDUCE_PLANE && t4a::unit_plan_fits(rd, output_len) &&
               block.z == 1 && threads <= 512u &&
               (block.y == 1 ||
                (block.x <= static_cast<unsigned>(t4a::kWarp) && (block.x & (block.x - 1)) == 0 &&
                 threads == static_cast<unsigned>(t4a::kBlock) &&
                 t4a::grid_stride_fits(output_len, grid.x,
                                       4ull * block.y)))) {
      const t4a::UnitPlan up = t4a::unit_plan(rd, t4a::VecLanes<T>::value, false);
      launch_plane_lean<T>(op, grid, block, static_cast<hipStream_t>(stream), out, in, up,
                           static_cast<unsigned int>(output_len));
    } else if (strategy == T4A_CUDA_REDUCE_UNIT && flat_blocks &&
               threads == static_cast<unsigned>(t4a::kBlock)) {
      hipLaunchKernelGGL((t4a::reduce_unit_kernel<T, t4a::kBlock>), grid, block, 0,
                         static_cast<hipStream_t>(stream), out, in, op, rd, output_len);
    } else if (strategy == T4A_CUDA_REDUCE_UNIT && flat_blocks &&
               threads == static_cast<unsigned>(t4a::kUnitSmallBlock)) {
      hipLaunchKernelGGL((t4a::reduce_unit_kernel<T, t4a::kUnitSmallBlock>), grid, block, 0,
                         static_cast<hipStream_t>(stream), out, in, op, rd, output_len);
    } else {
      hipLaunchKernelGGL(t4a::reduce_kernel<T>, grid, block, 0,
                         static_cast<hipStream_t>(stream), out, in, op, strategy, rd,
                         output_len);
    }
    return status_of_last_launch();
  });
}

namespace {

// The lean pass-1 kernel for (K, fold, linear), all chosen on the host.
template <typename T, int K, typename Fold>
void launch_lean_k(bool linear, dim3 grid, dim3 block, hipStream_t s, void* partials,
                   const void* in, const t4a::LeanPlan& lp) {
  if (linear)
    hipLaunchKernelGGL((t4a::partials_lean_kernel<T, K, Fold, true>), grid, block, 0, s,
                       partials, in, lp);
  else
    hipLaunchKernelGGL((t4a::partials_lean_kernel<T, K, Fold, false>), grid, block, 0, s,
                       partials, in, lp);
}

template <typename T, typename Fold>
void launch_lean_fold(int k, bool linear, dim3 grid, dim3 block, hipStream_t s, void* partials,
                      const void* in, const t4a::LeanPlan& lp) {
  switch (k) {
    case 1: launch_lean_k<T, 1, Fold>(linear, grid, block, s, partials, in, lp); break;
    case 2: launch_lean_k<T, 2, Fold>(linear, grid, block, s, partials, in, lp); break;
    case 3: launch_lean_k<T, 3, Fold>(linear, grid, block, s, partials, in, lp); break;
    default: launch_lean_k<T, 4, Fold>(linear, grid, block, s, partials, in, lp); break;
  }
}

// The lean mapping serves the regroupable folds (every op but PROD) of the
// reference's matrix for T.
template <typename T>
void launch_lean(int k, int op, bool linear, dim3 grid, dim3 block, hipStream_t s,
                 void* partials, const void* in, const t4a::LeanPlan& lp) {
  constexpr bool kFloat = std::is_same_v<T, float> || std::is_same_v<T, double>;
  switch (op) {
    case T4A_CUDA_REDUCE_SUM:
      launch_lean_fold<T, t4a::SumFold>(k, linear, grid, block, s, partials, in, lp);
      break;
    case T4A_CUDA_REDUCE_SUM_SQUARES:
      if constexpr (kFloat)
        launch_lean_fold<T, t4a::SumSquaresFold>(k, linear, grid, block, s, partials, in, lp);
      break;
    case T4A_CUDA_REDUCE_MAX:
      launch_lean_fold<T, t4a::MaxFold>(k, linear, grid, block, s, partials, in, lp);
      break;
    case T4A_CUDA_REDUCE_MIN:
      launch_lean_fold<T, t4a::MinFold>(k, linear, grid, block, s, partials, in, lp);
      break;
    default: break;
  }
}

}  // namespace

extern "C" int t4a_hip_reduce_partials(void* partials, const void* in, int dtype, int op,
                                       const t4a_cuda_layout* partials_layout,
                                       const t4a_cuda_layout* in_layout, int axis,
                                       long long output_len, long long splits,
                                       long long chunk_len, const t4a_launch* launch,
                                       void* stream) {
  if (launch == nullptr || partials_layout == nullptr || in_layout == nullptr)
    return T4A_HIP_ERR_NULL_ARGUMENT;
  if (launch_empty(launch)) return T4A_OK;
  if (partials == nullptr || in == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  const unsigned threads = launch->block[0] * launch->block[1] * launch->block[2];
  const int w = threads <= 32u ? static_cast<int>(threads) : t4a::kWarp;
  // The wavefront-wide mappings run in the planner's kBlock-thread blocks.
  const bool whole_waves = launch->block[1] == 1 && launch->block[2] == 1 &&
                           threads == static_cast<unsigned>(t4a::kBlock);
  const uintptr_t address = reinterpret_cast<uintptr_t>(in);
  const int align = (address & 15) == 0 ? 16 : (address & 7) == 0 ? 8 : (address & 3) == 0 ? 4 : 1;
  t4a::PartialsPlan pp;
  t4a::partials_plan(&pp, *partials_layout, *in_layout, axis, output_len, splits, w,
                     whole_waves && t4a::sideways_dtype(dtype), t4a::dtype_size(dtype), align);
  const dim3 grid(launch->grid[0], launch->grid[1], launch->grid[2]);
  const dim3 block(launch->block[0], launch->block[1], launch->block[2]);
  const bool sideways = pp.mode != t4a::kPartialsPlane;
  const bool aligned_in = (reinterpret_cast<uintptr_t>(in) & 15) == 0;
  // The lean mapping walks cubes with 32-bit indices, a grid stride of eight
  // planes per block.
  const int lean = !sideways && whole_waves && aligned_in &&
                           t4a::grid_stride_fits(pp.units, launch->grid[0],
                                                 t4a::kBlock / t4a::kWarp)
                       ? t4a::lean_slots(pp, dtype, op, splits, chunk_len, w)
                       : 0;
  const bool stream_mode = !lean && !sideways && whole_waves && aligned_in &&
                           t4a::stream_applies(pp, dtype, op, chunk_len, w);
  // Streaming planes split the cubes evenly over the launched planes (whole
  // wavefronts, so at least two planes per block).
  long long per_plane = 1;
  if (stream_mode) {
    const long long planes = static_cast<long long>(grid.x) * (threads / t4a::kWarp);
    per_plane = (output_len * splits + planes - 1) / planes;
  }
  return with_dtype(dtype, [&](auto* tag) {
    using T = std::remove_pointer_t<decltype(tag)>;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (lean > 0) {
      if constexpr (t4a::VecLanes<T>::value > 0) {
        const t4a::LeanPlan lp = t4a::lean_plan(pp, splits, chunk_len);
        launch_lean<T>(lean, op, lp.linear, grid, block, s, partials, in, lp);
      }
    } else if (stream_mode) {
      hipLaunchKernelGGL(t4a::partials_stream_kernel<T>, grid, block, 0,
                         static_cast<hipStream_t>(stream), partials, in, op, pp, output_len,
                         splits, chunk_len, per_plane);
    } else if (sideways) {
      if constexpr (t4a::VecLanes<T>::value > 0) {
        // sideways modes are planned for real and integer types only
        const t4a::SidePlan sp = t4a::side_plan(pp, splits, chunk_len);
        if (pp.mode == t4a::kPartialsTiles) {
          if (pp.cpl == 2)
            hipLaunchKernelGGL((t4a::partials_tiles_kernel<T, 2>), grid, block, 0, s, partials,
                               in, op, sp);
          else
            hipLaunchKernelGGL((t4a::partials_tiles_kernel<T, 1>), grid, block, 0, s, partials,
                               in, op, sp);
        } else if (pp.mode == t4a::kPartialsVecRows) {
          if (pp.cpl == 4)
            hipLaunchKernelGGL((t4a::partials_vecrows_kernel<T, 4>), grid, block, 0, s,
                               partials, in, op, sp);
          else
            hipLaunchKernelGGL((t4a::partials_vecrows_kernel<T, 2>), grid, block, 0, s,
                               partials, in, op, sp);
        } else {
          switch (pp.columns) {
            case 2:
              hipLaunchKernelGGL((t4a::partials_rows_kernel<T, 1>), grid, block, 0, s, partials,
                                 in, op, pp, splits, chunk_len);
              break;
            case 4:
              hipLaunchKernelGGL((t4a::partials_rows_kernel<T, 2>), grid, block, 0, s, partials,
                                 in, op, pp, splits, chunk_len);
              break;
            case 8:
              hipLaunchKernelGGL((t4a::partials_rows_kernel<T, 4>), grid, block, 0, s, partials,
                                 in, op, pp, splits, chunk_len);
              break;
            case 16:
              hipLaunchKernelGGL((t4a::partials_rows_kernel<T, 8>), grid, block, 0, s, partials,
                                 in, op, pp, splits, chunk_len);
              break;
            default:
              hipLaunchKernelGGL((t4a::partials_rows_kernel<T, 16>), grid, block, 0, s,
                                 partials, in, op, pp, splits, chunk_len);
              break;
          }
        }
      }
    } else {
      hipLaunchKernelGGL(t4a::partials_plane_kernel<T>, grid, block, 0,
                         static_cast<hipStream_t>(stream), partials, in, op, pp, output_len,
                         splits, chunk_len);
    }
    return status_of_last_launch();
  });
}

// ---- a whole planned reduction ---------------------------------------------------

namespace {

template <typename T, int K, typename Fold, typename CFold, int C>
void launch_joined_kernel(unsigned int grid, hipStream_t s, void* partials, const void* in,
                          const t4a::LeanPlan& lp, const t4a::JoinedOut& jo) {
  hipLaunchKernelGGL((t4a::reduction_joined_kernel<T, K, Fold, CFold, C>), dim3(grid),
                     dim3(t4a::kBlock), 0, s, partials, in, lp, jo);
}

template <typename T, int K, typename Fold, typename CFold>
void launch_joined_k(int c, unsigned int grid, hipStream_t s, void* partials, const void* in,
                     const t4a::LeanPlan& lp, const t4a::JoinedOut& jo) {
  switch (c) {
    case 1: launch_joined_kernel<T, K, Fold, CFold, 1>(grid, s, partials, in, lp, jo); break;
    case 2: launch_joined_kernel<T, K, Fold, CFold, 2>(grid, s, partials, in, lp, jo); break;
    case 3: launch_joined_kernel<T, K, Fold, CFold, 3>(grid, s, partials, in, lp, jo); break;
    default: launch_joined_kernel<T, K, Fold, CFold, 4>(grid, s, partials, in, lp, jo); break;
  }
}

// How a Split plan runs joined (pass 1 and the combine in one launch): a unit
// combine over at most 32 partials, the lean linear pass 1 (contiguous axis,
// end-to-end equal chunks, 16-byte aligned input) and finals at offset +
// o * stride, and at most eight 16-byte loads a lane once a block's eight
// planes hold all of an output's chunks (heavier shares cost more than the
// combine launch they save: i64 and f64 over 32 splits measured slower). Fills
// the lean plan, the slot count, the chunks per plane, the grid and the
// finals' place; false when the plan does not join.
struct Joined {
  t4a::LeanPlan lp;
  t4a::JoinedOut jo;
  int k;
  int c;
  unsigned int grid;
};

template <typename T, typename Fold, typename CFold>
void launch_joined_fold(const Joined& j, hipStream_t s, void* partials, const void* in) {
  switch (j.k) {
    case 1: launch_joined_k<T, 1, Fold, CFold>(j.c, j.grid, s, partials, in, j.lp, j.jo);
            break;
    case 2: launch_joined_k<T, 2, Fold, CFold>(j.c, j.grid, s, partials, in, j.lp, j.jo);
            break;
    case 3: launch_joined_k<T, 3, Fold, CFold>(j.c, j.grid, s, partials, in, j.lp, j.jo);
            break;
    default:
      launch_joined_k<T, 4, Fold, CFold>(j.c, j.grid, s, partials, in, j.lp, j.jo);
      break;
  }
}

bool joined_applies(const void* in, int dtype, int op, const t4a_cuda_layout& out_layout,
                    const t4a_cuda_layout& in_layout, const t4a_cuda_layout& partials_layout,
                    int axis, long long output_len, const t4a_reduction_plan& plan, Joined* j) {
  const t4a_launch& l = plan.pass1;
  const long long splits = plan.split.splits;
  if (plan.kind != T4A_PLAN_SPLIT || plan.combine_strategy != T4A_CUDA_REDUCE_UNIT ||
      splits < 1 || splits > t4a::kWarp || l.block[0] != static_cast<unsigned>(t4a::kBlock) ||
      l.block[1] != 1 || l.block[2] != 1 || !t4a::sideways_dtype(dtype) || output_len < 1 ||
      (reinterpret_cast<uintptr_t>(in) & 15) != 0)
    return false;
  t4a::PartialsPlan pp;
  t4a::partials_plan(&pp, partials_layout, in_layout, axis, output_len, splits, t4a::kWarp, 1,
                     t4a::dtype_size(dtype), 16);
  if (pp.mode != t4a::kPartialsPlane) return false;
  j->k = t4a::lean_slots(pp, dtype, op, splits, plan.split.chunk_len, t4a::kWarp);
  if (j->k == 0) return false;
  j->lp = t4a::lean_plan(pp, splits, plan.split.chunk_len);
  if (!j->lp.linear) return false;
  // The finals: output o at offset + o * stride (at most one fused dim, the
  // partials' own).
  t4a::ReduceDims ro;
  t4a::reduce_dims(&ro, out_layout, in_layout, axis);
  if (ro.n > 1 || ro.n != pp.dims.n || (ro.n == 1 && ro.ext[0] != pp.dims.ext[0])) return false;
  j->jo.offset = ro.out_offset;
  j->jo.stride = ro.n == 1 ? ro.os[0] : 0;
  constexpr int kLoads = 8;
  constexpr long long kPlanes = t4a::kBlock / t4a::kWarp;
  j->c = static_cast<int>((splits + kPlanes - 1) / kPlanes);
  if (j->c * j->k > kLoads) return false;
  j->jo.outputs = static_cast<unsigned int>(kPlanes * j->c / splits);
  j->grid = static_cast<unsigned int>((output_len + j->jo.outputs - 1) / j->jo.outputs);
  return true;
}

// The joined launch when the plan allows it: returns -1 (no launch) otherwise.
int try_joined(void* out, const void* in, void* partials, int dtype, int op,
               const t4a_cuda_layout& out_layout, const t4a_cuda_layout& in_layout,
               const t4a_cuda_layout& partials_layout, int axis, long long output_len,
               const t4a_reduction_plan& plan, void* stream) {
  Joined j;
  if (!joined_applies(in, dtype, op, out_layout, in_layout, partials_layout, axis, output_len,
                      plan, &j))
    return -1;
  j.jo.out = out;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  return with_dtype(dtype, [&](auto* tag) {
    using T = std::remove_pointer_t<decltype(tag)>;
    if constexpr (t4a::VecLanes<T>::value > 0) {
      constexpr bool kFloat = std::is_same_v<T, float> || std::is_same_v<T, double>;
      switch (op) {
        case T4A_CUDA_REDUCE_SUM:
          launch_joined_fold<T, t4a::SumFold, t4a::SumFold>(j, s, partials, in);
          break;
        case T4A_CUDA_REDUCE_SUM_SQUARES:
          if constexpr (kFloat)
            launch_joined_fold<T, t4a::SumSquaresFold, t4a::SumFold>(j, s, partials, in);
          break;
        case T4A_CUDA_REDUCE_MAX:
          launch_joined_fold<T, t4a::MaxFold, t4a::MaxFold>(j, s, partials, in);
          break;
        case T4A_CUDA_REDUCE_MIN:
          launch_joined_fold<T, t4a::MinFold, t4a::MinFold>(j, s, partials, in);
          break;
        default: return -1;
      }
      return status_of_last_launch();
    }
    return -1;
  });
}

}  // namespace

extern "C" int t4a_hip_reduction(void* out, const void* in, void* partials, int dtype, int op,
                                 const t4a_cuda_layout* out_layout,
                                 const t4a_cuda_layout* in_layout, int axis, long long output_len,
                                 const t4a_reduction_plan* plan, void* stream) {
  if (plan == nullptr || out_layout == nullptr || in_layout == nullptr)
    return T4A_HIP_ERR_NULL_ARGUMENT;
  if (plan->kind == T4A_PLAN_DIRECT)
    return t4a_hip_reduce(out, in, dtype, op, plan->strategy, out_layout, in_layout, axis,
                          output_len, &plan->launch, stream);
  t4a_cuda_layout pl;
  if (int st = t4a_reduction_partials_layout(in_layout, static_cast<unsigned>(axis),
                                             plan->split.splits, &pl))
    return st;
  if (launch_empty(&plan->pass1)) return T4A_OK;
  if (out == nullptr || in == nullptr || partials == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  const int joined = try_joined(out, in, partials, dtype, op, *out_layout, *in_layout, pl, axis,
                                output_len, *plan, stream);
  if (joined >= 0) return joined;
  if (int st = t4a_hip_reduce_partials(partials, in, dtype, op, &pl, in_layout, axis, output_len,
                                       plan->split.splits, plan->split.chunk_len, &plan->pass1,
                                       stream))
    return st;
  return t4a_hip_reduce(out, partials, dtype, plan->combine_op, plan->combine_strategy,
                        out_layout, &pl, axis, output_len, &plan->pass2, stream);
}

extern "C" int t4a_hip_reduction_joins(const void* in, int dtype, int op,
                                       const t4a_cuda_layout* out_layout,
                                       const t4a_cuda_layout* in_layout, int axis,
                                       long long output_len, const t4a_reduction_plan* plan) {
  if (plan == nullptr || out_layout == nullptr || in_layout == nullptr || in == nullptr ||
      plan->kind != T4A_PLAN_SPLIT)
    return 0;
  t4a_cuda_layout pl;
  if (t4a_reduction_partials_layout(in_layout, static_cast<unsigned>(axis), plan->split.splits,
                                    &pl) != T4A_OK)
    return 0;
  Joined j;
  return joined_applies(in, dtype, op, *out_layout, *in_layout, pl, axis, output_len, *plan, &j)
             ? 1
             : 0;
}

// ---- a whole planned reduction that allocates nothing -----------------------------
//
// The partials workspace of t4a_hip_reduction_scratch: one array per GPU,
// loaded with this library's code and held until the process ends. In host
// code `scratch` names a host-side stand-in, not the device array: its device
// address comes from hipGetSymbolAddress, once per device, and only that
// address is ever passed to a kernel.
static __device__ __align__(256) unsigned char scratch[T4A_HIP_SCRATCH_BYTES];

namespace {

constexpr int kScratchDevices = 64;
std::mutex scratch_mutex;
void* scratch_address[kScratchDevices];  // per device; nullptr until first looked up

// The current device's address of `scratch` (looked up on the device's first
// call, with that device current).
int scratch_of_current_device(void** address) {
  int device = -1;
  if (int st = t4a::status_of_hip(static_cast<int>(hipGetDevice(&device)))) return st;
  if (device < 0 || device >= kScratchDevices) return T4A_HIP_ERR_NOT_FOUND;
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (scratch_address[device] == nullptr) {
    void* p = nullptr;
    if (int st = t4a::status_of_hip(
            static_cast<int>(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)))))
      return st;
    if (p == nullptr) return T4A_HIP_ERR_NOT_FOUND;
    scratch_address[device] = p;
  }
  *address = scratch_address[device];
  return T4A_OK;
}

}  // namespace

extern "C" int t4a_hip_reduction_scratch(void* out, const void* in, int dtype, int op,
                                         const t4a_cuda_layout* out_layout,
                                         const t4a_cuda_layout* in_layout, int axis,
                                         long long output_len, const t4a_reduction_plan* plan,
                                         void* stream) {
  if (plan == nullptr || out_layout == nullptr || in_layout == nullptr)
    return T4A_HIP_ERR_NULL_ARGUMENT;
  if (plan->kind == T4A_PLAN_DIRECT)  // one pass: no workspace
    return t4a_hip_reduction(out, in, nullptr, dtype, op, out_layout, in_layout, axis,
                             output_len, plan, stream);
  // The partials' size is checked before the device is touched.
  t4a_cuda_layout pl;
  if (int st = t4a_reduction_partials_layout(in_layout, static_cast<unsigned>(axis),
                                             plan->split.splits, &pl))
    return st;
  long long count = 0;
  if (int st = t4a_layout_element_count(&pl, &count)) return st;
  const long long esize = t4a::dtype_size(dtype);
  if (esize == 0) return T4A_OK;  // unknown tag: no work, as t4a_hip_reduction
  if (count > static_cast<long long>(T4A_HIP_SCRATCH_BYTES) / esize)
    return T4A_HIP_ERR_SCRATCH_LIMIT;
  if (launch_empty(&plan->pass1)) return T4A_OK;
  void* partials = nullptr;
  if (int st = scratch_of_current_device(&partials)) return st;
  return t4a_hip_reduction(out, in, partials, dtype, op, out_layout, in_layout, axis,
                           output_len, plan, stream);
}

// The general-rank twins on the caller's stream with a planned geometry (any
// t4a_plan_*_any geometry: the twins stride over their work).
extern "C" int t4a_hip_reduce_any(void* out, const void* in, int dtype, int op, int strategy,
                                  const t4a_cuda_layout_any* out_layout,
                                  const t4a_cuda_layout_any* in_layout, int axis,
                                  long long output_len, const t4a_launch* launch, void* stream) {
  if (launch == nullptr || out_layout == nullptr || in_layout == nullptr)
    return T4A_HIP_ERR_NULL_ARGUMENT;
  if (launch_empty(launch)) return T4A_OK;
  if (out == nullptr || in == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  const dim3 grid(launch->grid[0], launch->grid[1], launch->grid[2]);
  const dim3 block(launch->block[0], launch->block[1], launch->block[2]);
  hipLaunchKernelGGL(t4a_cuda_reduce_any, grid, block, 0, static_cast<hipStream_t>(stream), out,
                     in, dtype, op, strategy, *out_layout, *in_layout, axis, output_len);
  return status_of_last_launch();
}

extern "C" int t4a_hip_reduce_partials_any(void* partials, const void* in, int dtype, int op,
                                           const t4a_cuda_layout_any* partials_layout,
                                           const t4a_cuda_layout_any* in_layout, int axis,
                                           long long output_len, long long splits,
                                           long long chunk_len, const t4a_launch* launch,
                                           void* stream) {
  if (launch == nullptr || partials_layout == nullptr || in_layout == nullptr)
    return T4A_HIP_ERR_NULL_ARGUMENT;
  if (launch_empty(launch)) return T4A_OK;
  if (partials == nullptr || in == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  const dim3 grid(launch->grid[0], launch->grid[1], launch->grid[2]);
  const dim3 block(launch->block[0], launch->block[1], launch->block[2]);
  hipLaunchKernelGGL(t4a_cuda_reduce_partials_any, grid, block, 0,
                     static_cast<hipStream_t>(stream), partials, in, dtype, op,
                     *partials_layout, *in_layout, axis, output_len, splits, chunk_len);
  return status_of_last_launch();
}
