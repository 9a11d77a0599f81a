// Device element arithmetic, fold objects and 32-lane plane collectives for
// gfx950.
//
// The arithmetic restates the reference's element semantics
// (reference cuda/include/t4a/abi.cuh:590-818): wrapping integer sum and
// product, IEEE float and componentwise complex arithmetic, a square rounded
// before it is added, and NaN-propagating extrema that order -0 below +0. All
// HIP sources are built with -ffp-contract=off, so every rounding is the one
// written here; the complex product spells out its fused multiply-adds.
#ifndef T4A_DEVICE_H_
#define T4A_DEVICE_H_

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "geometry.h"

namespace t4a {

// Threads per block: the launcher's compile-time block size BS, or, for BS = 0
// (the geometry-agnostic reference entries), blockDim.x. blockDim is an
// implicit kernel argument that a wavefront fetches with a vector memory load,
// so a short-lived wavefront that reads it waits one memory round trip before
// its first data load; a constant costs nothing.
template <int BS>
__device__ __forceinline__ int block_threads() {
  if constexpr (BS > 0) {
    return BS;
  } else {
    return static_cast<int>(blockDim.x);
  }
}

// The reference-named entries plan inside the kernel: thread 0 of each block
// derives the plan from the entry's arguments before the block's first load.
// Under the reference planner's geometry -- a thread per element or per
// output, 65,536 blocks for a 16M-element move -- that planning would run once
// per block, round after round of resident blocks. So an entry keeps at most
// kEntryWaves wavefronts' worth of blocks of the grid's first row working
// (blocks past that, and blocks off the first row, return before planning),
// and the kept blocks walk all of the work with their own count as the grid
// stride. The movement entries keep 2048 wavefronts (512 blocks of 256
// threads): about half of what their registers and LDS let the chip hold, so
// the returning blocks pass through the remaining slots while the working
// ones stream (a cap at full residency measured slower: the returning blocks
// then wait for the work to finish). The reduction entries keep 8192, the
// chip's whole wavefront capacity: their plane walks wait on each cube's
// loads in turn, so every working plane adds loads in flight, and their
// planning is a few dozen instructions.
constexpr unsigned int kMoveEntryWaves = 2048;
constexpr unsigned int kReduceEntryWaves = 8192;

// The launchers' persistent tile walk takes as many blocks as the device
// holds at once; this is the count for MI355X (256 CUs x 8 blocks of 256
// threads) when the runtime cannot be asked.
constexpr unsigned int kTileWalkBlocks = 2048;

// A grid of at most this many wavefronts (four of the entry kernels' blocks
// of 256 threads per CU, what their registers and LDS let the chip hold) has
// no block waiting for a slot: every block of its first row works, whatever
// the cap. This build's planner gives the entries such grids where it can
// (TILED plans); the reference's per-element grids are far larger.
constexpr unsigned int kEntryResidentWaves = 4096;

__device__ __forceinline__ unsigned int entry_blocks(unsigned int waves) {
  const unsigned int waves_per_block = (blockDim.x * blockDim.y * blockDim.z + 63u) / 64u;
  const unsigned int wpb = waves_per_block ? waves_per_block : 1u;
  if (static_cast<unsigned long long>(gridDim.x) * wpb <= kEntryResidentWaves) return gridDim.x;
  unsigned int cap = waves / wpb;
  if (cap == 0) cap = 1;
  return gridDim.x < cap ? gridDim.x : cap;
}

// The pass-1 entries: blocks of one wavefront or less (the reference
// geometry's one-plane blocks, 262,144 of them for C2) keep 2048 working
// blocks, so that the returning blocks still find slots (and each working
// plane keeps several cubes in flight); larger blocks keep 8192 wavefronts'
// worth, as the other reduction entries do. C2's f32 sums under the reference
// geometry (both passes) took 106-111 us with 2048, 113-116 with 4096,
// 118-128 with 8192 and 118-137 with 1024.
__device__ __forceinline__ unsigned int partials_entry_waves() {
  return blockDim.x * blockDim.y * blockDim.z <= 64u ? 2048u : kReduceEntryWaves;
}

__device__ __forceinline__ bool entry_block_idle(unsigned int waves) {
  return blockIdx.y != 0 || blockIdx.z != 0 || blockIdx.x >= entry_blocks(waves);
}

using c32 = t4a_cuda_c32;
using c64 = t4a_cuda_c64;

// ---- element arithmetic ------------------------------------------------------

template <typename T>
__device__ __forceinline__ T add(T a, T b) { return a + b; }
template <>
__device__ __forceinline__ int add<int>(int a, int b) {
  return static_cast<int>(static_cast<unsigned>(a) + static_cast<unsigned>(b));
}
template <>
__device__ __forceinline__ long long add<long long>(long long a, long long b) {
  return static_cast<long long>(static_cast<unsigned long long>(a) +
                                static_cast<unsigned long long>(b));
}
template <>
__device__ __forceinline__ c32 add<c32>(c32 a, c32 b) { return c32{a.re + b.re, a.im + b.im}; }
template <>
__device__ __forceinline__ c64 add<c64>(c64 a, c64 b) { return c64{a.re + b.re, a.im + b.im}; }

template <typename T>
__device__ __forceinline__ T mul(T a, T b) { return a * b; }
template <>
__device__ __forceinline__ int mul<int>(int a, int b) {
  return static_cast<int>(static_cast<unsigned>(a) * static_cast<unsigned>(b));
}
template <>
__device__ __forceinline__ long long mul<long long>(long long a, long long b) {
  return static_cast<long long>(static_cast<unsigned long long>(a) *
                                static_cast<unsigned long long>(b));
}
// (a.re*b.re - a.im*b.im, a.re*b.im + a.im*b.re) with one product of each
// component fused: re = fma(a.re, b.re, -(a.im*b.im)), im = fma(a.im, b.re,
// a.re*b.im). This is the rounding of the reference build's contracted complex
// product, written out explicitly (the reference's A100 golden vectors select
// it among the possible contractions).
template <>
__device__ __forceinline__ c32 mul<c32>(c32 a, c32 b) {
  const float ii = a.im * b.im;
  const float ri = a.re * b.im;
  return c32{__builtin_fmaf(a.re, b.re, -ii), __builtin_fmaf(a.im, b.re, ri)};
}
template <>
__device__ __forceinline__ c64 mul<c64>(c64 a, c64 b) {
  const double ii = a.im * b.im;
  const double ri = a.re * b.im;
  return c64{__builtin_fma(a.re, b.re, -ii), __builtin_fma(a.im, b.re, ri)};
}

// A square rounded once, before any later addition.
template <typename T>
__device__ __forceinline__ T square(T v) { return v; }
template <>
__device__ __forceinline__ float square<float>(float v) { return __builtin_fmaf(v, v, 0.0f); }
template <>
__device__ __forceinline__ double square<double>(double v) { return __builtin_fma(v, v, 0.0); }

// NaN wins (lhs first); equal operands differ at most in the sign of zero, and
// the maximum keeps +0 (AND of the bit patterns), the minimum -0 (OR).
__device__ __forceinline__ float fmax_nan(float l, float r) {
  const float both = __uint_as_float(__float_as_uint(l) & __float_as_uint(r));
  const float ordered = l == r ? both : (r > l ? r : l);
  const float right = r != r ? r : ordered;
  return l != l ? l : right;
}
__device__ __forceinline__ float fmin_nan(float l, float r) {
  const float either = __uint_as_float(__float_as_uint(l) | __float_as_uint(r));
  const float ordered = l == r ? either : (r < l ? r : l);
  const float right = r != r ? r : ordered;
  return l != l ? l : right;
}
__device__ __forceinline__ double fmax_nan(double l, double r) {
  const double both =
      __longlong_as_double(__double_as_longlong(l) & __double_as_longlong(r));
  const double ordered = l == r ? both : (r > l ? r : l);
  const double right = r != r ? r : ordered;
  return l != l ? l : right;
}
__device__ __forceinline__ double fmin_nan(double l, double r) {
  const double either =
      __longlong_as_double(__double_as_longlong(l) | __double_as_longlong(r));
  const double ordered = l == r ? either : (r < l ? r : l);
  const double right = r != r ? r : ordered;
  return l != l ? l : right;
}

template <typename T>
__device__ __forceinline__ T vmax(T a, T b) { return a > b ? a : b; }
template <typename T>
__device__ __forceinline__ T vmin(T a, T b) { return a < b ? a : b; }
template <>
__device__ __forceinline__ float vmax<float>(float a, float b) { return fmax_nan(a, b); }
template <>
__device__ __forceinline__ float vmin<float>(float a, float b) { return fmin_nan(a, b); }
template <>
__device__ __forceinline__ double vmax<double>(double a, double b) { return fmax_nan(a, b); }
template <>
__device__ __forceinline__ double vmin<double>(double a, double b) { return fmin_nan(a, b); }

// IEEE 754-2019 maximum / minimum: NaN-propagating, -0 below +0
// (v_maximum3_f32 / v_minimum3_f32 on gfx950, three operands per instruction).
// Among non-NaN operands the select-form extrema above pick the same bits in any
// order (equal values AND / OR their bits, which orders -0 below +0), so a Max
// or Min fold without a NaN may take any order through these; a NaN result
// sends the caller back to the select form, whose NaN choice is
// order-dependent.
template <typename T>
__device__ __forceinline__ T ieee_maximum(T a, T b) {
  return __builtin_elementwise_maximum(a, b);
}
template <typename T>
__device__ __forceinline__ T ieee_minimum(T a, T b) {
  return __builtin_elementwise_minimum(a, b);
}

// ---- folds ---------------------------------------------------------------------
// seed(v): the accumulator's first value; fold(acc, v): one more element;
// combine(a, b): two accumulators. Only SUM_SQUARES tells fold and combine apart
// (reference cuda/src/reduce.cu:25-108). kRegroup: pass 1 may take the grouped
// walk (every fold except PROD).

struct SumFold {
  static constexpr bool kRegroup = true;
  template <typename T> __device__ __forceinline__ T seed(T v) const { return v; }
  template <typename T> __device__ __forceinline__ T fold(T a, T v) const { return add(a, v); }
  template <typename T> __device__ __forceinline__ T combine(T a, T b) const { return add(a, b); }
};
struct ProdFold {
  static constexpr bool kRegroup = false;
  template <typename T> __device__ __forceinline__ T seed(T v) const { return v; }
  template <typename T> __device__ __forceinline__ T fold(T a, T v) const { return mul(a, v); }
  template <typename T> __device__ __forceinline__ T combine(T a, T b) const { return mul(a, b); }
};
struct SumSquaresFold {
  static constexpr bool kRegroup = true;
  template <typename T> __device__ __forceinline__ T seed(T v) const { return square(v); }
  template <typename T> __device__ __forceinline__ T fold(T a, T v) const { return add(a, square(v)); }
  template <typename T> __device__ __forceinline__ T combine(T a, T b) const { return add(a, b); }
};
struct MaxFold {
  static constexpr bool kRegroup = true;
  template <typename T> __device__ __forceinline__ T seed(T v) const { return v; }
  template <typename T> __device__ __forceinline__ T fold(T a, T v) const { return vmax(a, v); }
  template <typename T> __device__ __forceinline__ T combine(T a, T b) const { return vmax(a, b); }
};
struct MinFold {
  static constexpr bool kRegroup = true;
  template <typename T> __device__ __forceinline__ T seed(T v) const { return v; }
  template <typename T> __device__ __forceinline__ T fold(T a, T v) const { return vmin(a, v); }
  template <typename T> __device__ __forceinline__ T combine(T a, T b) const { return vmin(a, b); }
};

// ---- lane exchange ---------------------------------------------------------------
// xor exchange inside aligned groups of `width` lanes of the 64-lane wavefront.

__device__ __forceinline__ float shfl_xor(float v, int m, int w) { return __shfl_xor(v, m, w); }
__device__ __forceinline__ double shfl_xor(double v, int m, int w) { return __shfl_xor(v, m, w); }
__device__ __forceinline__ int shfl_xor(int v, int m, int w) { return __shfl_xor(v, m, w); }
__device__ __forceinline__ long long shfl_xor(long long v, int m, int w) {
  return __shfl_xor(v, m, w);
}
__device__ __forceinline__ c32 shfl_xor(c32 v, int m, int w) {
  return c32{__shfl_xor(v.re, m, w), __shfl_xor(v.im, m, w)};
}
__device__ __forceinline__ c64 shfl_xor(c64 v, int m, int w) {
  return c64{__shfl_xor(v.re, m, w), __shfl_xor(v.im, m, w)};
}

// The plane xor tree: offsets 1, 2, 4, ... < width, each lane combining its own
// value (left) with its partner's (reference reduce.cu:148-157). Lane 0 ends
// with the own-left pairwise tree of the plane's lanes.
template <typename Fold, typename T>
__device__ __forceinline__ T plane_tree(T v, int width, Fold f) {
  for (int off = 1; off < width; off <<= 1) v = f.combine(v, shfl_xor(v, off, width));
  return v;
}

// The any-order twin of a float Max / Min fold (see ieee_maximum), or void.
template <typename Fold, typename T>
struct AnyOrder {
  using type = void;
};
struct AnyOrderMax {
  template <typename T> __device__ __forceinline__ T seed(T v) const { return v; }
  template <typename T> __device__ __forceinline__ T fold(T a, T v) const {
    return ieee_maximum(a, v);
  }
  template <typename T> __device__ __forceinline__ T combine(T a, T b) const {
    return ieee_maximum(a, b);
  }
};
struct AnyOrderMin {
  template <typename T> __device__ __forceinline__ T seed(T v) const { return v; }
  template <typename T> __device__ __forceinline__ T fold(T a, T v) const {
    return ieee_minimum(a, v);
  }
  template <typename T> __device__ __forceinline__ T combine(T a, T b) const {
    return ieee_minimum(a, b);
  }
};
template <> struct AnyOrder<MaxFold, float> { using type = AnyOrderMax; };
template <> struct AnyOrder<MaxFold, double> { using type = AnyOrderMax; };
template <> struct AnyOrder<MinFold, float> { using type = AnyOrderMin; };
template <> struct AnyOrder<MinFold, double> { using type = AnyOrderMin; };

// Folds whose combine is commutative bit for bit whenever the result is not a
// NaN: real and integer additions (SUM, and SUM_SQUARES's combine), integer
// extrema and the any-order float extrema. Their plane tree can pair lanes
// with DPP moves instead of xor shuffles through LDS.
template <typename Fold, typename T>
struct Commutes {
  static constexpr bool value = false;
};
template <typename T>
constexpr bool kRealOrInt = std::is_same_v<T, float> || std::is_same_v<T, double> ||
                            std::is_same_v<T, int> || std::is_same_v<T, long long>;
template <typename T> struct Commutes<SumFold, T> { static constexpr bool value = kRealOrInt<T>; };
template <typename T> struct Commutes<SumSquaresFold, T> {
  static constexpr bool value = kRealOrInt<T>;
};
template <typename T> struct Commutes<MaxFold, T> {
  static constexpr bool value = std::is_same_v<T, int> || std::is_same_v<T, long long>;
};
template <typename T> struct Commutes<MinFold, T> {
  static constexpr bool value = std::is_same_v<T, int> || std::is_same_v<T, long long>;
};
template <typename T> struct Commutes<AnyOrderMax, T> {
  static constexpr bool value = std::is_same_v<T, float> || std::is_same_v<T, double>;
};
template <typename T> struct Commutes<AnyOrderMin, T> {
  static constexpr bool value = std::is_same_v<T, float> || std::is_same_v<T, double>;
};

// A DPP lane move of a 4- or 8-byte value (Ctrl: the DPP control word).
template <int Ctrl, typename T>
__device__ __forceinline__ T dpp_move(T v) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "one or two words");
  int w[sizeof(T) / 4];
  __builtin_memcpy(w, &v, sizeof(T));
#pragma unroll
  for (int k = 0; k < static_cast<int>(sizeof(T) / 4); ++k)
    w[k] = __builtin_amdgcn_update_dpp(0, w[k], Ctrl, 0xF, 0xF, false);
  __builtin_memcpy(&v, w, sizeof(T));
  return v;
}

template <typename T>
__device__ __forceinline__ T read_lane(T v, int lane) {
  int w[sizeof(T) / 4];
  __builtin_memcpy(w, &v, sizeof(T));
#pragma unroll
  for (int k = 0; k < static_cast<int>(sizeof(T) / 4); ++k)
    w[k] = __builtin_amdgcn_readlane(w[k], lane);
  __builtin_memcpy(&v, w, sizeof(T));
  return v;
}

// The plane tree of a 32-lane plane (lanes 0-31 or 32-63 of the wavefront)
// for a commuting fold; every lane of the plane ends with the result. The pairs
// are the xor tree's: after offsets 1 and 2 (quad_perm moves) each quad holds
// one value -- the two lanes of a pair compute combine(a, b) and combine(b,
// a), equal for a commuting fold -- so row_half_mirror (lane i takes lane
// 7 - i) pairs each quad with its xor-4 partner and, the eight lanes then
// holding one value, row_mirror (i takes 15 - i) pairs each eight with its
// xor-8 partner; offset 16 combines lanes 0 and 16 (or 32 and 48), read as
// scalars. No LDS traffic and no waits, where an xor shuffle is an LDS permute
// per offset. A float result that is a NaN (then so on every lane of the
// plane) is recomputed by the own-left xor tree, whose NaN payload is the
// reference's: commutativity holds only for non-NaN results. Every lane of the
// plane must be active.
template <typename Fold, typename T>
__device__ __forceinline__ T plane_tree32(T v, Fold f) {
  if constexpr (Commutes<Fold, T>::value) {
    T r = f.combine(v, dpp_move<0xB1>(v));  // quad_perm [1, 0, 3, 2]: xor 1
    r = f.combine(r, dpp_move<0x4E>(r));    // quad_perm [2, 3, 0, 1]: xor 2
    r = f.combine(r, dpp_move<0x141>(r));   // row_half_mirror
    r = f.combine(r, dpp_move<0x140>(r));   // row_mirror
    // All four reads first: a read inside a conditional arm becomes a branch.
    const T r0 = read_lane(r, 0);
    const T r16 = read_lane(r, 16);
    const T r32 = read_lane(r, 32);
    const T r48 = read_lane(r, 48);
    const bool upper = (threadIdx.x & 32) != 0;
    r = f.combine(upper ? r32 : r0, upper ? r48 : r16);
    if constexpr (std::is_same_v<T, float> || std::is_same_v<T, double>) {
      if (r != r) r = plane_tree(v, kWarp, f);
    }
    return r;
  } else {
    return plane_tree(v, kWarp, f);
  }
}

// Pairwise own-left tree over `n` register values (n a power of two); the
// value of lane 0 of a plane whose lanes are held by one thread.
template <int N, typename Fold, typename T>
__device__ __forceinline__ T register_tree(T* v, Fold f) {
#pragma unroll
  for (int off = 1; off < N; off <<= 1) {
#pragma unroll
    for (int l = 0; l < N; l += 2 * off) v[l] = f.combine(v[l], v[l + off]);
  }
  return v[0];
}

// ---- vector payloads -----------------------------------------------------------

struct alignas(16) Bits128 {
  unsigned long long lo, hi;
};
// A 16-byte element that is only 8-byte aligned (c64).
struct alignas(8) Elem16 {
  unsigned long long lo, hi;
};

// V payloads moved as one access: a 16-byte vector when V > 1, else the
// payload at its own alignment (a c64 element is only 8-byte aligned).
template <typename P, int V>
struct alignas(V > 1 ? sizeof(P) * V : alignof(P)) Vec {
  P v[V];
};

// Streaming (non-temporal) loads and stores of a Vec: data moved once is not
// kept in the caches. The access width is the Vec's size, split into 8-byte
// halves when the Vec is only 8-byte aligned.
using u32x4 = unsigned int __attribute__((ext_vector_type(4)));
using u32x2 = unsigned int __attribute__((ext_vector_type(2)));

template <typename P, int V>
__device__ __forceinline__ Vec<P, V> nt_load(const P* p) {
  constexpr int kBytes = static_cast<int>(sizeof(P)) * V;
  Vec<P, V> out;
  if constexpr (kBytes == 16 && alignof(Vec<P, V>) == 16) {
    const u32x4 r = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    __builtin_memcpy(&out, &r, 16);
  } else if constexpr (kBytes == 16) {
    const u32x2 lo = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
    const u32x2 hi = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p) + 1);
    __builtin_memcpy(&out, &lo, 8);
    __builtin_memcpy(reinterpret_cast<char*>(&out) + 8, &hi, 8);
  } else if constexpr (kBytes == 8) {
    const u32x2 r = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
    __builtin_memcpy(&out, &r, 8);
  } else if constexpr (kBytes == 4) {
    const unsigned r = __builtin_nontemporal_load(reinterpret_cast<const unsigned*>(p));
    __builtin_memcpy(&out, &r, 4);
  } else {
    out = *reinterpret_cast<const Vec<P, V>*>(p);
  }
  return out;
}

template <typename P, int V>
__device__ __forceinline__ void nt_store(P* p, const Vec<P, V>& x) {
  constexpr int kBytes = static_cast<int>(sizeof(P)) * V;
  if constexpr (kBytes == 16 && alignof(Vec<P, V>) == 16) {
    u32x4 r;
    __builtin_memcpy(&r, &x, 16);
    __builtin_nontemporal_store(r, reinterpret_cast<u32x4*>(p));
  } else if constexpr (kBytes == 16) {
    u32x2 lo, hi;
    __builtin_memcpy(&lo, &x, 8);
    __builtin_memcpy(&hi, reinterpret_cast<const char*>(&x) + 8, 8);
    __builtin_nontemporal_store(lo, reinterpret_cast<u32x2*>(p));
    __builtin_nontemporal_store(hi, reinterpret_cast<u32x2*>(p) + 1);
  } else if constexpr (kBytes == 8) {
    u32x2 r;
    __builtin_memcpy(&r, &x, 8);
    __builtin_nontemporal_store(r, reinterpret_cast<u32x2*>(p));
  } else if constexpr (kBytes == 4) {
    unsigned r;
    __builtin_memcpy(&r, &x, 4);
    __builtin_nontemporal_store(r, reinterpret_cast<unsigned*>(p));
  } else {
    *reinterpret_cast<Vec<P, V>*>(p) = x;
  }
}

}  // namespace t4a

#endif  // T4A_DEVICE_H_
