// Launch-independent work decompositions shared by the host planner and the
// gfx950 kernels. Every function here is a pure function of an entry's
// arguments, so the planner (which sizes the grid) and the kernel (which walks
// the work) always agree. The kernels walk their work items with grid-stride
// loops, so any geometry computes the same result; the planned one is the fast
// one.
//
// Nothing here changes *what* an entry computes: movement is a bijection of
// logical coordinates, and the reductions keep the reference's per-element fold
// order (which lane of which plane folds which element, reference
// cuda/src/reduce.cu:343-633). Only the mapping of that work onto MI355X
// wavefronts is chosen here.
#ifndef T4A_GEOMETRY_H_
#define T4A_GEOMETRY_H_

#include "t4a/abi.h"

#if defined(__HIP__)
#define T4A_HD __host__ __device__ __forceinline__
#else
#define T4A_HD inline
#endif

namespace t4a {

// Threads per block of the MI355X launches this library plans (four 64-lane
// wavefronts; the tiled transpose runs eight).
constexpr int kBlock = 256;
// Unit reductions over a few thousand outputs (combine passes) run one
// wavefront per block so that they spread over more CUs.
constexpr int kUnitSmallBlock = 64;
constexpr int kTransposeBlock = 512;
constexpr int kWave = 64;
// Lanes of a reference "warp": planes wider than this cross it (reduce.cu:140).
constexpr int kWarp = 32;

T4A_HD int dtype_size(int dtype) {
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

// ---- tiled transpose ----------------------------------------------------------
//
// dst[b*S + i + j*M] = src[src_offset + b*S + i*N + j] (reference
// docs/abi/c-kernel-abi.md:151-159). A tile is tile_m source rows (i) by
// tile_n source columns (j), staged through LDS by one 512-thread block; the
// batch is the grid's z coordinate, like the reference's (x, y, z) grid.
struct TransposeTiling {
  int tile_m;
  int tile_n;
  long long tiles_m;
  long long tiles_n;
  long long total;  // tiles over all batches
};

T4A_HD TransposeTiling transpose_tiling(long long m, long long n, long long batches,
                                        int esize) {
  TransposeTiling t;
  // About 64 KiB of LDS per tile: 128 x 128 elements up to 4 bytes, 128 x 64
  // of 8 bytes, 64 x 64 of 16 bytes.
  t.tile_m = esize >= 16 ? 64 : 128;
  t.tile_n = esize >= 8 ? 64 : 128;
  t.tiles_m = (m + t.tile_m - 1) / t.tile_m;
  t.tiles_n = (n + t.tile_n - 1) / t.tile_n;
  t.total = t.tiles_m * t.tiles_n * batches;
  return t;
}

// ---- strided movement -----------------------------------------------------------
//
// Both movement entries copy every logical coordinate of a shared extent set
// from a source layout to a destination layout. The plan fuses the axes into at
// most eight "dims" (extent-one axes dropped, axes contiguous in both layouts
// merged), then picks:
//   TILED   the destination-contiguous run (dims chained from the dim of
//           destination stride 1) differs from the source-contiguous run
//           (chained from the dim of source stride 1): an LA x LB tile through
//           LDS, read along the source run and written along the destination run;
//   CONTIG  the same dim is contiguous on both sides: row copies;
//   GENERIC anything else (broadcast or reversed fast axes): per-element decode.
enum MoveMode { kMoveEmpty = 0, kMoveGeneric = 1, kMoveContig = 2, kMoveTiled = 3 };

constexpr int kMaxDims = T4A_CUDA_MAX_RANK;
// Longest run of a movement tile (entries of each LDS offset table) and the
// LDS bytes of its padded tile: 64 x 33 16-byte elements, 128 x 33 8-byte ones.
constexpr long long kMoveRunMax = 128;
constexpr long long kMoveTileBytes = 64 * 33 * 16;

// Division of x < 2^31 by an invariant d >= 1 as a multiply-high, an add and a
// shift (Granlund and Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, section 4): with l = ceil(log2 d) and
// m = floor(2^32 (2^l - d) / d) + 1, q = (mulhi(m, x) + x) >> l; x < 2^31 keeps
// the sum inside 32 bits. AMD GPUs have no integer divide instruction: a
// runtime 32-bit division is a dozen dependent instructions.
struct FastDiv {
  unsigned int d;
  unsigned int m;
  int shift;
};

T4A_HD FastDiv fast_div(unsigned int d) {
  FastDiv f;
  if (d == 0) d = 1;  // no divisor of an empty walk is ever used; keep it defined
  f.d = d;
  if (d > 0x80000000u) {
    // Every dividend (x < 2^31) is below d: the quotient is 0, which m = 0 and
    // a shift of 31 give exactly (the general form would shift by 32).
    f.m = 0;
    f.shift = 31;
    return f;
  }
  int l = 0;
  while ((1ull << l) < d) ++l;
  f.shift = l;
  f.m = static_cast<unsigned int>((((1ull << l) - d) << 32) / d + 1);
  return f;
}

T4A_HD unsigned int div_by(unsigned int x, const FastDiv& f) {
#if defined(__HIP_DEVICE_COMPILE__)
  const unsigned int t = __umulhi(f.m, x);
#else
  const unsigned int t =
      static_cast<unsigned int>((static_cast<unsigned long long>(f.m) * x) >> 32);
#endif
  return (t + x) >> f.shift;
}

struct MovePlan {
  int mode;
  int n;                      // fused dims
  long long ext[kMaxDims];
  long long ss[kMaxDims];     // source strides
  long long ds[kMaxDims];     // destination strides
  long long src_offset;
  long long dst_offset;
  long long len;              // logical elements
  // TILED: the A chain (destination run) is dims a_dims[0..na), the last one
  // tiled by a_tile; the B chain (source run) is b_dims[0..nb), the last tiled
  // by b_tile. la/lb are the run lengths of a full tile.
  int na, nb;
  int a_dims[kMaxDims];
  int b_dims[kMaxDims];
  long long a_tile, b_tile;
  long long la, lb;
  long long a_inner, b_inner;  // product of full extents before the tiled dim
  // Batch dims: every dim outside both chains, plus the two tiled dims' tile
  // counts, walked with the A tile count fastest.
  int nbatch;
  int batch_dims[kMaxDims];
  long long a_tiles, b_tiles;
  long long tiles;            // total work items (tiles, rows or elements)
  // Tile coordinates as 32-bit quotients when tiles < 2^30: the divisors of
  // the coordinate extents in walk order (A tiles, B tiles, batch dims).
  bool coords32;
  FastDiv coord_div[kMaxDims + 2];
  // CONTIG: dim `row_dim` is contiguous on both sides; rows are decoded over
  // the other dims.
  int row_dim;
  long long row_len;
  long long rows;
};

T4A_HD int move_chain_contains(const int* dims, int count, int dim) {
  for (int i = 0; i < count; ++i) {
    if (dims[i] == dim) return 1;
  }
  return 0;
}

// Fused movement geometry of any rank: every axis of extent 1 dropped, and an
// axis whose source and destination strides both continue the previous kept
// axis's span merged into it (axis 0 first). `src(k)` / `dst(k)` give axis k's
// strides (called once per axis, in axis order). Writes at most `cap` fused
// axes to fe / fs / fd and returns their count, or -1 when more remain. With
// no extent 0 every fused axis has extent >= 2, so a layout of fewer than 2^63
// elements fuses to at most 62 axes.
constexpr int kMaxFusedDims = 64;

// The element count a movement may touch: `len` (the caller's count) capped at
// the product of the `n` extents, so a count past the layout's elements never
// walks an axis past its extent. An extent <= 0 leaves nothing.
T4A_HD long long clamp_count(int n, const long long* ext, long long len) {
  if (len <= 0) return 0;
  for (int k = 0; k < n; ++k) {
    if (ext[k] <= 0) return 0;
  }
  long long c = 1;
  for (int k = 0; k < n; ++k) {
    if (c > len / ext[k]) return len;
    c *= ext[k];
  }
  return c < len ? c : len;
}

template <typename SrcStride, typename DstStride>
T4A_HD int fuse_move_by(int rank, const long long* ext, SrcStride src, DstStride dst,
                        long long* fe, long long* fs, long long* fd, int cap) {
  int n = 0;
  for (int k = 0; k < rank; ++k) {
    const long long e = ext[k];
    const long long s = src(k);
    const long long d = dst(k);
    if (e == 1) continue;
    if (n > 0 && s == fs[n - 1] * fe[n - 1] && d == fd[n - 1] * fe[n - 1]) {
      fe[n - 1] *= e;
      continue;
    }
    if (n == cap) return -1;
    fe[n] = e;
    fs[n] = s;
    fd[n] = d;
    ++n;
  }
  return n;
}

// Strides of a compact layout over `ext`, axis by axis in order (the running
// extent product; a stateful functor for fuse_move_by).
struct CompactStrides {
  const long long* ext;
  unsigned long long next;
  T4A_HD long long operator()(int k) {
    const long long s = static_cast<long long>(next);
    next *= static_cast<unsigned long long>(ext[k]);
    return s;
  }
};

// Array strides, or (null) those of the compact layout over `ext`.
struct StridesOf {
  const long long* strides;
  CompactStrides compact;
  T4A_HD long long operator()(int k) { return strides ? strides[k] : compact(k); }
};

T4A_HD StridesOf strides_of(const long long* strides, const long long* ext) {
  return StridesOf{strides, CompactStrides{ext, 1}};
}

// broadcast_in_dim's source seen over the destination's axes (reference
// cuda/src/movement.cu:409-434): destination axis k reads input axis i where
// dims[i] = k with that axis's stride, or stride 0 (broadcast) when no input
// axis maps to k or the input extent there is one.
struct BroadcastStrides {
  const long long* dims;
  int dims_rank;
  const long long* in_ext;
  const long long* in_st;
  T4A_HD long long operator()(int k) const {
    for (int i = 0; i < dims_rank; ++i) {
      if (dims[i] == k) return in_ext[i] == 1 ? 0 : in_st[i];
    }
    return 0;
  }
};

// Array strides, or the compact layout's when `strides` is null.
T4A_HD int fuse_move(int rank, const long long* ext, const long long* ss, const long long* ds,
                     long long* fe, long long* fs, long long* fd, int cap) {
  CompactStrides cs{ext, 1}, cd{ext, 1};
  return fuse_move_by(
      rank, ext, [&](int k) { return ss ? ss[k] : cs(k); },
      [&](int k) { return ds ? ds[k] : cd(k); }, fe, fs, fd, cap);
}

// GENERIC: one decode per element over the fused dims; in 32-bit arithmetic
// with multiply-high divisors (coord_div[k] for dim k) when the count and every
// extent are below 2^31 (a 64-bit division per dim per element otherwise).
T4A_HD void move_generic(MovePlan* p, long long len) {
  p->mode = kMoveGeneric;
  p->tiles = len;
  bool narrow = len < (1ll << 31);
  for (int k = 0; k < p->n; ++k) narrow = narrow && p->ext[k] < (1ll << 31);
  p->coords32 = narrow;
  if (narrow) {
    for (int k = 0; k < p->n; ++k)
      p->coord_div[k] = fast_div(static_cast<unsigned int>(p->ext[k]));
  }
}

// Tiles smaller than this many elements (two chains that end at a few
// elements each, as when a permute swaps small neighbouring axes) move
// faster one element at a time: an [8]^8 f32 permute swapping axis pairs
// (8 x 8 tiles) took 881 us through the general tiled kernel.
constexpr long long kMoveMinTile = 256;

// `dst_strides == nullptr` means the compact destination of materialize_strided.
// The source is `rank` axes of extents `src_ext` and strides `src_str` (at most
// kMaxDims are read) from `src_offset`.
T4A_HD void move_plan_view(MovePlan* p, int rank, long long src_offset, const long long* src_ext,
                           const long long* src_str, const long long* dst_strides,
                           long long dst_offset, long long len, int esize) {
  p->mode = kMoveEmpty;
  p->coords32 = false;
  p->n = 0;
  p->len = len;
  p->src_offset = src_offset;
  p->dst_offset = dst_offset;
  p->na = p->nb = p->nbatch = 0;
  p->tiles = 0;
  p->row_dim = -1;
  if (rank < 0) rank = 0;
  if (rank > kMaxDims) rank = kMaxDims;
  len = clamp_count(rank, src_ext, len);
  p->len = len;
  if (len <= 0) return;
  long long compact = 1;
  for (int k = 0; k < rank; ++k) {
    const long long e = src_ext[k];
    const long long s = src_str[k];
    const long long d = dst_strides ? dst_strides[k] : compact;
    compact *= e;
    if (e == 1) continue;
    if (p->n > 0) {
      const int last = p->n - 1;
      if (s == p->ss[last] * p->ext[last] && d == p->ds[last] * p->ext[last]) {
        p->ext[last] *= e;
        continue;
      }
    }
    p->ext[p->n] = e;
    p->ss[p->n] = s;
    p->ds[p->n] = d;
    ++p->n;
  }
  if (p->n == 0) {  // one element (rank 0 or all extents one)
    p->mode = kMoveGeneric;
    p->tiles = 1;
    return;
  }
  int a = -1, b = -1;
  for (int k = 0; k < p->n; ++k) {
    if (p->ds[k] == 1 && a < 0) a = k;
    if (p->ss[k] == 1 && b < 0) b = k;
  }
  if (a >= 0 && a == b) {
    p->mode = kMoveContig;
    p->row_dim = a;
    p->row_len = p->ext[a];
    p->rows = len / p->row_len;
    p->tiles = p->rows;
    return;
  }
  if (a < 0 || b < 0) {
    move_generic(p, len);
    return;
  }
  // Tile budget: 16 KiB of elements -- 4096 of 4 bytes or less (runs aiming
  // for 64 x 64), 2048 of 8 bytes (64 x 32), 1024 of 16 bytes (32 x 32): a
  // tile per block with more blocks per CU measured faster than larger tiles.
  // A run whose chain ends short leaves its share of the budget to the other
  // run, up to kMoveRunMax elements (a power of two), as long as the padded
  // tile fits kMoveTileBytes: a 16-element source run then feeds 128-element
  // destination runs.
  const long long budget = esize >= 16 ? 1024 : esize >= 8 ? 2048 : 4096;
  long long target_a = esize >= 16 ? 32 : 64;
  long long target_b = esize >= 8 ? 32 : 64;
  p->a_dims[0] = a;
  p->na = 1;
  p->b_dims[0] = b;
  p->nb = 1;
  // Grow a run along its chain: each next dim's stride on that side equals the
  // run's span so far; a dim of the other chain ends it.
  auto grow_a = [&](long long target) {
    long long span = 1;
    for (int i = 0; i < p->na; ++i) span *= p->ext[p->a_dims[i]];
    while (span < target && p->na < kMaxDims) {
      int next = -1;
      for (int k = 0; k < p->n; ++k) {
        if (p->ds[k] == span && !move_chain_contains(p->a_dims, p->na, k) &&
            !move_chain_contains(p->b_dims, p->nb, k))
          next = k;
      }
      if (next < 0) break;
      p->a_dims[p->na++] = next;
      span *= p->ext[next];
    }
    return span;
  };
  auto grow_b = [&](long long target) {
    long long span = 1;
    for (int i = 0; i < p->nb; ++i) span *= p->ext[p->b_dims[i]];
    while (span < target && p->nb < kMaxDims) {
      int next = -1;
      for (int k = 0; k < p->n; ++k) {
        if (p->ss[k] == span && !move_chain_contains(p->b_dims, p->nb, k) &&
            !move_chain_contains(p->a_dims, p->na, k))
          next = k;
      }
      if (next < 0) break;
      p->b_dims[p->nb++] = next;
      span *= p->ext[next];
    }
    return span;
  };
  auto pow2_floor = [](long long v) {
    long long r = 1;
    while (r * 2 <= v) r *= 2;
    return r;
  };
  auto fits = [&](long long la, long long lb) {
    return la <= kMoveRunMax && lb <= kMoveRunMax && la * lb <= budget &&
           la * (lb + 1) * esize <= kMoveTileBytes;
  };
  const long long span_a = grow_a(target_a);
  const long long span_b = grow_b(target_b);
  const long long run_a = span_a < target_a ? span_a : target_a;
  const long long run_b = span_b < target_b ? span_b : target_b;
  if (run_b < target_b) {
    long long t = pow2_floor(budget / run_b);
    while (t > target_a && !fits(t, run_b)) t /= 2;
    if (t > target_a) {
      grow_a(t);
      target_a = t;
    }
  } else if (run_a < target_a) {
    long long t = pow2_floor(budget / run_a);
    while (t > target_b && !fits(run_a, t)) t /= 2;
    if (t > target_b) {
      grow_b(t);
      target_b = t;
    }
  }
  // Tile the last dim of each chain so that the run stays near its target.
  p->a_inner = 1;
  for (int i = 0; i + 1 < p->na; ++i) p->a_inner *= p->ext[p->a_dims[i]];
  {
    const long long last = p->ext[p->a_dims[p->na - 1]];
    long long t = target_a / p->a_inner;
    if (t < 1) t = 1;
    if (t > last) t = last;
    p->a_tile = t;
    p->a_tiles = (last + t - 1) / t;
    p->la = p->a_inner * t;
  }
  p->b_inner = 1;
  for (int i = 0; i + 1 < p->nb; ++i) p->b_inner *= p->ext[p->b_dims[i]];
  {
    const long long last = p->ext[p->b_dims[p->nb - 1]];
    long long t = target_b / p->b_inner;
    if (t < 1) t = 1;
    if (t > last) t = last;
    p->b_tile = t;
    p->b_tiles = (last + t - 1) / t;
    p->lb = p->b_inner * t;
  }
  if (p->la * p->lb < kMoveMinTile) {
    p->na = p->nb = 0;
    move_generic(p, len);
    return;
  }
  long long tiles = p->a_tiles * p->b_tiles;
  for (int k = 0; k < p->n; ++k) {
    if (move_chain_contains(p->a_dims, p->na, k) || move_chain_contains(p->b_dims, p->nb, k))
      continue;
    p->batch_dims[p->nbatch++] = k;
    tiles *= p->ext[k];
  }
  p->mode = kMoveTiled;
  p->tiles = tiles;
  p->coords32 = tiles < (1ll << 30);
  if (p->coords32) {
    p->coord_div[0] = fast_div(static_cast<unsigned int>(p->a_tiles));
    p->coord_div[1] = fast_div(static_cast<unsigned int>(p->b_tiles));
    for (int q = 0; q < p->nbatch; ++q)
      p->coord_div[q + 2] = fast_div(static_cast<unsigned int>(p->ext[p->batch_dims[q]]));
  }
}

T4A_HD void move_plan(MovePlan* p, const t4a_cuda_layout& src, const long long* dst_strides,
                      long long dst_offset, long long len, int esize) {
  move_plan_view(p, src.rank, src.offset, src.extents, src.strides, dst_strides, dst_offset, len,
                 esize);
}

// The plan of a move over derived geometry (the general-rank entries'
// in-kernel planning; host use: its arrays are 1.5 KiB of stack). False when
// more than kMaxDims fused axes remain (the general twins decode those per
// element).
template <typename SrcStride, typename DstStride>
T4A_HD bool move_plan_by(MovePlan* p, int rank, const long long* ext, SrcStride src,
                         long long src_offset, DstStride dst, long long dst_offset, long long len,
                         int esize) {
  long long fe[kMaxFusedDims], fs[kMaxFusedDims], fd[kMaxFusedDims];
  const int n = len > 0 ? fuse_move_by(rank, ext, src, dst, fe, fs, fd, kMaxFusedDims) : 0;
  if (n < 0 || n > kMaxDims) return false;
  move_plan_view(p, n, src_offset, fe, fs, fd, dst_offset, len, esize);
  return true;
}

// A TILED plan that is one compact 2-D transpose: dim a contiguous in the
// destination (extent m, source stride n), dim b contiguous in the source
// (extent n, destination stride m). Then dst[dst_offset + i + j*m] =
// src[src_offset + i*n + j], the tiled transpose's map with one matrix, and
// the launchers route it to that kernel's 128 x 128 tiles (16 KiB tiles of the
// general tiled walk move a square transpose about a tenth slower).
struct TransposeRoute {
  long long m, n, src_offset, dst_offset;
};

T4A_HD bool transpose_route(const MovePlan& p, TransposeRoute* r) {
  if (p.mode != kMoveTiled || p.n != 2) return false;
  const int a = p.ds[0] == 1 ? 0 : p.ds[1] == 1 ? 1 : -1;
  if (a < 0) return false;
  const int b = 1 - a;
  if (p.ss[b] != 1 || p.ss[a] != p.ext[b] || p.ds[b] != p.ext[a]) return false;
  if (p.src_offset < 0 || p.dst_offset < 0) return false;
  r->m = p.ext[a];
  r->n = p.ext[b];
  r->src_offset = p.src_offset;
  r->dst_offset = p.dst_offset;
  const TransposeTiling t = transpose_tiling(r->m, r->n, 1, 16);  // the smallest tiles
  return t.total < (1ll << 30) && r->m < (1ll << 31) && r->n < (1ll << 31);
}

// A CONTIG plan of one fused dim: one run contiguous on both sides from the
// two offsets, which the launchers move as copy_exact moves a buffer.
T4A_HD bool linear_route(const MovePlan& p) { return p.mode == kMoveContig && p.n == 1; }

// The launchers' form of a CONTIG plan: rows cut into units of V elements (a
// 16-byte vector when V > 1), one unit per thread of a one-dimensional grid.
// Unit u is column u % vpr of row u / vpr; the row index is decoded over the
// other dims, first dim fastest. Every quotient is 32-bit (units < 2^31), so
// each division is a multiply-high by a precomputed FastDiv.
struct RowPlan {
  long long src_offset, dst_offset;
  unsigned int units;  // rows * vpr
  unsigned int vpr;    // units per row
  FastDiv row_div;     // by vpr
  int n;               // dims other than the row dim
  FastDiv div[kMaxDims];
  long long ss[kMaxDims], ds[kMaxDims];
  bool reread;  // a source stride 0 across rows: the source stays cached
};

// V = 16 / element size for 1-, 4- and 8-byte elements (1 otherwise) when the
// rows, offsets and strides keep every unit on V-element boundaries (the
// launcher also checks the pointers); else 1. False when the plan is not
// CONTIG or the units reach 2^31.
T4A_HD bool row_plan(RowPlan* r, const MovePlan& p, int esize, bool vectors) {
  if (p.mode != kMoveContig || p.row_len <= 0) return false;
  long long v = vectors && (esize == 1 || esize == 4 || esize == 8) ? 16 / esize : 1;
  if (v > 1 && (p.row_len % v != 0 || p.src_offset % v != 0 || p.dst_offset % v != 0)) v = 1;
  for (int k = 0; k < p.n && v > 1; ++k) {
    if (k != p.row_dim && (p.ss[k] % v != 0 || p.ds[k] % v != 0)) v = 1;
  }
  const long long vpr = p.row_len / v;
  if (p.rows <= 0 || vpr >= (1ll << 31) || p.rows > ((1ll << 31) - 1) / vpr) return false;
  r->src_offset = p.src_offset;
  r->dst_offset = p.dst_offset;
  r->units = static_cast<unsigned int>(p.rows * vpr);
  r->vpr = static_cast<unsigned int>(vpr);
  r->row_div = fast_div(r->vpr);
  r->n = 0;
  r->reread = false;
  for (int k = 0; k < p.n; ++k) {
    if (k == p.row_dim) continue;
    r->div[r->n] = fast_div(static_cast<unsigned int>(p.ext[k]));
    r->ss[r->n] = p.ss[k];
    r->ds[r->n] = p.ds[k];
    if (p.ss[k] == 0) r->reread = true;
    ++r->n;
  }
  for (int k = r->n; k < kMaxDims; ++k) {
    r->div[k] = fast_div(1);
    r->ss[k] = r->ds[k] = 0;
  }
  return true;
}

// fill_zero_view: the view's fused axes (fuse_move with the view's strides on
// both sides), the stride-1 axis, if any, moved first so that consecutive flat
// indices are consecutive addresses (every element gets the same zero, so the
// order of the walk is free). At most kMaxDims axes; the general-rank entry
// decodes wider views itself.
struct FillPlan {
  int n;
  long long ext[kMaxDims];
  long long st[kMaxDims];
  FastDiv div[kMaxDims];  // by ext[k], when narrow
  long long offset;
  long long len;
  bool narrow;  // len below 2^31: 32-bit quotients by multiply-high
};

T4A_HD bool fill_plan(FillPlan* p, int n, const long long* fe, const long long* fs,
                      long long offset, long long len) {
  if (n < 0 || n > kMaxDims) return false;
  len = clamp_count(n, fe, len);
  if (len == 0) n = 0;
  p->n = n;
  p->offset = offset;
  p->len = len;
  p->narrow = len >= 0 && len < (1ll << 31);
  int unit = -1;
  for (int k = 0; k < n; ++k) {
    if (fs[k] == 1 && unit < 0) unit = k;
  }
  int w = 0;
  if (unit >= 0) {
    p->ext[w] = fe[unit];
    p->st[w] = fs[unit];
    ++w;
  }
  for (int k = 0; k < n; ++k) {
    if (k == unit) continue;
    p->ext[w] = fe[k];
    p->st[w] = fs[k];
    ++w;
  }
  for (int k = n; k < kMaxDims; ++k) {
    p->ext[k] = 1;
    p->st[k] = 0;
  }
  for (int k = 0; k < kMaxDims; ++k)
    p->div[k] = fast_div(p->narrow ? static_cast<unsigned int>(p->ext[k]) : 1u);
  return true;
}

// Whether V consecutive flat indices are V consecutive, V-aligned elements:
// the first axis contiguous with an extent that V divides, and the offset and
// every other stride multiples of V (the pointer's alignment is the caller's).
T4A_HD bool fill_vectorizable(const FillPlan& p, int v) {
  if (v <= 1 || p.n == 0 || p.st[0] != 1 || p.ext[0] % v != 0 || p.offset % v != 0)
    return false;
  for (int k = 1; k < p.n; ++k) {
    if (p.st[k] % v != 0) return false;
  }
  return true;
}

// The TilePlan form of a TILED plan: tile t decoded from its index by
// precomputed divisors and moved whole, all of a thread's loads issued before
// its first LDS write, the tile shape a compile-time LA x LB. It applies when
// each chain has at most two dims (an inner one at full extent, the tiled
// outer one), the tile count is below 2^30 (32-bit coordinates) and (la, lb)
// is one of the shapes below.
// NC: the coordinate slots. The planner fills the full form (every fused dim
// can be a batch coordinate); a plan of at most four coordinates (C3 and C5
// have four) also travels in the compact form, whose 216 bytes of kernel
// arguments leave the tile kernels scalar registers for eight wavefronts per
// SIMD -- the full 384 bytes held them to seven.
template <int NC>
struct TilePlanN {
  static constexpr int kCoords = NC;
  long long src_offset, dst_offset;
  long long a_ss0, a_ss1;  // source strides of the A chain's inner and outer dims
  long long b_ds0, b_ds1;  // destination strides of the B chain's inner and outer dims
  FastDiv a_in, b_in;      // the inner dims' extents (1 for a one-dim chain)
  unsigned int a_tile, b_tile;  // tile extents along the outer dims
  unsigned int a_last, b_last;  // the outer dims' extents
  int ncoord;                   // coordinates of the tile walk: A tile, B tile, batch dims
  int skew_first, skew_second;  // diagonal order (see the persistent walk), -1 if none
  FastDiv coord[NC];
  long long coord_ss[NC];  // source / destination offset per unit of a coordinate
  long long coord_ds[NC];
};
using TilePlan = TilePlanN<kMaxDims + 2>;
constexpr int kCompactCoords = 4;
using TilePlanCompact = TilePlanN<kCompactCoords>;

// Whether the in-tile offsets of the valid slots -- the source offset of row
// i plus a column, the destination offset of column j plus a row, for an LA x
// LB tile of esize-byte elements -- span fewer than 2^31 bytes on each side.
T4A_HD bool tile_offsets_narrow(const TilePlan& tp, int la, int lb, int esize) {
  auto mag = [](long long v) { return v < 0 ? -static_cast<double>(v) : static_cast<double>(v); };
  const double src = mag(tp.a_ss0) * (tp.a_in.d - 1.0) + mag(tp.a_ss1) * (tp.a_tile - 1.0) + lb;
  const double dst = mag(tp.b_ds0) * (tp.b_in.d - 1.0) + mag(tp.b_ds1) * (tp.b_tile - 1.0) + la;
  return src * esize < 2147483648.0 && dst * esize < 2147483648.0;
}

// The compact form of a plan of at most kCompactCoords coordinates.
T4A_HD TilePlanCompact compact_tile_plan(const TilePlan& tp) {
  TilePlanCompact c;
  c.src_offset = tp.src_offset;
  c.dst_offset = tp.dst_offset;
  c.a_ss0 = tp.a_ss0;
  c.a_ss1 = tp.a_ss1;
  c.b_ds0 = tp.b_ds0;
  c.b_ds1 = tp.b_ds1;
  c.a_in = tp.a_in;
  c.b_in = tp.b_in;
  c.a_tile = tp.a_tile;
  c.b_tile = tp.b_tile;
  c.a_last = tp.a_last;
  c.b_last = tp.b_last;
  c.ncoord = tp.ncoord;
  c.skew_first = tp.skew_first;
  c.skew_second = tp.skew_second;
  for (int q = 0; q < kCompactCoords; ++q) {
    const bool used = q < tp.ncoord;
    c.coord[q] = used ? tp.coord[q] : fast_div(1);
    c.coord_ss[q] = used ? tp.coord_ss[q] : 0;
    c.coord_ds[q] = used ? tp.coord_ds[q] : 0;
  }
  return c;
}

// Compile-time tile shapes (LA x LB: A the destination run, B the source
// run). The balanced shape of each element size is the planner's full tile
// when both chains reach their targets: 64 x 64 for 4-byte elements, 64 x 32
// for 8-byte ones and 32 x 32 for 16-byte ones; every walk (the launchers'
// and the entries') has it. When one chain ends at 16 or 32 elements the
// planner hands the tile budget to the other run, and the launchers also walk
// those long-and-short shapes, with compact narrow plans (a TILED move with a
// 32-element source run, as a reversed-view f32 permute has, otherwise takes
// the general tiled kernel at two thirds of the speed).
T4A_HD bool tile_balanced_shape(long long la, long long lb, int esize) {
  if (esize == 4) return la == 64 && lb == 64;
  if (esize == 8) return la == 64 && lb == 32;
  if (esize == 16) return la == 32 && lb == 32;
  return false;
}

T4A_HD bool tile_long_short_shape(long long la, long long lb, int esize) {
  if (esize == 4)
    return (la == 128 && (lb == 32 || lb == 16)) || (lb == 128 && (la == 32 || la == 16));
  if (esize == 8) return (la == 128 && lb == 16) || (la == 16 && lb == 128) || (la == 32 && lb == 64);
  if (esize == 16) return (la == 64 && lb == 16) || (la == 16 && lb == 64);
  return false;
}

T4A_HD bool tile_once_shape(long long la, long long lb, int esize) {
  return tile_balanced_shape(la, lb, esize) || tile_long_short_shape(la, lb, esize);
}

T4A_HD bool tile_plan(TilePlan* tp, const MovePlan& p, int esize) {
  if (p.mode != kMoveTiled || !p.coords32 || p.na > 2 || p.nb > 2 ||
      !tile_once_shape(p.la, p.lb, esize))
    return false;
  tp->src_offset = p.src_offset;
  tp->dst_offset = p.dst_offset;
  const int a_outer = p.a_dims[p.na - 1];
  const int b_outer = p.b_dims[p.nb - 1];
  tp->a_in = fast_div(p.na == 2 ? static_cast<unsigned int>(p.ext[p.a_dims[0]]) : 1u);
  tp->a_ss0 = p.na == 2 ? p.ss[p.a_dims[0]] : 0;
  tp->a_ss1 = p.ss[a_outer];
  tp->b_in = fast_div(p.nb == 2 ? static_cast<unsigned int>(p.ext[p.b_dims[0]]) : 1u);
  tp->b_ds0 = p.nb == 2 ? p.ds[p.b_dims[0]] : 0;
  tp->b_ds1 = p.ds[b_outer];
  tp->a_tile = static_cast<unsigned int>(p.a_tile);
  tp->b_tile = static_cast<unsigned int>(p.b_tile);
  tp->a_last = static_cast<unsigned int>(p.ext[a_outer]);
  tp->b_last = static_cast<unsigned int>(p.ext[b_outer]);
  tp->ncoord = 2 + p.nbatch;
  long long ext[kMaxDims + 2];
  ext[0] = p.a_tiles;
  ext[1] = p.b_tiles;
  tp->coord_ss[0] = p.a_tile * p.ss[a_outer];
  tp->coord_ds[0] = p.a_tile * p.ds[a_outer];
  tp->coord_ss[1] = p.b_tile * p.ss[b_outer];
  tp->coord_ds[1] = p.b_tile * p.ds[b_outer];
  for (int q = 0; q < p.nbatch; ++q) {
    const int k = p.batch_dims[q];
    ext[q + 2] = p.ext[k];
    tp->coord_ss[q + 2] = p.ss[k];
    tp->coord_ds[q + 2] = p.ds[k];
  }
  // Diagonal order only between the A and B tile coordinates (a transpose's
  // tiles): skewing one batch dim by another scatters the writes of blocks
  // that run together, which measured slower.
  tp->skew_first = tp->skew_second = -1;
  if (ext[0] > 1 && ext[1] > 1) {
    tp->skew_first = 0;
    tp->skew_second = 1;
  }
  for (int q = 0; q < tp->ncoord; ++q) tp->coord[q] = p.coord_div[q];
  return true;
}

// Whether the launchers walk a tile plan with one of the walk kernels: the
// balanced shape in any plan form, a long-and-short one in the compact narrow
// form only (anything else takes the general tiled kernel).
T4A_HD bool tile_walk_applies(const MovePlan& p, const TilePlan& tp, int esize) {
  if (tile_balanced_shape(p.la, p.lb, esize)) return true;
  return tile_long_short_shape(p.la, p.lb, esize) && tp.ncoord <= kCompactCoords &&
         tile_offsets_narrow(tp, static_cast<int>(p.la), static_cast<int>(p.lb), esize);
}

// ---- reductions ---------------------------------------------------------------
//
// The non-axis axes of a reduction, fused: extent-one axes dropped and
// neighbours merged where both the input and the output (or partials) strides
// continue each other. The output index decodes over them in axis order, as
// reduce.cu:110-130 decodes it over the output layout.
// The fused non-axis dims of a reduction, at most N of them: ReduceDims (N =
// kMaxDims) for the by-value entries and plans, ReduceDimsWide for the
// general-rank `_any` entries, built in LDS.
template <int N>
struct ReduceDimsN {
  static constexpr int kDims = N;
  int n;
  long long ext[N];
  long long is[N];  // input strides
  long long os[N];  // output / partials strides
  long long in_offset;
  long long out_offset;
  long long axis_len;
  long long axis_stride;
  long long out_axis_stride;  // partials stride of the split coordinate
  bool narrow;                // the product of ext[] is below 2^32
};
using ReduceDims = ReduceDimsN<kMaxDims>;
using ReduceDimsWide = ReduceDimsN<kMaxFusedDims>;

// Fuse the non-axis dims of a reduction of any rank (extent-1 dims dropped,
// a dim merged into the previous kept one when its input and output strides
// both continue that one's span; the axis is skipped, so dims on its two sides
// may merge) into r. `out_ext` gives the non-axis extents; the axis takes its
// length and stride from the input and its output stride (the partials' split
// stride, or the keepdims output's) from the output. False, with r->n = -1,
// when more than N dims remain.
template <int N>
T4A_HD bool reduce_dims_view(ReduceDimsN<N>* r, int rank, int axis, long long out_offset,
                             const long long* out_ext, const long long* out_str,
                             long long in_offset, const long long* in_ext,
                             const long long* in_str) {
  r->n = 0;
  r->in_offset = in_offset;
  r->out_offset = out_offset;
  r->axis_len = in_ext[axis];
  r->axis_stride = in_str[axis];
  r->out_axis_stride = out_str[axis];
  for (int k = 0; k < rank; ++k) {
    if (k == axis) continue;
    const long long e = out_ext[k];
    if (e == 1) continue;
    const long long s = in_str[k];
    const long long o = out_str[k];
    if (r->n > 0) {
      const int last = r->n - 1;
      if (s == r->is[last] * r->ext[last] && o == r->os[last] * r->ext[last]) {
        r->ext[last] *= e;
        continue;
      }
    }
    if (r->n == N) {
      r->n = -1;
      return false;
    }
    r->ext[r->n] = e;
    r->is[r->n] = s;
    r->os[r->n] = o;
    ++r->n;
  }
  unsigned long long total = 1;
  r->narrow = true;
  for (int k = 0; k < r->n; ++k) {
    const unsigned long long e = static_cast<unsigned long long>(r->ext[k]);
    if (e != 0 && total > 0xffffffffull / e) r->narrow = false;
    total *= e;
    if (total > 0xffffffffull) r->narrow = false;
  }
  return true;
}

T4A_HD void reduce_dims(ReduceDims* r, const t4a_cuda_layout& out,
                        const t4a_cuda_layout& in, int axis) {
  int rank = out.rank;
  if (rank > kMaxDims) rank = kMaxDims;
  reduce_dims_view(r, rank, axis, out.offset, out.extents, out.strides, in.offset, in.extents,
                   in.strides);
}


// The unit kernels' compact plan: at most three fused output dims with
// precomputed divisors, 32-bit output indices. `vector`: the axis is contiguous
// and every output's start a multiple of v = 16 / esize elements (the launcher
// also checks the pointer's alignment).
struct UnitPlan {
  long long in_offset;
  long long out_offset;
  long long axis_stride;
  long long is[3];
  long long os[3];
  FastDiv ext[3];
  int n;
  int axis_len;
  bool vector;
};

T4A_HD bool unit_plan_fits(const ReduceDims& rd, long long output_len) {
  return rd.n <= 3 && output_len < (1ll << 31) && rd.axis_len < (1ll << 31);
}

// A 32-bit grid-stride walk over `items` (index i < items, then i + S with
// S = blocks * per_block) never wraps when items + S < 2^32. The lean kernels
// walk their outputs or cubes that way, and any caller's grid reaches them, so
// their launchers check it.
T4A_HD bool grid_stride_fits(long long items, unsigned int blocks, unsigned long long per_block) {
  if (items < 0) return false;
  return static_cast<unsigned long long>(items) + per_block * blocks < (1ull << 32);
}

// The lean unit kernel's walk: a lane's outputs below run + 64 *
// kUnitOutputsPerThread, runs kUnitOutputsPerThread * S apart (S = blocks *
// threads).
T4A_HD bool unit_lean_fits(long long output_len, unsigned int blocks, unsigned int threads);

T4A_HD UnitPlan unit_plan(const ReduceDims& rd, int v, bool aligned) {
  UnitPlan up;
  up.in_offset = rd.in_offset;
  up.out_offset = rd.out_offset;
  up.axis_stride = rd.axis_stride;
  up.axis_len = static_cast<int>(rd.axis_len);
  up.n = rd.n;
  for (int k = 0; k < 3; ++k) {
    const bool used = k < rd.n;
    up.is[k] = used ? rd.is[k] : 0;
    up.os[k] = used ? rd.os[k] : 0;
    up.ext[k] = fast_div(used ? static_cast<unsigned int>(rd.ext[k]) : 1u);
  }
  bool vector = v > 0 && aligned && rd.axis_stride == 1 && rd.axis_len >= v &&
                rd.in_offset % v == 0;
  for (int k = 0; k < rd.n; ++k) vector = vector && rd.is[k] % v == 0;
  up.vector = vector;
  return up;
}

// A unit reduction whose axis is one 16-byte group (V <= len < 2V contiguous
// elements of a 4- or 8-byte real or integer type, every output's start a
// multiple of V): each wavefront takes runs of 64 * kUnitOutputsPerThread
// consecutive outputs, lane l the outputs run + l + 64u, so that every load and
// store instruction covers one contiguous span; a lane's loads are issued
// together. (Two outputs a lane measured fastest on C4's 2^25-output i32
// product: 103 us against 107-111 us for one, four or eight, and 128 us for
// four outputs a whole grid apart.)
constexpr int kUnitOutputsPerThread = 2;

T4A_HD bool unit_lean_fits(long long output_len, unsigned int blocks, unsigned int threads) {
  return grid_stride_fits(output_len, blocks,
                          static_cast<unsigned long long>(kUnitOutputsPerThread) * threads);
}

T4A_HD bool unit_one_group(const ReduceDims& rd, int dtype) {
  const int es = dtype_size(dtype);
  const bool real_or_int = dtype == T4A_CUDA_F32 || dtype == T4A_CUDA_F64 ||
                           dtype == T4A_CUDA_I32 || dtype == T4A_CUDA_I64;
  if (!real_or_int) return false;
  const long long v = 16 / es;
  if (rd.axis_stride != 1 || rd.axis_len < v || rd.axis_len >= 2 * v || rd.in_offset % v != 0)
    return false;
  for (int k = 0; k < rd.n; ++k) {
    if (rd.is[k] % v != 0) return false;
  }
  return true;
}

// Element types the sideways pass-1 mappings serve (real and integer; complex
// keeps the plane mapping).
T4A_HD bool sideways_dtype(int dtype) {
  return dtype == T4A_CUDA_F32 || dtype == T4A_CUDA_F64 || dtype == T4A_CUDA_I32 ||
         dtype == T4A_CUDA_I64;
}

// Pass-1 work mapping (t4a_cuda_reduce_partials). All of them keep the
// reference's per-plane topology -- plane lane l folds rows start + l + 32k in k
// order, then the own-left xor tree -- and differ only in which hardware lanes
// hold which plane lanes:
//   PLANE      one 32-lane half-wavefront per (output, split) cube, as the
//              reference warp (any width 8/16/32);
//   TILES      a strided axis whose fastest non-axis dim (input stride 1) has
//              at least 64 columns: a block of four wavefronts per (column
//              block, split); lane t holds `cpl` adjacent columns (one 8-byte
//              load for two 4-byte columns) and wavefront w the plane lanes
//              8w..8w+7 of those columns' cubes; the four wavefronts' subtrees
//              meet through LDS;
//   VECROWS    rows of c = 2 or 4 contiguous elements (8 or 16 bytes): a 32-lane
//              plane per (split, other) takes all c columns, each plane lane
//              loading whole rows, one xor tree per column;
//   ROWS       2..32 columns (a power of two) otherwise: 64 / C rows per
//              wavefront load, each lane holding the 32 / (64 / C) plane lanes of
//              its row residue.
// The wavefront mappings need 32-lane planes and kBlock-thread blocks.
enum PartialsMode {
  kPartialsPlane = 0,
  kPartialsRows = 2,
  kPartialsTiles = 3,
  kPartialsVecRows = 4
};

struct PartialsPlan {
  int mode;
  ReduceDims dims;
  int col_dim;          // fused dim of input stride 1 (TILES/VECROWS/ROWS)
  int cpl;              // columns per lane: TILES 1 or 2, VECROWS c
  long long columns;    // its extent
  long long col_os;     // partials stride of that dim
  long long col_blocks; // column blocks of 64 * cpl (TILES), else 1
  long long others;     // product of the other fused extents
  long long units;      // blocks (TILES), planes (VECROWS), wavefronts (ROWS), cubes
};

// A reduction's layouts as a rank <= 8 pair with the same fused dims (for
// partials_plan): the layouts themselves up to rank 8, else the non-axis dims
// fused (reduce_dims_view, into `work`) with the axis appended last. False when
// more than seven non-axis dims remain. Arrays may be host or device memory;
// on the device, `work` and the outputs live in LDS (as locals their runtime
// subscripts would take per-lane scratch memory).
T4A_HD bool reduction_pair_view(int rank, long long out_offset, const long long* out_ext,
                                const long long* out_str, long long in_offset,
                                const long long* in_ext, const long long* in_str, int axis,
                                t4a_cuda_layout* o8, t4a_cuda_layout* i8, int* axis8,
                                ReduceDimsN<kMaxDims - 1>* work) {
  o8->rank = i8->rank = 0;
  o8->offset = out_offset;
  i8->offset = in_offset;
  for (int k = 0; k < kMaxDims; ++k) {
    o8->extents[k] = o8->strides[k] = i8->extents[k] = i8->strides[k] = 0;
  }
  if (rank <= kMaxDims) {
    o8->rank = i8->rank = rank;
    for (int k = 0; k < rank; ++k) {
      o8->extents[k] = out_ext[k];
      o8->strides[k] = out_str[k];
      i8->extents[k] = in_ext[k];
      i8->strides[k] = in_str[k];
    }
    *axis8 = axis;
    return true;
  }
  ReduceDimsN<kMaxDims - 1>& rd = *work;
  if (!reduce_dims_view(&rd, rank, axis, out_offset, out_ext, out_str, in_offset, in_ext,
                        in_str))
    return false;
  o8->rank = i8->rank = rd.n + 1;
  for (int k = 0; k < rd.n; ++k) {
    o8->extents[k] = i8->extents[k] = rd.ext[k];
    o8->strides[k] = rd.os[k];
    i8->strides[k] = rd.is[k];
  }
  o8->extents[rd.n] = out_ext[axis];
  o8->strides[rd.n] = out_str[axis];
  i8->extents[rd.n] = in_ext[axis];
  i8->strides[rd.n] = in_str[axis];
  *axis8 = rd.n;
  return true;
}

// `align`: the input pointer's alignment in bytes (the planner, which has no
// pointer, assumes 16; the launcher passes the real one). A plan made for a
// better-aligned pointer still runs correctly through the launcher, which
// re-plans, because every mapping walks its units grid-stride.
T4A_HD void partials_plan(PartialsPlan* p, const t4a_cuda_layout& partials,
                          const t4a_cuda_layout& in, int axis, long long output_len,
                          long long splits, int plane_width, int whole_waves, int esize,
                          int align) {
  reduce_dims(&p->dims, partials, in, axis);
  const ReduceDims& d = p->dims;
  p->mode = kPartialsPlane;
  p->col_dim = -1;
  p->cpl = 1;
  p->columns = 0;
  p->col_os = 0;
  p->col_blocks = 0;
  p->others = 0;
  p->units = output_len * splits;
  if (plane_width != kWarp || !whole_waves || d.axis_stride == 1 || output_len <= 0) return;
  int col = -1;
  for (int k = 0; k < d.n; ++k) {
    if (d.is[k] == 1) col = k;
  }
  if (col < 0) return;
  const long long c = d.ext[col];
  long long others = 1;
  for (int k = 0; k < d.n; ++k) {
    if (k != col) others *= d.ext[k];
  }
  // Every row start of the column dim a multiple of v elements from the base.
  auto rows_multiple_of = [&](long long v) {
    if (d.in_offset % v != 0 || d.axis_stride % v != 0) return false;
    for (int k = 0; k < d.n; ++k) {
      if (k != col && d.is[k] % v != 0) return false;
    }
    return true;
  };
  if (c >= kWave) {
    p->mode = kPartialsTiles;
    p->cpl = esize == 4 && align >= 8 && c % 2 == 0 && rows_multiple_of(2) ? 2 : 1;
    p->col_blocks = (c + kWave * p->cpl - 1) / (kWave * p->cpl);
  } else if ((c * esize == 8 || c * esize == 16) && align >= c * esize && rows_multiple_of(c)) {
    p->mode = kPartialsVecRows;
    p->cpl = static_cast<int>(c);
    p->col_blocks = 1;
  } else if (c >= 2 && (c & (c - 1)) == 0) {
    p->mode = kPartialsRows;
    p->col_blocks = 1;
  } else {
    return;
  }
  p->col_dim = col;
  p->columns = c;
  p->col_os = d.os[col];
  p->others = others;
  p->units = p->col_blocks * others * splits;
  // TILES and VECROWS walk a SidePlan: at most two other dims, 32-bit counts.
  if ((p->mode == kPartialsTiles || p->mode == kPartialsVecRows) &&
      (d.n > 3 || d.axis_len >= (1ll << 31) || p->units >= (1ll << 31))) {
    p->mode = kPartialsPlane;
    p->units = output_len * splits;
  }
}

// Whether pass 1 can stream whole runs of cubes through the grouped walk: a
// regroupable fold over a 4- or 8-byte real or integer type, 32-lane planes, a
// contiguous axis, every chunk holding at least 32 groups of V = 16 / size
// elements, and every chunk start a multiple of V elements from the base (the
// base pointer's own 16-byte alignment is the launcher's to check).
T4A_HD bool stream_applies(const PartialsPlan& p, int dtype, int op, long long chunk_len,
                           int plane_width) {
  if (!sideways_dtype(dtype) || op == T4A_CUDA_REDUCE_PROD) return false;
  if (op < T4A_CUDA_REDUCE_SUM || op > T4A_CUDA_REDUCE_MIN) return false;
  if (p.mode != kPartialsPlane || plane_width != kWarp || p.dims.axis_stride != 1) return false;
  const long long v = 16 / dtype_size(dtype);
  if (chunk_len / v < kWarp || chunk_len % v != 0 || p.dims.in_offset % v != 0) return false;
  for (int k = 0; k < p.dims.n; ++k) {
    if (p.dims.is[k] % v != 0) return false;
  }
  return true;
}

// Batch slots (groups per lane, 1..4) of the lean pass-1 mapping, or 0 where it
// does not apply: the streaming conditions above, and the longest chunk (the
// last one, which absorbs the remainder) holding at most 4 * 32 groups, so each
// lane's share is the grouped walk's first batch alone.
T4A_HD int lean_slots(const PartialsPlan& p, int dtype, int op, long long splits,
                      long long chunk_len, int plane_width) {
  if (!stream_applies(p, dtype, op, chunk_len, plane_width)) return 0;
  // The lean plan's decode: at most three fused non-axis dims, cube and output
  // indices below 2^31 (32-bit quotients).
  if (p.dims.n > 3 || p.units >= (1ll << 31)) return 0;
  const long long v = 16 / dtype_size(dtype);
  const long long last = p.dims.axis_len - (splits - 1) * chunk_len;
  const long long slots = (last / v + kWarp - 1) / kWarp;
  return slots <= 4 ? static_cast<int>(slots) : 0;
}

// The lean mapping's own plan: the fused non-axis dims (at most three) with
// their divisors precomputed, and the split walk.
struct LeanPlan {
  // First, next to each other: what a wavefront needs before its first load
  // (the cube count it tests against, the chunk's place), so that one scalar
  // load fetches them all.
  unsigned int cubes;
  long long in_offset;
  long long chunk_len;
  long long out_offset;
  long long out_axis_stride;
  long long is[3];
  long long os[3];
  FastDiv ext[3];
  FastDiv splits;
  int n;
  int last_len;
  // Equal chunks laid end to end in cube order on both sides (an inner axis
  // of a compact input, compact partials): cube c's chunk starts at
  // in_offset + c * chunk_len and its partial at out_offset + c * out_axis_stride.
  bool linear;
};

T4A_HD LeanPlan lean_plan(const PartialsPlan& p, long long splits, long long chunk_len) {
  LeanPlan lp;
  lp.cubes = static_cast<unsigned int>(p.units);
  const ReduceDims& rd = p.dims;
  lp.in_offset = rd.in_offset;
  lp.out_offset = rd.out_offset;
  lp.n = rd.n;
  for (int k = 0; k < 3; ++k) {
    const bool used = k < rd.n;
    lp.is[k] = used ? rd.is[k] : 0;
    lp.os[k] = used ? rd.os[k] : 0;
    lp.ext[k] = fast_div(used ? static_cast<unsigned int>(rd.ext[k]) : 1u);
  }
  lp.splits = fast_div(static_cast<unsigned int>(splits));
  lp.last_len = static_cast<int>(rd.axis_len - (splits - 1) * chunk_len);
  lp.chunk_len = chunk_len;
  lp.out_axis_stride = rd.out_axis_stride;
  lp.linear = rd.n <= 1 && lp.last_len == chunk_len &&
              (rd.n == 0 ||
               (rd.is[0] == splits * chunk_len && rd.os[0] == splits * rd.out_axis_stride));
  return lp;
}

// The TILES / VECROWS mappings' own plan: unit u = (column block, split,
// other) decoded with precomputed divisors over at most two other fused dims,
// the rest as element offsets and strides.
struct SidePlan {
  long long in_offset;
  long long out_offset;
  long long axis_stride;      // input elements between rows
  long long out_axis_stride;  // partials elements between splits
  long long col_os;           // partials elements between columns
  long long is[2];
  long long os[2];
  FastDiv ext[2];
  FastDiv col_blocks;
  FastDiv splits;
  int n_other;
  int chunk_len;
  int last_len;
  long long columns;
  long long units;
};

// Written through a pointer: a kernel's thread 0 builds it in LDS, where the
// runtime-subscripted writes below need no per-lane scratch memory (a local
// SidePlan would).
T4A_HD void side_plan_into(SidePlan* out, const PartialsPlan& p, long long splits,
                           long long chunk_len) {
  SidePlan& sp = *out;
  const ReduceDims& d = p.dims;
  sp.in_offset = d.in_offset;
  sp.out_offset = d.out_offset;
  sp.axis_stride = d.axis_stride;
  sp.out_axis_stride = d.out_axis_stride;
  sp.col_os = p.col_os;
  sp.n_other = 0;
  for (int k = 0; k < 2; ++k) {
    sp.is[k] = 0;
    sp.os[k] = 0;
    sp.ext[k] = fast_div(1);
  }
  for (int k = 0; k < d.n; ++k) {
    if (k == p.col_dim || sp.n_other == 2) continue;
    sp.is[sp.n_other] = d.is[k];
    sp.os[sp.n_other] = d.os[k];
    sp.ext[sp.n_other] = fast_div(static_cast<unsigned int>(d.ext[k]));
    ++sp.n_other;
  }
  sp.col_blocks = fast_div(static_cast<unsigned int>(p.col_blocks));
  sp.splits = fast_div(static_cast<unsigned int>(splits));
  sp.chunk_len = static_cast<int>(chunk_len);
  sp.last_len = static_cast<int>(d.axis_len - (splits - 1) * chunk_len);
  sp.columns = p.columns;
  sp.units = p.units;
}

T4A_HD SidePlan side_plan(const PartialsPlan& p, long long splits, long long chunk_len) {
  SidePlan sp;
  side_plan_into(&sp, p, splits, chunk_len);
  return sp;
}

// Cubes each streaming plane takes: enough planes to fill the chip (16384, four
// wavefronts of two planes on each of 256 CUs, twice over), at most 8 cubes.
T4A_HD long long stream_cubes_per_plane(long long cubes) {
  long long per = cubes / 16384;
  if (per < 1) per = 1;
  if (per > 8) per = 8;
  return per;
}

}  // namespace t4a

#endif  // T4A_GEOMETRY_H_
