// gfx950 movement kernels: tiled transpose, materialize_strided and
// strided_to_strided, exported under the reference entry names and argument
// lists (reference cuda/src/movement.cu:535-610).
//
// Movement is a bijection of logical coordinates, so every kernel here copies
// each element's bits exactly once and the work order is free. The MI355X
// design: elements are moved as raw 1/4/8/16-byte payloads; both sides of a
// permute are made contiguous by staging an LA x LB tile through LDS (read along
// the source-contiguous run, written along the destination-contiguous run) with
// 16-byte vector accesses where alignment allows; tiles are walked with
// grid-stride loops, so a block plans once and then streams tiles.
#include <hip/hip_runtime.h>

#include <atomic>
#include <type_traits>

#include "device.h"
#include "geometry.h"
#include "t4a/t4a.h"

namespace t4a {
namespace {

// One LDS arena per block, shared by every payload width's instantiation.
// Movement: two run-offset tables of kMoveRunMax entries plus the largest padded
// tile, kMoveTileBytes (128 x 33 payloads of 8 bytes, 64 x 33 of 16 bytes).
// Transpose: one tile of TransposeShape below, at most 128 x 65 8-byte payloads.
constexpr int kMoveLdsBytes = 2 * kMoveRunMax * 8 + kMoveTileBytes;
constexpr int kTransposeLdsBytes = 128 * 65 * 8;

// ---- tiled transpose ---------------------------------------------------------------

// dst[b*S + i + j*M] = src[src_offset + b*S + i*N + j] for the batch of
// blockIdx.z. A tile is TM source rows (i) by TN source columns (j), about 64
// KiB of LDS. Tiles are visited in diagonal order -- tile t takes i-tile
// t % tiles_m and j-tile (t / tiles_m + i-tile) % tiles_n -- so the tiles in
// flight at once start at different column offsets: with the power-of-two row
// pitches of typical matrices, i-tile-major order sends every concurrent tile's
// rows to the same few HBM channels. Both sides stream with non-temporal 16-byte
// accesses. VL / VS: elements per load / store (a 16-byte vector, or 1).
template <typename P>
struct TransposeShape {
  static constexpr int TM = sizeof(P) >= 16 ? 64 : 128;
  static constexpr int TN = sizeof(P) >= 8 ? 64 : 128;
};

// BS: the launcher's compile-time block size (0: read blockDim, for the
// geometry-agnostic entry). With BS known, a whole tile takes the unrolled path:
// each thread issues all of its loads before the first LDS write and all of its
// LDS reads before the first store, with no edge tests; edge tiles and the
// entry take the general loops.
// The launcher's tile order: tiles of M and of N as precomputed divisors, the
// tile count of one matrix (below 2^30, so every quotient input stays below
// 2^31) and the grid's block count (gridDim.x costs two hidden-argument loads,
// a scalar round trip after the alignment tests and before the first load).
struct TileOrder {
  FastDiv tiles_m;
  FastDiv tiles_n;
  unsigned int per_batch;
  unsigned int blocks;
};

template <typename P, int VL, int VS, int BS, bool Ordered>
__device__ __forceinline__ void transpose_tiles(P* __restrict__ dst, const P* __restrict__ src,
                                                long long src_offset, long long S, long long M,
                                                long long N, const TileOrder& order,
                                                unsigned char* lds) {
  constexpr int TM = TransposeShape<P>::TM;
  constexpr int TN = TransposeShape<P>::TN;
  constexpr int PITCH = TN + 1;
  P* tile = reinterpret_cast<P*>(lds);
  const long long tiles_m = (M + TM - 1) / TM;
  const long long tiles_n = (N + TN - 1) / TN;
  const long long per_batch = tiles_m * tiles_n;
  const long long b = blockIdx.z;
  const P* s = src + src_offset + b * S;
  P* d = dst + b * S;
  // Threads and blocks are numbered flat over x and y, so the reference's 2-D
  // geometry (grid (tiles of M, tiles of N, batches), block (tile / vw, rows))
  // and this build's 1-D one both cover every tile exactly once.
  const int tid = threadIdx.x + threadIdx.y * (BS > 0 ? BS : blockDim.x);
  const int nthreads = BS > 0 ? BS : blockDim.x * blockDim.y;
  // Tile t of the matrix, in diagonal order: tm = t mod tiles_m, tn = (t div
  // tiles_m + tm) mod tiles_n.
  auto tile_body = [&](long long tm, long long tn) {
    const long long i0 = tm * TM;
    const long long j0 = tn * TN;
    const int rows = static_cast<int>(M - i0 < TM ? M - i0 : TM);
    const int cols = static_cast<int>(N - j0 < TN ? N - j0 : TN);
    constexpr int kLoads = BS > 0 ? TM * (TN / VL) / BS : 0;
    constexpr int kStores = BS > 0 ? TN * (TM / VS) / BS : 0;
    // The unrolled path holds a thread's whole share in registers: only for
    // vector accesses (at most eight of them per side).
    if constexpr (BS > 0 && kLoads <= 8 && kStores <= 8) {
      static_assert(kLoads * BS == TM * (TN / VL) && kStores * BS == TN * (TM / VS),
                    "the block divides the tile");
      if (rows == TM && cols == TN) {
        Vec<P, VL> x[kLoads];
#pragma unroll
        for (int r = 0; r < kLoads; ++r) {
          const int e = tid + r * BS;
          const int i = e / (TN / VL);
          const int j = (e % (TN / VL)) * VL;
          x[r] = nt_load<P, VL>(s + (i0 + i) * N + j0 + j);
        }
#pragma unroll
        for (int r = 0; r < kLoads; ++r) {
          const int e = tid + r * BS;
          const int i = e / (TN / VL);
          const int j = (e % (TN / VL)) * VL;
#pragma unroll
          for (int k = 0; k < VL; ++k) tile[i * PITCH + j + k] = x[r].v[k];
        }
        __syncthreads();
        Vec<P, VS> y[kStores];
#pragma unroll
        for (int r = 0; r < kStores; ++r) {
          const int e = tid + r * BS;
          const int j = e / (TM / VS);
          const int i = (e % (TM / VS)) * VS;
#pragma unroll
          for (int k = 0; k < VS; ++k) y[r].v[k] = tile[(i + k) * PITCH + j];
        }
#pragma unroll
        for (int r = 0; r < kStores; ++r) {
          const int e = tid + r * BS;
          const int j = e / (TM / VS);
          const int i = (e % (TM / VS)) * VS;
          nt_store<P, VS>(d + (j0 + j) * M + i0 + i, y[r]);
        }
        __syncthreads();
        return;
      }
    }
    // Source rows: runs of TN along j. VL divides N and src_offset, so a vector
    // is wholly inside or wholly past the matrix edge.
    for (int e = tid; e < TM * (TN / VL); e += nthreads) {
      const int i = e / (TN / VL);
      const int j = (e % (TN / VL)) * VL;
      if (i < rows && j < cols) {
        const Vec<P, VL> x = nt_load<P, VL>(s + (i0 + i) * N + j0 + j);
#pragma unroll
        for (int k = 0; k < VL; ++k) tile[i * PITCH + j + k] = x.v[k];
      }
    }
    __syncthreads();
    // Destination rows: runs of TM along i.
    for (int e = tid; e < TN * (TM / VS); e += nthreads) {
      const int j = e / (TM / VS);
      const int i = (e % (TM / VS)) * VS;
      if (i < rows && j < cols) {
        Vec<P, VS> x;
#pragma unroll
        for (int k = 0; k < VS; ++k) x.v[k] = tile[(i + k) * PITCH + j];
        nt_store<P, VS>(d + (j0 + j) * M + i0 + i, x);
      }
    }
    __syncthreads();
  };
  if constexpr (Ordered) {
    // The launcher's 1-D grid over one matrix's tiles: 32-bit tile indices and
    // precomputed divisors.
    for (unsigned int t = blockIdx.x; t < order.per_batch; t += order.blocks) {
      const unsigned int q = div_by(t, order.tiles_m);
      const unsigned int tm = t - q * order.tiles_m.d;
      const unsigned int u = q + tm;
      tile_body(tm, u - div_by(u, order.tiles_n) * order.tiles_n.d);
    }
  } else {
    const long long nblocks = static_cast<long long>(gridDim.x) * gridDim.y;
    for (long long t = blockIdx.x + static_cast<long long>(blockIdx.y) * gridDim.x;
         t < per_batch; t += nblocks) {
      const long long tm = t % tiles_m;
      tile_body(tm, (t / tiles_m + tm) % tiles_n);
    }
  }
}

template <typename P, int BS, bool Ordered = false>
__device__ __forceinline__ void transpose_dispatch(void* dst, const void* src,
                                                   long long src_offset, long long S,
                                                   long long M, long long N,
                                                   unsigned char* lds,
                                                   const TileOrder& order = TileOrder{}) {
  constexpr int V = sizeof(P) <= 8 ? 16 / static_cast<int>(sizeof(P)) : 1;
  const bool vl = V > 1 && (reinterpret_cast<uintptr_t>(src) & 15) == 0 && N % V == 0 &&
                  src_offset % V == 0;
  const bool vs = V > 1 && (reinterpret_cast<uintptr_t>(dst) & 15) == 0 && M % V == 0;
  P* d = static_cast<P*>(dst);
  const P* s = static_cast<const P*>(src);
  if (vl && vs) {
    transpose_tiles<P, V, V, BS, Ordered>(d, s, src_offset, S, M, N, order, lds);
  } else if (vl) {
    transpose_tiles<P, V, 1, BS, Ordered>(d, s, src_offset, S, M, N, order, lds);
  } else if (vs) {
    transpose_tiles<P, 1, V, BS, Ordered>(d, s, src_offset, S, M, N, order, lds);
  } else {
    transpose_tiles<P, 1, 1, BS, Ordered>(d, s, src_offset, S, M, N, order, lds);
  }
}

__device__ __forceinline__ bool transpose_config_valid(const t4a_cuda_transpose_config& c) {
  const bool tile = c.tile == 8 || c.tile == 16 || c.tile == 32;
  const bool rows = c.block_rows == 4 || c.block_rows == 8 || c.block_rows == 16;
  const bool pad = c.padding == 0 || c.padding == 1;
  const bool vw = c.vector_width == 1 || c.vector_width == 2 || c.vector_width == 4;
  return tile && rows && pad && vw && c.tile % c.vector_width == 0;
}

// ---- strided movement --------------------------------------------------------------

// TILED: an la x lb tile; element (i, j) sits at src_base + src_a[i] + j and at
// dst_base + i + dst_b[j]. VL / VS: elements per load / store.
//
// A block walks tiles t, t + blocks, ... and keeps a tile's loads in flight
// while it writes the previous one: it loads tile t into registers, parks them
// in LDS, then issues tile t+1's loads before reading tile t back out of LDS
// and storing it. Tile coordinates are A-tile fastest, then B-tile, then the
// batch dims; the second coordinate of extent > 1 is skewed by the first
// (diagonal order), so tiles in flight together start at different offsets
// along both runs.
struct TileCoords {
  long long sbase, dbase;
  int va, vb;  // valid run lengths of this tile
};

__device__ __forceinline__ TileCoords tile_coords(const MovePlan& p, long long t) {
  const int a_last = p.a_dims[p.na - 1];
  const int b_last = p.b_dims[p.nb - 1];
  long long rest = t;
  long long first = 0;
  int seen = 0;
  // Coordinate q of the walk (extent `extent`): 32-bit quotients by the plan's
  // precomputed divisors when the tile count is below 2^30 (every rest, and a
  // coordinate plus the first one, then stays below 2^31), else 64-bit ones.
  auto coord = [&](int q, long long extent) {
    long long c;
    if (p.coords32) {
      const unsigned int r = static_cast<unsigned int>(rest);
      const unsigned int quot = div_by(r, p.coord_div[q]);
      c = r - quot * p.coord_div[q].d;
      rest = quot;
    } else {
      c = rest % extent;
      rest /= extent;
    }
    if (extent > 1) {
      if (seen == 1) {
        if (p.coords32) {
          const unsigned int u = static_cast<unsigned int>(c + first);
          c = u - div_by(u, p.coord_div[q]) * p.coord_div[q].d;
        } else {
          c = (c + first) % extent;
        }
      }
      if (seen == 0) first = c;
      ++seen;
    }
    return c;
  };
  const long long ta = coord(0, p.a_tiles);
  const long long tb = coord(1, p.b_tiles);
  TileCoords tc;
  tc.sbase = p.src_offset + ta * p.a_tile * p.ss[a_last] + tb * p.b_tile * p.ss[b_last];
  tc.dbase = p.dst_offset + ta * p.a_tile * p.ds[a_last] + tb * p.b_tile * p.ds[b_last];
  for (int q = 0; q < p.nbatch; ++q) {
    const int k = p.batch_dims[q];
    const long long c = coord(q + 2, p.ext[k]);
    tc.sbase += c * p.ss[k];
    tc.dbase += c * p.ds[k];
  }
  const long long a_left = p.ext[a_last] - ta * p.a_tile;
  const long long b_left = p.ext[b_last] - tb * p.b_tile;
  tc.va = static_cast<int>(p.a_inner * (a_left < p.a_tile ? a_left : p.a_tile));
  tc.vb = static_cast<int>(p.b_inner * (b_left < p.b_tile ? b_left : p.b_tile));
  return tc;
}

// Threads of a pipelined tile block, and the largest tile (elements) of each
// payload width: the register stage holds a tile's share per thread.
constexpr int kTileThreads = 256;
template <typename P>
constexpr int max_tile_elems() {
  return sizeof(P) >= 16 ? 32 * 32 : sizeof(P) >= 8 ? 64 * 32 : 64 * 64;
}

// `Pipelined`: with kTileThreads threads a block holds the next tile's loads in
// registers while it stores the current one (the launchers' kernel); the
// entries, which carry every plan's code in one kernel, take the tile-at-a-
// time walk, whose registers do not cap the occupancy of all their paths.
template <typename P, int VL, int VS, bool Pipelined>
__device__ __forceinline__ void move_tiles(P* __restrict__ dst, const P* __restrict__ src,
                                           const MovePlan& p, const long long* src_a,
                                           const long long* dst_b, P* tile,
                                           unsigned int blocks) {
  const int la = static_cast<int>(p.la);
  const int lb = static_cast<int>(p.lb);
  const int pitch = lb + 1;
  const int tid = threadIdx.x;
  const int lbv = lb / VL;
  const int lav = la / VS;
  auto store_tile = [&](const TileCoords& tc) {
    P* d = dst + tc.dbase;
    for (int e = tid; e < lb * lav; e += blockDim.x) {
      const int j = e / lav;
      const int i = (e - j * lav) * VS;
      if (i < tc.va && j < tc.vb) {
        Vec<P, VS> x;
#pragma unroll
        for (int k = 0; k < VS; ++k) x.v[k] = tile[(i + k) * pitch + j];
        nt_store<P, VS>(d + i + dst_b[j], x);
      }
    }
  };
  long long t = blockIdx.x;
  if (!Pipelined || blockDim.x != kTileThreads) {
    // Any other block size: load, park, store, one tile at a time.
    for (; t < p.tiles; t += blocks) {
      const TileCoords tc = tile_coords(p, t);
      const P* s = src + tc.sbase;
      for (int e = tid; e < la * lbv; e += blockDim.x) {
        const int i = e / lbv;
        const int j = (e - i * lbv) * VL;
        if (i < tc.va && j < tc.vb) {
          const Vec<P, VL> x = nt_load<P, VL>(s + src_a[i] + j);
#pragma unroll
          for (int k = 0; k < VL; ++k) tile[i * pitch + j + k] = x.v[k];
        }
      }
      __syncthreads();
      store_tile(tc);
      __syncthreads();
    }
    return;
  }
  constexpr int R = max_tile_elems<P>() / VL / kTileThreads;  // register vectors per thread
  // This thread's tile slots (row i, column j) are the same for every tile.
  int slot_i[R], slot_j[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int e = tid + r * kTileThreads;
    slot_i[r] = e < la * lbv ? e / lbv : la;  // la: no slot
    slot_j[r] = e < la * lbv ? (e - slot_i[r] * lbv) * VL : 0;
  }
  Vec<P, VL> regs[R];
  auto load_tile = [&](const TileCoords& tc) {
    const P* s = src + tc.sbase;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (slot_i[r] < tc.va && slot_j[r] < tc.vb)
        regs[r] = nt_load<P, VL>(s + src_a[slot_i[r]] + slot_j[r]);
    }
  };
  if (t >= p.tiles) return;
  TileCoords cur = tile_coords(p, t);
  load_tile(cur);
  for (;;) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (slot_i[r] < cur.va && slot_j[r] < cur.vb) {
#pragma unroll
        for (int k = 0; k < VL; ++k) tile[slot_i[r] * pitch + slot_j[r] + k] = regs[r].v[k];
      }
    }
    __syncthreads();
    const long long next = t + blocks;
    TileCoords nxt = cur;
    if (next < p.tiles) {
      nxt = tile_coords(p, next);
      load_tile(nxt);  // in flight while this tile is stored
    }
    store_tile(cur);
    __syncthreads();
    if (next >= p.tiles) break;
    t = next;
    cur = nxt;
  }
}

// The TilePlan body: tile t's coordinates by precomputed divisors (uniform,
// scalar), then every load of the thread issued before its first LDS write,
// as in the tiled transpose; element (i, j) of the LA x LB tile sits at
// src_base + src_a(i) + j and dst_base + i + dst_b(j), the chain offsets
// decoded per slot (at most two digits). A partial tile's empty slots load
// the tile's first element instead (so no branch separates the loads) and are
// neither parked nor stored.
// Where element (i, j) of the LA x LB tile sits in LDS. The
// LDS serves a wave's 8-byte reads 32 lanes a pass over 64 banks of 4 bytes
// and its 8-byte writes 16 lanes a pass over 32 banks (measured on gfx950
// with SQ_LDS_BANK_CONFLICT over fixed lane patterns). Rows padded by one
// element serve every access pattern of 4- and 16-byte elements without
// conflict. For 8-byte elements (64 x 32) they do not: a 16-byte store vector
// reads rows 2n and 2n + 1 of a column (n = 0..31 over 32 lanes), which the
// pad puts on 16 bank pairs, two lanes each, and a 16-byte load vector (VL =
// 2) writes columns 2m + k of a row (m = 0..15 over 16 lanes), on 8 bank
// pairs mod 32: every such read and write took two passes. Those tiles are
// unpadded: column j of row i sits at g(j) ^ (i % 32) ^ (i / 32), where g
// interleaves the even columns before the odd ones when VL = 2 (identity
// otherwise). The XOR term sends any 32 consecutive rows, and the 32 even and
// the 32 odd rows, of a column to 32 distinct bank pairs; g puts the 16
// columns 2m + k that 16 lanes write at once on 16 consecutive words.
template <typename P, int LA, int LB, int VL>
struct TileSlots {
  static constexpr bool kSwizzled = sizeof(P) == 8 && LB == 32 && LA == 2 * LB;
  static constexpr int kElems = kSwizzled ? LA * LB : LA * (LB + 1);
  static __device__ __forceinline__ int at(int i, int j) {
    if constexpr (kSwizzled) {
      const int g = VL == 2 ? (j >> 1) | ((j & 1) << 4) : j;
      return i * LB + (g ^ (i & (LB - 1)) ^ (i / LB));
    } else {
      return i * (LB + 1) + j;
    }
  }
};

// The source and destination bases of tile `t` and its valid extents (in
// elements) along the A and B sides; uniform over the block.
struct TileBase {
  long long sb, db;
  int va, vb;
};

template <typename TP>
__device__ __forceinline__ TileBase tile_base(const TP& tp, unsigned int t) {
  unsigned int rest = t, first = 0, ta = 0, tb = 0;
  TileBase b;
  b.sb = tp.src_offset;
  b.db = tp.dst_offset;
#pragma unroll
  for (int q = 0; q < TP::kCoords; ++q) {
    if (q < tp.ncoord) {
      const unsigned int quot = div_by(rest, tp.coord[q]);
      unsigned int c = rest - quot * tp.coord[q].d;
      rest = quot;
      if (q == tp.skew_second) {
        const unsigned int u = c + first;
        c = u - div_by(u, tp.coord[q]) * tp.coord[q].d;
      }
      if (q == tp.skew_first) first = c;
      if (q == 0) ta = c;
      if (q == 1) tb = c;
      b.sb += static_cast<long long>(c) * tp.coord_ss[q];
      b.db += static_cast<long long>(c) * tp.coord_ds[q];
    }
  }
  const unsigned int a_left = tp.a_last - ta * tp.a_tile;
  const unsigned int b_left = tp.b_last - tb * tp.b_tile;
  b.va = static_cast<int>(tp.a_in.d * (a_left < tp.a_tile ? a_left : tp.a_tile));
  b.vb = static_cast<int>(tp.b_in.d * (b_left < tp.b_tile ? b_left : tp.b_tile));
  return b;
}

// Offset of tile row i from the tile's source base (the A chain's two digits
// times their source strides), and of tile column j from its destination base.
template <typename TP>
__device__ __forceinline__ long long tile_src_a(const TP& tp, int i) {
  const unsigned int o = div_by(static_cast<unsigned int>(i), tp.a_in);
  return static_cast<long long>(i - static_cast<int>(o * tp.a_in.d)) * tp.a_ss0 +
         static_cast<long long>(o) * tp.a_ss1;
}
template <typename TP>
__device__ __forceinline__ long long tile_dst_b(const TP& tp, int j) {
  const unsigned int o = div_by(static_cast<unsigned int>(j), tp.b_in);
  return static_cast<long long>(j - static_cast<int>(o * tp.b_in.d)) * tp.b_ds0 +
         static_cast<long long>(o) * tp.b_ds1;
}

// Persistent walk: the block moves tiles blockIdx.x, blockIdx.x + blocks, ...
// and issues the next tile's loads before it stores the current tile from LDS
// (so loads stay in flight through the store phase instead of waiting for a
// new block: C5's permute in 97 us against 102 with a block per tile). Every
// wave of a block takes the same branches (the tile count and bases are
// uniform).
// Each slot's offset inside a tile, the same for every tile, is computed once
// per thread; `Narrow`: their byte span fits 31 bits (tile_offsets_narrow),
// and each takes one register instead of two.
// Not `Pipelined` (the entries, which carry every plan's code in one kernel
// and whose occupancy the walk's registers would cap): one tile at a time,
// loaded, parked and stored before the next, its offsets computed per tile.
template <typename P, int VL, int VS, int LA, int LB, typename TP, bool Narrow,
          bool Pipelined = true>
__device__ __forceinline__ void move_tile_walk(P* __restrict__ dst, const P* __restrict__ src,
                                               const TP& tp, P* tile, unsigned int tiles,
                                               unsigned int blocks) {
  constexpr int BS = kBlock;
  using Slots = TileSlots<P, LA, LB, VL>;
  constexpr int LBV = LB / VL;
  constexpr int LAV = LA / VS;
  constexpr int RL = LA * LBV / BS;
  constexpr int RS = LB * LAV / BS;
  static_assert(RL * BS == LA * LBV && RS * BS == LB * LAV, "the block divides the tile");
  const int tid = threadIdx.x;
  if constexpr (!Pipelined) {
    // The tile count is below 2^30 (tile_plan), so t + blocks cannot wrap.
    for (unsigned int t = blockIdx.x; t < tiles; t += blocks) {
      const TileBase b = tile_base(tp, t);
      const P* s = src + b.sb;
      P* d = dst + b.db;
      Vec<P, VL> x[RL];
#pragma unroll
      for (int r = 0; r < RL; ++r) {
        const int e = tid + r * BS;
        const int i = e / LBV;
        const int j = (e % LBV) * VL;
        x[r] = nt_load<P, VL>(i < b.va && j < b.vb ? s + tile_src_a(tp, i) + j : s);
      }
#pragma unroll
      for (int r = 0; r < RL; ++r) {
        const int e = tid + r * BS;
        const int i = e / LBV;
        const int j = (e % LBV) * VL;
        if (i < b.va && j < b.vb) {
#pragma unroll
          for (int k = 0; k < VL; ++k) tile[Slots::at(i, j + k)] = x[r].v[k];
        }
      }
      __syncthreads();
#pragma unroll
      for (int r = 0; r < RS; ++r) {
        const int e = tid + r * BS;
        const int j = e / LAV;
        const int i = (e % LAV) * VS;
        if (i < b.va && j < b.vb) {
          Vec<P, VS> y;
#pragma unroll
          for (int k = 0; k < VS; ++k) y.v[k] = tile[Slots::at(i + k, j)];
          nt_store<P, VS>(d + i + tile_dst_b(tp, j), y);
        }
      }
      __syncthreads();  // the next tile is parked over this one
    }
    return;
  }
  unsigned int t = blockIdx.x;
  if (t >= tiles) return;
  // Narrow: each slot's offset is kept as an unsigned 32-bit byte offset from
  // a uniform corner of the tile (the base moved by the in-tile strides'
  // negative parts), so every access is a scalar base plus a 32-bit lane
  // offset; otherwise as a 64-bit element offset from the tile's base.
  using Off = std::conditional_t<Narrow, unsigned int, long long>;
  long long s_shift = 0, d_shift = 0;
  if constexpr (Narrow) {
    auto low = [](long long stride, unsigned int count) {
      return stride < 0 ? stride * static_cast<long long>(count - 1) : 0ll;
    };
    s_shift = low(tp.a_ss0, tp.a_in.d) + low(tp.a_ss1, tp.a_tile);
    d_shift = low(tp.b_ds0, tp.b_in.d) + low(tp.b_ds1, tp.b_tile);
  }
  auto narrow = [](long long elements) {
    return static_cast<Off>(Narrow ? elements * static_cast<long long>(sizeof(P)) : elements);
  };
  Off soff[RL], doff[RS];
#pragma unroll
  for (int r = 0; r < RL; ++r) {
    const int e = tid + r * BS;
    soff[r] = narrow(tile_src_a(tp, e / LBV) + (e % LBV) * VL - s_shift);
  }
#pragma unroll
  for (int r = 0; r < RS; ++r) {
    const int e = tid + r * BS;
    doff[r] = narrow((e % LAV) * VS + tile_dst_b(tp, e / LAV) - d_shift);
  }
  // The first element of the tile (the load of an empty slot, the store of
  // an empty slot's stand-in), at offset -shift.
  const Off s_first = narrow(-s_shift);
  const Off d_first = narrow(-d_shift);
  auto at = [](auto* base, long long corner, Off off) {
    using Q = std::remove_pointer_t<decltype(base)>;
    if constexpr (Narrow) {
      using B = std::conditional_t<std::is_const_v<Q>, const char, char>;
      return reinterpret_cast<Q*>(reinterpret_cast<B*>(base + corner) + off);
    } else {
      return base + corner + off;
    }
  };
  Vec<P, VL> x[RL];
  auto load = [&](const TileBase& b) {
#pragma unroll
    for (int r = 0; r < RL; ++r) {
      const int e = tid + r * BS;
      const bool valid = e / LBV < b.va && (e % LBV) * VL < b.vb;
      x[r] = nt_load<P, VL>(at(src, b.sb + s_shift, valid ? soff[r] : s_first));
    }
  };
  auto park = [&](const TileBase& b) {
#pragma unroll
    for (int r = 0; r < RL; ++r) {
      const int e = tid + r * BS;
      const int i = e / LBV;
      const int j = (e % LBV) * VL;
      if (i < b.va && j < b.vb) {
#pragma unroll
        for (int k = 0; k < VL; ++k) tile[Slots::at(i, j + k)] = x[r].v[k];
      }
    }
  };
  // Every slot stores: an empty slot of a partial tile stores the tile's
  // first vector (elements 0 .. VS - 1 of column 0, valid in any non-empty
  // tile: a partial tile's valid length is a multiple of VS) over itself, the
  // same bytes its own slot writes. With no branch around them, the compiler
  // counts exactly RS stores after the next tile's loads and waits for those
  // loads alone before parking them (a branch would make it wait for the
  // stores as well).
  auto store = [&](const TileBase& b) {
#pragma unroll
    for (int r = 0; r < RS; ++r) {
      const int e = tid + r * BS;
      const bool valid = e / LAV < b.vb && (e % LAV) * VS < b.va;
      const int j = valid ? e / LAV : 0;
      const int i = valid ? (e % LAV) * VS : 0;
      Vec<P, VS> y;
#pragma unroll
      for (int k = 0; k < VS; ++k) y.v[k] = tile[Slots::at(i + k, j)];
      nt_store<P, VS>(at(dst, b.db + d_shift, valid ? doff[r] : d_first), y);
    }
  };
  TileBase cur = tile_base(tp, t);
  load(cur);
  park(cur);
  __syncthreads();
  for (;;) {
    // t < tiles, so tiles - t cannot wrap, and neither can t + blocks.
    if (!(blocks < tiles - t)) {
      store(cur);
      return;
    }
    t += blocks;
    const TileBase nb = tile_base(tp, t);
    load(nb);
    store(cur);
    __syncthreads();  // every wave has read the tile before it is overwritten
    park(nb);
    __syncthreads();
    cur = nb;
  }
}

// Offsets of run position `i` along a chain: mixed-radix digits over the
// chain's extents (the last digit bounded by the tile), times the other side's
// strides.
__host__ __device__ inline long long chain_offset(const MovePlan& p, const int* dims, int count,
                                                  long long last_tile, const long long* strides,
                                                  long long i) {
  long long off = 0;
  for (int c = 0; c < count; ++c) {
    const int k = dims[c];
    const long long e = c + 1 < count ? p.ext[k] : last_tile;
    off += (i % e) * strides[k];
    i /= e;
  }
  return off;
}

// 16-byte accesses along a run need every run start to be a multiple of V:
// the base offset, every stride outside the run, the tile step of the run's
// tiled dim, and every partial tile's valid length.
__host__ __device__ inline bool run_vectorizable(const MovePlan& p, const int* dims, int count,
                                                 long long inner, long long tile,
                                                 const long long* strides, long long offset,
                                                 int v, const void* ptr) {
  if (v <= 1 || (reinterpret_cast<uintptr_t>(ptr) & 15) != 0) return false;
  if (offset % v != 0) return false;
  const int last = dims[count - 1];
  const bool tail_ok = inner % v == 0 || (tile % v == 0 && p.ext[last] % v == 0);
  if (!tail_ok) return false;
  if ((tile * inner) % v != 0) return false;
  for (int k = 0; k < p.n; ++k) {
    if (move_chain_contains(dims, count, k)) continue;
    if (strides[k] % v != 0) return false;
  }
  return true;
}

// The vector width (elements per 16-byte access) of a payload on the tiled
// path, and whether the source (VL) and destination (VS) runs take it.
template <typename P>
constexpr int tile_vector() {
  return sizeof(P) <= 8 && sizeof(P) >= 4 ? 16 / static_cast<int>(sizeof(P)) : 1;
}

__host__ __device__ inline void tile_vectorizable(const MovePlan& p, int v, const void* dst,
                                                  const void* src, bool* vl, bool* vs) {
  *vl = run_vectorizable(p, p.b_dims, p.nb, p.b_inner, p.b_tile, p.ss, p.src_offset, v, src);
  *vs = run_vectorizable(p, p.a_dims, p.na, p.a_inner, p.a_tile, p.ds, p.dst_offset, v, dst);
}

// LDS layout of a tiled block: the two run-offset tables, then the tile.
__device__ __forceinline__ void tile_tables(const MovePlan& p, unsigned char* lds) {
  long long* src_a = reinterpret_cast<long long*>(lds);
  long long* dst_b = src_a + kMoveRunMax;
  for (int i = threadIdx.x; i < p.la; i += blockDim.x)
    src_a[i] = chain_offset(p, p.a_dims, p.na, p.a_tile, p.ss, i);
  for (int j = threadIdx.x; j < p.lb; j += blockDim.x)
    dst_b[j] = chain_offset(p, p.b_dims, p.nb, p.b_tile, p.ds, j);
  __syncthreads();
}

template <typename P, int VL, int VS, bool Pipelined>
__device__ __forceinline__ void move_tiled_as(void* dst, const void* src, const MovePlan& p,
                                              unsigned char* lds, unsigned int blocks) {
  tile_tables(p, lds);
  const long long* src_a = reinterpret_cast<const long long*>(lds);
  move_tiles<P, VL, VS, Pipelined>(static_cast<P*>(dst), static_cast<const P*>(src), p, src_a,
                        src_a + kMoveRunMax,
                        reinterpret_cast<P*>(lds + 2 * kMoveRunMax * sizeof(long long)), blocks);
}

// The entries' tiled walk (one tile at a time).
template <typename P>
__device__ __forceinline__ void move_tiled(void* dst, const void* src, const MovePlan& p,
                                           unsigned char* lds, unsigned int blocks) {
  constexpr int V = tile_vector<P>();
  bool vl, vs;
  tile_vectorizable(p, V, dst, src, &vl, &vs);
  if (vl && vs) {
    move_tiled_as<P, V, V, false>(dst, src, p, lds, blocks);
  } else if (vl) {
    move_tiled_as<P, V, 1, false>(dst, src, p, lds, blocks);
  } else if (vs) {
    move_tiled_as<P, 1, V, false>(dst, src, p, lds, blocks);
  } else {
    move_tiled_as<P, 1, 1, false>(dst, src, p, lds, blocks);
  }
}

// CONTIG: rows along the fused dim `row_dim`, contiguous on both sides.
template <typename P, int BS>
__device__ __forceinline__ void move_rows(void* dst, const void* src, const MovePlan& p,
                                          unsigned int blocks) {
  P* d = static_cast<P*>(dst);
  const P* s = static_cast<const P*>(src);
  const int bs = block_threads<BS>();
  const long long gstride = static_cast<long long>(blocks) * bs;
  for (long long f = static_cast<long long>(blockIdx.x) * bs + threadIdx.x; f < p.len;
       f += gstride) {
    long long rest = f / p.row_len;
    long long so = p.src_offset + (f - rest * p.row_len);
    long long dof = p.dst_offset + (f - rest * p.row_len);
    for (int k = 0; k < p.n; ++k) {
      if (k == p.row_dim) continue;
      const long long c = rest % p.ext[k];
      rest /= p.ext[k];
      so += c * p.ss[k];
      dof += c * p.ds[k];
    }
    d[dof] = s[so];
  }
}

// CONTIG rows through a RowPlan (the launchers): one unit of V elements per
// thread of a kBlock-thread grid of `blocks` <= 2^23 blocks (so the 32-bit
// unit index and its grid stride stay below 2^32), the row decoded with
// 32-bit multiply-high quotients; the store streams past the caches, the load
// too unless the source is read again across rows (a broadcast).
template <typename P, int V, bool NTL, int NR>
__device__ __forceinline__ void move_row_units(void* dst, const void* src, const RowPlan& rp,
                                               unsigned int blocks) {
  P* d = static_cast<P*>(dst);
  const P* s = static_cast<const P*>(src);
  const unsigned int gstride = blocks * static_cast<unsigned int>(kBlock);
  for (unsigned int u = blockIdx.x * static_cast<unsigned int>(kBlock) + threadIdx.x;
       u < rp.units; u += gstride) {
    const unsigned int row = div_by(u, rp.row_div);
    const unsigned int col = u - row * rp.vpr;
    long long so = rp.src_offset + static_cast<long long>(col) * V;
    long long dof = rp.dst_offset + static_cast<long long>(col) * V;
    unsigned int r = row;
#pragma unroll
    for (int k = 0; k < (NR >= 0 ? NR : kMaxDims); ++k) {
      if (NR < 0 && k >= rp.n) break;
      const unsigned int q = div_by(r, rp.div[k]);
      const long long c = static_cast<long long>(r - q * rp.div[k].d);
      so += c * rp.ss[k];
      dof += c * rp.ds[k];
      r = q;
    }
    Vec<P, V> x;
    if constexpr (NTL) {
      x = nt_load<P, V>(s + so);
    } else {
      x = *reinterpret_cast<const Vec<P, V>*>(s + so);
    }
    nt_store<P, V>(d + dof, x);
  }
}

// GENERIC: one decode per element on both sides.
template <typename P, int BS>
__device__ __forceinline__ void move_elements(void* dst, const void* src, const MovePlan& p,
                                              unsigned int blocks) {
  P* d = static_cast<P*>(dst);
  const P* s = static_cast<const P*>(src);
  const int bs = block_threads<BS>();
  const long long gstride = static_cast<long long>(blocks) * bs;
  if (p.coords32 && gstride < (1ll << 31)) {
    // f < len < 2^31 and f + gstride < 2^32: 32-bit indices and divisors.
    const unsigned int len = static_cast<unsigned int>(p.len);
    for (unsigned int f = blockIdx.x * bs + threadIdx.x; f < len;
         f += static_cast<unsigned int>(gstride)) {
      unsigned int rest = f;
      long long so = p.src_offset;
      long long dof = p.dst_offset;
      for (int k = 0; k < p.n; ++k) {
        const unsigned int q = div_by(rest, p.coord_div[k]);
        const unsigned int c = rest - q * p.coord_div[k].d;
        rest = q;
        so += static_cast<long long>(c) * p.ss[k];
        dof += static_cast<long long>(c) * p.ds[k];
      }
      d[dof] = s[so];
    }
    return;
  }
  for (long long f = static_cast<long long>(blockIdx.x) * bs + threadIdx.x; f < p.len;
       f += gstride) {
    long long rest = f;
    long long so = p.src_offset;
    long long dof = p.dst_offset;
    for (int k = 0; k < p.n; ++k) {
      const long long c = rest % p.ext[k];
      rest /= p.ext[k];
      so += c * p.ss[k];
      dof += c * p.ds[k];
    }
    d[dof] = s[so];
  }
}

// A value every lane holds alike, read out of LDS into scalar registers (one
// readfirstlane per dword), so that a loop reads it without LDS traffic.
template <typename T>
__device__ __forceinline__ T uniform_copy(const T& shared_value) {
  static_assert(sizeof(T) % 4 == 0, "whole dwords");
  unsigned int words[sizeof(T) / 4];
  __builtin_memcpy(words, &shared_value, sizeof(T));
#pragma unroll
  for (int i = 0; i < static_cast<int>(sizeof(T) / 4); ++i)
    words[i] = __builtin_amdgcn_readfirstlane(words[i]);
  T out;
  __builtin_memcpy(&out, words, sizeof(T));
  return out;
}

// TILED inside the entries: when the plan has a TilePlan form (tile_plan),
// thread 0 writes it into the block's move scratch behind the tile, and the
// block moves tiles blockIdx.x, blockIdx.x + blocks, ... with the launchers'
// tile body, one tile at a time, so a persistent grid plans once per block;
// other plans and block sizes take the general tile walk.
template <typename P>
__device__ __forceinline__ void move_tiled_entry(void* dst, const void* src, const MovePlan& p,
                                                 unsigned char* lds, unsigned int blocks) {
  if constexpr (sizeof(P) >= 4) {
    constexpr int LA = sizeof(P) >= 16 ? 32 : 64;
    constexpr int LB = sizeof(P) >= 8 ? 32 : 64;
    constexpr int kTileBytes = TileSlots<P, LA, LB, 1>::kElems * static_cast<int>(sizeof(P));
    static_assert(kTileBytes + static_cast<int>(sizeof(TilePlan)) <= kMoveLdsBytes,
                  "the tile and its plan share the move scratch");
    if (blockDim.x == static_cast<unsigned>(kBlock)) {
      TilePlan* shared_tp = reinterpret_cast<TilePlan*>(lds + kTileBytes);
      // 0: no TilePlan form; 1: wide slot offsets; 2: narrow ones.
      __shared__ int once_ok;
      // The entries walk the balanced shape only.
      if (threadIdx.x == 0) {
        once_ok = p.la == LA && p.lb == LB && tile_plan(shared_tp, p, static_cast<int>(sizeof(P)))
                      ? (tile_offsets_narrow(*shared_tp, LA, LB, static_cast<int>(sizeof(P))) ? 2
                                                                                          : 1)
                      : 0;
      }
      __syncthreads();
      if (once_ok) {
        constexpr int V = tile_vector<P>();
        bool vl, vs;
        tile_vectorizable(p, V, dst, src, &vl, &vs);
        P* tile = reinterpret_cast<P*>(lds);
        const unsigned int tiles = static_cast<unsigned int>(p.tiles);
        // Read from LDS: copied to scalar registers, the plan overflows the
        // scalar file, and the spills into vector registers halve the
        // occupancy of every path of the entry kernel.
        const TilePlan& tp = *shared_tp;
        // Every block of a grid the chip holds at once works (this build's
        // planned grids): the fully vectorized shapes then take the
        // launchers' pipelined walk. Under the reference's per-element grids,
        // where returning blocks need the free slots, one tile at a time
        // measured faster.
        const bool resident = blocks == gridDim.x &&
                              static_cast<unsigned long long>(gridDim.x) *
                                      ((blockDim.x + 63u) / 64u) <=
                                  kEntryResidentWaves;
        const bool narrow = once_ok == 2;
        auto walk = [&](auto vl_tag, auto vs_tag) {
          constexpr int VLt = decltype(vl_tag)::value;
          constexpr int VSt = decltype(vs_tag)::value;
          if constexpr (VLt == V && VSt == V) {
            if (resident && narrow) {
              move_tile_walk<P, VLt, VSt, LA, LB, TilePlan, true, true>(
                  static_cast<P*>(dst), static_cast<const P*>(src), tp, tile, tiles, blocks);
              return;
            }
          }
          move_tile_walk<P, VLt, VSt, LA, LB, TilePlan, false, false>(
              static_cast<P*>(dst), static_cast<const P*>(src), tp, tile, tiles, blocks);
        };
        using VV = std::integral_constant<int, V>;
        using V1 = std::integral_constant<int, 1>;
        if (vl && vs) walk(VV{}, VV{});
        else if (vl) walk(VV{}, V1{});
        else if (vs) walk(V1{}, VV{});
        else walk(V1{}, V1{});
        return;
      }
    }
  }
  move_tiled<P>(dst, src, p, lds, blocks);
}


// CONTIG inside the entries: thread 0 turns the LDS plan into the launchers'
// RowPlan (in the block's move scratch, unused by rows), every lane copies it
// to scalar registers and walks 16-byte row units as the launchers do. Other
// block sizes, and plans the row walk cannot take, decode per element.
template <typename P>
__device__ __forceinline__ void move_rows_entry(void* dst, const void* src, const MovePlan& p,
                                                unsigned char* lds, unsigned int blocks) {
  if (blockDim.x != static_cast<unsigned>(kBlock) || blocks > (1u << 23)) {
    move_rows<P, 0>(dst, src, p, blocks);
    return;
  }
  RowPlan* shared_rp = reinterpret_cast<RowPlan*>(lds);
  __shared__ int rows_ok;
  if (threadIdx.x == 0) {
    const bool aligned =
        ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) & 15) == 0;
    rows_ok = row_plan(shared_rp, p, static_cast<int>(sizeof(P)), aligned) ? 1 : 0;
  }
  __syncthreads();
  if (!rows_ok) {
    move_rows<P, 0>(dst, src, p, blocks);
    return;
  }
  const RowPlan rp = uniform_copy(*shared_rp);
  constexpr int V = sizeof(P) == 1 ? 16 : sizeof(P) == 4 ? 4 : sizeof(P) == 8 ? 2 : 1;
  const bool vec = V > 1 && p.row_len == static_cast<long long>(rp.vpr) * V;
  if (vec && rp.reread)
    move_row_units<P, V, false, -1>(dst, src, rp, blocks);
  else if (vec)
    move_row_units<P, V, true, -1>(dst, src, rp, blocks);
  else if (rp.reread)
    move_row_units<P, 1, false, -1>(dst, src, rp, blocks);
  else
    move_row_units<P, 1, true, -1>(dst, src, rp, blocks);
}

template <typename P>
__device__ __forceinline__ void move_dispatch(void* dst, const void* src, const MovePlan& p,
                                              unsigned char* lds, unsigned int blocks) {
  switch (p.mode) {
    case kMoveTiled: move_tiled_entry<P>(dst, src, p, lds, blocks); break;
    case kMoveContig: move_rows_entry<P>(dst, src, p, lds, blocks); break;
    case kMoveGeneric: move_elements<P, 0>(dst, src, p, blocks); break;
    default: break;
  }
}

__device__ __forceinline__ void move_entry(void* dst, const void* src, int dtype,
                                           const t4a_cuda_layout& src_layout,
                                           const long long* dst_strides, long long dst_offset,
                                           long long len) {
  const int es = dtype_size(dtype);
  if (es == 0) return;  // unknown tag: no work (reference c-kernel-abi.md:107-108)
  if (entry_block_idle(kMoveEntryWaves)) return;
  const unsigned int blocks = entry_blocks(kMoveEntryWaves);
  __shared__ MovePlan plan;
  __shared__ alignas(16) unsigned char lds[kMoveLdsBytes];
  if (threadIdx.x == 0) move_plan(&plan, src_layout, dst_strides, dst_offset, len, es);
  __syncthreads();
  switch (es) {
    case 1: move_dispatch<uint8_t>(dst, src, plan, lds, blocks); break;
    case 4: move_dispatch<uint32_t>(dst, src, plan, lds, blocks); break;
    case 8: move_dispatch<unsigned long long>(dst, src, plan, lds, blocks); break;
    case 16: move_dispatch<Elem16>(dst, src, plan, lds, blocks); break;
    default: break;
  }
}

// General-rank movement (reference movement.cu:620-646, docs/abi/c-kernel-abi.md
// "Dynamic rank"): the geometry arrays live in caller-owned device memory.
// Thread 0 fuses them into LDS (extent-1 axes dropped, chained axes merged);
// at most kMaxDims fused axes take the by-value entries' plan and mappings,
// more (at most 62: each has extent >= 2) a per-element decode over the fused
// axes, axis 0 first, as the reference decodes.
template <typename P>
__device__ __forceinline__ void move_elements_wide(void* dst, const void* src, int n,
                                                   const long long* fe, const long long* fs,
                                                   const long long* fd, long long src_offset,
                                                   long long dst_offset, long long len,
                                                   unsigned int blocks) {
  P* d = static_cast<P*>(dst);
  const P* s = static_cast<const P*>(src);
  const long long gstride = static_cast<long long>(blocks) * blockDim.x;
  for (long long f = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; f < len;
       f += gstride) {
    long long rest = f;
    long long so = src_offset;
    long long dof = dst_offset;
    for (int k = 0; k < n; ++k) {
      const long long c = rest % fe[k];
      rest /= fe[k];
      so += c * fs[k];
      dof += c * fd[k];
    }
    d[dof] = s[so];
  }
}

// A move over derived geometry, planned by thread 0 in LDS: `rank` axes of
// extents `ext` (device memory, read once), source strides src(k) from
// `src_offset`, destination strides dst(k) from `dst_offset` (callables, axis
// by axis in order). `ok` false does no work.
template <typename SrcStride, typename DstStride>
__device__ __forceinline__ void move_entry_by(void* dst, const void* src, int dtype, bool ok,
                                              int rank, const long long* ext, SrcStride src_st,
                                              long long src_offset, DstStride dst_st,
                                              long long dst_offset, long long len) {
  const int es = dtype_size(dtype);
  if (es == 0 || len <= 0 || !ok || rank < 0) return;
  if (entry_block_idle(kMoveEntryWaves)) return;
  const unsigned int blocks = entry_blocks(kMoveEntryWaves);
  __shared__ MovePlan plan;
  __shared__ long long fe[kMaxFusedDims], fs[kMaxFusedDims], fd[kMaxFusedDims];
  __shared__ int fused;
  __shared__ long long count;
  __shared__ alignas(16) unsigned char lds[kMoveLdsBytes];
  if (threadIdx.x == 0) {
    fused = fuse_move_by(rank, ext, src_st, dst_st, fe, fs, fd, kMaxFusedDims);
    count = fused >= 0 ? clamp_count(fused, fe, len) : 0;
    if (fused >= 0 && fused <= kMaxDims)
      move_plan_view(&plan, fused, src_offset, fe, fs, fd, dst_offset, len, es);
  }
  __syncthreads();
  if (fused < 0) return;
  auto run = [&](auto* tag) {
    using P = std::remove_pointer_t<decltype(tag)>;
    if (fused <= kMaxDims) {
      move_dispatch<P>(dst, src, plan, lds, blocks);
    } else {
      move_elements_wide<P>(dst, src, fused, fe, fs, fd, src_offset, dst_offset, count, blocks);
    }
  };
  switch (es) {
    case 1: run(static_cast<uint8_t*>(nullptr)); break;
    case 4: run(static_cast<uint32_t*>(nullptr)); break;
    case 8: run(static_cast<unsigned long long*>(nullptr)); break;
    case 16: run(static_cast<Elem16*>(nullptr)); break;
    default: break;
  }
}

// `dst_layout == nullptr`: the compact destination of materialize_strided.
// Ranks that differ do no work.
__device__ __forceinline__ void move_entry_any(void* dst, const void* src, int dtype,
                                               const t4a_cuda_layout_any& src_layout,
                                               const t4a_cuda_layout_any* dst_layout,
                                               long long len) {
  const bool ok = dst_layout == nullptr || dst_layout->rank == src_layout.rank;
  move_entry_by(dst, src, dtype, ok, src_layout.rank, src_layout.extents,
                strides_of(src_layout.strides, src_layout.extents), src_layout.offset,
                strides_of(dst_layout ? dst_layout->strides : nullptr, src_layout.extents),
                dst_layout ? dst_layout->offset : 0, len);
}

// ---- copy_exact -----------------------------------------------------------------------
// A bit-preserving copy of len elements (reference movement.cu:91-97, entry
// 528-533). With both pointers 16-byte aligned the bytes stream as non-temporal
// 16-byte vectors, one per thread of the planned grid: on this part a copy
// reaches HBM speed through many short-lived wavefronts with one load and one
// store each (several vectors per thread measured 5-8 % slower, the extra
// stores waiting behind each other). A smaller grid (the reference's geometry
// through the module entry) strides over the rest. The elements after the last
// whole vector, and unaligned buffers, go element by element.
template <typename P, int BS>
__device__ __forceinline__ void copy_elements(void* dst, const void* src, long long first,
                                              long long len, unsigned int blocks) {
  P* d = static_cast<P*>(dst);
  const P* s = static_cast<const P*>(src);
  const int bs = block_threads<BS>();
  const long long gstride = static_cast<long long>(blocks) * bs;
  for (long long i = first + static_cast<long long>(blockIdx.x) * bs + threadIdx.x; i < len;
       i += gstride)
    d[i] = s[i];
}

// `blocks`: the grid's block count, an argument for the launcher's kernel
// (gridDim.x costs hidden-argument loads, a second scalar round trip before
// the first vector load), gridDim.x for the entry.
template <typename P, int BS>
__device__ __forceinline__ void copy_body(void* dst, const void* src, long long len,
                                          unsigned int blocks) {
  const bool aligned = ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) &
                        15) == 0;
  if (!aligned || sizeof(P) > 16) {
    copy_elements<P, BS>(dst, src, 0, len, blocks);
    return;
  }
  const long long vectors = len * static_cast<long long>(sizeof(P)) / 16;
  Bits128* d = static_cast<Bits128*>(dst);
  const Bits128* s = static_cast<const Bits128*>(src);
  const int bs = block_threads<BS>();
  for (long long i = static_cast<long long>(blockIdx.x) * bs + threadIdx.x; i < vectors;
       i += static_cast<long long>(blocks) * bs)
    nt_store<Bits128, 1>(d + i, nt_load<Bits128, 1>(s + i));
  // Elements after the last whole vector.
  copy_elements<P, BS>(dst, src, vectors * 16 / static_cast<long long>(sizeof(P)), len,
                       blocks);
}

// ---- fill_zero / fill_zero_view -------------------------------------------------------
// Every element type's zero is all-zero bits (reference t4a_cuda_zero,
// cuda/include/t4a/abi.cuh:520-538: 0, +0.0, {+0.0, +0.0}). fill_zero writes
// len contiguous elements as the copy streams them: one non-temporal 16-byte
// vector per thread when the buffer is 16-byte aligned, element by element
// after the last whole vector and otherwise (reference movement.cu:70-76).
template <typename P, int BS>
__device__ __forceinline__ void fill_body(void* out, long long len, unsigned int blocks) {
  const int bs = block_threads<BS>();
  const long long gstride = static_cast<long long>(blocks) * bs;
  long long first = 0;
  if ((reinterpret_cast<uintptr_t>(out) & 15) == 0 && sizeof(P) <= 16) {
    const long long vectors = len * static_cast<long long>(sizeof(P)) / 16;
    Bits128* o = static_cast<Bits128*>(out);
    const Vec<Bits128, 1> zero{};
    for (long long i = static_cast<long long>(blockIdx.x) * bs + threadIdx.x; i < vectors;
         i += gstride)
      nt_store<Bits128, 1>(o + i, zero);
    first = vectors * 16 / static_cast<long long>(sizeof(P));
  }
  P* o = static_cast<P*>(out);
  for (long long i = first + static_cast<long long>(blockIdx.x) * bs + threadIdx.x; i < len;
       i += gstride)
    o[i] = P{};
}

// fill_zero_view over a FillPlan: V flat indices per thread, stored as one
// vector when fill_vectorizable (reference movement.cu:78-96 zeroes one element
// per thread at its decoded address).
template <typename P, int V, int BS>
__device__ __forceinline__ void fill_view_body(void* out, const FillPlan& fp, unsigned int blocks) {
  P* o = static_cast<P*>(out) + fp.offset;
  const long long units = fp.len / V;
  const int bs = block_threads<BS>();
  const long long gstride = static_cast<long long>(blocks) * bs;
  const Vec<P, V> zero{};
  for (long long u = static_cast<long long>(blockIdx.x) * bs + threadIdx.x; u < units;
       u += gstride) {
    long long off = 0;
    if (fp.narrow) {
      unsigned int r = static_cast<unsigned int>(u * V);
#pragma unroll
      for (int k = 0; k < kMaxDims; ++k) {
        if (k >= fp.n) break;
        const unsigned int q = div_by(r, fp.div[k]);
        off += static_cast<long long>(r - q * fp.div[k].d) * fp.st[k];
        r = q;
      }
    } else {
      long long r = u * V;
#pragma unroll
      for (int k = 0; k < kMaxDims; ++k) {
        if (k >= fp.n) break;
        off += (r % fp.ext[k]) * fp.st[k];
        r /= fp.ext[k];
      }
    }
    nt_store<P, V>(o + off, zero);
  }
}

// A fused view wider than kMaxDims axes (the general-rank entry): one element
// per thread, decoded over the LDS-resident axes.
template <typename P>
__device__ __forceinline__ void fill_view_wide(void* out, int n, const long long* fe,
                                               const long long* fs, long long offset,
                                               long long len, unsigned int blocks) {
  P* o = static_cast<P*>(out);
  const long long gstride = static_cast<long long>(blocks) * blockDim.x;
  for (long long f = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; f < len;
       f += gstride) {
    long long rest = f;
    long long off = offset;
    for (int k = 0; k < n; ++k) {
      off += (rest % fe[k]) * fs[k];
      rest /= fe[k];
    }
    o[off] = P{};
  }
}

// The entries' fill: thread 0 fuses the view (any rank, arrays read once)
// into LDS and builds the plan; 16-byte stores where the plan and pointer
// allow.
__device__ __forceinline__ void fill_view_entry(void* out, int dtype, int rank, long long offset,
                                                const long long* ext, const long long* st,
                                                long long len) {
  const int es = dtype_size(dtype);
  if (es == 0 || len <= 0 || rank < 0) return;
  if (entry_block_idle(kMoveEntryWaves)) return;
  const unsigned int blocks = entry_blocks(kMoveEntryWaves);
  __shared__ FillPlan plan;
  __shared__ long long fe[kMaxFusedDims], fs[kMaxFusedDims], fd[kMaxFusedDims];
  __shared__ int fused;
  __shared__ long long count;
  if (threadIdx.x == 0) {
    fused = fuse_move(rank, ext, st, st, fe, fs, fd, kMaxFusedDims);
    count = fused >= 0 ? clamp_count(fused, fe, len) : 0;
    if (fused >= 0 && fused <= kMaxDims) fill_plan(&plan, fused, fe, fs, offset, len);
  }
  __syncthreads();
  if (fused < 0) return;
  auto run = [&](auto* tag) {
    using P = std::remove_pointer_t<decltype(tag)>;
    constexpr int V = sizeof(P) <= 8 && sizeof(P) >= 4 ? 16 / static_cast<int>(sizeof(P)) : 1;
    if (fused > kMaxDims) {
      fill_view_wide<P>(out, fused, fe, fs, offset, count, blocks);
    } else if (V > 1 && (reinterpret_cast<uintptr_t>(out) & 15) == 0 &&
               fill_vectorizable(plan, V)) {
      fill_view_body<P, V, 0>(out, plan, blocks);
    } else {
      fill_view_body<P, 1, 0>(out, plan, blocks);
    }
  };
  switch (es) {
    case 1: run(static_cast<uint8_t*>(nullptr)); break;
    case 4: run(static_cast<uint32_t*>(nullptr)); break;
    case 8: run(static_cast<unsigned long long*>(nullptr)); break;
    case 16: run(static_cast<Elem16*>(nullptr)); break;
    default: break;
  }
}

// ---- kernels the launchers use: one per payload width, the plan computed on
// the host and passed by value. ----

template <typename P, int BS>
__global__ void __launch_bounds__(256)
    copy_kernel(void* dst, const void* src, long long len, unsigned int blocks) {
  copy_body<P, BS>(dst, src, len, blocks);
}

template <typename P, int BS, bool Ordered>
__global__ void __launch_bounds__(512)
    transpose_kernel(void* dst, const void* src, long long src_offset, long long batch_stride,
                     long long dst_fast_extent, long long src_fast_extent, TileOrder order) {
  __shared__ alignas(16) unsigned char lds[kTransposeLdsBytes];
  transpose_dispatch<P, BS, Ordered>(dst, src, src_offset, batch_stride, dst_fast_extent,
                                     src_fast_extent, lds, order);
}

template <typename P, int VL, int VS>
__global__ void __launch_bounds__(256)
    move_tiled_kernel(void* dst, const void* src, MovePlan plan) {
  __shared__ alignas(16) unsigned char lds[kMoveLdsBytes];
  move_tiled_as<P, VL, VS, true>(dst, src, plan, lds, gridDim.x);
}

template <typename P, int BS>
__global__ void __launch_bounds__(256)
    fill_kernel(void* out, long long len, unsigned int blocks) {
  fill_body<P, BS>(out, len, blocks);
}

template <typename P, int V, int BS>
__global__ void __launch_bounds__(256)
    fill_view_kernel(void* out, FillPlan fp, unsigned int blocks) {
  fill_view_body<P, V, BS>(out, fp, blocks);
}

// NR: the row plan's other-dim count when 0, 1 or 2 (the loop unrolled to
// exactly those), -1 for any count.
template <typename P, int V, bool NTL, int NR>
__global__ void __launch_bounds__(kBlock)
    move_rows_kernel(void* dst, const void* src, RowPlan rp, unsigned int blocks) {
  move_row_units<P, V, NTL, NR>(dst, src, rp, blocks);
}

// Eight wavefronts per SIMD for the narrow walk of 16-byte elements: its
// scalar registers (102) otherwise hold it to seven, and a grid of seven
// blocks per CU leaves C5's 16,384 tiles 9.14 rounds, a tenth round in which
// one block in seven works (97.2 against 100.2 us with the request, which
// moves 32 scalar registers to vector lanes). The 8-byte walk already has
// eight (99 scalar registers); the request made it spill 74 and run 3 %
// slower on C3.
template <typename P>
constexpr int walk_waves(bool narrow) {
  return narrow && sizeof(P) == 16 ? 8 : 1;
}

template <typename P, int VL, int VS, int LA, int LB, typename TP, bool Narrow>
__global__ void __launch_bounds__(kBlock, walk_waves<P>(Narrow))
    move_tile_walk_kernel(void* dst, const void* src, TP tp, unsigned int tiles) {
  __shared__ P tile[TileSlots<P, LA, LB, VL>::kElems];
  move_tile_walk<P, VL, VS, LA, LB, TP, Narrow>(static_cast<P*>(dst),
                                                static_cast<const P*>(src), tp, tile, tiles,
                                                gridDim.x);
}

template <typename P, int BS>
__global__ void __launch_bounds__(256) move_flat_kernel(void* dst, const void* src, MovePlan plan) {
  if (plan.mode == kMoveContig) {
    move_rows<P, BS>(dst, src, plan, gridDim.x);
  } else {
    move_elements<P, BS>(dst, src, plan, gridDim.x);
  }
}

}  // namespace
}  // namespace t4a

using t4a::kBlock;

extern "C" __global__ void __launch_bounds__(512)
    t4a_cuda_tiled_transpose(void* dst, const void* src, int dtype, long long src_offset,
                             long long batch_stride, long long dst_fast_extent,
                             long long src_fast_extent, t4a_cuda_transpose_config config) {
  // An unsupported configuration or dtype performs no work, as in the reference
  // (movement.cu:264-266); the MI355X tile does not depend on the config.
  if (!t4a::transpose_config_valid(config)) return;
  __shared__ alignas(16) unsigned char lds[t4a::kTransposeLdsBytes];
  switch (t4a::dtype_size(dtype)) {
    case 1:
      t4a::transpose_dispatch<uint8_t, 0>(dst, src, src_offset, batch_stride, dst_fast_extent,
                                       src_fast_extent, lds);
      break;
    case 4:
      t4a::transpose_dispatch<uint32_t, 0>(dst, src, src_offset, batch_stride, dst_fast_extent,
                                        src_fast_extent, lds);
      break;
    case 8:
      t4a::transpose_dispatch<unsigned long long, 0>(dst, src, src_offset, batch_stride,
                                                  dst_fast_extent, src_fast_extent, lds);
      break;
    case 16:
      t4a::transpose_dispatch<t4a::Elem16, 0>(dst, src, src_offset, batch_stride, dst_fast_extent,
                                           src_fast_extent, lds);
      break;
    default:
      break;
  }
}

extern "C" __global__ void __launch_bounds__(256)
    t4a_cuda_copy_exact(void* dst, const void* src, int dtype, long long len) {
  switch (t4a::dtype_size(dtype)) {
    case 1: t4a::copy_body<uint8_t, 0>(dst, src, len, gridDim.x); break;
    case 4: t4a::copy_body<uint32_t, 0>(dst, src, len, gridDim.x); break;
    case 8: t4a::copy_body<unsigned long long, 0>(dst, src, len, gridDim.x); break;
    case 16: t4a::copy_body<t4a::Elem16, 0>(dst, src, len, gridDim.x); break;
    default: break;
  }
}

extern "C" __global__ void __launch_bounds__(256)
    t4a_cuda_materialize_strided(void* dst, const void* src, int dtype,
                                 t4a_cuda_layout src_layout, long long len) {
  t4a::move_entry(dst, src, dtype, src_layout, nullptr, 0, len);
}

extern "C" __global__ void __launch_bounds__(256)
    t4a_cuda_strided_to_strided(void* dst, const void* src, int dtype,
                                t4a_cuda_layout src_layout, t4a_cuda_layout dst_layout,
                                long long len) {
  // Both layouts share the source's extents (reference movement.cu:139-141).
  t4a::move_entry(dst, src, dtype, src_layout, dst_layout.strides, dst_layout.offset, len);
}

extern "C" __global__ void __launch_bounds__(256)
    t4a_cuda_materialize_strided_any(void* dst, const void* src, int dtype,
                                     t4a_cuda_layout_any src_layout, long long len) {
  t4a::move_entry_any(dst, src, dtype, src_layout, nullptr, len);
}

extern "C" __global__ void __launch_bounds__(256)
    t4a_cuda_strided_to_strided_any(void* dst, const void* src, int dtype,
                                    t4a_cuda_layout_any src_layout,
                                    t4a_cuda_layout_any dst_layout, long long len) {
  t4a::move_entry_any(dst, src, dtype, src_layout, &dst_layout, len);
}

// ---- the rest of the reference movement entries (movement.cu:514-551, 612-685) ----------

extern "C" __global__ void __launch_bounds__(256)
    t4a_cuda_fill_zero(void* out, int dtype, long long len) {
  switch (t4a::dtype_size(dtype)) {
    case 1: t4a::fill_body<uint8_t, 0>(out, len, gridDim.x); break;
    case 4: t4a::fill_body<uint32_t, 0>(out, len, gridDim.x); break;
    case 8: t4a::fill_body<unsigned long long, 0>(out, len, gridDim.x); break;
    case 16: t4a::fill_body<t4a::Elem16, 0>(out, len, gridDim.x); break;
    default: break;
  }
}

extern "C" __global__ void __launch_bounds__(256)
    t4a_cuda_fill_zero_view(void* out, int dtype, t4a_cuda_layout layout, long long len) {
  t4a::fill_view_entry(out, dtype, layout.rank <= t4a::kMaxDims ? layout.rank : -1,
                       layout.offset, layout.extents, layout.strides, len);
}

extern "C" __global__ void __launch_bounds__(256)
    t4a_cuda_fill_zero_view_any(void* out, int dtype, t4a_cuda_layout_any layout,
                                long long len) {
  t4a::fill_view_entry(out, dtype, layout.rank, layout.offset, layout.extents, layout.strides,
                       len);
}

// contiguous_to_view: dst[decode(f, dst_layout)] = src[f] (reference
// movement.cu:112-125): a move from the compact layout over the view's extents.
extern "C" __global__ void __launch_bounds__(256)
    t4a_cuda_contiguous_to_view(void* dst, const void* src, int dtype,
                                t4a_cuda_layout dst_layout, long long len) {
  const bool ok = dst_layout.rank >= 0 && dst_layout.rank <= t4a::kMaxDims;
  t4a::move_entry_by(dst, src, dtype, ok, dst_layout.rank, dst_layout.extents,
                     t4a::strides_of(nullptr, dst_layout.extents), 0,
                     t4a::strides_of(dst_layout.strides, dst_layout.extents), dst_layout.offset,
                     len);
}

extern "C" __global__ void __launch_bounds__(256)
    t4a_cuda_contiguous_to_view_any(void* dst, const void* src, int dtype,
                                    t4a_cuda_layout_any dst_layout, long long len) {
  t4a::move_entry_by(dst, src, dtype, true, dst_layout.rank, dst_layout.extents,
                     t4a::strides_of(nullptr, dst_layout.extents), 0,
                     t4a::strides_of(dst_layout.strides, dst_layout.extents), dst_layout.offset,
                     len);
}

// broadcast_in_dim: out[f] = in[sum over input axes i of coordinate(f, dims[i])
// * in.strides[i], coordinate 0 where the input extent is one] into a compact
// destination (reference movement.cu:409-434): a move whose source has the
// destination's extents and stride 0 on broadcast axes.
extern "C" __global__ void __launch_bounds__(256)
    t4a_cuda_broadcast_in_dim(void* out, const void* in, int dtype, t4a_cuda_layout out_layout,
                              t4a_cuda_layout in_layout, t4a_cuda_axis_values dims,
                              long long out_len) {
  const bool ok = out_layout.rank >= 0 && out_layout.rank <= t4a::kMaxDims && dims.rank >= 0 &&
                  dims.rank <= t4a::kMaxDims;
  t4a::move_entry_by(out, in, dtype, ok, out_layout.rank, out_layout.extents,
                     t4a::BroadcastStrides{dims.values, dims.rank, in_layout.extents,
                                           in_layout.strides},
                     in_layout.offset, t4a::strides_of(nullptr, out_layout.extents), 0, out_len);
}

extern "C" __global__ void __launch_bounds__(256)
    t4a_cuda_broadcast_in_dim_any(void* out, const void* in, int dtype,
                                  t4a_cuda_layout_any out_layout, t4a_cuda_layout_any in_layout,
                                  t4a_cuda_axis_values_any dims, long long out_len) {
  t4a::move_entry_by(out, in, dtype, dims.rank >= 0, out_layout.rank, out_layout.extents,
                     t4a::BroadcastStrides{dims.values, dims.rank, in_layout.extents,
                                           in_layout.strides},
                     in_layout.offset, t4a::strides_of(nullptr, out_layout.extents), 0, out_len);
}

// concatenate_copy: out[decode(f shifted by axis_offset along axis, out)] =
// in[f] for the compact input (reference movement.cu:436-465): a move from the
// input into the destination's strides from the shifted origin.
extern "C" __global__ void __launch_bounds__(256)
    t4a_cuda_concatenate_copy(void* out, const void* in, int dtype, t4a_cuda_layout out_layout,
                              t4a_cuda_layout in_layout, int axis, long long axis_offset,
                              long long in_len) {
  const bool ok = in_layout.rank >= 0 && in_layout.rank <= t4a::kMaxDims &&
                  out_layout.rank == in_layout.rank && axis >= 0 && axis < in_layout.rank;
  const long long origin = ok ? out_layout.offset + axis_offset * out_layout.strides[axis] : 0;
  t4a::move_entry_by(out, in, dtype, ok, in_layout.rank, in_layout.extents,
                     t4a::strides_of(nullptr, in_layout.extents), 0,
                     t4a::strides_of(out_layout.strides, in_layout.extents), origin, in_len);
}

extern "C" __global__ void __launch_bounds__(256)
    t4a_cuda_concatenate_copy_any(void* out, const void* in, int dtype,
                                  t4a_cuda_layout_any out_layout, t4a_cuda_layout_any in_layout,
                                  int axis, long long axis_offset, long long in_len) {
  const bool ok = out_layout.rank == in_layout.rank && axis >= 0 && axis < in_layout.rank;
  __shared__ long long origin;
  if (threadIdx.x == 0)
    origin = ok ? out_layout.offset + axis_offset * out_layout.strides[axis] : 0;
  __syncthreads();
  t4a::move_entry_by(out, in, dtype, ok, in_layout.rank, in_layout.extents,
                     t4a::strides_of(nullptr, in_layout.extents), 0,
                     t4a::strides_of(out_layout.strides, in_layout.extents), origin, in_len);
}

// ---- launchers -----------------------------------------------------------------------

namespace {
thread_local int last_launch_error = 0;
std::atomic<unsigned long long> launch_count{0};
}  // namespace

namespace t4a {
// Called once right after every kernel launch of every t4a_hip_* launcher.
int status_of_last_launch() {
  launch_count.fetch_add(1, std::memory_order_relaxed);
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return T4A_OK;
  last_launch_error = static_cast<int>(e);
  return T4A_HIP_ERR_LAUNCH;
}

int status_of_hip(int error) {
  if (error == static_cast<int>(hipSuccess)) return T4A_OK;
  last_launch_error = error;
  return T4A_HIP_ERR_LAUNCH;
}
}  // namespace t4a

extern "C" int t4a_hip_last_error(void) { return last_launch_error; }

extern "C" unsigned long long t4a_hip_launch_count(void) {
  return launch_count.load(std::memory_order_relaxed);
}

namespace {
using t4a::status_of_last_launch;

bool launch_empty(const t4a_launch* l) {
  return l->grid[0] == 0 || l->grid[1] == 0 || l->grid[2] == 0;
}

// A block of exactly `threads` threads along x: the block-size-specialised
// kernels number their threads by threadIdx.x alone (any other block shape
// takes the kernels that read blockDim).
bool one_dim(const dim3& block, int threads) {
  return block.x == static_cast<unsigned>(threads) && block.y == 1 && block.z == 1;
}


template <typename Fn>
int with_payload(int dtype, Fn&& fn) {
  switch (t4a::dtype_size(dtype)) {
    case 1: return fn(static_cast<uint8_t*>(nullptr));
    case 4: return fn(static_cast<uint32_t*>(nullptr));
    case 8: return fn(static_cast<unsigned long long*>(nullptr));
    case 16: return fn(static_cast<t4a::Elem16*>(nullptr));
    default: return T4A_OK;  // unknown tag: no work, as the reference entry
  }
}

bool config_valid(const t4a_cuda_transpose_config& c) {
  t4a_cuda_transpose_config checked;
  return t4a_transpose_config_new(c.tile, c.block_rows, c.padding, c.vector_width, &checked) ==
         T4A_OK;
}

// Blocks of Kernel (kBlock threads, no dynamic LDS) that the current device
// holds at once -- its occupancy per CU times the CU count -- queried once
// per device; kTileWalkBlocks if the runtime cannot say.
template <auto Kernel>
unsigned int resident_blocks() {
  static std::atomic<unsigned int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return t4a::kTileWalkBlocks;
  unsigned int v = cache[dev].load(std::memory_order_relaxed);
  if (v != 0) return v;
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, Kernel, t4a::kBlock, 0) !=
          hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      per_cu <= 0 || cus <= 0)
    return t4a::kTileWalkBlocks;
  v = static_cast<unsigned int>(per_cu) * static_cast<unsigned int>(cus);
  cache[dev].store(v, std::memory_order_relaxed);
  return v;
}

// The tile walk's own grid, whatever the caller's geometry (one block per
// tile) was: as many blocks as the device holds at once (a larger grid would
// leave its last blocks a whole walk to do after the others finish), at most
// one per tile.
template <auto Kernel, typename TP>
void launch_tile_walk(unsigned int tiles, hipStream_t s, void* dst, const void* src,
                      const TP& tp) {
  const unsigned int resident = resident_blocks<Kernel>();
  hipLaunchKernelGGL(Kernel, dim3(tiles < resident ? tiles : resident), dim3(t4a::kBlock), 0, s,
                     dst, src, tp, tiles);
}

// A long-and-short LA x LB tile: compact narrow plans only
// (t4a::tile_walk_applies has checked the form), one block per tile (the walk
// then moves one tile a block). On six such moves (2^25 elements of 4, 8 and
// 16 bytes, a 16-element run on either side) that measured 8-12 % faster than
// the resident grid; the balanced tiles keep the resident grid,
// which C5's permute needs (97 us against 107 with a block per tile), although
// other balanced moves ran 0-13 % faster with a block per tile.
template <typename P, int VL, int VS, int LA, int LB>
void launch_walk_compact(unsigned int tiles, hipStream_t s, void* dst, const void* src,
                         const t4a::TilePlan& tp) {
  hipLaunchKernelGGL(
      (t4a::move_tile_walk_kernel<P, VL, VS, LA, LB, t4a::TilePlanCompact, true>), dim3(tiles),
      dim3(t4a::kBlock), 0, s, dst, src, t4a::compact_tile_plan(tp), tiles);
}

// The walk kernel of the plan's tile shape (la x lb, one of
// t4a::tile_once_shape's) and vector widths.
template <typename P, int VL, int VS>
void launch_tile_shape(long long la, long long lb, unsigned int tiles, hipStream_t s, void* dst,
                       const void* src, const t4a::TilePlan& tp) {
  constexpr int LA = sizeof(P) >= 16 ? 32 : 64;
  constexpr int LB = sizeof(P) >= 8 ? 32 : 64;
  if (la == LA && lb == LB) {
    if (tp.ncoord <= t4a::kCompactCoords &&
        t4a::tile_offsets_narrow(tp, LA, LB, static_cast<int>(sizeof(P))))
      launch_tile_walk<t4a::move_tile_walk_kernel<P, VL, VS, LA, LB, t4a::TilePlanCompact, true>>(
          tiles, s, dst, src, t4a::compact_tile_plan(tp));
    else
      launch_tile_walk<t4a::move_tile_walk_kernel<P, VL, VS, LA, LB, t4a::TilePlan, false>>(
          tiles, s, dst, src, tp);
    return;
  }
  if constexpr (sizeof(P) == 4) {
    if (la == 128 && lb == 32) return launch_walk_compact<P, VL, VS, 128, 32>(tiles, s, dst, src, tp);
    if (la == 128 && lb == 16) return launch_walk_compact<P, VL, VS, 128, 16>(tiles, s, dst, src, tp);
    if (la == 32 && lb == 128) return launch_walk_compact<P, VL, VS, 32, 128>(tiles, s, dst, src, tp);
    if (la == 16 && lb == 128) return launch_walk_compact<P, VL, VS, 16, 128>(tiles, s, dst, src, tp);
  } else if constexpr (sizeof(P) == 8) {
    if (la == 128 && lb == 16) return launch_walk_compact<P, VL, VS, 128, 16>(tiles, s, dst, src, tp);
    if (la == 16 && lb == 128) return launch_walk_compact<P, VL, VS, 16, 128>(tiles, s, dst, src, tp);
    if (la == 32 && lb == 64) return launch_walk_compact<P, VL, VS, 32, 64>(tiles, s, dst, src, tp);
  } else if constexpr (sizeof(P) == 16) {
    if (la == 64 && lb == 16) return launch_walk_compact<P, VL, VS, 64, 16>(tiles, s, dst, src, tp);
    if (la == 16 && lb == 64) return launch_walk_compact<P, VL, VS, 16, 64>(tiles, s, dst, src, tp);
  }
}

// The walk kernels by vector widths.
template <typename P, int V>
void launch_tile_once(bool vl, bool vs, long long la, long long lb, unsigned int tiles,
                      hipStream_t s, void* dst, const void* src, const t4a::TilePlan& tp) {
  if constexpr (V > 1) {
    if (vl && vs) return launch_tile_shape<P, V, V>(la, lb, tiles, s, dst, src, tp);
    if (vl) return launch_tile_shape<P, V, 1>(la, lb, tiles, s, dst, src, tp);
    if (vs) return launch_tile_shape<P, 1, V>(la, lb, tiles, s, dst, src, tp);
  }
  launch_tile_shape<P, 1, 1>(la, lb, tiles, s, dst, src, tp);
}

// A compact 2-D transpose found in a movement plan, on the tiled transpose's
// kernel: 512-thread blocks, one per tile, in the ordered (diagonal) walk.
template <typename P>
int launch_transpose_route(void* dst, const void* src, const t4a::TransposeRoute& r,
                           hipStream_t s) {
  constexpr long long TM = t4a::TransposeShape<P>::TM;
  constexpr long long TN = t4a::TransposeShape<P>::TN;
  const long long tiles_m = (r.m + TM - 1) / TM;
  const long long tiles_n = (r.n + TN - 1) / TN;
  t4a::TileOrder order{};
  order.tiles_m = t4a::fast_div(static_cast<unsigned int>(tiles_m));
  order.tiles_n = t4a::fast_div(static_cast<unsigned int>(tiles_n));
  order.per_batch = static_cast<unsigned int>(tiles_m * tiles_n);
  order.blocks = order.per_batch;
  P* d = static_cast<P*>(dst) + r.dst_offset;
  hipLaunchKernelGGL((t4a::transpose_kernel<P, t4a::kTransposeBlock, true>),
                     dim3(order.per_batch), dim3(t4a::kTransposeBlock), 0, s, d, src, r.src_offset,
                     r.m * r.n, r.m, r.n, order);
  return status_of_last_launch();
}

int launch_move(void* dst, const void* src, const t4a::MovePlan& plan,
                const t4a_launch* launch, void* stream, int dtype) {
  const dim3 grid(launch->grid[0], launch->grid[1], launch->grid[2]);
  const dim3 block(launch->block[0], launch->block[1], launch->block[2]);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  return with_payload(dtype, [&](auto* tag) {
    using P = std::remove_pointer_t<decltype(tag)>;
    const bool flat_grid = block.x == static_cast<unsigned>(t4a::kBlock) && block.y == 1 &&
                           block.z == 1 && grid.y == 1 && grid.z == 1;
    if (flat_grid && t4a::linear_route(plan)) {
      hipLaunchKernelGGL((t4a::copy_kernel<P, t4a::kBlock>), grid, block, 0, s,
                         static_cast<P*>(dst) + plan.dst_offset,
                         static_cast<const P*>(src) + plan.src_offset, plan.len, grid.x);
      return status_of_last_launch();
    }
    t4a::RowPlan rp;
    if (plan.mode == t4a::kMoveContig && block.x == static_cast<unsigned>(t4a::kBlock) &&
        block.y == 1 && block.z == 1 && grid.y == 1 && grid.z == 1 && grid.x <= (1u << 23) &&
        t4a::row_plan(&rp, plan, static_cast<int>(sizeof(P)),
                      ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) &
                       15) == 0)) {
      constexpr int V = sizeof(P) == 1 ? 16 : sizeof(P) == 4 ? 4 : sizeof(P) == 8 ? 2 : 1;
      const bool vec = V > 1 && plan.row_len == static_cast<long long>(rp.vpr) * V;
      auto go = [&](auto v_tag, auto ntl_tag) {
        constexpr int VV = decltype(v_tag)::value;
        constexpr bool NTL = decltype(ntl_tag)::value;
        switch (rp.n) {
          case 0:
            hipLaunchKernelGGL((t4a::move_rows_kernel<P, VV, NTL, 0>), grid, block, 0, s, dst,
                               src, rp, grid.x);
            break;
          case 1:
            hipLaunchKernelGGL((t4a::move_rows_kernel<P, VV, NTL, 1>), grid, block, 0, s, dst,
                               src, rp, grid.x);
            break;
          case 2:
            hipLaunchKernelGGL((t4a::move_rows_kernel<P, VV, NTL, 2>), grid, block, 0, s, dst,
                               src, rp, grid.x);
            break;
          default:
            hipLaunchKernelGGL((t4a::move_rows_kernel<P, VV, NTL, -1>), grid, block, 0, s, dst,
                               src, rp, grid.x);
            break;
        }
      };
      using Vt = std::integral_constant<int, V>;
      using V1 = std::integral_constant<int, 1>;
      using Nt = std::true_type;
      using Nf = std::false_type;
      if (vec && rp.reread) go(Vt{}, Nf{});
      else if (vec) go(Vt{}, Nt{});
      else if (rp.reread) go(V1{}, Nf{});
      else go(V1{}, Nt{});
      return status_of_last_launch();
    }
    if (plan.mode != t4a::kMoveTiled) {
      if (one_dim(block, t4a::kBlock))
        hipLaunchKernelGGL((t4a::move_flat_kernel<P, t4a::kBlock>), grid, block, 0, s, dst, src,
                           plan);
      else
        hipLaunchKernelGGL((t4a::move_flat_kernel<P, 0>), grid, block, 0, s, dst, src, plan);
      return status_of_last_launch();
    }
    // A planned tiled geometry whose plan is one compact 2-D transpose takes
    // the transpose kernel, with that kernel's own grid.
    t4a::TransposeRoute route;
    if (block.x == static_cast<unsigned>(t4a::kBlock) && block.y == 1 && block.z == 1 &&
        grid.y == 1 && grid.z == 1 && t4a::transpose_route(plan, &route))
      return launch_transpose_route<P>(dst, src, route, s);
    constexpr int V = t4a::tile_vector<P>();
    bool vl, vs;
    t4a::tile_vectorizable(plan, V, dst, src, &vl, &vs);
    if constexpr (sizeof(P) >= 4) {
      t4a::TilePlan tp;
      if (block.x == static_cast<unsigned>(t4a::kBlock) && block.y == 1 && block.z == 1 &&
          grid.y == 1 && grid.z == 1 && t4a::tile_plan(&tp, plan, static_cast<int>(sizeof(P))) &&
          t4a::tile_walk_applies(plan, tp, static_cast<int>(sizeof(P)))) {
        launch_tile_once<P, V>(vl, vs, plan.la, plan.lb, static_cast<unsigned int>(plan.tiles), s,
                               dst, src, tp);
        return status_of_last_launch();
      }
    }
    if (vl && vs) {
      hipLaunchKernelGGL((t4a::move_tiled_kernel<P, V, V>), grid, block, 0, s, dst, src, plan);
    } else if (vl) {
      hipLaunchKernelGGL((t4a::move_tiled_kernel<P, V, 1>), grid, block, 0, s, dst, src, plan);
    } else if (vs) {
      hipLaunchKernelGGL((t4a::move_tiled_kernel<P, 1, V>), grid, block, 0, s, dst, src, plan);
    } else {
      hipLaunchKernelGGL((t4a::move_tiled_kernel<P, 1, 1>), grid, block, 0, s, dst, src, plan);
    }
    return status_of_last_launch();
  });
}

}  // namespace

extern "C" int t4a_hip_tiled_transpose(void* dst, const void* src, int dtype,
                                       long long src_offset, long long batch_stride,
                                       long long dst_fast_extent, long long src_fast_extent,
                                       t4a_cuda_transpose_config config,
                                       const t4a_launch* launch, void* stream) {
  if (launch == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (launch_empty(launch)) return T4A_OK;
  if (dst == nullptr || src == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  // An unsupported configuration performs no work (reference movement.cu:264-266).
  if (!config_valid(config)) return T4A_OK;
  // The batch index is the grid's z coordinate, as in the reference launch.
  const dim3 grid(launch->grid[0], launch->grid[1], launch->grid[2]);
  const dim3 block(launch->block[0], launch->block[1], launch->block[2]);
  return with_payload(dtype, [&](auto* tag) {
    using P = std::remove_pointer_t<decltype(tag)>;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    // The planned geometry (one 1-D grid per matrix, 512 threads) takes the
    // ordered kernel when one matrix has fewer than 2^30 tiles.
    constexpr long long TM = t4a::TransposeShape<P>::TM;
    constexpr long long TN = t4a::TransposeShape<P>::TN;
    const long long tiles_m = (dst_fast_extent + TM - 1) / TM;
    const long long tiles_n = (src_fast_extent + TN - 1) / TN;
    t4a::TileOrder order{};
    const bool planned = one_dim(block, t4a::kTransposeBlock);
    if (planned && grid.y == 1 && tiles_m > 0 && tiles_n > 0 &&
        tiles_m * tiles_n < (1ll << 30)) {
      order.tiles_m = t4a::fast_div(static_cast<unsigned int>(tiles_m));
      order.tiles_n = t4a::fast_div(static_cast<unsigned int>(tiles_n));
      order.per_batch = static_cast<unsigned int>(tiles_m * tiles_n);
      order.blocks = grid.x;
      hipLaunchKernelGGL((t4a::transpose_kernel<P, t4a::kTransposeBlock, true>), grid, block, 0,
                         s, dst, src, src_offset, batch_stride, dst_fast_extent, src_fast_extent,
                         order);
    } else if (planned) {
      hipLaunchKernelGGL((t4a::transpose_kernel<P, t4a::kTransposeBlock, false>), grid, block, 0,
                         s, dst, src, src_offset, batch_stride, dst_fast_extent, src_fast_extent,
                         order);
    } else {
      hipLaunchKernelGGL((t4a::transpose_kernel<P, 0, false>), grid, block, 0, s, dst, src,
                         src_offset, batch_stride, dst_fast_extent, src_fast_extent, order);
    }
    return status_of_last_launch();
  });
}

extern "C" int t4a_hip_copy_exact(void* dst, const void* src, int dtype, long long len,
                                  const t4a_launch* launch, void* stream) {
  if (launch == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (launch_empty(launch)) return T4A_OK;
  if (dst == nullptr || src == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  const dim3 grid(launch->grid[0], launch->grid[1], launch->grid[2]);
  const dim3 block(launch->block[0], launch->block[1], launch->block[2]);
  return with_payload(dtype, [&](auto* tag) {
    using P = std::remove_pointer_t<decltype(tag)>;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (one_dim(block, t4a::kBlock))
      hipLaunchKernelGGL((t4a::copy_kernel<P, t4a::kBlock>), grid, block, 0, s, dst, src, len,
                         grid.x);
    else
      hipLaunchKernelGGL((t4a::copy_kernel<P, 0>), grid, block, 0, s, dst, src, len, grid.x);
    return status_of_last_launch();
  });
}

extern "C" int t4a_hip_materialize_strided(void* dst, const void* src, int dtype,
                                           const t4a_cuda_layout* src_layout, long long len,
                                           const t4a_launch* launch, void* stream) {
  if (launch == nullptr || src_layout == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (launch_empty(launch)) return T4A_OK;
  if (dst == nullptr || src == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  t4a::MovePlan plan;
  t4a::move_plan(&plan, *src_layout, nullptr, 0, len, t4a::dtype_size(dtype));
  return launch_move(dst, src, plan, launch, stream, dtype);
}

extern "C" int t4a_hip_strided_to_strided(void* dst, const void* src, int dtype,
                                          const t4a_cuda_layout* src_layout,
                                          const t4a_cuda_layout* dst_layout, long long len,
                                          const t4a_launch* launch, void* stream) {
  if (launch == nullptr || src_layout == nullptr || dst_layout == nullptr)
    return T4A_HIP_ERR_NULL_ARGUMENT;
  if (launch_empty(launch)) return T4A_OK;
  if (dst == nullptr || src == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  t4a::MovePlan plan;
  t4a::move_plan(&plan, *src_layout, dst_layout->strides, dst_layout->offset, len,
                 t4a::dtype_size(dtype));
  return launch_move(dst, src, plan, launch, stream, dtype);
}

// The general-rank twins on the caller's stream with a planned geometry (any
// t4a_plan_*_any geometry: the twins stride over their work).
extern "C" int t4a_hip_materialize_strided_any(void* dst, const void* src, int dtype,
                                               const t4a_cuda_layout_any* src_layout,
                                               long long len, const t4a_launch* launch,
                                               void* stream) {
  if (launch == nullptr || src_layout == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (launch_empty(launch)) return T4A_OK;
  if (dst == nullptr || src == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  const dim3 grid(launch->grid[0], launch->grid[1], launch->grid[2]);
  const dim3 block(launch->block[0], launch->block[1], launch->block[2]);
  hipLaunchKernelGGL(t4a_cuda_materialize_strided_any, grid, block, 0,
                     static_cast<hipStream_t>(stream), dst, src, dtype, *src_layout, len);
  return status_of_last_launch();
}

extern "C" int t4a_hip_strided_to_strided_any(void* dst, const void* src, int dtype,
                                              const t4a_cuda_layout_any* src_layout,
                                              const t4a_cuda_layout_any* dst_layout,
                                              long long len, const t4a_launch* launch,
                                              void* stream) {
  if (launch == nullptr || src_layout == nullptr || dst_layout == nullptr)
    return T4A_HIP_ERR_NULL_ARGUMENT;
  if (launch_empty(launch)) return T4A_OK;
  if (dst == nullptr || src == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  const dim3 grid(launch->grid[0], launch->grid[1], launch->grid[2]);
  const dim3 block(launch->block[0], launch->block[1], launch->block[2]);
  hipLaunchKernelGGL(t4a_cuda_strided_to_strided_any, grid, block, 0,
                     static_cast<hipStream_t>(stream), dst, src, dtype, *src_layout, *dst_layout,
                     len);
  return status_of_last_launch();
}

// ---- the rest of the movement entries ---------------------------------------------------

extern "C" int t4a_hip_fill_zero(void* out, int dtype, long long len, const t4a_launch* launch,
                                 void* stream) {
  if (launch == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (launch_empty(launch)) return T4A_OK;
  if (out == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  const dim3 grid(launch->grid[0], launch->grid[1], launch->grid[2]);
  const dim3 block(launch->block[0], launch->block[1], launch->block[2]);
  return with_payload(dtype, [&](auto* tag) {
    using P = std::remove_pointer_t<decltype(tag)>;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (one_dim(block, t4a::kBlock))
      hipLaunchKernelGGL((t4a::fill_kernel<P, t4a::kBlock>), grid, block, 0, s, out, len,
                         grid.x);
    else
      hipLaunchKernelGGL((t4a::fill_kernel<P, 0>), grid, block, 0, s, out, len, grid.x);
    return status_of_last_launch();
  });
}

extern "C" int t4a_hip_fill_zero_view(void* out, int dtype, const t4a_cuda_layout* layout,
                                      long long len, const t4a_launch* launch, void* stream) {
  if (launch == nullptr || layout == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (launch_empty(launch)) return T4A_OK;
  if (out == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  long long fe[t4a::kMaxFusedDims], fs[t4a::kMaxFusedDims], fd[t4a::kMaxFusedDims];
  const int rank = layout->rank < 0 ? 0 : layout->rank > t4a::kMaxDims ? t4a::kMaxDims
                                                                         : layout->rank;
  const int n = t4a::fuse_move(rank, layout->extents, layout->strides, layout->strides, fe, fs,
                               fd, t4a::kMaxFusedDims);
  t4a::FillPlan fp;
  if (!t4a::fill_plan(&fp, n, fe, fs, layout->offset, len)) return T4A_OK;
  const dim3 grid(launch->grid[0], launch->grid[1], launch->grid[2]);
  const dim3 block(launch->block[0], launch->block[1], launch->block[2]);
  return with_payload(dtype, [&](auto* tag) {
    using P = std::remove_pointer_t<decltype(tag)>;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    constexpr int V = t4a::tile_vector<P>();
    const bool vec =
        V > 1 && (reinterpret_cast<uintptr_t>(out) & 15) == 0 && t4a::fill_vectorizable(fp, V);
    const bool planned = one_dim(block, t4a::kBlock);
    if (vec && planned)
      hipLaunchKernelGGL((t4a::fill_view_kernel<P, V, t4a::kBlock>), grid, block, 0, s, out, fp,
                         grid.x);
    else if (vec)
      hipLaunchKernelGGL((t4a::fill_view_kernel<P, V, 0>), grid, block, 0, s, out, fp, grid.x);
    else if (planned)
      hipLaunchKernelGGL((t4a::fill_view_kernel<P, 1, t4a::kBlock>), grid, block, 0, s, out, fp,
                         grid.x);
    else
      hipLaunchKernelGGL((t4a::fill_view_kernel<P, 1, 0>), grid, block, 0, s, out, fp, grid.x);
    return status_of_last_launch();
  });
}

// The copy-style entries: the same move machinery as strided_to_strided over
// the geometry the entry implies (the planner derives the same plan).
namespace {

template <typename SrcStride, typename DstStride>
int launch_derived(void* dst, const void* src, int dtype, int rank, const long long* ext,
                   SrcStride src_st, long long src_offset, DstStride dst_st, long long dst_offset,
                   long long len, const t4a_launch* launch, void* stream) {
  if (rank < 0 || rank > t4a::kMaxDims) return T4A_OK;
  t4a::MovePlan plan;
  if (!t4a::move_plan_by(&plan, rank, ext, src_st, src_offset, dst_st, dst_offset, len,
                         t4a::dtype_size(dtype)))
    return T4A_OK;
  return launch_move(dst, src, plan, launch, stream, dtype);
}

}  // namespace

extern "C" int t4a_hip_contiguous_to_view(void* dst, const void* src, int dtype,
                                          const t4a_cuda_layout* dst_layout, long long len,
                                          const t4a_launch* launch, void* stream) {
  if (launch == nullptr || dst_layout == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (launch_empty(launch)) return T4A_OK;
  if (dst == nullptr || src == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  return launch_derived(dst, src, dtype, dst_layout->rank, dst_layout->extents,
                        t4a::strides_of(nullptr, dst_layout->extents), 0,
                        t4a::strides_of(dst_layout->strides, dst_layout->extents),
                        dst_layout->offset, len, launch, stream);
}

extern "C" int t4a_hip_broadcast_in_dim(void* out, const void* in, int dtype,
                                        const t4a_cuda_layout* out_layout,
                                        const t4a_cuda_layout* in_layout,
                                        const t4a_cuda_axis_values* dims, long long out_len,
                                        const t4a_launch* launch, void* stream) {
  if (launch == nullptr || out_layout == nullptr || in_layout == nullptr || dims == nullptr)
    return T4A_HIP_ERR_NULL_ARGUMENT;
  if (launch_empty(launch)) return T4A_OK;
  if (out == nullptr || in == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (dims->rank < 0 || dims->rank > t4a::kMaxDims) return T4A_OK;
  return launch_derived(out, in, dtype, out_layout->rank, out_layout->extents,
                        t4a::BroadcastStrides{dims->values, dims->rank, in_layout->extents,
                                              in_layout->strides},
                        in_layout->offset, t4a::strides_of(nullptr, out_layout->extents), 0,
                        out_len, launch, stream);
}

extern "C" int t4a_hip_concatenate_copy(void* out, const void* in, int dtype,
                                        const t4a_cuda_layout* out_layout,
                                        const t4a_cuda_layout* in_layout, int axis,
                                        long long axis_offset, long long in_len,
                                        const t4a_launch* launch, void* stream) {
  if (launch == nullptr || out_layout == nullptr || in_layout == nullptr)
    return T4A_HIP_ERR_NULL_ARGUMENT;
  if (launch_empty(launch)) return T4A_OK;
  if (out == nullptr || in == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (in_layout->rank > t4a::kMaxDims || axis < 0 || axis >= in_layout->rank ||
      out_layout->rank != in_layout->rank)
    return T4A_OK;
  return launch_derived(out, in, dtype, in_layout->rank, in_layout->extents,
                        t4a::strides_of(nullptr, in_layout->extents), 0,
                        t4a::strides_of(out_layout->strides, in_layout->extents),
                        out_layout->offset + axis_offset * out_layout->strides[axis], in_len,
                        launch, stream);
}

// The general-rank twins of these entries: the kernels plan in LDS.
#define T4A_ANY_LAUNCH(kernel, ...)                                                        \
  do {                                                                                     \
    if (launch_empty(launch)) return T4A_OK;                                               \
    const dim3 grid(launch->grid[0], launch->grid[1], launch->grid[2]);                    \
    const dim3 block(launch->block[0], launch->block[1], launch->block[2]);                \
    hipLaunchKernelGGL(kernel, grid, block, 0, static_cast<hipStream_t>(stream), __VA_ARGS__); \
    return status_of_last_launch();                                                        \
  } while (0)

extern "C" int t4a_hip_fill_zero_view_any(void* out, int dtype,
                                          const t4a_cuda_layout_any* layout, long long len,
                                          const t4a_launch* launch, void* stream) {
  if (launch == nullptr || layout == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (!launch_empty(launch) && out == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  T4A_ANY_LAUNCH(t4a_cuda_fill_zero_view_any, out, dtype, *layout, len);
}

extern "C" int t4a_hip_contiguous_to_view_any(void* dst, const void* src, int dtype,
                                              const t4a_cuda_layout_any* dst_layout,
                                              long long len, const t4a_launch* launch,
                                              void* stream) {
  if (launch == nullptr || dst_layout == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  if (!launch_empty(launch) && (dst == nullptr || src == nullptr))
    return T4A_HIP_ERR_NULL_ARGUMENT;
  T4A_ANY_LAUNCH(t4a_cuda_contiguous_to_view_any, dst, src, dtype, *dst_layout, len);
}

extern "C" int t4a_hip_broadcast_in_dim_any(void* out, const void* in, int dtype,
                                            const t4a_cuda_layout_any* out_layout,
                                            const t4a_cuda_layout_any* in_layout,
                                            const t4a_cuda_axis_values_any* dims,
                                            long long out_len, const t4a_launch* launch,
                                            void* stream) {
  if (launch == nullptr || out_layout == nullptr || in_layout == nullptr || dims == nullptr)
    return T4A_HIP_ERR_NULL_ARGUMENT;
  if (!launch_empty(launch) && (out == nullptr || in == nullptr))
    return T4A_HIP_ERR_NULL_ARGUMENT;
  T4A_ANY_LAUNCH(t4a_cuda_broadcast_in_dim_any, out, in, dtype, *out_layout, *in_layout, *dims,
                 out_len);
}

extern "C" int t4a_hip_concatenate_copy_any(void* out, const void* in, int dtype,
                                            const t4a_cuda_layout_any* out_layout,
                                            const t4a_cuda_layout_any* in_layout, int axis,
                                            long long axis_offset, long long in_len,
                                            const t4a_launch* launch, void* stream) {
  if (launch == nullptr || out_layout == nullptr || in_layout == nullptr)
    return T4A_HIP_ERR_NULL_ARGUMENT;
  if (!launch_empty(launch) && (out == nullptr || in == nullptr))
    return T4A_HIP_ERR_NULL_ARGUMENT;
  T4A_ANY_LAUNCH(t4a_cuda_concatenate_copy_any, out, in, dtype, *out_layout, *in_layout, axis,
                 axis_offset, in_len);
}

#undef T4A_ANY_LAUNCH
