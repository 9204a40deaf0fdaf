// Backward of rows longer than 32 elements, from the forward's final hulls.
//
// Replaces the reference's long-row gradient (reference src/torchisotonic/csrc/grad.cuh:
// 165-195 tile summaries, 346-370 ATen tile scan, 200-290 fill), which reads starts, g and w
// twice and runs about fifteen ATen kernels in between. Here the forward's final hulls (in its
// workspace, or copied out of it by ti_keep) give every block's weight and fit; only the block
// sums of g are new, and they are differences of a prefix sum of g taken at the hull's vertices:
//
//   gsum_kernel    per tile (two to a workgroup, their loads in flight together): reads g
//                  once; the tile's total, and the prefix of g (within the tile, double-double)
//                  at each hull vertex inside it, by the vertex's rank (a tile inside one block,
//                  the common case, needs only its total);
//   gscan kernels  exclusive scans of the tile totals: within groups of 256 tiles, then over
//                  the groups of a row;
//   gfill_kernel   per tile: for each block overlapping the tile, G = difference of the row
//                  prefix of g at its two vertices, W and the fit from the forward's vertices
//                  (so the clamp mask is the forward's, bit for bit); then reads w (and y) once
//                  and writes gy = w * mask * G / W and gw = (y - fit) * mask * G / W.
// Rows of at most 2048 elements (one tile) take one kernel instead:
//
//   gpack_kernel   whole rows packed into a workgroup; a segmented scan of g over its elements
//                  (reset at each block start) leaves every block's sum at its last element,
//                  then as gfill_kernel, per block and per element.
// A row holding a NaN is one block (its fit is NaN), as in the reference's CPU path.
#include <type_traits>

#include "ti_common.h"
#include "ti_kernels.h"
#include "ti_tile.h"

namespace ti {

namespace {

constexpr int kScanTiles = 256;

struct GradPlan {
  int64_t tpr, ngroups, cap_final;
  size_t off_tg, off_lp, off_gt, off_gp, off_lv, bytes;
};

// kept_maxc > 0: the final hulls come from a kept state, at most that many vertices a row
GradPlan grad_plan(int64_t batch, int64_t n, bool weighted, bool lo, int64_t kept_maxc) {
  const LongPlan lp = long_plan(batch, n, weighted, lo);
  GradPlan g{};
  g.tpr = lp.tiles_per_row;
  g.ngroups = (g.tpr + kScanTiles - 1) / kScanTiles;
  // a row's slots (room for any final hull), or the kept hulls' largest
  g.cap_final = kept_maxc > 0 ? kept_maxc : lp.npr[0] * (lp.span0 + 1);
  size_t off = 0;
  g.off_tg = off;
  off += align256(static_cast<size_t>(batch * g.tpr) * 16);
  g.off_lp = off;
  off += align256(static_cast<size_t>(batch * g.tpr) * 16);
  g.off_gt = off;
  off += align256(static_cast<size_t>(batch * g.ngroups) * 16);
  g.off_gp = off;
  off += align256(static_cast<size_t>(batch * (g.ngroups + 1)) * 16);
  g.off_lv = off;
  off += align256(static_cast<size_t>(batch * g.cap_final) * 16);
  g.bytes = off;
  return g;
}

struct GradKArgs {
  const uint32_t* starts;
  const void* g;
  const void* w;
  const void* y;
  void* gy;
  void* gw;
  int64_t batch, n, tpr, ngroups, cap_final;
  unsigned flags;
  double lo, hi;
  NodeLevel hulls;       // the forward's final level
  const TileRec* tiles;  // the forward's per-tile records
  double* tg;            // [batch * tpr][2]: tile totals of g
  double* lp;            // [batch * tpr][2]: exclusive prefix within the tile's group
  double* gt;            // [batch * ngroups][2]: group totals
  double* gp;            // [batch * (ngroups + 1)][2]: exclusive prefix of groups, then total
  double* lv;            // [batch * cap_final][2]: prefix of g within its tile at each vertex
  RowMap map;            // ragged rows of one block: g, w, y, gy, gw in the packed layout
};


// Exclusive double-double scan over a 256-thread workgroup; returns the exclusive prefix and
// sets `total`.
__device__ DD block_scan_dd(DD v, DD* wave_tot, DD& total) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const DD inc = wave_incl_dd(v);
  const DD exc = wave_shr1_dd(inc);
  if (lane == kWave - 1) wave_tot[wave] = inc;
  __syncthreads();
  DD pre{0.0, 0.0};
  for (int w2 = 0; w2 < wave; ++w2) pre = dd_add(pre, wave_tot[w2]);
  total = DD{0.0, 0.0};
  for (int w2 = 0; w2 < kWaves256; ++w2) total = dd_add(total, wave_tot[w2]);
  __syncthreads();
  return dd_add(pre, exc);
}

__device__ __forceinline__ uint32_t tile_bits(const uint32_t* srow, int x, int E) {
  const uint32_t mask = E == 32 ? 0xFFFFFFFFu : ((1u << E) - 1u);
  return (srow[x >> 5] >> (x & 31)) & mask;
}

// A tile's total of g; for rows of one tile also the scans' results (no scan kernel runs then):
// the tile's prefix within its group and the group's within the row are 0, the row total is
// the tile's.
__device__ __forceinline__ void put_tile_total(const GradKArgs& a, int64_t gt, DD total) {
  a.tg[2 * gt] = total.hi;
  a.tg[2 * gt + 1] = total.lo;
  if (a.tpr == 1) {
    a.lp[2 * gt] = 0.0;
    a.lp[2 * gt + 1] = 0.0;
    a.gp[4 * gt] = 0.0;
    a.gp[4 * gt + 1] = 0.0;
    a.gp[4 * gt + 2] = total.hi;
    a.gp[4 * gt + 3] = total.lo;
  }
}

// Tiles per gsum workgroup: their loads are all in flight before the first tile is summed.
constexpr int kGsumTiles = 2;

// Over a 256-thread workgroup, one barrier: the exclusive scan of v (double-double) and of c
// (an int), and v's total. wave_tot and wave_cnt are this call's own (no later call in the
// kernel writes them, so no barrier follows).
// PR false (float32 g): v.hi alone, scanned in float64, the results' lo parts zero. A tile's
// 2048 sums then carry a relative error near 2^-42, far below float32's 2^-24 (the reference
// sums its tiles in float64 too, grad.cuh:187-190); the scans across a row's tiles stay
// double-double.
template <bool PR>
__device__ __forceinline__ DD block_scan2(DD v, int c, DD* wave_tot, int* wave_cnt, DD& total, int& cbefore) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  if constexpr (!PR) {
    const double inc = wave_incl_f64(v.hi);
    const int cinc = wave_incl_i32(c);
    const double exc = dpp_f64<0x138, 0xF>(inc);
    if (lane == kWave - 1) {
      wave_tot[wave] = DD{inc, 0.0};
      wave_cnt[wave] = cinc;
    }
    __syncthreads();
    double pre = 0.0, tot = 0.0;
    int cpre = 0;
#pragma unroll
    for (int w2 = 0; w2 < kWaves256; ++w2) {
      const double t = wave_tot[w2].hi;
      if (w2 < wave) {
        pre += t;
        cpre += wave_cnt[w2];
      }
      tot += t;
    }
    cbefore = cpre + cinc - c;
    total = DD{tot, 0.0};
    return DD{pre + exc, 0.0};
  }
  const DD inc = wave_incl_dd(v);
  const int cinc = wave_incl_i32(c);
  const DD exc = wave_shr1_dd(inc);
  if (lane == kWave - 1) {
    wave_tot[wave] = inc;
    wave_cnt[wave] = cinc;
  }
  __syncthreads();
  DD pre{0.0, 0.0};
  total = DD{0.0, 0.0};
  int cpre = 0;
#pragma unroll
  for (int w2 = 0; w2 < kWaves256; ++w2) {
    const DD t = wave_tot[w2];
    if (w2 < wave) {
      pre = dd_add(pre, t);
      cpre += wave_cnt[w2];
    }
    total = dd_add(total, t);
  }
  cbefore = cpre + cinc - c;
  return dd_add(pre, exc);
}

template <typename T, bool W, bool MAP = false>
__global__ __launch_bounds__(256) void gsum_kernel(GradKArgs a) {
  using C = TileCfg<W>;
  constexpr int E = C::kE;
  // float32 g: a thread's prefix over E values is kept in float64 (its error is far below the
  // data's); float64 g carries the rounding errors (double-double)
  constexpr bool PR = sizeof(T) == 8;
  __shared__ DD wtot[kGsumTiles][kWaves256];  // (per tile: no barrier between the tiles' scans)
  __shared__ int wcnt[kGsumTiles][kWaves256];
  const int tid = threadIdx.x;
  const int64_t ntiles = a.batch * a.tpr;
  const int64_t gt0 = static_cast<int64_t>(blockIdx.x) * kGsumTiles;
  const int t0 = tid * E;
  // every tile's loads first (a tile's own small reads would each cost a memory round trip):
  // g and the tile's record (the hull's ranks around it, the row's NaN flag and last vertex,
  // whether a vertex starts it)
  T gv[kGsumTiles][E];
  int rA[kGsumTiles], rB[kGsumTiles], badu[kGsumTiles], lastu[kGsumTiles], head[kGsumTiles];
  // each tile's row and place in it: one division, then steps (a 64-bit division by a runtime
  // value is a long scalar sequence)
  int64_t rowu[kGsumTiles], tileu[kGsumTiles];
  {
    int64_t row = gt0 / a.tpr, tile = gt0 - row * a.tpr;
#pragma unroll
    for (int u = 0; u < kGsumTiles; ++u) {
      rowu[u] = row;
      tileu[u] = tile;
      if (++tile == a.tpr && row + 1 < a.batch) {
        tile = 0;
        ++row;
      }
    }
  }
#pragma unroll
  for (int u = 0; u < kGsumTiles; ++u) {
    const int64_t gt = min(gt0 + u, ntiles - 1);
    const int64_t row = rowu[u];
    const int64_t tile = tileu[u];
    const int64_t first = tile * C::kN;
    const int len = static_cast<int>(min<int64_t>(C::kN, a.n - first));
    // (ragged rows: the row's own elements from its packed place, g = 0 for the pad's)
    int64_t rfirst = row * a.n, rlen = a.n;
    if constexpr (MAP) map_row(a.map, row, a.n, rfirst, rlen);
    const int lc = static_cast<int>(max<int64_t>(0, min<int64_t>(E, min<int64_t>(len, rlen - first) - t0)));
    load_elems_zero<T, E>(static_cast<const T*>(a.g) + rfirst + first + t0, lc, gv[u]);
    const TileRec rec = a.tiles[gt];
    rA[u] = rec.ra;
    rB[u] = rec.rb;
    badu[u] = rec.flags & kTileBad;
    lastu[u] = rec.last;
    head[u] = (rec.flags & kTileHead) ? 1 : 0;
  }
#pragma unroll
  for (int u = 0; u < kGsumTiles; ++u) {
    const int64_t gt = gt0 + u;
    if (gt >= ntiles) break;
    const int64_t row = rowu[u];
    const int64_t tile = tileu[u];
    const int64_t first = tile * C::kN;
    const int len = static_cast<int>(min<int64_t>(C::kN, a.n - first));
    const int ecount = max(0, min(E, len - t0));
    const int bad = badu[u];
    double* lv = a.lv + 2 * row * a.cap_final;
    // the thread's sum; its prefixes are formed again, in the same order, where a vertex needs
    // one (keeping them would hold E more float64 registers through the tile); elements past
    // the tile's or the row's end were loaded as zeros, which leave a sum as it is
    auto add = [&](DD& acc, int k) {
      if constexpr (PR) acc = dd_add(acc, static_cast<double>(gv[u][k]));
      else acc.hi += static_cast<double>(gv[u][k]);
    };
    DD acc{0.0, 0.0};
#pragma unroll
    for (int k = 0; k < E; ++k) add(acc, k);
    if (bad || rB[u] == rA[u] + 1) {
      // no vertex inside the tile (the common case on long rows): its total, a zero prefix for
      // a vertex at its first element, and on the row's last tile the row's end point
      int unused;
      DD total;
      block_scan2<PR>(acc, 0, wtot[u], wcnt[u], total, unused);
      if (tid == 0) {
        put_tile_total(a, gt, total);
        if (!bad) {
          if (head[u]) {  // vertex rA is the tile's first element
            lv[2 * rA[u]] = 0.0;
            lv[2 * rA[u] + 1] = 0.0;
          }
          if (tile == a.tpr - 1) {
            const int last = lastu[u];
            lv[2 * last] = total.hi;
            lv[2 * last + 1] = total.lo;
          }
        }
      }
      continue;
    }
    // the hull vertices inside the tile, by rank: rA, less one if rA is the tile's first element
    // (the prefix of g and the vertex ranks in one scan)
    const uint32_t* srow = a.starts + row * ((a.n + 31) / 32);
    uint32_t mybits = ecount > 0 ? tile_bits(srow, static_cast<int>(first + t0), E) : 0u;
    const int at_start = head[u];
    if (ecount > 0 && ecount < E) mybits &= (1u << ecount) - 1u;
    if (first + t0 == 0) mybits |= 1u;
    const int pc = __builtin_popcount(mybits);
    DD total;
    int before;
    const DD off = block_scan2<PR>(acc, pc, wtot[u], wcnt[u], total, before);
    if (tid == 0) put_tile_total(a, gt, total);
    int rank = rA[u] - at_start + before;
    DD run{0.0, 0.0};
#pragma unroll
    for (int k = 0; k < E; ++k) {
      if ((mybits >> k) & 1u) {
        ++rank;
        const DD p = PR ? dd_add(off, run) : DD{off.hi + run.hi, 0.0};
        lv[2 * rank] = p.hi;
        lv[2 * rank + 1] = p.lo;
      }
      add(run, k);
    }
    if (tile == a.tpr - 1 && tid == 0) {  // the row's end point: the last vertex
      const int last = lastu[u];
      lv[2 * last] = total.hi;
      lv[2 * last + 1] = total.lo;
    }
  }
}

// Exclusive scan of tile totals within groups of 256 tiles; group totals.
__global__ __launch_bounds__(256) void gscan_local_kernel(GradKArgs a) {
  __shared__ DD wtot[kWaves256];
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x / a.ngroups;
  const int64_t grp = blockIdx.x - row * a.ngroups;
  const int64_t tile = grp * kScanTiles + tid;
  DD v{0.0, 0.0};
  if (tile < a.tpr) v = DD{a.tg[2 * (row * a.tpr + tile)], a.tg[2 * (row * a.tpr + tile) + 1]};
  DD total;
  const DD ex = block_scan_dd(v, wtot, total);
  if (tile < a.tpr) {
    a.lp[2 * (row * a.tpr + tile)] = ex.hi;
    a.lp[2 * (row * a.tpr + tile) + 1] = ex.lo;
  }
  if (tid == 0) {
    a.gt[2 * blockIdx.x] = total.hi;
    a.gt[2 * blockIdx.x + 1] = total.lo;
    if (a.ngroups == 1) {  // (rows of one group: gscan_groups_kernel's results, which then does not run)
      a.gp[4 * row] = 0.0;
      a.gp[4 * row + 1] = 0.0;
      a.gp[4 * row + 2] = total.hi;
      a.gp[4 * row + 3] = total.lo;
    }
  }
}

// Exclusive scan of group totals per row (chunks of 256 groups with a carry); [ngroups] = total.
__global__ __launch_bounds__(256) void gscan_groups_kernel(GradKArgs a) {
  __shared__ DD wtot[kWaves256];
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  DD carry{0.0, 0.0};
  for (int64_t g0 = 0; g0 < a.ngroups; g0 += 256) {
    const int64_t gi = g0 + tid;
    DD v{0.0, 0.0};
    if (gi < a.ngroups) v = DD{a.gt[2 * (row * a.ngroups + gi)], a.gt[2 * (row * a.ngroups + gi) + 1]};
    DD total;
    const DD ex = dd_add(carry, block_scan_dd(v, wtot, total));
    if (gi < a.ngroups) {
      a.gp[2 * (row * (a.ngroups + 1) + gi)] = ex.hi;
      a.gp[2 * (row * (a.ngroups + 1) + gi) + 1] = ex.lo;
    }
    carry = dd_add(carry, total);
  }
  if (tid == 0) {
    a.gp[2 * (row * (a.ngroups + 1) + a.ngroups)] = carry.hi;
    a.gp[2 * (row * (a.ngroups + 1) + a.ngroups) + 1] = carry.lo;
  }
}

template <bool W>
__device__ __forceinline__ DD vertex_w(const NodeOut& f, int r) {
  if constexpr (W) return DD{f.whi[r], lo_at(f.wlo, r)};
  else return DD{static_cast<double>(f.idx[r]), 0.0};
}

template <typename T, bool W, bool MAP = false>
__global__ __launch_bounds__(256) void gfill_kernel(GradKArgs a) {
  using C = TileCfg<W>;
  constexpr int E = C::kE;
  constexpr int NT = C::kThreads;
  __shared__ double qv[C::kN + 2];
  __shared__ T mv[C::kN + 2];
  __shared__ int rank_scan[kWaves256];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int64_t row = blockIdx.x / a.tpr;
  const int64_t tile = blockIdx.x - row * a.tpr;
  const int64_t first = tile * C::kN;
  const int len = static_cast<int>(min<int64_t>(C::kN, a.n - first));
  const int t0 = tid * E;
  const int ecount = max(0, min(E, len - t0));
  const NodeOut fin = node_out(a.hulls, W, row);
  const TileRec rec = a.tiles[blockIdx.x];
  const bool bad = (rec.flags & kTileBad) != 0;
  const int count = rec.last + 1;
  const bool use_lo = a.flags & TI_CLIP_MIN, use_hi = a.flags & TI_CLIP_MAX;
  const T lo = static_cast<T>(a.lo), hi = static_cast<T>(a.hi);
  // the forward's hull is of sgn * y: its slopes are sgn * fit
  const double sgn = (a.flags & TI_INCREASING) ? 1.0 : -1.0;
  const double* lv = a.lv + 2 * row * a.cap_final;
  const double* gp = a.gp + 2 * row * (a.ngroups + 1);
  const double* lpr = a.lp + 2 * row * a.tpr;
  // the row prefix of g at vertex r
  auto pg = [&](int r) -> DD {
    const int x = fin.idx[r];
    const int64_t tl = min<int64_t>(x / C::kN, a.tpr - 1);
    const int64_t grp = tl / kScanTiles;
    DD p = dd_add(DD{gp[2 * grp], gp[2 * grp + 1]}, DD{lpr[2 * tl], lpr[2 * tl + 1]});
    return dd_add(p, DD{lv[2 * r], lv[2 * r + 1]});
  };
  const int rA = rec.ra, rB = rec.rb;
  if (bad) {  // one block over the whole row, fit NaN
    if (tid == 0) {
      const DD gtot{gp[2 * a.ngroups], gp[2 * a.ngroups + 1]};
      const double wsum = dd_diff(vertex_w<W>(fin, count - 1), vertex_w<W>(fin, 0));
      qv[0] = (use_lo || use_hi) ? 0.0 : (gtot.hi + gtot.lo) / wsum;
      mv[0] = quiet_nan<T>();
    }
  } else {
    for (int jb = rA + tid; jb < rB; jb += NT) {
      const DD ga = pg(jb), gb = pg(jb + 1);
      const double G = dd_diff(gb, ga);
      double dW, dS;
      dW = dd_diff(vertex_w<W>(fin, jb + 1), vertex_w<W>(fin, jb));
      dS = dd_diff(DD{fin.shi[jb + 1], lo_at(fin.slo, jb + 1)}, DD{fin.shi[jb], lo_at(fin.slo, jb)});
      const T mean = static_cast<T>(sgn * slope_div(dS, dW));
      double q = G / dW;
      if ((use_lo || use_hi) && !clip_passes(mean, use_lo, lo, use_hi, hi)) q = 0.0;
      qv[jb - rA] = q;
      mv[jb - rA] = mean;
    }
  }
  // the block of each element: vertex bits of the tile, ranked
  const uint32_t* srow = a.starts + row * ((a.n + 31) / 32);
  uint32_t mybits = ecount > 0 ? tile_bits(srow, static_cast<int>(first + t0), E) : 0u;
  if (ecount > 0 && ecount < E) mybits &= (1u << ecount) - 1u;
  if (first + t0 == 0) mybits |= 1u;
  if (bad) mybits = 0u;
  const int pc = __builtin_popcount(mybits);
  const int incl = wave_incl_i32(pc);
  if (lane == kWave - 1) rank_scan[wave] = incl;
  __syncthreads();
  int before = incl - pc;
  for (int w2 = 0; w2 < wave; ++w2) before += rank_scan[w2];
  const int at_start = bad ? 0 : ((rec.flags & kTileHead) ? 1 : 0);
  int jj = bad ? 0 : before + static_cast<int>(mybits & 1u) - at_start;
  T wv[W ? E : 1], yv[E];
  const bool need_y = a.gw != nullptr;
  // (ragged rows: the row's own elements from and to their packed places; the pad's gradients
  // are not stored, nor their w and y read)
  int64_t rfirst = row * a.n, rlen = a.n;
  if constexpr (MAP) map_row(a.map, row, a.n, rfirst, rlen);
  const int lc = MAP ? static_cast<int>(max<int64_t>(0, min<int64_t>(ecount, min<int64_t>(len, rlen - first) - t0)))
                     : ecount;
  if constexpr (W) load_elems_any<T, E>(static_cast<const T*>(a.w) + rfirst + first + t0, lc, wv);
  if (need_y) load_elems_any<T, E>(static_cast<const T*>(a.y) + rfirst + first + t0, lc, yv);
  T oy[E], ow[E];
#pragma unroll
  for (int k = 0; k < E; ++k) {
    if (k > 0) jj += (mybits >> k) & 1u;
    const double q = qv[jj];
    const double wk = W ? static_cast<double>(wv[W ? k : 0]) : 1.0;
    oy[k] = static_cast<T>(wk * q);
    if (need_y) ow[k] = static_cast<T>((static_cast<double>(yv[k]) - static_cast<double>(mv[jj])) * q);
  }
  if (a.gy != nullptr) store_elems_any<T, E>(static_cast<T*>(a.gy) + rfirst + first + t0, lc, oy);
  if (a.gw != nullptr) store_elems_any<T, E>(static_cast<T*>(a.gw) + rfirst + first + t0, lc, ow);
}

// Rows of at most 2048 elements: whole rows packed into a workgroup of 256 threads, E
// consecutive elements a thread (E = 4 for rows up to 1024 elements, 8 up to 2048; the larger
// E is slower for short rows, the smaller leaves half a workgroup idle above 1024).
template <int E>
struct PackCfg {
  static constexpr int kElems = 256 * E;                                   // elements a workgroup
  static constexpr int kRows = kElems / (static_cast<int>(kShortMax) + 1);  // rows a workgroup, n > 32
  static_assert(kRows < 256, "row indices in uint8_t");
  static_assert(kElems <= TileCfg<true>::kN && kElems <= TileCfg<false>::kN, "rows of one tile");
};
constexpr int kPackMaxN = PackCfg<8>::kElems;

// segmented sum: b's value unless b holds a block start, else a's plus b's
__device__ __forceinline__ void seg_combine(double as, int ac, double& bs, int& bc) {
  bs = bc > 0 ? bs : as + bs;
  bc += ac;
}

// One kernel for the backward of such rows (no per-tile pass, no scan kernels): one segmented
// scan of g over the workgroup's elements, reset at every block start, leaves each block's sum
// G at its last element; a pass over the workgroup's blocks then takes each block's weight and
// fit from the forward's hull vertices (as gfill_kernel does) and forms q = mask * G / W; each
// element writes gy = w * q and gw = (y - fit) * q. A NaN row is one block (fit NaN).
template <typename T, bool W, int E, bool MAP = false>
__global__ __launch_bounds__(256) void gpack_kernel(GradKArgs a, int rows_per_wg) {
  using C = PackCfg<E>;
  __shared__ double qv[C::kElems];       // per block of the workgroup: G, then mask * G / W
  __shared__ T mv[C::kElems];            // per block: its fit
  __shared__ uint8_t brow[C::kElems];    // per block: its row within the workgroup
  __shared__ int rowbase[C::kRows];      // per row: its first block's index in the workgroup
  __shared__ uint8_t rowbad[C::kRows];   // per row: NaN row (one block)
  __shared__ double wave_s[kWaves256];
  __shared__ int wave_c[kWaves256];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int n = static_cast<int>(a.n);
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * rows_per_wg;
  const int rows = static_cast<int>(min<int64_t>(rows_per_wg, a.batch - row0));
  const int count = rows * n;
  const int64_t base = row0 * a.n;
  const int e0 = tid * E;
  const int ecount = max(0, min(E, count - e0));
  const DivBy div(static_cast<uint32_t>(n));  // (e, n <= 2048: e * n < 2^32)
  const int64_t wpr = (a.n + 31) / 32;
  const bool use_lo = a.flags & TI_CLIP_MIN, use_hi = a.flags & TI_CLIP_MAX;
  const bool need_y = a.gw != nullptr;

  T gv[E], wv[W ? E : 1], yv[E];
  // Ragged rows: element e0 + k is element i_k of the workgroup's row r_k, at its packed place
  // for i_k below the row's length, else the pad's (g = 0; w and y unused: its gradients are not
  // stored). Rows are longer than 32 elements and a thread holds at most 8, so a thread's
  // elements lie in at most two rows, whose descriptors it reads once.
  constexpr bool mapped = MAP;
  int64_t mf[2] = {0, 0}, ml[2] = {0, 0};
  int ra = 0;
  if (mapped) {
    ra = ecount > 0 ? static_cast<int>(div(static_cast<uint32_t>(e0))) : 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (ra + h < rows) map_row(a.map, row0 + ra + h, a.n, mf[h], ml[h]);
    }
  }
  // (the packed index of element k, or -1 for the pad's and past the workgroup's elements)
  auto mapped_at = [&](int k) -> int64_t {
    const int e = e0 + k;
    if (k >= ecount) return -1;
    const int i = e - ra * n;
    const int h = i >= n ? 1 : 0;
    const int ih = i - h * n;
    return ih < ml[h] ? mf[h] + ih : int64_t{-1};
  };
  if (mapped) {
#pragma unroll
    for (int k = 0; k < E; ++k) {
      const int64_t p = mapped_at(k);
      gv[k] = p >= 0 ? static_cast<const T*>(a.g)[p] : T(0);
      if constexpr (W) wv[W ? k : 0] = p >= 0 ? static_cast<const T*>(a.w)[p] : T(1);
      if (need_y) yv[k] = p >= 0 ? static_cast<const T*>(a.y)[p] : T(0);
    }
  } else {
    load_elems_any<T, E>(static_cast<const T*>(a.g) + base + e0, ecount, gv);
    if constexpr (W) load_elems_any<T, E>(static_cast<const T*>(a.w) + base + e0, ecount, wv);
    if (need_y) load_elems_any<T, E>(static_cast<const T*>(a.y) + base + e0, ecount, yv);
  }
  if (tid < rows) rowbad[tid] = (a.tiles[row0 + tid].flags & kTileBad) ? 1 : 0;
  __syncthreads();

  // block starts of elements e0 .. e0 + E (past the workgroup's last element: an end)
  bool f[E + 1];
  int er[E];  // each element's row within the workgroup
#pragma unroll
  for (int k = 0; k <= E; ++k) {
    const int e = e0 + k;
    if (e < count) {
      const int r = static_cast<int>(div(static_cast<uint32_t>(e)));
      const int i = e - r * n;
      if (k < E) er[k] = r;
      f[k] = i == 0 || (!rowbad[r] && ((a.starts[(row0 + r) * wpr + (i >> 5)] >> (i & 31)) & 1u));
    } else {
      f[k] = true;
      if (k < E) er[k] = 0;
    }
  }

  // the thread's segmented aggregate, then the workgroup's exclusive scan of them
  double s = 0.0;
  int c = 0;
#pragma unroll
  for (int k = 0; k < E; ++k) {
    if (k < ecount) {
      if (f[k]) {
        s = 0.0;
        ++c;
      }
      s += static_cast<double>(gv[k]);
    }
  }
  // (DPP steps: a lane without a source gets (0, 0), which seg_combine passes through)
  auto step = [&](double os, int oc) { seg_combine(os, oc, s, c); };
  step(dpp_f64<0x111, 0xF>(s), dpp_i32<0x111, 0xF>(c));
  step(dpp_f64<0x112, 0xF>(s), dpp_i32<0x112, 0xF>(c));
  step(dpp_f64<0x114, 0xF>(s), dpp_i32<0x114, 0xF>(c));
  step(dpp_f64<0x118, 0xF>(s), dpp_i32<0x118, 0xF>(c));
  step(dpp_f64<0x142, 0xA>(s), dpp_i32<0x142, 0xA>(c));
  step(dpp_f64<0x143, 0xC>(s), dpp_i32<0x143, 0xC>(c));
  if (lane == kWave - 1) {
    wave_s[wave] = s;
    wave_c[wave] = c;
  }
  double xs = dpp_f64<0x138, 0xF>(s);
  int xc = wave_shr1_i32(c);
  __syncthreads();
  double ps = 0.0;
  int pc = 0, nb = 0;
  for (int v = 0; v < kWaves256; ++v) {
    if (v < wave) {
      double ts = wave_s[v];
      int tc = wave_c[v];
      seg_combine(ps, pc, ts, tc);
      ps = ts;
      pc = tc;
    }
    nb += wave_c[v];
  }
  seg_combine(ps, pc, xs, xc);

  // each block's sum at its last element; each row's first block
  int eb[E];
#pragma unroll
  for (int k = 0; k < E; ++k) {
    eb[k] = 0;
    if (k < ecount) {
      if (f[k]) {
        xs = 0.0;
        ++xc;
        const int i = e0 + k - er[k] * n;
        if (i == 0) rowbase[er[k]] = xc - 1;
      }
      xs += static_cast<double>(gv[k]);
      eb[k] = xc - 1;
      if (f[k + 1]) {
        qv[xc - 1] = xs;
        brow[xc - 1] = static_cast<uint8_t>(er[k]);
      }
    }
  }
  __syncthreads();

  // per block: q and the fit, from the forward's hull of its row
  const double sgn = (a.flags & TI_INCREASING) ? 1.0 : -1.0;
  const T lo = static_cast<T>(a.lo), hi = static_cast<T>(a.hi);
  for (int b = tid; b < nb; b += 256) {
    const int r = brow[b];
    const int64_t row = row0 + r;
    const NodeOut fin = node_out(a.hulls, W, row);
    const double G = qv[b];
    double q;
    T mean;
    if (rowbad[r]) {
      const int last = a.tiles[row].last;
      const double wsum = dd_diff(vertex_w<W>(fin, last), vertex_w<W>(fin, 0));
      q = (use_lo || use_hi) ? 0.0 : G / wsum;
      mean = quiet_nan<T>();
    } else {
      const int j = b - rowbase[r];
      const double dW = dd_diff(vertex_w<W>(fin, j + 1), vertex_w<W>(fin, j));
      const double dS = dd_diff(DD{fin.shi[j + 1], lo_at(fin.slo, j + 1)}, DD{fin.shi[j], lo_at(fin.slo, j)});
      mean = static_cast<T>(sgn * slope_div(dS, dW));
      q = G / dW;
      if ((use_lo || use_hi) && !clip_passes(mean, use_lo, lo, use_hi, hi)) q = 0.0;
    }
    qv[b] = q;
    mv[b] = mean;
  }
  __syncthreads();

  T oy[E], ow[E];
#pragma unroll
  for (int k = 0; k < E; ++k) {
    const double q = qv[eb[k]];
    const double wk = W ? static_cast<double>(wv[W ? k : 0]) : 1.0;
    oy[k] = static_cast<T>(wk * q);
    if (need_y) ow[k] = static_cast<T>((static_cast<double>(yv[k]) - static_cast<double>(mv[eb[k]])) * q);
  }
  if (mapped) {
#pragma unroll
    for (int k = 0; k < E; ++k) {
      const int64_t p = mapped_at(k);
      if (p >= 0) {
        if (a.gy != nullptr) static_cast<T*>(a.gy)[p] = oy[k];
        if (a.gw != nullptr) static_cast<T*>(a.gw)[p] = ow[k];
      }
    }
    return;
  }
  if (a.gy != nullptr) store_elems_any<T, E>(static_cast<T*>(a.gy) + base + e0, ecount, oy);
  if (a.gw != nullptr) store_elems_any<T, E>(static_cast<T*>(a.gw) + base + e0, ecount, ow);
}

}  // namespace

size_t long_grad_bytes(int64_t batch, int64_t n, bool weighted, bool lo, int64_t kept_maxc) {
  return grad_plan(batch, n, weighted, lo, kept_maxc).bytes;
}

hipError_t long_grad(const LongGradArgs& in, const LongPlan& p, void* ws) {
  const bool W = in.w != nullptr;
  const int64_t kmaxc = in.kept != nullptr ? in.kept_maxc : 0;
  const bool lo = in.dtype == TI_F64;
  const GradPlan gpn = grad_plan(in.batch, in.n, W, lo, kmaxc);
  char* base = static_cast<char*>(ws);
  const char* fbase = static_cast<const char*>(in.fwd_ws);
  GradKArgs a;
  a.starts = in.starts;
  a.g = in.g;
  a.w = in.w;
  a.y = in.y;
  a.gy = in.gy;
  a.gw = in.gw;
  a.batch = in.batch;
  a.n = in.n;
  a.map = in.map;
  a.tpr = gpn.tpr;
  a.ngroups = gpn.ngroups;
  a.cap_final = gpn.cap_final;
  a.flags = in.flags;
  a.lo = in.lo;
  a.hi = in.hi;
  if (in.kept != nullptr) {
    const KeepPlan kp = keep_plan(in.batch, in.n, W, lo, kmaxc);
    a.hulls = kp.level(const_cast<void*>(in.kept));
    a.tiles = reinterpret_cast<const TileRec*>(static_cast<const char*>(in.kept) + kp.off_tiles);
  } else {
    a.hulls = p.level(const_cast<char*>(fbase), p.levels);
    a.tiles = reinterpret_cast<const TileRec*>(fbase + p.off_rank);
  }
  a.tg = reinterpret_cast<double*>(base + gpn.off_tg);
  a.lp = reinterpret_cast<double*>(base + gpn.off_lp);
  a.gt = reinterpret_cast<double*>(base + gpn.off_gt);
  a.gp = reinterpret_cast<double*>(base + gpn.off_gp);
  a.lv = reinterpret_cast<double*>(base + gpn.off_lv);
  if (in.n <= kPackMaxN) {  // (then one tile a row)
    auto launch = [&](auto E_) -> hipError_t {
      constexpr int E = decltype(E_)::value;
      const int rpw = PackCfg<E>::kElems / static_cast<int>(in.n);
      const unsigned blocks = static_cast<unsigned>((in.batch + rpw - 1) / rpw);
      if (in.dtype == TI_F32) {
        // (ragged rows of a block: float32 only)
        if (in.map.rows != nullptr) {
          if (W) gpack_kernel<float, true, E, true><<<dim3(blocks), dim3(256), 0, in.stream>>>(a, rpw);
          else gpack_kernel<float, false, E, true><<<dim3(blocks), dim3(256), 0, in.stream>>>(a, rpw);
        } else if (W) {
          gpack_kernel<float, true, E><<<dim3(blocks), dim3(256), 0, in.stream>>>(a, rpw);
        } else {
          gpack_kernel<float, false, E><<<dim3(blocks), dim3(256), 0, in.stream>>>(a, rpw);
        }
      } else {
        if (W) gpack_kernel<double, true, E><<<dim3(blocks), dim3(256), 0, in.stream>>>(a, rpw);
        else gpack_kernel<double, false, E><<<dim3(blocks), dim3(256), 0, in.stream>>>(a, rpw);
      }
      return hipGetLastError();
    };
    if (in.n <= PackCfg<4>::kElems) return launch(std::integral_constant<int, 4>{});
    return launch(std::integral_constant<int, 8>{});
  }
  const unsigned tiles = static_cast<unsigned>(in.batch * gpn.tpr);
  const unsigned gsum_blocks = (tiles + kGsumTiles - 1) / kGsumTiles;
  if (in.dtype == TI_F32) {
    if (in.map.rows != nullptr) {  // (ragged rows of a block: float32 only)
      if (W) gsum_kernel<float, true, true><<<dim3(gsum_blocks), dim3(256), 0, in.stream>>>(a);
      else gsum_kernel<float, false, true><<<dim3(gsum_blocks), dim3(256), 0, in.stream>>>(a);
    } else if (W) {
      gsum_kernel<float, true><<<dim3(gsum_blocks), dim3(256), 0, in.stream>>>(a);
    } else {
      gsum_kernel<float, false><<<dim3(gsum_blocks), dim3(256), 0, in.stream>>>(a);
    }
  } else {
    if (W) gsum_kernel<double, true><<<dim3(gsum_blocks), dim3(256), 0, in.stream>>>(a);
    else gsum_kernel<double, false><<<dim3(gsum_blocks), dim3(256), 0, in.stream>>>(a);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (gpn.tpr > 1) {  // (rows of one tile: gsum wrote the scans' results)
    gscan_local_kernel<<<dim3(static_cast<unsigned>(in.batch * gpn.ngroups)), dim3(256), 0, in.stream>>>(a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (gpn.ngroups > 1) {
      gscan_groups_kernel<<<dim3(static_cast<unsigned>(in.batch)), dim3(256), 0, in.stream>>>(a);
      e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
  }
  if (in.dtype == TI_F32) {
    if (in.map.rows != nullptr) {  // (ragged rows of a block: float32 only)
      if (W) gfill_kernel<float, true, true><<<dim3(tiles), dim3(256), 0, in.stream>>>(a);
      else gfill_kernel<float, false, true><<<dim3(tiles), dim3(256), 0, in.stream>>>(a);
    } else if (W) {
      gfill_kernel<float, true><<<dim3(tiles), dim3(256), 0, in.stream>>>(a);
    } else {
      gfill_kernel<float, false><<<dim3(tiles), dim3(256), 0, in.stream>>>(a);
    }
  } else {
    if (W) gfill_kernel<double, true><<<dim3(tiles), dim3(256), 0, in.stream>>>(a);
    else gfill_kernel<double, false><<<dim3(tiles), dim3(256), 0, in.stream>>>(a);
  }
  return hipGetLastError();
}

}  // namespace ti
