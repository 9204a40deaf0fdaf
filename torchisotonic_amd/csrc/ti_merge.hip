// Rows longer than 32 elements: the cross-span merge and the expansion.
//
// Replaces the reference's chunk-start prefix, merge rounds and fit stages (reference
// src/torchisotonic/csrc/tiles.cuh:1680-1725, 1524-1537 + 1728-1743, 1541-1667): instead of
// one launch per pairwise round over segment lists, a workgroup merges G = 64 neighbouring
// hulls at a time, six rounds in LDS, so a row of 1e8 elements (390,625 span hulls of 256
// elements) needs four merge launches.
//
//   merge_kernel   G child hulls (compact arrays, double-double coordinates relative to the
//                  child) -> one parent hull relative to the parent. Children are laid end to
//                  end with their shared boundary point stored once, so a merge whose junction
//                  is already convex moves nothing; a bridge moves the right part's surviving
//                  suffix down. Works in LDS when the children's vertices fit (the case for
//                  noisy data, where hulls are small), else in the parent's own global array.
//   expand_kernel  per tile of the row (four to a workgroup): the final hull's vertices around
//                  the tile (ranks from rank_kernel), edge slopes in float64 rounded once, every
//                  element the slope of its edge with the clamp fused, and the start bits. y is
//                  not read again.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "ti_common.h"
#include "ti_expand.h"
#include "ti_kernels.h"
#include "ti_slots.h"
#include "ti_gmerge.h"
#include "ti_tile.h"

namespace ti {

namespace {



// Float32 data keeps its hull sums rounded to float64 in the vertex store (NodeOut). Rounded one
// by one, a hull that the double-double merges found convex can turn slightly non-convex in the
// stored values where points are nearly collinear, and the fit (its slopes) would step down
// there. Each final hull is made convex in the stored values: by the workgroup that merged it
// (repair_row, at the end of the last merge launch) where rows end two or more merge levels up
// and are many, else in two launches after the merges:
//
//   convex_check_kernel  `chunks` workgroups a row test every vertex against its neighbours; a
//                        vertex on or above the chord between them marks its row (flag = the
//                        call's epoch, so the flags need no clearing between calls);
//   repair_kernel        one workgroup a marked row: a vertex on or above the chord between its
//                        neighbours is no vertex of the lower hull of the stored points, so every
//                        such vertex goes at once, and the row is tested again. The removal
//                        compacts the row in place a chunk at a time, the chunk's original
//                        vertices (and its neighbours outside it) staged in LDS before any of its
//                        slots is written.
constexpr int kRepairThreads = 256;

template <bool W>
__global__ __launch_bounds__(kRepairThreads) void convex_check_kernel(NodeLevel fin, int chunks, unsigned epoch,
                                                                      unsigned* __restrict__ flag) {
  const int64_t row = blockIdx.x / chunks;
  const int c = static_cast<int>(blockIdx.x - row * chunks);
  const NodeOut o = node_out(fin, W, row);
  if (*o.bad != 0) return;  // (a NaN row's fit is NaN whatever its hull)
  const int cnt = *o.count;
  const VArr v = dvarr_of(o);
  bool found = false;
  for (int i = 1 + c * kRepairThreads + static_cast<int>(threadIdx.x); i < cnt - 1; i += chunks * kRepairThreads)
    found |= vpools<W>(vload<W>(v, i - 1), vload<W>(v, i), vload<W>(v, i + 1));
  if (found) flag[row] = epoch;
}

// (repair_row's removal, written out for one 256-thread workgroup a marked row: through
// repair_row, whose check keeps four vertices a thread in flight, C3's float32 forward took 5 us
// longer)
template <bool W>
__global__ __launch_bounds__(kRepairThreads) void repair_kernel(NodeLevel fin, unsigned epoch,
                                                                const unsigned* __restrict__ flag, int passes) {
  __shared__ int any;
  __shared__ int wcount[kRepairThreads / kWave];
  __shared__ VPt tile[kRepairThreads + 2];
  __shared__ VPt prev;  // the original vertex before the chunk
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int64_t row = blockIdx.x;
  if (flag[row] != epoch) return;  // (convex already)
  const NodeOut o = node_out(fin, W, row);
  if (*o.bad != 0) return;
  const VArr v = dvarr_of(o);
  int cnt = *o.count;
  bool convex = false;
  for (int pass = 0; pass <= passes; ++pass) {
    if (tid == 0) any = 0;
    __syncthreads();
    bool found = false;
    for (int i = 1 + tid; i < cnt - 1; i += kRepairThreads)
      found |= vpools<W>(vload<W>(v, i - 1), vload<W>(v, i), vload<W>(v, i + 1));
    if (__any(found) && lane == 0) any = 1;
    __syncthreads();
    if (any == 0) {
      convex = true;
      break;
    }
    if (pass == passes) break;  // (still not convex: chain_row below)
    int base = 0;
    for (int c0 = 0; c0 < cnt; c0 += kRepairThreads) {
      const int i = c0 + tid;
      if (i < cnt) tile[tid + 1] = vload<W>(v, i);
      if (tid == 0) {
        if (c0 > 0) tile[0] = prev;
        if (c0 + kRepairThreads < cnt) tile[kRepairThreads + 1] = vload<W>(v, c0 + kRepairThreads);
      }
      __syncthreads();
      const bool keep = i < cnt && (i == 0 || i == cnt - 1 || !vpools<W>(tile[tid], tile[tid + 1], tile[tid + 2]));
      const uint64_t m = __ballot(keep);
      if (lane == 0) wcount[wave] = __popcll(m);
      __syncthreads();
      int before = base, all = 0;
      for (int k = 0; k < kRepairThreads / kWave; ++k) {
        before += k < wave ? wcount[k] : 0;
        all += wcount[k];
      }
      const VPt x = tile[tid + 1];
      if (tid == kRepairThreads - 1) prev = x;  // (read in the next chunk, after its barrier)
      __syncthreads();  // every read of this chunk's slots is done
      if (keep) vstore<W>(v, before + __popcll(m & ((uint64_t{1} << lane) - 1)), x);
      base += all;
    }
    cnt = base;
    __syncthreads();
  }
  if (!convex) cnt = chain_row<W, kRepairThreads>(v, cnt, tile);
  if (tid == 0) *o.count = cnt;
}

// Per merge: the children (vertex counts, first slots, offsets within the parent) and the
// fallback's pairwise-round bookkeeping.
// The merge in LDS: the children's vertices into slots (every thread's loads in flight
// together), the pairwise rounds, and the survivors out to the parent's arrays.
template <bool W, bool PR, int NT, int G>
__device__ void merge_lds(const MergeArgs& a, const MergeSmall& sm, MergeRounds& rs, const Slots<W, PR>& v,
                          int64_t row, int64_t c0, int nch, const NodeOut& pout) {
  const int tid = threadIdx.x;
  const int total = sm.total;
  // slots per thread with their loads in flight together (fewer in large workgroups, whose
  // threads have fewer registers and fewer slots each)
  constexpr int B = NT >= 1024 ? 2 : NT >= 256 ? 4 : 8;
  for (int s0 = 0; s0 < total; s0 += NT * B) {
    HPt p[B];
    int cs[B];
#pragma unroll
    for (int u = 0; u < B; ++u) {
      // (slots past the end load the last slot again, so the loads need no branches)
      const int s = min(s0 + u * NT + tid, total - 1);
      cs[u] = child_of_slot(sm, nch, s);
      p[u] = child_vertex<W, PR>(a, sm, row, c0, cs[u], s - sm.off[cs[u]]);
    }
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int s = s0 + u * NT + tid;
      if (s < total) {
        sput(v, s, p[u]);
        v.cid[s] = static_cast<uint8_t>(cs[u]);
      }
    }
  }
  for (int c = tid; c < nch; c += NT) rs.seg[0][c] = sm.off[c] + sm.cnt[c] - 1;
  __syncthreads();
  const int count = merge_rounds<W, PR, NT, G>(v, rs, total, nch);
  for (int s = tid; s < count; s += NT) {
    const HPt x = sget(v, s);
    pout.idx[s] = x.i;
    put_dd(pout.shi, pout.slo, s, x.s, x.sl);
    if constexpr (W) put_dd(pout.whi, pout.wlo, s, x.w, x.wl);
  }
  if (tid == 0) *pout.count = count;
}

// One workgroup of NT threads per parent node: G = 64 children (fewer at a row's end) -> the
// parent's hull. NT grows where few parents share the GPU (the upper levels), so that their
// larger hulls still take few slots per thread.
// Rows enough for their final merge workgroups to read their hulls at the GPU's bandwidth.
constexpr bool batch_fills_gpu(int64_t batch) { return batch >= 256; }

// LDS repair_row takes with NT threads (carved from a merge kernel's slots once they are free).
constexpr size_t repair_lds_bytes(int nt) { return (nt + 2) * sizeof(VPt) + (nt / kWave + 1) * sizeof(int); }

// fix > 0: the launch makes the final hulls of float32 data, which the workgroup then makes convex
// in their stored values (repair_row, with fix - 1 removal passes before its chain), so no check
// launch follows.
// TX (float or double: the fit's type) with the final level of rows enough to fill the GPU: the
// workgroup then expands its row's final hull too (expand_row, with x.lds_bytes of its dynamic
// LDS), in place of the rank and expansion launches.
// DF: a deferring level, tab its parents' DeferTabs (see merge_global).
template <bool W, bool PR, int NT, int G, typename TX = void, bool DF = false>
__global__ __launch_bounds__(NT) void merge_kernel(MergeArgs a, int cap_lds, int fix, RowExpand x, DeferTab* tab) {
  __shared__ MergeSmall sm;
  __shared__ MergeRounds rs;
  extern __shared__ __align__(16) char lds_dyn[];
  const int tid = threadIdx.x;
  if (DF && tid == 0) tab[blockIdx.x].deferred = 0;
  if (a.mark != nullptr && blockIdx.x == 0 && tid == 0)
    __hip_atomic_store(a.mark, a.mark_value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  const int64_t row = blockIdx.x / a.out.npr;
  const int64_t j = blockIdx.x - row * a.out.npr;
  const int64_t c0 = j * kGroup;  // first child within the row
  const int nch = static_cast<int>(min<int64_t>(kGroup, a.in.npr - c0));
  const NodeOut pout = node_out(a.out, W, row * a.out.npr + j);
  // (a first child's count of -1: the span kernel merged this group already)
  if (*node_out(a.in, W, row * a.in.npr + c0).count < 0) return;

  // Children (first wave): counts, NaN flags, and offsets within the parent (double-double scan).
  if (tid < kWave) {
    const int lane = tid;
    int cnt = 0, bad = 0;
    DD tw{0.0, 0.0}, ts{0.0, 0.0};
    if (lane < nch) {
      const NodeOut ci = node_out(a.in, W, row * a.in.npr + c0 + lane);
      cnt = *ci.count;
      bad = *ci.bad;
      tw = DD{ci.tot[0], ci.tot[1]};
      ts = DD{ci.tot[2], ci.tot[3]};
    }
    // inclusive scans: totals (dd) and slots (count - 1, the shared point stored once)
    const DD iw = wave_incl_dd(tw), is = wave_incl_dd(ts);
    const int islot = wave_incl_i32(max(cnt - 1, 0));
    const int anybad = __any(bad != 0);
    const DD ew = wave_shr1_dd(iw), es = wave_shr1_dd(is);
    if (lane < nch) {
      sm.cnt[lane] = cnt;
      sm.off[lane] = islot - max(cnt - 1, 0);
      sm.tot[0][lane] = ew.hi;
      sm.tot[1][lane] = ew.lo;
      sm.tot[2][lane] = es.hi;
      sm.tot[3][lane] = es.lo;
    }
    if (lane == nch - 1) {
      sm.tot[0][nch] = iw.hi;
      sm.tot[1][nch] = iw.lo;
      sm.tot[2][nch] = is.hi;
      sm.tot[3][nch] = is.lo;
      sm.total = islot + 1;  // slots
    }
    if (lane == 0) sm.bad = anybad;
  }
  __syncthreads();

  if (sm.total <= cap_lds) {
    merge_lds<W, PR, NT, G>(a, sm, rs, slots_carve<W, PR>(lds_dyn, cap_lds), row, c0, nch, pout);
  } else {
    __shared__ MergeRanges mr;
    merge_global<W, PR, NT, DF>(a, sm, mr.rlo, mr.rhi, mr.pre, row, c0, nch, pout, DF ? tab + blockIdx.x : nullptr);
  }
  if (tid == 0) {
    *pout.bad = sm.bad;
    pout.tot[0] = sm.tot[0][nch];
    pout.tot[1] = sm.tot[1][nch];
    pout.tot[2] = sm.tot[2][nch];
    pout.tot[3] = sm.tot[3][nch];
  }
  if (fix != 0 && sm.bad == 0) {
    __syncthreads();  // the hull written by every thread, the slots read
    VPt* tile = reinterpret_cast<VPt*>(lds_dyn);
    int* wcount = reinterpret_cast<int*>(tile + NT + 2);
    repair_row<W, NT>(pout, tile, wcount, wcount[NT / kWave], fix - 1);
  }
  if constexpr (!std::is_void_v<TX>) expand_row<TX, W, false, NT>(x, pout, sm.bad != 0, row, lds_dyn);
}

// The survivors of a deferring level's parents that merge_global left to it (their children's
// kept ranges and offsets in each parent's DeferTab), written into the parents' arrays, which
// lie in the other store than the children's: per_parent workgroups a parent, each a stretch of
// its slots, in no order (no slot of the parent's array is a source). A slot's vertex is the
// kept vertex of the last child whose survivors start at or before it, its coordinates rebased
// into the parent's as the merge's own pass does (child_vertex); four slots a thread at a time,
// their loads in flight together.
constexpr int64_t kSurvivorBlocks = 2048;

template <bool W, bool PR>
__global__ __launch_bounds__(256) void survivors_kernel(MergeArgs a, const DeferTab* __restrict__ tab,
                                                        int per_parent) {
  constexpr int NT = 256, U = 4;
  __shared__ MergeSmall sm;  // (its tot only: child_vertex's offsets)
  __shared__ int rlo[kGroup], pre[kGroup];
  const int tid = threadIdx.x;
  const int64_t parent = blockIdx.x / per_parent;
  const int part = static_cast<int>(blockIdx.x - parent * per_parent);
  const DeferTab* tp = tab + parent;
  const int64_t row = parent / a.out.npr;
  const int64_t c0 = (parent - row * a.out.npr) * kGroup;
  const int nch = static_cast<int>(min<int64_t>(kGroup, a.in.npr - c0));
  // (the flag, the count and the table in one round trip: a parent the merge finished, the
  // common case, costs its workgroups no more)
  const int deferred = tp->deferred;
  const int64_t total = tp->total;
  for (int c = tid; c < nch; c += NT) {
    rlo[c] = tp->rlo[c];
    pre[c] = tp->pre[c];
#pragma unroll
    for (int q = 0; q < 4; ++q) sm.tot[q][c] = tp->tot[q][c];
  }
  if (deferred == 0) return;
  __syncthreads();
  const int64_t chunk = ((total + per_parent - 1) / per_parent + NT * U - 1) / (NT * U) * (NT * U);
  const int s_end = static_cast<int>(min<int64_t>(total, (part + 1) * chunk));
  const VArr v = dvarr_of(node_out(a.out, W, parent));
  for (int s0 = static_cast<int>(min<int64_t>(total, part * chunk)); s0 < s_end; s0 += NT * U) {
    HPt h[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = s0 + u * NT + tid;
      if (s < s_end) {
        int lo = 0, hi = nch - 1;
        while (lo < hi) {
          const int mid = (lo + hi + 1) >> 1;
          if (pre[mid] <= s) lo = mid;
          else hi = mid - 1;
        }
        h[u] = child_vertex<W, PR>(a, sm, row, c0, lo, rlo[lo] + (s - pre[lo]));
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = s0 + u * NT + tid;
      if (s < s_end) {
        VPt p;
        p.i = h[u].i;
        p.s = DD{h[u].s, h[u].sl};
        p.w = W ? DD{h[u].w, h[u].wl} : DD{static_cast<double>(h[u].i), 0.0};
        vstore<W>(v, s, p);
      }
    }
  }
}

// Per expansion tile of tile_n elements (one thread each): the final hull's last vertex at or
// before the tile's first element, and its first vertex at or after the tile's end, by binary
// searches over the row's hull (which runs from index 0 to n), with the row's flags and, where
// one edge covers the tile, its slope. All tiles search at once, so the expansion and the
// backward start from one read per tile.
template <bool W>
__global__ __launch_bounds__(256) void rank_kernel(NodeLevel hulls, int64_t batch, int64_t n,
                                                   int64_t tile_n, int64_t tpr, TileRec* tiles) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (g >= batch * tpr) return;
  const int64_t row = g / tpr;
  const int64_t ta = (g - row * tpr) * tile_n;
  const int64_t tb = min(ta + tile_n, n);
  const NodeOut fin = node_out(hulls, W, row);
  const int* idx = fin.idx;
  const int count = *fin.count;
  const bool bad = *fin.bad != 0;
  TileRec r;
  int lo = 0, hi = count - 1;  // idx[0] = 0 <= ta
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (idx[mid] <= ta) lo = mid;
    else hi = mid - 1;
  }
  r.ra = lo;
  hi = count - 1;  // idx[count - 1] = n >= tb
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (idx[mid] >= tb) hi = mid;
    else lo = mid + 1;
  }
  r.rb = lo;
  r.last = count - 1;
  const bool head = bad ? ta == 0 : idx[r.ra] == ta;
  r.flags = (bad ? kTileBad : 0) | (head ? kTileHead : 0);
  r.slope = 0.0;
  r.unused = 0.0;
  if (!bad && r.rb == r.ra + 1) {
    const VArr v = dvarr_of(fin);
    double dW, dS;
    vdiff<W>(vload<W>(v, r.ra), vload<W>(v, r.ra + 1), dW, dS);
    r.slope = slope_div(dS, dW);
  }
  tiles[g] = r;
}

// Tiles per expansion workgroup: their records are read together, so a workgroup waits for one
// memory round trip, not one per tile.
constexpr int kExpandTiles = 4;

// Per tile: the fit from the row's final hull.
// NTS: the fit written with non-temporal stores (TI_STREAM_OUT), its lines leaving the caches
// as they are written instead of draining under the next kernel's reads.
template <typename T, bool W, bool NTS, bool MAP = false>
__global__ __launch_bounds__(256) void expand_kernel(ExpandArgs a) {
  using C = TileCfg<W>;
  constexpr int E = C::kE;
  constexpr int NT = C::kThreads;
  constexpr int K = kExpandTiles;
  constexpr int NW = C::kN / 32;       // bitmap words a tile
  constexpr int V = 16 / sizeof(T);    // elements a 16-byte piece
  constexpr int G = E / V;             // pieces a thread
  static_assert(NW <= NT, "a thread per bitmap word");
  __shared__ T sl[C::kN + 2];  // sgn * slope per edge, rounded once to T
  __shared__ uint32_t bits[NW];
  __shared__ int wpre[NW];
  __shared__ int rank_scan[kWaves256];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int64_t ntiles = a.batch * a.tiles_per_row;
  const int64_t blk0 = static_cast<int64_t>(blockIdx.x) * K;
  const T tsgn = static_cast<T>((a.flags & TI_INCREASING) ? 1.0 : -1.0);
  const bool use_lo = a.flags & TI_CLIP_MIN, use_hi = a.flags & TI_CLIP_MAX;
  const T lo = static_cast<T>(a.lo), hi = static_cast<T>(a.hi);
  const int t0 = tid * E;
  const int64_t wpr = (a.n + 31) / 32;

  // each tile's row and place in it: one division, then steps (a 64-bit division by a runtime
  // value is a long scalar sequence)
  int64_t rowu[K], tileu[K];
  {
    int64_t row = blk0 / a.tiles_per_row, tile = blk0 - row * a.tiles_per_row;
#pragma unroll
    for (int u = 0; u < K; ++u) {
      rowu[u] = row;
      tileu[u] = tile;
      if (++tile == a.tiles_per_row && row + 1 < a.batch) {
        tile = 0;
        ++row;
      }
    }
  }
  // every tile's record first: one memory round trip for the workgroup
  TileRec rec[K];
#pragma unroll
  for (int u = 0; u < K; ++u) rec[u] = a.tiles[min(blk0 + u, ntiles - 1)];

#pragma unroll
  for (int u = 0; u < K; ++u) {
    const int64_t blk = blk0 + u;
    if (blk >= ntiles) break;
    const int64_t row = rowu[u];
    const int64_t tile = tileu[u];
    const int64_t first = tile * C::kN;
    const int len = static_cast<int>(min<int64_t>(C::kN, a.n - first));
    const bool row_bad = (rec[u].flags & kTileBad) != 0;
    const int ta = static_cast<int>(first);
    const int rA = rec[u].ra;
    const int ecount = max(0, min(E, len - t0));
    // (ragged rows: the row's place in the packed output, and slen, the tile's elements that are
    // the row's own: the pad's are not stored)
    int64_t rfirst = row * a.n, rlen = a.n;
    if constexpr (MAP) map_row(a.map, row, a.n, rfirst, rlen);
    const int slen = MAP ? static_cast<int>(max<int64_t>(0, min<int64_t>(len, rlen - first))) : len;
    T* out = static_cast<T*>(a.out) + rfirst + first;
    auto write_starts = [&](uint32_t sb) {
      if (a.starts == nullptr || ecount <= 0) return;
      if (ecount < E) sb &= (1u << ecount) - 1u;
      if constexpr (E == 16) {
        uint16_t* s16 = reinterpret_cast<uint16_t*>(a.starts + row * wpr);
        s16[(first + t0) >> 4] = static_cast<uint16_t>(sb);
      } else {
        uint8_t* s8 = reinterpret_cast<uint8_t*>(a.starts + row * wpr);
        s8[(first + t0) >> 3] = static_cast<uint8_t>(sb);
      }
    };

    if (rec[u].rb == rA + 1) {
      // One hull edge covers the whole tile (the common case on long rows, whose hulls have far
      // fewer vertices than tiles): the edge's slope from the record, no LDS, no barriers. The
      // only possible start is the tile's first element.
      const T val = row_bad ? quiet_nan<T>() : tsgn * static_cast<T>(rec[u].slope);
      fill_elems<T, E, NT, NTS>(out, slen, tid, clip(val, use_lo, lo, use_hi, hi));
      write_starts((t0 == 0 && (rec[u].flags & kTileHead)) ? 1u : 0u);
      continue;
    }
    const VArr v = dvarr_of(node_out(a.hulls, W, row));
    // (holds for any well-formed hull; it keeps the reads in bounds regardless)
    const int rB = min(min(rec[u].rb, rA + C::kN + 1), rec[u].last);

    // Edge slopes rA .. rB-1 and the vertex bits of the tile.
    for (int wd = tid; wd < C::kN / 32; wd += NT) bits[wd] = 0u;
    __syncthreads();
    for (int e = rA + tid; e < rB; e += NT) {
      const VPt p = vload<W>(v, e), q = vload<W>(v, e + 1);
      double dW, dS;
      vdiff<W>(p, q, dW, dS);
      sl[e - rA] = tsgn * static_cast<T>(slope_div(dS, dW));
      if (p.i >= ta) atomicOr(&bits[(p.i - ta) >> 5], 1u << ((p.i - ta) & 31));
    }
    __syncthreads();
    // per bitmap word: the tile's vertices before it (a scan of the words' counts)
    {
      const int c = tid < NW ? __popc(bits[tid]) : 0;
      const int incl = wave_incl_i32(c);
      if (lane == kWave - 1) rank_scan[wave] = incl;
      __syncthreads();
      int before = incl - c;
      for (int w2 = 0; w2 < wave; ++w2) before += rank_scan[w2];
      if (tid < NW) wpre[tid] = before;
    }
    __syncthreads();
    // An element's edge (from rA) is the tile's vertices at or before it, less one if a vertex
    // starts the tile. Each thread takes G pieces of V consecutive elements, each store
    // instruction of a wave one contiguous run of 64 pieces (16 bytes each); every piece's word
    // and count are read at once, then its elements' slopes.
    const int at_start = (v.idx[rA] == ta) ? 1 : 0;
    int g0[G], cnt[G];
    uint32_t wb[G];
#pragma unroll
    for (int j = 0; j < G; ++j) {
      g0[j] = j * NT * V + tid * V;
      const uint32_t word = bits[g0[j] >> 5];
      wb[j] = word >> (g0[j] & 31);
      cnt[j] = wpre[g0[j] >> 5] + __popc(word & ((1u << (g0[j] & 31)) - 1u)) - at_start;
    }
    T fit[G][V];
#pragma unroll
    for (int j = 0; j < G; ++j) {
#pragma unroll
      for (int k = 0; k < V; ++k) {
        cnt[j] += (wb[j] >> k) & 1u;  // (zero past the row's end: the last edge again)
        const T val = row_bad ? quiet_nan<T>() : sl[cnt[j]];
        fit[j][k] = clip(val, use_lo, lo, use_hi, hi);
      }
    }
    const bool aligned = (reinterpret_cast<uintptr_t>(out) & 15) == 0;
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const int m = slen - g0[j];
      if (m >= V && aligned) {
        using VT = T __attribute__((ext_vector_type(V)));
        VT x;
#pragma unroll
        for (int k = 0; k < V; ++k) x[k] = fit[j][k];
        if constexpr (NTS) __builtin_nontemporal_store(x, reinterpret_cast<VT*>(out + g0[j]));
        else *reinterpret_cast<VT*>(out + g0[j]) = x;
      } else {
#pragma unroll
        for (int k = 0; k < V; ++k)
          if (k < m) out[g0[j] + k] = fit[j][k];
      }
    }
    // start bits: the tile's words (a NaN row: its first element only)
    if (a.starts != nullptr) {
      for (int wd = tid; wd < (len + 31) / 32; wd += NT)
        a.starts[row * wpr + (first >> 5) + wd] = row_bad ? ((first == 0 && wd == 0) ? 1u : 0u) : bits[wd];
    }
    __syncthreads();  // sl, bits, wpre and rank_scan are reused by the next tile
  }
}

// Rows of at most 2048 elements (one tile) in place of rank_kernel and expand_kernel, whose
// one-tile-a-row layout leaves most threads of a workgroup idle on such rows: whole rows packed
// into a workgroup of 256 threads, E consecutive elements a thread (E = 4 for rows up to 1024
// elements, 8 up to 2048). Per row (one lane each): its record, as rank_kernel forms it for a
// row of one tile, and its edge count; per edge: its fit (the slope rounded once, then clamped,
// as expand_kernel forms it), its first element and that element's start bit, in LDS; per
// element: its edge (a binary search for a thread's first element, then at most one step per
// element). A NaN row is one edge, fit NaN.
constexpr int kXpackMaxN = 2048;

template <typename T, bool W, int E, bool MAP = false>
__global__ __launch_bounds__(256) void xpack_kernel(ExpandArgs a, TileRec* tiles, int rows_per_wg) {
  constexpr int NE = 256 * E;                  // elements a workgroup
  constexpr int NR = NE / (kShortMax + 1);     // rows a workgroup (n > 32)
  static_assert(NR <= kWave, "one lane per row");
  __shared__ T sl[NE];                         // per edge of the workgroup's rows: the fit
  __shared__ int16_t est[NE];                  // per edge: its first element within its row (< 2048)
  __shared__ int roff[NR + 1];                 // per row: its first edge; [rows]: the edges in all
  __shared__ uint8_t rbad[NR];
  __shared__ uint32_t sbits[NE / 32 + NR];     // the rows' start-bit words, in order
  __shared__ int64_t rmf[NR];                  // (ragged rows) per row: its first packed element
  __shared__ int rml[NR];                      // and its length
  const int tid = threadIdx.x;
  constexpr bool mapped = MAP;
  const int n = static_cast<int>(a.n);
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * rows_per_wg;
  const int rows = static_cast<int>(min<int64_t>(rows_per_wg, a.batch - row0));
  const int wpr = (n + 31) / 32;
  const T tsgn = static_cast<T>((a.flags & TI_INCREASING) ? 1.0 : -1.0);
  const bool use_lo = a.flags & TI_CLIP_MIN, use_hi = a.flags & TI_CLIP_MAX;
  const T lo = static_cast<T>(a.lo), hi = static_cast<T>(a.hi);

  if (tid < kWave) {
    int ne = 0;
    if (tid < rows) {
      const int64_t row = row0 + tid;
      const NodeOut fin = node_out(a.hulls, W, row);
      const int count = *fin.count;
      const bool bad = *fin.bad != 0;
      TileRec r;
      r.ra = 0;
      r.rb = count - 1;
      r.last = count - 1;
      r.flags = kTileHead | (bad ? kTileBad : 0);
      r.slope = 0.0;
      r.unused = 0.0;
      if (!bad && count == 2) {
        const VArr v = dvarr_of(fin);
        double dW, dS;
        vdiff<W>(vload<W>(v, 0), vload<W>(v, 1), dW, dS);
        r.slope = slope_div(dS, dW);
      }
      tiles[row] = r;
      ne = bad ? 1 : count - 1;
      rbad[tid] = bad ? 1 : 0;
      if constexpr (MAP) {
        int64_t f, l;
        map_row(a.map, row, a.n, f, l);
        rmf[tid] = f;
        rml[tid] = static_cast<int>(l);
      }
    }
    const int inc = wave_incl_i32(ne);
    if (tid < rows) roff[tid] = inc - ne;
    if (tid == rows - 1) roff[rows] = inc;
  }
  for (int wd = tid; wd < rows * wpr; wd += 256) sbits[wd] = 0u;
  __syncthreads();

  // edges: fit, first element, start bit
  const int ntot = roff[rows];
  for (int b = tid; b < ntot; b += 256) {
    int rl = 0, rh = rows - 1;  // the row of edge b: the last with roff <= b
    while (rl < rh) {
      const int mid = (rl + rh + 1) >> 1;
      if (roff[mid] <= b) rl = mid;
      else rh = mid - 1;
    }
    int first = 0;
    T val = quiet_nan<T>();
    if (!rbad[rl]) {
      const VArr v = dvarr_of(node_out(a.hulls, W, row0 + rl));
      const int j = b - roff[rl];
      const VPt p = vload<W>(v, j), q = vload<W>(v, j + 1);
      double dW, dS;
      vdiff<W>(p, q, dW, dS);
      val = tsgn * static_cast<T>(slope_div(dS, dW));
      first = p.i;
    }
    sl[b] = clip(val, use_lo, lo, use_hi, hi);
    est[b] = static_cast<int16_t>(first);
    atomicOr(&sbits[rl * wpr + (first >> 5)], 1u << (first & 31));
  }
  __syncthreads();

  // elements
  const int count = rows * n;
  const int e0 = tid * E;
  const int ecount = max(0, min(E, count - e0));
  T fit[E];
  if (ecount > 0) {
    const DivBy div(static_cast<uint32_t>(n));  // (e, n <= 2048: e * n < 2^32)
    int r = static_cast<int>(div(static_cast<uint32_t>(e0)));
    int i = e0 - r * n;
    int jl = roff[r], jh = roff[r + 1] - 1;  // the last edge of row r starting at or before i
    while (jl < jh) {
      const int mid = (jl + jh + 1) >> 1;
      if (est[mid] <= i) jl = mid;
      else jh = mid - 1;
    }
    int jj = jl;
#pragma unroll
    for (int k = 0; k < E; ++k) {
      if (k < ecount) {
        if (k > 0) {
          if (++i == n) {
            i = 0;
            jj = roff[++r];
          } else if (jj + 1 < roff[r + 1] && est[jj + 1] <= i) {
            ++jj;
          }
        }
        fit[k] = sl[jj];
        // (ragged rows: the row's own elements to their packed places)
        if (mapped && i < rml[r]) static_cast<T*>(a.out)[rmf[r] + i] = fit[k];
      }
    }
  }
  if (!mapped) store_elems_any<T, E>(static_cast<T*>(a.out) + row0 * a.n + e0, ecount, fit);
  if (a.starts != nullptr) {
    for (int wd = tid; wd < rows * wpr; wd += 256) a.starts[row0 * wpr + wd] = sbits[wd];
  }
}

// A bound on the final hulls' vertex counts: the largest over the rows of a row's vertices at
// `level` (the sum of its nodes' counts there, a row's final hull having no vertex its nodes'
// hulls lack), at most n + 1. One workgroup writes it to *out (which may be pinned host memory:
// one store); with more rows, each workgroup's maximum goes to partial[blockIdx.x] and a second
// launch of one workgroup takes the maximum of those.
constexpr int kMaxcBlocks = 256;
constexpr int64_t kMaxcRowsOne = 256 * 64;  // rows one workgroup takes alone

__device__ __forceinline__ int64_t block_max_i64(int64_t v, int64_t* sh) {
#pragma unroll
  for (int d = kWave / 2; d >= 1; d >>= 1) {
    const int64_t o = __shfl_xor(v, d, kWave);
    v = o > v ? o : v;
  }
  if ((threadIdx.x & (kWave - 1)) == 0) sh[threadIdx.x / kWave] = v;
  __syncthreads();
  int64_t m = sh[0];
#pragma unroll
  for (int k = 1; k < kWaves256; ++k) m = sh[k] > m ? sh[k] : m;
  return m;
}

// P lanes a row (a power of two up to 64, at least the row's node count where that is at most
// 64), 256 / P rows a workgroup, the workgroups striding over the rows.
__global__ __launch_bounds__(256) void maxc_rows_kernel(const int* __restrict__ count, int64_t batch, int64_t npr,
                                                        int lg_p, int64_t cap, int64_t* __restrict__ out,
                                                        int64_t* __restrict__ partial) {
  __shared__ int64_t sh[kWaves256];
  const int P = 1 << lg_p;
  const int sub = threadIdx.x & (P - 1);
  const int64_t rows_per_wg = 256 >> lg_p;
  int64_t v = 0;
  // (sixteen stretches of rows at a time, their loads in flight together: a thousand rows of a
  // few groups in one memory round trip)
  constexpr int U = 16;
  for (int64_t r0 = blockIdx.x * rows_per_wg; r0 < batch; r0 += U * rows_per_wg * gridDim.x) {
    int64_t t[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t r = r0 + u * rows_per_wg * gridDim.x + (threadIdx.x >> lg_p);
      t[u] = 0;
      if (r < batch) {
        for (int64_t j = sub; j < npr; j += P) t[u] += count[r * npr + j];
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      for (int d = P / 2; d >= 1; d >>= 1) t[u] += __shfl_xor(t[u], d, kWave);
      v = t[u] > v ? t[u] : v;
    }
  }
  const int64_t m = block_max_i64(v, sh);
  // (a store that goes to host memory directly where out is there: its caller may poll it)
  if (threadIdx.x == 0) {
    if (gridDim.x == 1) __hip_atomic_store(out, m < cap ? m : cap, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    else partial[blockIdx.x] = m;
  }
}

__global__ __launch_bounds__(256) void maxc_final_kernel(const int64_t* __restrict__ partial, int parts, int64_t cap,
                                                         int64_t* __restrict__ out) {
  __shared__ int64_t sh[kWaves256];
  int64_t v = 0;
  for (int k = threadIdx.x; k < parts; k += 256) v = partial[k] > v ? partial[k] : v;
  const int64_t m = block_max_i64(v, sh);
  if (threadIdx.x == 0) __hip_atomic_store(out, m < cap ? m : cap, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// The first hull_blocks workgroups: cpr of them a row, 256 slots each, the row's final hull
// (vertices; and, in the row's first, its count, NaN flag and totals) into the kept layout, whose
// rows hold maxc slots (a longer hull, which a wrong maxc would mean, is cut there). The others:
// the tile records, four 16-byte words a thread, every load before any store.
template <bool W>
__global__ __launch_bounds__(256) void keep_kernel(NodeLevel fin, NodeLevel kept, int64_t maxc, int64_t cpr,
                                                   int64_t hull_blocks, const uint4* __restrict__ tiles_in,
                                                   uint4* __restrict__ tiles_out, int64_t tile_words) {
  const int64_t blk = blockIdx.x;
  if (blk < hull_blocks) {
    const int64_t row = blk / cpr;
    const int64_t chunk = blk - row * cpr;
    const NodeOut s = node_out(fin, W, row);
    const NodeOut d = node_out(kept, W, row);
    const int q = static_cast<int>(chunk * 256) + threadIdx.x;
    // (the slot is read before the count is known, so the two reads overlap: slots below maxc
    // lie within the row's store, whose span0 + 1 slots a span exceed n + 1)
    HPt x{};
    if (q < maxc) {
      x.i = s.idx[q];
      x.s = s.shi[q];
      x.sl = lo_at(s.slo, q);
      if constexpr (W) {
        x.w = s.whi[q];
        x.wl = lo_at(s.wlo, q);
      }
    }
    const int cnt = static_cast<int>(min<int64_t>(*s.count, maxc));
    if (q < cnt) {
      d.idx[q] = x.i;
      put_dd(d.shi, d.slo, q, x.s, x.sl);
      if constexpr (W) put_dd(d.whi, d.wlo, q, x.w, x.wl);
    }
    if (chunk == 0) {
      if (threadIdx.x < 4) d.tot[threadIdx.x] = s.tot[threadIdx.x];
      if (threadIdx.x == 0) {
        *d.count = cnt;
        *d.bad = *s.bad;
      }
    }
    return;
  }
  const int64_t k0 = (blk - hull_blocks) * 1024 + threadIdx.x;
  uint4 v[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int64_t k = k0 + u * 256;
    if (k < tile_words) v[u] = tiles_in[k];
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int64_t k = k0 + u * 256;
    if (k < tile_words) tiles_out[k] = v[u];
  }
}

}  // namespace

LongPlan long_plan(int64_t batch, int64_t n, bool weighted, bool lo) {
  LongPlan p{};
  p.lo = lo;
  const int64_t tn = tile_elems(weighted);
  p.tiles_per_row = (n + tn - 1) / tn;
  // The longest span that still gives the span kernel about 2^17 lanes (two waves per SIMD),
  // within [kSpanMin, kSpanMax]: long spans mean fewer hulls to merge, short ones more lanes.
  int64_t span0 = kSpanMax;
  while (span0 > kSpanMin && batch * ((n + span0 - 1) / span0) < (int64_t{1} << 17)) span0 >>= 1;
  // Where spans of up to kSpanMax make a row one group, and that still leaves 2^15 lanes, take
  // them: the span kernel's group merge then finishes each row, and no merge launch follows
  // (1000 rows of 5000 float64: 150 -> 108 us). The span is the row split 64 ways (rounded up
  // to 4 elements, 16-byte aligned spans), so the wave's lanes are all busy and each span is as
  // short as one group allows (1000 rows of 5000: spans of 80 on 63 lanes, not 128 on 40;
  // float64 108 -> 93 us).
  int64_t one_group = (((n + kGroup - 1) / kGroup) + 3) & ~int64_t{3};
  if (one_group < kSpanMin) one_group = kSpanMin;
  if (one_group <= kSpanMax && (n + one_group - 1) / one_group <= kGroup && batch * ((n + one_group - 1) / one_group) >= (int64_t{1} << 15))
    span0 = span0 > one_group ? span0 : one_group;
  // Rows of at most kSpanMax elements in batches of thousands: one span per row, so the span
  // kernel runs one row per lane and 64 rows a wave (a wave per row would keep a few lanes busy;
  // 100000 rows of 64: 0.93 ms that way), and the span hulls are the final hulls.
  if (n <= kSpanMax && batch >= 8192) {
    int64_t s = kSpanMin;
    while (s < n) s <<= 1;
    span0 = span0 > s ? span0 : s;
  }
  // Rows of at most 2048 elements (which one wave's lanes cannot all share with spans of
  // kSpanMin or more): several rows a wave, k lanes each (a power of two up to 32), the smallest
  // k that gives about 2^17 lanes, each span at least 8 elements and none empty. Each row's k
  // span hulls are merged in the wave (log2 k rounds), so the span kernel finishes the rows, with
  // k times the lanes of one row per lane and no idle lanes (10000 rows of 256: 135 -> 89 us;
  // 5000 rows of 100: 87 -> 49 us, float64 weighted 148 -> 44 us).
  // Where that leaves spans longer than kSpanMin and the GPU short of lanes, one row a wave with
  // spans of kSpanMin does better (shorter spans, the same idle SIMDs); and one row a lane
  // ("packed", above) does better in batches of 32768 rows or more, or for rows of at most 64
  // elements, where the GPU has lanes enough without splitting rows (100000 rows of 128: 117 us
  // packed, 158 us two lanes a row; float64 weighted 200 and 314 us).
  p.rows_per_wave = 1;
  const bool packed_better = n <= kSpanMax && batch >= 8192 && (batch >= 32768 || n <= 64);
  if (n <= 2048 && !packed_better) {
    int64_t kmin = 1;
    while (kmin * kSpanMax < n) kmin <<= 1;
    int64_t k = kmin;
    while (k < 32 && batch * k < (int64_t{1} << 17)) k <<= 1;
    auto fits = [&](int64_t kk) {
      const int64_t s = (n + kk - 1) / kk;
      return s >= 8 && (kk - 1) * s < n;
    };
    while (k > kmin && !fits(k)) k >>= 1;
    if (k > 1 && fits(k) && ((n + k - 1) / k <= kSpanMin || batch * k >= (int64_t{1} << 17))) {
      span0 = (n + k - 1) / k;
      p.rows_per_wave = static_cast<int>(kGroup / k);
    }
  }
  p.span0 = span0;
  p.batch = batch;
  p.weighted = weighted;
  int64_t npr = (n + span0 - 1) / span0;
  int64_t span = span0;  // elements per node at this level
  int64_t spn = 1;       // spans per node at this level
  size_t off = 0;
  int level = 0;
  for (;;) {
    p.npr[level] = npr;
    p.span[level] = span;
    p.spn[level] = spn;
    p.off_meta[level] = off;
    off += align256(node_meta_bytes(batch * npr));
    if (npr == 1) break;
    npr = (npr + kGroup - 1) / kGroup;
    span *= kGroup;
    spn *= kGroup;
    ++level;
  }
  p.levels = level;  // merge launches; the final hulls are at level p.levels
  // the level whose vertex counts bound the final hulls' for a caller keeping them (ti_keep): two
  // below the final level (its merges, and then the expansion, overlap that caller's wait and
  // allocation), but not level 0, whose counts the span kernel's fused merge overwrites
  p.keep_level = p.levels <= 1 ? p.levels : std::max(1, p.levels - 2);
  p.slots = batch * p.npr[0] * (span0 + 1);
  bool any_defer = false, alt = false;
  for (int l = 0; l <= p.levels; ++l) {
    p.defer[l] = l >= 2 && batch * p.npr[l] < kDeferParents && p.span[l] >= kDeferSpan;
    if (p.defer[l]) alt = !alt;
    p.alt[l] = alt;
    any_defer = any_defer || p.defer[l];
  }
  p.off_store = off;
  off += align256(vertex_store_bytes(p.slots, weighted, lo));
  p.off_store2 = off;
  if (any_defer) off += align256(vertex_store_bytes(p.slots, weighted, lo));
  p.off_defer = off;
  if (any_defer) off += align256(static_cast<size_t>(kDeferParents) * sizeof(DeferTab));
  p.off_rank = off;
  p.off_maxc = p.off_rank + align256(static_cast<size_t>(batch * p.tiles_per_row) * sizeof(TileRec));
  p.off_rflag = p.off_maxc + align256(kMaxcBlocks * sizeof(int64_t));
  p.bytes = p.off_rflag + align256(static_cast<size_t>(batch) * sizeof(unsigned));
  return p;
}

KeepPlan keep_plan(int64_t batch, int64_t n, bool weighted, bool lo, int64_t maxc) {
  KeepPlan k{};
  k.lo = lo;
  k.batch = batch;
  k.maxc = maxc;
  k.tiles = batch * long_plan(batch, n, weighted, lo).tiles_per_row;
  size_t off = 0;
  k.off_meta = off;
  off += align256(node_meta_bytes(batch));
  k.off_store = off;
  off += align256(vertex_store_bytes(batch * maxc, weighted, lo));
  k.off_tiles = off;
  off += align256(static_cast<size_t>(k.tiles) * sizeof(TileRec));
  k.bytes = off;
  return k;
}

hipError_t long_keep(const LongPlan& p, const void* ws, const KeepPlan& k, void* kept, hipStream_t stream) {
  const NodeLevel fin = p.level(const_cast<void*>(ws), p.levels);
  const NodeLevel kl = k.level(kept);
  const int64_t words = k.tiles * static_cast<int64_t>(sizeof(TileRec) / sizeof(uint4));
  const auto* tin = reinterpret_cast<const uint4*>(static_cast<const char*>(ws) + p.off_rank);
  auto* tout = reinterpret_cast<uint4*>(static_cast<char*>(kept) + k.off_tiles);
  const int64_t cpr = (k.maxc + 255) / 256;
  const int64_t hull_blocks = k.batch * cpr;
  const int64_t grid = hull_blocks + (words + 1023) / 1024;
  if (grid > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
  if (p.weighted)
    keep_kernel<true><<<dim3(static_cast<unsigned>(grid)), dim3(256), 0, stream>>>(fin, kl, k.maxc, cpr, hull_blocks,
                                                                                tin, tout, words);
  else
    keep_kernel<false><<<dim3(static_cast<unsigned>(grid)), dim3(256), 0, stream>>>(fin, kl, k.maxc, cpr, hull_blocks,
                                                                                 tin, tout, words);
  return hipGetLastError();
}

hipError_t long_fit(const TileArgs& t, const LongPlan& p, void* ws) {
  const bool W = t.w != nullptr;
  char* base = static_cast<char*>(ws);
  const NodeLevel fin = p.level(ws, p.levels);
  // level 0: span hulls (and the first merge level, fused, where there is one)
  // Float32 data: the final hulls made convex in their stored values. Rows of one merge level
  // get theirs from the span kernel (or, for a multi-row wave's overflowing spans, the level-1
  // launch), whose waves check and repair them in place (span_fold); a final level of two or
  // more launches up has a merge workgroup for every row, which does it at its end (fold) where
  // rows are enough to spread those workgroups over the GPU (one workgroup reading a hull of
  // millions of vertices would take milliseconds); otherwise two launches after the merges do.
  const int repair_passes = (t.flags & TI_REPAIR_CHAIN) != 0 ? 0 : kRepairPasses;
  const bool span_fold = !p.lo && p.levels == 1;
  const bool fold = !p.lo && p.levels >= 2 && batch_fills_gpu(t.batch);
  // Rows of one merge level, one row a wave: the wave that builds a row's final hull also writes
  // its tile records, start bits and fit (span_expand), so no rank or expansion launch follows.
  const bool span_expand = p.levels == 1 && p.rows_per_wave == 1;
  TileRec* const recs_at = reinterpret_cast<TileRec*>(base + p.off_rank);
  hipError_t e = span_run(t, p.level(ws, 0), p.span0, p.level(ws, p.levels >= 1 ? 1 : 0), p.rows_per_wave,
                          span_fold ? 1 + repair_passes : 0, span_expand ? recs_at : nullptr);
  if (e != hipSuccess) return e;
  // the span kernel has read every weight (and set the flag if one is not positive)
  if (t.weights_read != nullptr && (e = hipEventRecord(t.weights_read, t.stream)) != hipSuccess) return e;
  // (the weights' mark: stored by the first merge launch as it starts, or by a kernel of its own
  // where no merge launch follows the span kernel)
  uint32_t* pending_mark = t.weights_mark;
  // for a caller that keeps only the final hulls: a bound on their vertex counts, from the
  // counts of level keep_level once it is merged
  auto report = [&](int l) -> hipError_t {
    if (l != p.keep_level) return hipSuccess;
    if (t.max_vertices != nullptr) {
      const NodeLevel kl = p.level(ws, l);
      int lg_p = 0;
      while (lg_p < 6 && (int64_t{1} << lg_p) < p.npr[l]) ++lg_p;
      const int64_t rows_one = kMaxcRowsOne >> lg_p;  // (a workgroup's 256 / P rows, 64 times over)
      const int parts = static_cast<int>(
          t.batch <= rows_one ? 1 : std::min<int64_t>(kMaxcBlocks, (t.batch + rows_one - 1) / rows_one));
      int64_t* partial = reinterpret_cast<int64_t*>(base + p.off_maxc);
      maxc_rows_kernel<<<dim3(parts), dim3(256), 0, t.stream>>>(reinterpret_cast<const int*>(kl.meta), t.batch,
                                                                p.npr[l], lg_p, t.n + 1, t.max_vertices, partial);
      if (parts > 1) maxc_final_kernel<<<dim3(1), dim3(256), 0, t.stream>>>(partial, parts, t.n + 1, t.max_vertices);
      const hipError_t le = hipGetLastError();
      if (le != hipSuccess) return le;
    }
    return t.hulls_ready != nullptr ? hipEventRecord(t.hulls_ready, t.stream) : hipSuccess;
  };
  if ((e = report(0)) != hipSuccess) return e;
  bool expanded = false;  // (the final merge launch expanded the rows)
  for (int l = 1; l <= p.levels; ++l) {
    // (one row a wave: the span kernel merged every group, in LDS or, where its hulls do not
    // fit, in the group's global array; a multi-row wave's overflowing spans wait for a launch)
    if (l == 1 && p.rows_per_wave == 1) {
      if ((e = report(l)) != hipSuccess) return e;
      continue;
    }
    MergeArgs m;
    m.in = p.level(ws, l - 1);
    m.out = p.level(ws, l);
    m.child_elems = p.span[l - 1];
    m.mark = pending_mark;
    m.mark_value = t.mark_value;
    pending_mark = nullptr;
    const unsigned grid = static_cast<unsigned>(t.batch * p.npr[l]);
    // Workgroup size and LDS slots by how many merges share the GPU: one wave and 768 slots
    // (64 noisy span hulls take 300-500) where there are thousands, else 256 or 1024 threads
    // and up to 56 KB of slots for the fewer, larger hulls of the upper levels.
    // (the final level of float32 data repairs its hulls in the merge launch: fold)
    const int fix = (fold || span_fold) && l == p.levels ? 1 + repair_passes : 0;
    // The final level of rows enough to fill the GPU, one workgroup a row (dense rows whose
    // bitmap, counts and a pass's edges fit the launch's LDS): the workgroup expands its row.
    // Only from the second level on: a first-level launch merges just the rows of multi-row
    // waves whose spans overflowed, the span kernel's waves having finished the others.
    const bool last_fills =
        l == p.levels && l >= 2 && batch_fills_gpu(t.batch) && grid >= 64 && t.map.rows == nullptr;
    RowExpand x{};
    x.n = t.n;
    x.out = t.out;
    x.starts = t.starts;
    x.tiles = recs_at;
    x.tpr = p.tiles_per_row;
    x.tile_n = static_cast<int>(tile_elems(W));
    x.flags = t.flags;
    x.lo = t.lo;
    x.hi = t.hi;
    const int tb = t.dtype == TI_F32 ? 4 : 8;
    DeferTab* const tab_l = p.defer[l] ? reinterpret_cast<DeferTab*>(base + p.off_defer) : nullptr;
    // (a deferring level has fewer than kDeferParents parents: a 256- or 1024-thread launch, DF)
    static_assert(kDeferParents <= 1024, "a deferring level's launch has 256 or 1024 threads");
    auto launch = [&](auto k64, auto k256, auto k1024, auto x64f, auto x256f, auto x64d, auto x256d, auto k256df,
                      auto k1024df, size_t vb) {
      const int big = static_cast<int>((56 * 1024 / vb) & ~size_t(63));
      if (grid >= 1024) {
        const size_t lds = std::max(768 * vb, repair_lds_bytes(64));
        x.lds_bytes = static_cast<int>(lds);
        if (last_fills && static_cast<int>(lds) >= expand_lds_min(t.n, 64, tb)) {
          expanded = true;
          if (tb == 4) x64f<<<dim3(grid), dim3(64), lds, t.stream>>>(m, 768, fix, x, tab_l);
          else x64d<<<dim3(grid), dim3(64), lds, t.stream>>>(m, 768, fix, x, tab_l);
        } else {
          k64<<<dim3(grid), dim3(64), lds, t.stream>>>(m, 768, fix, x, tab_l);
        }
      } else if (grid >= 64) {
        const size_t lds = std::max(big * vb, repair_lds_bytes(256));
        x.lds_bytes = static_cast<int>(lds);
        if (last_fills && static_cast<int>(lds) >= expand_lds_min(t.n, 256, tb)) {
          expanded = true;
          if (tb == 4) x256f<<<dim3(grid), dim3(256), lds, t.stream>>>(m, big, fix, x, tab_l);
          else x256d<<<dim3(grid), dim3(256), lds, t.stream>>>(m, big, fix, x, tab_l);
        } else if (tab_l != nullptr) {
          k256df<<<dim3(grid), dim3(256), lds, t.stream>>>(m, big, fix, x, tab_l);
        } else {
          k256<<<dim3(grid), dim3(256), lds, t.stream>>>(m, big, fix, x, tab_l);
        }
      } else {
        const size_t lds = std::max(big * vb, repair_lds_bytes(1024));
        if (tab_l != nullptr) k1024df<<<dim3(grid), dim3(1024), lds, t.stream>>>(m, big, fix, x, tab_l);
        else k1024<<<dim3(grid), dim3(1024), lds, t.stream>>>(m, big, fix, x, tab_l);
      }
    };
#define TI_MERGE_LAUNCH(Wv, PRv)                                                                            \
  launch(merge_kernel<Wv, PRv, 64, 4>, merge_kernel<Wv, PRv, 256, 2>, merge_kernel<Wv, PRv, 1024, 2>,           \
         merge_kernel<Wv, PRv, 64, 4, float>, merge_kernel<Wv, PRv, 256, 2, float>,                            \
         merge_kernel<Wv, PRv, 64, 4, double>, merge_kernel<Wv, PRv, 256, 2, double>,                           \
         merge_kernel<Wv, PRv, 256, 2, void, true>, merge_kernel<Wv, PRv, 1024, 2, void, true>, slot_bytes<Wv, PRv>())
    // (node arrays and slots are double-double for both dtypes: see child_vertex)
    if (W) TI_MERGE_LAUNCH(true, true);
    else TI_MERGE_LAUNCH(false, true);
#undef TI_MERGE_LAUNCH
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (tab_l != nullptr) {
      // the deferred parents' survivors: about kSurvivorBlocks workgroups over the launch's parents
      const int per = static_cast<int>(std::max<int64_t>(1, kSurvivorBlocks / grid));
      const dim3 sgrid(static_cast<unsigned>(grid * per));
      if (W) survivors_kernel<true, true><<<sgrid, dim3(256), 0, t.stream>>>(m, tab_l, per);
      else survivors_kernel<false, true><<<sgrid, dim3(256), 0, t.stream>>>(m, tab_l, per);
      e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
    if ((e = report(l)) != hipSuccess) return e;
  }
  if (pending_mark != nullptr && (e = mark_run(pending_mark, t.mark_value, t.stream)) != hipSuccess) return e;
  if (!p.lo && p.levels >= 1 && !fold && !span_fold) {
    // (float32 data: the final hulls convex in their stored values; span hulls, the final hulls
    // of rows of one span, are exact and convex already). Enough check workgroups a row for a
    // hull of every element (4096 vertices each), at most 256 a row, or about 4096 in all where
    // the rows are few (one row of 1e8 with 3.8e7 vertices: 290 us of checks at 256).
    static std::atomic<unsigned> calls{0};
    const unsigned epoch = calls.fetch_add(1, std::memory_order_relaxed) * 2u + 1u;  // (odd: never 0)
    const int64_t most = std::max<int64_t>(256, 4096 / t.batch);
    const int chunks = static_cast<int>(std::min<int64_t>(most, std::max<int64_t>(1, (t.n + 4096) / 4096)));
    unsigned* flag = reinterpret_cast<unsigned*>(base + p.off_rflag);
    const dim3 cgrid(static_cast<unsigned>(t.batch * chunks)), rgrid(static_cast<unsigned>(t.batch));
    if (W) {
      convex_check_kernel<true><<<cgrid, dim3(kRepairThreads), 0, t.stream>>>(fin, chunks, epoch, flag);
      repair_kernel<true><<<rgrid, dim3(kRepairThreads), 0, t.stream>>>(fin, epoch, flag, repair_passes);
    } else {
      convex_check_kernel<false><<<cgrid, dim3(kRepairThreads), 0, t.stream>>>(fin, chunks, epoch, flag);
      repair_kernel<false><<<rgrid, dim3(kRepairThreads), 0, t.stream>>>(fin, epoch, flag, repair_passes);
    }
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (span_expand || expanded) return hipSuccess;
  if (t.n <= kXpackMaxN) {
    // rows of one tile: records and fit together, whole rows a workgroup
    ExpandArgs x;
    x.hulls = fin;
    x.batch = t.batch;
    x.n = t.n;
    x.tiles_per_row = 1;
    x.out = t.out;
    x.starts = t.starts;
    x.tiles = nullptr;
    x.flags = t.flags;
    x.lo = t.lo;
    x.hi = t.hi;
    x.map = t.map;
    TileRec* recs = reinterpret_cast<TileRec*>(base + p.off_rank);
    auto go = [&](auto E_) {
      constexpr int E = decltype(E_)::value;
      const int rpw = 256 * E / static_cast<int>(t.n);
      const dim3 grid(static_cast<unsigned>((t.batch + rpw - 1) / rpw));
      if (t.dtype == TI_F32) {
        // (ragged rows of a block: float32 only)
        if (t.map.rows != nullptr) {
          if (W) xpack_kernel<float, true, E, true><<<grid, dim3(256), 0, t.stream>>>(x, recs, rpw);
          else xpack_kernel<float, false, E, true><<<grid, dim3(256), 0, t.stream>>>(x, recs, rpw);
        } else if (W) {
          xpack_kernel<float, true, E><<<grid, dim3(256), 0, t.stream>>>(x, recs, rpw);
        } else {
          xpack_kernel<float, false, E><<<grid, dim3(256), 0, t.stream>>>(x, recs, rpw);
        }
      } else {
        if (W) xpack_kernel<double, true, E><<<grid, dim3(256), 0, t.stream>>>(x, recs, rpw);
        else xpack_kernel<double, false, E><<<grid, dim3(256), 0, t.stream>>>(x, recs, rpw);
      }
      return hipGetLastError();
    };
    return t.n <= 1024 ? go(std::integral_constant<int, 4>{}) : go(std::integral_constant<int, 8>{});
  }
  {
    const int64_t tiles = t.batch * p.tiles_per_row;
    const dim3 grid(static_cast<unsigned>((tiles + 255) / 256));
    TileRec* recs = reinterpret_cast<TileRec*>(base + p.off_rank);
    if (W) {
      rank_kernel<true><<<grid, dim3(256), 0, t.stream>>>(fin, t.batch, t.n, tile_elems(W), p.tiles_per_row, recs);
    } else {
      rank_kernel<false><<<grid, dim3(256), 0, t.stream>>>(fin, t.batch, t.n, tile_elems(W), p.tiles_per_row, recs);
    }
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  ExpandArgs x;
  x.hulls = fin;
  x.batch = t.batch;
  x.n = t.n;
  x.tiles_per_row = p.tiles_per_row;
  x.out = t.out;
  x.starts = t.starts;
  x.tiles = reinterpret_cast<const TileRec*>(base + p.off_rank);
  x.flags = t.flags;
  x.lo = t.lo;
  x.hi = t.hi;
  x.map = t.map;
  const unsigned grid = static_cast<unsigned>((t.batch * p.tiles_per_row + kExpandTiles - 1) / kExpandTiles);
  auto go = [&](auto k) { k<<<dim3(grid), dim3(256), 0, t.stream>>>(x); };
  const bool nts = (t.flags & TI_STREAM_OUT) != 0;
  if (t.dtype == TI_F32) {
    if (t.map.rows != nullptr) {  // (ragged rows of a block: float32 only)
      if (W) go(expand_kernel<float, true, false, true>);
      else go(expand_kernel<float, false, false, true>);
    } else if (W) {
      nts ? go(expand_kernel<float, true, true>) : go(expand_kernel<float, true, false>);
    } else {
      nts ? go(expand_kernel<float, false, true>) : go(expand_kernel<float, false, false>);
    }
  } else {
    if (W) nts ? go(expand_kernel<double, true, true>) : go(expand_kernel<double, true, false>);
    else nts ? go(expand_kernel<double, false, true>) : go(expand_kernel<double, false, false>);
  }
  return hipGetLastError();
}

}  // namespace ti
