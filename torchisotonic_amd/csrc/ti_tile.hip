// Rows longer than the short-row limit: one workgroup per tile of a row.
//
// A tile is 256 threads x E consecutive elements (E = 16 unweighted, 8 weighted: 4096 or 2048
// elements). Replaces the reference's chunk stage (reference src/torchisotonic/csrc/
// tiles.cuh:665-913, chunk_kernel) with a wave64/LDS design:
//
//   1. each thread loads its E elements (16-byte loads where aligned), forms float64
//      cumulative sums of w*y and w over them, and the workgroup scans the thread totals in
//      double-double to place every thread in the tile;
//   2. each thread builds the lower hull of its E + 1 points (the same prefiltered monotone
//      chain as the short rows), stored compactly in its own LDS slots;
//   3. eight rounds of pairwise merges join the thread hulls: a leader per pair finds the
//      bridge (a walk from the shared point, or a nested binary search when the walk runs
//      long) and the pair's threads move the right hull's surviving suffix next to the left
//      hull's surviving prefix;
//   4. a row that fits in one tile is finished here: edge slopes in float64, rounded once,
//      one per thread, then every element takes the slope of its edge (clamp fused) and the
//      vertex bits become the row's start bits. A longer row writes its tile hull (double-
//      double coordinates relative to the tile) for the cross-tile merge.
//
// Coordinates: a point is (owner thread, float64 sums relative to the owner's first point);
// owners are placed by double-double offsets, so the difference of two nearby points keeps
// the precision of the difference (the cancellation that tiny weights would otherwise expose).
#include <type_traits>

#include "ti_common.h"
#include "ti_kernels.h"
#include "ti_tile.h"

namespace ti {

namespace {

template <typename T, bool W>
struct TileShared {
  using C = TileCfg<W>;
  static constexpr bool kPairs = sizeof(T) == 8;
  double ls[C::kSlots];              // cumulative w*y, relative to the point's owner thread
  double lw[W ? C::kSlots : 1];      // cumulative w, likewise (unweighted: the index)
  float ls_lo[kPairs ? C::kSlots : 1];  // float64 data: the sums' rounding errors
  float lw_lo[kPairs && W ? C::kSlots : 1];
  int16_t idx[C::kSlots];            // the point's index within the tile
  double off_s[2][C::kThreads + 1];  // owner offsets (hi, lo); [kThreads]: the tile total
  double off_w[2][W ? C::kThreads + 1 : 1];
  int cnt[C::kThreads];              // vertex count of the part led by each thread
  int keep[C::kThreads];             // per merge (by leader): vertices kept from the left part
  int from[C::kThreads];             // per merge: first vertex kept from the right part
  uint32_t bits[C::kN / 32];         // the final hull's vertices as bits (single-tile rows)
  double wsum[4][kWaves256];         // wave totals of the offset scans
  int rank_scan[kWaves256];
  int bad;
  int wbad;
};

// A point of the tile: index, and sums relative to its owner thread (index >> kLogE); for
// float64 data each sum is hi + lo (lo kept as float32 in LDS), so that the difference of
// neighbouring points is the product w*y itself.
struct Pt {
  int i;
  double w, s;
  double wl, sl;
};

template <typename T, bool W>
struct TileOps {
  using C = TileCfg<W>;
  using Sh = TileShared<T, W>;

  static constexpr bool kPairs = Sh::kPairs;

  __device__ static Pt load(const Sh& sh, int slot) {
    Pt p;
    p.i = sh.idx[slot];
    p.s = sh.ls[slot];
    p.w = W ? sh.lw[W ? slot : 0] : 0.0;
    p.sl = kPairs ? static_cast<double>(sh.ls_lo[kPairs ? slot : 0]) : 0.0;
    p.wl = (kPairs && W) ? static_cast<double>(sh.lw_lo[(kPairs && W) ? slot : 0]) : 0.0;
    return p;
  }

  __device__ static void store(Sh& sh, int slot, const Pt& p) {
    sh.idx[slot] = static_cast<int16_t>(p.i);
    sh.ls[slot] = p.s;
    if constexpr (W) sh.lw[slot] = p.w;
    if constexpr (kPairs) sh.ls_lo[slot] = static_cast<float>(p.sl);
    if constexpr (kPairs && W) sh.lw_lo[slot] = static_cast<float>(p.wl);
  }

  // b - a as (dW, dS). Across owners the terms are taken in an order that keeps the
  // cancellation exact: the owners' offset difference (exact for nearby owners), minus a's local
  // sum (exact where the two nearly cancel, as for neighbouring points), then the small terms
  // (offset and local rounding errors, b's local sum), so the result is rounded about once.
  __device__ static void diff(const Sh& sh, const Pt& a, const Pt& b, double& dW, double& dS) {
    const int oa = a.i >> C::kLogE, ob = b.i >> C::kLogE;
    if (oa == ob) {
      dS = (b.s - a.s) + (b.sl - a.sl);
      if constexpr (W) dW = (b.w - a.w) + (b.wl - a.wl);
    } else {
      const double xs = (sh.off_s[0][ob] - sh.off_s[0][oa]) - a.s;
      dS = xs + (((sh.off_s[1][ob] - sh.off_s[1][oa]) + (b.sl - a.sl)) + b.s);
      if constexpr (W) {
        const double xw = (sh.off_w[0][ob] - sh.off_w[0][oa]) - a.w;
        dW = xw + (((sh.off_w[1][ob] - sh.off_w[1][oa]) + (b.wl - a.wl)) + b.w);
      }
    }
    if constexpr (!W) dW = static_cast<double>(b.i - a.i);
  }

  // B leaves the hull through A, B, C (equal slopes pool).
  __device__ static bool pools3(const Sh& sh, const Pt& a, const Pt& b, const Pt& c) {
    double dW1, dS1, dW2, dS2;
    diff(sh, a, b, dW1, dS1);
    diff(sh, b, c, dW2, dS2);
    return pools<true>(dS1, dW1, dS2, dW2);
  }

  // Bridge of the lower hulls A = slots [ba, ba + cA) and B = [bb, bb + cB), which share their
  // boundary point (A's last = B's first). The merged hull is A[0 .. keep) ++ B[from .. cB).
  __device__ static void bridge(const Sh& sh, int ba, int cA, int bb, int cB, int& keep, int& from) {
    if (cA == 0) {  // nothing on the left (cannot happen for a non-empty row): take B
      keep = 0;
      from = 0;
      return;
    }
    if (cB <= 1 || cA == 1) {  // B is only the shared point, or A is
      keep = cA;
      from = cB <= 1 ? cB : 1;
      if (cA == 1 && cB > 1) {
        keep = 0;
        from = 0;
      }
      return;
    }
    const Pt x = load(sh, ba + cA - 1);  // the shared point
    Pt a = load(sh, ba + cA - 2);
    Pt b = load(sh, bb + 1);
    if (!pools3(sh, a, x, b)) {  // already convex there: concatenate
      keep = cA;
      from = 1;
      return;
    }
    // Walk: drop A's last kept vertex while it is on or above the segment from its
    // predecessor to B's candidate, then B's candidate while it is on or above the segment from
    // A's candidate to its successor; both only move outwards.
    int i = cA - 2, j = 1;
    constexpr int kWalk = 24;
    int steps = 0;
    bool done = false;
    Pt ap = i > 0 ? load(sh, ba + i - 1) : a;
    Pt bn = j + 1 < cB ? load(sh, bb + j + 1) : b;
    while (steps < kWalk) {
      if (i > 0 && pools3(sh, ap, a, b)) {
        --i;
        a = ap;
        if (i > 0) ap = load(sh, ba + i - 1);
      } else if (j + 1 < cB && pools3(sh, a, b, bn)) {
        ++j;
        b = bn;
        if (j + 1 < cB) bn = load(sh, bb + j + 1);
      } else {
        done = true;
        break;
      }
      ++steps;
    }
    if (!done) {
      // Nested binary search: the bridge's left end is the first i whose tangent to B[1..]
      // (the last of equal-slope touch points) leaves A[i + 1] on or above it.
      int lo = 0, hi = cA - 2;
      int jbest = 1;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        const Pt am = load(sh, ba + mid);
        const int t = tangent(sh, am, bb, cB);
        if (pools3(sh, am, load(sh, ba + mid + 1), load(sh, bb + t))) {
          hi = mid;
          jbest = t;
        } else {
          lo = mid + 1;
        }
      }
      i = lo;
      j = tangent(sh, load(sh, ba + lo), bb, cB);
      (void)jbest;
    }
    keep = i + 1;
    from = j;
  }

  // The vertex of B[1 .. cB) touched by the lower tangent from p (left of B): the first j whose
  // successor lies strictly above the line p -> B[j] (the last of equal-slope candidates).
  __device__ static int tangent(const Sh& sh, const Pt& p, int bb, int cB) {
    int lo = 1, hi = cB - 1;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (!pools3(sh, p, load(sh, bb + mid), load(sh, bb + mid + 1))) hi = mid;
      else lo = mid + 1;
    }
    return lo;
  }
};

// Inclusive double-double scan over a wave.
__device__ __forceinline__ DD wave_scan_dd(DD v, int lane) {
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    DD o;
    o.hi = __shfl_up(v.hi, d, kWave);
    o.lo = __shfl_up(v.lo, d, kWave);
    if (lane >= d) v = dd_add(o, v);
  }
  return v;
}

__device__ __forceinline__ int wave_scan_int(int v, int lane) {
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int o = __shfl_up(v, d, kWave);
    if (lane >= d) v += o;
  }
  return v;
}

template <int E>
struct LocalMask {
  using type = typename std::conditional<(E < 32), uint32_t, uint64_t>::type;
};

template <typename T, bool W, int MODE>
__global__ __launch_bounds__(256) void tile_kernel(TileArgs a) {
  using C = TileCfg<W>;
  using Sh = TileShared<T, W>;
  using Ops = TileOps<T, W>;
  constexpr int E = C::kE;
  constexpr int NT = C::kThreads;
  constexpr bool EXACT_LOCAL = W || sizeof(T) == 8;
  __shared__ Sh sh;

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int64_t tiles_per_row = (a.n + C::kN - 1) / C::kN;
  const int64_t row = blockIdx.x / tiles_per_row;
  const int64_t tile = blockIdx.x - row * tiles_per_row;
  const int64_t first = tile * C::kN;  // first element of the tile within the row
  const int len = static_cast<int>(min<int64_t>(C::kN, a.n - first));
  const int t0 = tid * E;  // first element of this thread within the tile
  const int ecount = max(0, min(E, len - t0));
  const double sgn = (a.flags & TI_INCREASING) ? 1.0 : -1.0;

  const T* y = static_cast<const T*>(a.y) + row * a.n + first;
  const T* w = W ? static_cast<const T*>(a.w) + row * a.n + first : nullptr;

  if (tid == 0) {
    sh.bad = 0;
    sh.wbad = 0;
  }

  // 1. Elements and local cumulative sums.
  T yv[E];
  T wv[W ? E : 1];
  load_elems_any<T, E>(y + t0, ecount, yv);
  if constexpr (W) load_elems_any<T, E>(w + t0, ecount, wv);
  // (float64 data: each sum also carries its rounding errors, SL / PL)
  constexpr bool PAIRS = Sh::kPairs;
  double S[E + 1], SL[PAIRS ? E + 1 : 1];
  double P[W ? E + 1 : 1], PL[PAIRS && W ? E + 1 : 1];
  bool bad = false, wbad = false;
  S[0] = 0.0;
  if constexpr (PAIRS) SL[0] = 0.0;
  if constexpr (W) P[0] = 0.0;
  if constexpr (PAIRS && W) PL[0] = 0.0;
#pragma unroll
  for (int k = 0; k < E; ++k) {
    double term = 0.0, wk = 1.0;
    if (k < ecount) {
      const double yk = sgn * static_cast<double>(yv[k]);
      bad |= yk != yk;
      if constexpr (W) {
        wk = static_cast<double>(wv[k]);
        wbad |= !(wk > 0.0);
        term = wk * yk;
      } else {
        term = yk;
      }
    } else {
      wk = 0.0;
    }
    if constexpr (PAIRS) {
      const DD t = two_sum(S[k], term);
      S[k + 1] = t.hi;
      SL[k + 1] = SL[k] + t.lo;
    } else {
      S[k + 1] = S[k] + term;
    }
    if constexpr (W) {
      if constexpr (PAIRS) {
        const DD t = two_sum(P[k], wk);
        P[k + 1] = t.hi;
        PL[k + 1] = PL[k] + t.lo;
      } else {
        P[k + 1] = P[k] + wk;
      }
    }
  }
  auto sum_s = [&](int k) -> DD { return DD{S[k], PAIRS ? SL[PAIRS ? k : 0] : 0.0}; };
  auto sum_w = [&](int k) -> DD {
    if constexpr (W) return DD{P[k], PAIRS ? PL[PAIRS ? k : 0] : 0.0};
    else return DD{static_cast<double>(k), 0.0};
  };

  // Thread offsets within the tile: exclusive double-double scans of the thread totals.
  {
    DD vs = sum_s(E);
    DD is = wave_scan_dd(vs, lane);
    DD iw{0.0, 0.0};
    if constexpr (W) iw = wave_scan_dd(sum_w(E), lane);
    __syncthreads();  // sh.bad initialised before anyone ORs into it
    if (bad) sh.bad = 1;
    if (wbad) sh.wbad = 1;
    if (lane == kWave - 1) {
      sh.wsum[0][wave] = is.hi;
      sh.wsum[1][wave] = is.lo;
      if constexpr (W) {
        sh.wsum[2][wave] = iw.hi;
        sh.wsum[3][wave] = iw.lo;
      }
    }
    __syncthreads();
    DD ps{0.0, 0.0}, pw{0.0, 0.0};
    for (int v = 0; v < wave; ++v) {
      ps = dd_add(ps, DD{sh.wsum[0][v], sh.wsum[1][v]});
      if constexpr (W) pw = dd_add(pw, DD{sh.wsum[2][v], sh.wsum[3][v]});
    }
    // exclusive = preceding waves + inclusive - own
    DD es{__shfl_up(is.hi, 1, kWave), __shfl_up(is.lo, 1, kWave)};
    if (lane == 0) es = DD{0.0, 0.0};
    es = dd_add(ps, es);
    sh.off_s[0][tid] = es.hi;
    sh.off_s[1][tid] = es.lo;
    if constexpr (W) {
      DD ew{__shfl_up(iw.hi, 1, kWave), __shfl_up(iw.lo, 1, kWave)};
      if (lane == 0) ew = DD{0.0, 0.0};
      ew = dd_add(pw, ew);
      sh.off_w[0][tid] = ew.hi;
      sh.off_w[1][tid] = ew.lo;
    }
    if (tid == NT - 1) {
      const DD ts = dd_add(ps, is);
      sh.off_s[0][NT] = ts.hi;
      sh.off_s[1][NT] = ts.lo;
      if constexpr (W) {
        const DD tw = dd_add(pw, iw);
        sh.off_w[0][NT] = tw.hi;
        sh.off_w[1][NT] = tw.lo;
      }
    }
  }

  // 2. This thread's hull, in its slots [base, base + E + 1).
  const int base = tid * (E + 1);
  using Mask = typename LocalMask<E>::type;
  int count = 0;
  if (t0 <= len) {
#pragma unroll
    for (int k = 0; k <= E; ++k) {
      if (k <= ecount) {
        sh.idx[base + k] = static_cast<int16_t>(t0 + k);
        sh.ls[base + k] = S[k];
        if constexpr (W) sh.lw[base + k] = P[k];
        if constexpr (PAIRS) sh.ls_lo[base + k] = static_cast<float>(SL[k]);
        if constexpr (PAIRS && W) sh.lw_lo[base + k] = static_cast<float>(PL[k]);
      }
    }
    Mask m = 1;
    if (ecount > 0) {
      Mask cand = Mask(1) | (Mask(1) << ecount);
#pragma unroll
      for (int k = 1; k < E; ++k) {
        const bool lt = sgn > 0.0 ? yv[k - 1] < yv[k] : yv[k] < yv[k - 1];
        if (k < ecount && lt) cand |= Mask(1) << k;
      }
      // stack: t1 (last vertex), t2, t3 (< 0: none); their points p1, p2, p3 (local sums)
      auto lpt = [&](int kk) -> Pt {
        Pt p = Ops::load(sh, base + kk);
        p.i = kk;
        return p;
      };
      auto ldiff = [&](const Pt& a0, const Pt& b0, double& dW, double& dS) {
        dS = (b0.s - a0.s) + (b0.sl - a0.sl);
        if constexpr (W) dW = (b0.w - a0.w) + (b0.wl - a0.wl);
        else dW = static_cast<double>(b0.i - a0.i);
      };
      int t1 = 0, t2 = -1, t3 = -1;
      Pt p1 = lpt(0), p2 = p1, p3 = p1;
      Mask rest = cand & ~Mask(1);
      int k = __builtin_ctz(static_cast<uint32_t>(rest));
      rest &= rest - 1;
      Pt pk = lpt(k);
      int kn = rest ? static_cast<int>(__builtin_ctz(static_cast<uint32_t>(rest))) : -1;
      Pt pkn = pk;
      if (kn >= 0) pkn = lpt(kn);
      while (k >= 0) {
        bool pop = false;
        if (t2 >= 0) {
          double dW1, dS1, dW2, dS2;
          ldiff(p2, p1, dW1, dS1);
          ldiff(p1, pk, dW2, dS2);
          pop = pools<EXACT_LOCAL>(dS1, dW1, dS2, dW2);
        }
        if (pop) {
          m &= ~(Mask(1) << t1);
          t1 = t2;
          p1 = p2;
          t2 = t3;
          p2 = p3;
          if (t3 >= 0) {
            const Mask below = m & ((Mask(1) << t3) - Mask(1));
            t3 = below ? 31 - __builtin_clz(static_cast<uint32_t>(below)) : -1;
            if (t3 >= 0) p3 = lpt(t3);
          }
        } else {
          m |= Mask(1) << k;
          t3 = t2;
          p3 = p2;
          t2 = t1;
          p2 = p1;
          t1 = k;
          p1 = pk;
          k = kn;
          pk = pkn;
          if (kn >= 0) {
            rest &= rest - 1;
            kn = rest ? static_cast<int>(__builtin_ctz(static_cast<uint32_t>(rest))) : -1;
            if (kn >= 0) pkn = lpt(kn);
          }
        }
      }
    }
    // Compact the vertices to the front of the slots; a vertex at the thread's end point is
    // stored as the next thread's first point (sums 0), its canonical form.
    Mask v = m;
    while (v) {
      const int kk = __builtin_ctz(static_cast<uint32_t>(v));
      v &= v - 1;
      Pt p = Ops::load(sh, base + kk);
      p.i = t0 + kk;
      if (kk == E) {
        p.s = p.sl = 0.0;
        p.w = p.wl = 0.0;
      }
      Ops::store(sh, base + count, p);
      ++count;
    }
  }
  sh.cnt[tid] = count;
  __syncthreads();

  // 3. Pairwise merges of the thread hulls.
  constexpr int kBuf = E / 2 + 1;
#pragma unroll 1
  for (int span = 1; span < NT; span <<= 1) {
    const int leader = tid & ~(2 * span - 1);
    const int cB = sh.cnt[leader + span];
    if (tid == leader) {
      const int cA = sh.cnt[leader];
      int keep, from;
      Ops::bridge(sh, leader * (E + 1), cA, (leader + span) * (E + 1), cB, keep, from);
      sh.keep[leader] = keep;
      sh.from[leader] = from;
      sh.cnt[leader] = keep + (cB - from);
    }
    __syncthreads();
    const int keep = sh.keep[leader];
    const int from = sh.from[leader];
    const int mlen = cB - from;
    const int r = tid - leader;
    const int src = (leader + span) * (E + 1) + from;
    const int dst = leader * (E + 1) + keep;
    const int mine = r < mlen ? (mlen - r + 2 * span - 1) / (2 * span) : 0;  // my entries
    Pt buf[kBuf];
#pragma unroll
    for (int q = 0; q < kBuf; ++q) {
      if (q < mine) buf[q] = Ops::load(sh, src + r + q * 2 * span);
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kBuf; ++q) {
      if (q < mine) Ops::store(sh, dst + r + q * 2 * span, buf[q]);
    }
    __syncthreads();
  }

  const int hull = sh.cnt[0];  // vertices of the tile's hull, at slots [0, hull)
  if (tid == 0 && sh.wbad && a.bad_weight != nullptr) *a.bad_weight = 1u;

  if constexpr (MODE == kTileSingle) {
    // 4. The row is this tile: slopes, then the fit.
    const bool row_bad = sh.bad != 0;
    // vertex bits of elements 0 .. len-1
    for (int wd = tid; wd < C::kN / 32; wd += NT) sh.bits[wd] = 0u;
    __syncthreads();
    for (int j = tid; j < hull; j += NT) {
      const int i = sh.idx[j];
      if (i < len) atomicOr(&sh.bits[i >> 5], 1u << (i & 31));
    }
    // edge slopes into registers, then over the sums they came from
    constexpr int kMaxEdges = (C::kN + NT - 1) / NT;
    double sl[kMaxEdges];
#pragma unroll
    for (int q = 0; q < kMaxEdges; ++q) {
      const int j = tid + q * NT;
      if (j + 1 < hull) {
        double dW, dS;
        Ops::diff(sh, Ops::load(sh, j), Ops::load(sh, j + 1), dW, dS);
        sl[q] = slope_div(dS, dW);
      }
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kMaxEdges; ++q) {
      const int j = tid + q * NT;
      if (j + 1 < hull) sh.ls[j] = sl[q];
    }
    // rank of this thread's first element: vertices at indices <= t0, minus one
    constexpr int kWordsPerThread = E / 32 > 0 ? E / 32 : 1;
    uint32_t mybits;
    if constexpr (E == 16) mybits = (sh.bits[t0 >> 5] >> (t0 & 31)) & 0xFFFFu;
    else mybits = (sh.bits[t0 >> 5] >> (t0 & 31)) & 0xFFu;
    (void)kWordsPerThread;
    const int pc = __builtin_popcount(mybits);
    int incl = wave_scan_int(pc, lane);
    if (lane == kWave - 1) sh.rank_scan[wave] = incl;
    __syncthreads();
    int before = incl - pc;
    for (int v = 0; v < wave; ++v) before += sh.rank_scan[v];
    // edge of element t0: (vertices with index <= t0) - 1
    int j = before + static_cast<int>(mybits & 1u) - 1;
    const bool use_lo = a.flags & TI_CLIP_MIN, use_hi = a.flags & TI_CLIP_MAX;
    const T lo = static_cast<T>(a.lo), hi = static_cast<T>(a.hi);
    const T tsgn = static_cast<T>(sgn);
    T fit[E];
#pragma unroll
    for (int k = 0; k < E; ++k) {
      if (k > 0) j += (mybits >> k) & 1u;
      const T v = row_bad ? quiet_nan<T>() : tsgn * static_cast<T>(sh.ls[j]);
      fit[k] = clip(v, use_lo, lo, use_hi, hi);
    }
    T* out = static_cast<T*>(a.out) + row * a.n + first;
    store_elems_any<T, E>(out + t0, ecount, fit);
    if (a.starts != nullptr && ecount > 0) {
      uint32_t sb = row_bad ? (t0 == 0 ? 1u : 0u) : mybits;
      if (ecount < E) sb &= (1u << ecount) - 1u;
      const int64_t wpr = (a.n + 31) / 32;
      if constexpr (E == 16) {
        uint16_t* s16 = reinterpret_cast<uint16_t*>(a.starts + row * wpr);
        s16[(first + t0) >> 4] = static_cast<uint16_t>(sb);
      } else {
        uint8_t* s8 = reinterpret_cast<uint8_t*>(a.starts + row * wpr);
        s8[(first + t0) >> 3] = static_cast<uint8_t>(sb);
      }
    }
  } else {
    // 4'. A tile of a longer row: its hull, totals and NaN flag for the cross-tile merge.
    NodeOut o = node_out(a.scratch, a.tiles_total, a.cap, W, row * tiles_per_row + tile);
    if (tid == 0) {
      *o.count = hull;
      *o.bad = sh.bad;
      o.tot[0] = sh.off_w[0][W ? NT : 0];
      o.tot[1] = W ? sh.off_w[1][NT] : 0.0;
      if constexpr (!W) o.tot[0] = static_cast<double>(len);
      o.tot[2] = sh.off_s[0][NT];
      o.tot[3] = sh.off_s[1][NT];
    }
    for (int j = tid; j < hull; j += NT) {
      const Pt p = Ops::load(sh, j);
      const int ow = p.i >> C::kLogE;
      o.idx[j] = p.i;
      const DD s = dd_add(dd_add(DD{sh.off_s[0][ow], sh.off_s[1][ow]}, p.s), p.sl);
      o.shi[j] = s.hi;
      o.slo[j] = s.lo;
      if constexpr (W) {
        const DD ww = dd_add(dd_add(DD{sh.off_w[0][ow], sh.off_w[1][ow]}, p.w), p.wl);
        o.whi[j] = ww.hi;
        o.wlo[j] = ww.lo;
      }
    }
  }
}

template <typename T, bool W>
hipError_t launch_tiles(const TileArgs& a, int mode) {
  using C = TileCfg<W>;
  const int64_t tiles = a.batch * ((a.n + C::kN - 1) / C::kN);
  if (mode == kTileSingle)
    tile_kernel<T, W, kTileSingle><<<dim3(static_cast<unsigned>(tiles)), dim3(C::kThreads), 0, a.stream>>>(a);
  else
    tile_kernel<T, W, kTileHull><<<dim3(static_cast<unsigned>(tiles)), dim3(C::kThreads), 0, a.stream>>>(a);
  return hipGetLastError();
}

}  // namespace

int64_t tile_elems(bool weighted) { return weighted ? TileCfg<true>::kN : TileCfg<false>::kN; }

hipError_t tile_run(const TileArgs& a, int mode) {
  const bool weighted = a.w != nullptr;
  if (a.dtype == TI_F32) return weighted ? launch_tiles<float, true>(a, mode) : launch_tiles<float, false>(a, mode);
  return weighted ? launch_tiles<double, true>(a, mode) : launch_tiles<double, false>(a, mode);
}

}  // namespace ti
