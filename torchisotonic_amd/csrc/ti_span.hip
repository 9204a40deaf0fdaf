// Rows longer than 32 elements, first stage: one lane per span of span0 elements.
//
// Replaces the reference's chunk stage for long rows (reference src/torchisotonic/csrc/
// tiles.cuh:665-913, chunk_kernel, which builds small lane hulls and merges them across the
// block in rounds). A lane instead runs the monotone chain over its whole span by itself: no
// block-wide scans, no merge rounds, no barriers. The span streams through registers C elements
// at a time (the next block of LC loading meanwhile), in two phases:
//
//   1. uniform work per chunk: the cumulative sums (float64, relative to the span start;
//      float64 data also carries their rounding errors, two-sum) at every point, and the
//      candidate points appended to the lane's queue of Q slots in LDS;
//   2. before each chunk, an event loop in which every lane with queued candidates does one
//      stack operation per iteration - pop the top vertex, or push its next candidate - until
//      every queue has room for the chunk. Lanes advance independently, so one lane's run of
//      pops does not hold the others at a data-dependent loop, and a lane's queue lets it fall
//      behind by up to Q candidates before the wave waits for it.
//
// The stack lives in a ring of R LDS slots per lane; positions that fall out of it go to the
// span's hull array in global memory, where the finished hull ends anyway (noisy data seldom
// gets that deep).
//
// A point is a candidate only where the data rises into it (y_{k-1} < y_k): elsewhere the slope
// into it is at least the slope out of it, and equal slopes pool, so it is never a vertex. Grids
// of at most two waves a SIMD (FILT) also drop a point that lies clearly above the chord of its
// neighbours two elements away on either side: about 0.68 loop iterations per element of noisy
// data instead of 0.98, for some twenty more float64 operations per element.
//
// Output: the span hulls as the first node array of the cross-span merge (ti_merge.hip).
#include <atomic>

#include "ti_common.h"
#include "ti_expand.h"
#include "ti_gmerge.h"
#include "ti_kernels.h"
#include "ti_slots.h"
#include "ti_tile.h"

namespace ti {

namespace {

constexpr int kSpanLanes = 64;

struct SpanArgs {
  const void* y;
  const void* w;
  uint32_t* bad_weight;
  int64_t n, spr, nodes;  // row length, spans per row, spans in total
  int64_t gpr;            // groups of kGroup spans per row (one wave each)
  int rpw;                // > 1: rows per wave, 64 / rpw spans each (spr == 64 / rpw)
  int64_t span0;          // elements per span
  unsigned flags;
  NodeLevel hulls;        // the spans' level
  NodeLevel hulls1;       // the groups' (the first merge level; with rpw > 1, the rows')
  RowMap map;             // ragged rows of one block: y and w read from the packed arrays
  // > 0: the hulls this kernel merges are the rows' final hulls of float32 data, which the wave
  // then makes convex in their stored values (repair_row, fix - 1 removal passes before its
  // chain), so that no check launch follows
  int fix;
  // (rows of one merge level, one row a wave) the wave expands its row's final hull itself: the
  // fit, the start bits (if asked for) and the tile records, in place of the rank and expansion
  // launches
  bool expand;
  RowExpand xp;
  // (where given) mark_value stored to *mark by the kernel's first thread as it starts: the
  // caller's mark that a kernel before this one has read every weight
  uint32_t* mark;
  uint32_t mark_value;
};

// Per lane (columns [slot][lane], so lanes never share a bank row): the candidate queue (index
// and sums of each queued point) and the stack ring. Arrays a configuration does not use have
// no rows (a zero-length array, which only code under a false `if constexpr` or condition names).
template <typename T, bool W, int Q, int R>
struct SpanLds {
  static constexpr bool PR = sizeof(T) == 8;
  int qi[Q][kSpanLanes];
  double qs[Q][kSpanLanes];
  double qsl[PR ? Q : 0][kSpanLanes];
  double qw[W ? Q : 0][kSpanLanes];
  double qwl[W && PR ? Q : 0][kSpanLanes];
  int ri[R][kSpanLanes];
  double rs[R][kSpanLanes];
  double rsl[PR ? R : 0][kSpanLanes];
  double rw[W ? R : 0][kSpanLanes];
  double rwl[W && PR ? R : 0][kSpanLanes];
  // Weighted float32 runs two waves a SIMD (its registers allow no more), so eight waves share
  // a CU's 160 KB of LDS: the rest of a wave's 20 KB becomes merge slots for the group's merge
  // (C4's groups need up to about 420 slots).
  char pad[(W && !PR) ? 20480 - (Q + R) * (4 + 8 * 2) * kSpanLanes : 0];
};

// N consecutive values at byte offset `off` of a buffer resource, 16 bytes per load. Reads past
// the resource's end return zero and never fault, so a block is always loaded whole (its values
// past the span's end are never used) and the loads stay straight-line code.
template <typename T, int N>
__device__ __forceinline__ void load_block(__amdgpu_buffer_rsrc_t r, uint32_t off, T (&v)[N]) {
  constexpr int V = 16 / sizeof(T);
  using VT = T __attribute__((ext_vector_type(V)));
#pragma unroll
  for (int j = 0; j < N / V; ++j) {
    // (taken as a vector of T at once: element access on the builtin's integer-vector result
    // is what this compiler narrows to a single-dword load)
    const VT x = __builtin_bit_cast(VT, __builtin_amdgcn_raw_buffer_load_b128(r, off + j * 16, 0, 0));
#pragma unroll
    for (int t = 0; t < V; ++t) v[j * V + t] = x[t];
  }
}

template <typename T, bool W, int C, int Q, int R, int LC, bool INC, bool MAP = false, bool FILT = false>
__global__ __launch_bounds__(kSpanLanes) void span_kernel(SpanArgs a) {
  static_assert((R & (R - 1)) == 0 && (Q & (Q - 1)) == 0 && R >= 4, "ring and queue slots: powers of two");
  static_assert(C < Q, "a chunk's candidates fit the queue");
  static_assert(LC % C == 0, "a load block is a whole number of chunks");
  // PR: the span's own sums carry their rounding errors (float64 data). Within a span every
  // test and every later slope uses the same span-relative coordinates, so float32 data needs
  // none there; but a span's vertices moved into a larger frame (the group's, the row's) keep
  // the translation's low part whatever the dtype (the merge slots and node arrays are always
  // double-double): re-rounded there, a hull the span found convex can turn non-convex where
  // sums cancel, and the fit would step down.
  constexpr bool PR = sizeof(T) == 8;
  static_assert(kSpanLanes == kGroup, "a wave's spans are one group of the first merge level");
  __shared__ SpanLds<T, W, Q, R> L;
  const int lane = threadIdx.x;
  if (a.mark != nullptr && blockIdx.x == 0 && lane == 0)
    __hip_atomic_store(a.mark, a.mark_value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  // One wave per group of kGroup spans of one row (fewer at the row's end: the other lanes idle);
  // where a row is one span (spr == 1), one row per lane and 64 rows a wave ("packed"): each
  // span's hull is then its row's final hull, and there is nothing to merge; with rpw > 1, rpw
  // rows a wave of kl = 64 / rpw spans each ("multi"), every span non-empty: the wave merges
  // each row's spans into the row's hull.
  const bool packed = a.spr == 1;
  const bool multi = a.rpw > 1;
  const int kl = kSpanLanes / a.rpw;  // (multi) lanes, and spans, per row
  const int64_t batch = a.nodes / a.spr;
  const int64_t row = packed  ? static_cast<int64_t>(blockIdx.x) * kSpanLanes + lane
                      : multi ? static_cast<int64_t>(blockIdx.x) * a.rpw + lane / kl
                              : blockIdx.x / a.gpr;
  const int64_t grp = packed || multi ? 0 : blockIdx.x - row * a.gpr;
  const int64_t span = packed ? 0 : multi ? lane % kl : grp * kSpanLanes + lane;
  const bool active = packed || multi ? row < batch : span < a.spr;
  const int nch = multi ? static_cast<int>(min<int64_t>(a.rpw, batch - static_cast<int64_t>(blockIdx.x) * a.rpw)) * kl
                        : static_cast<int>(min<int64_t>(kSpanLanes, a.spr - grp * kSpanLanes));
  const int64_t node = packed ? (active ? row : 0) : active ? row * a.spr + span : 0;
  const int64_t first = span * a.span0;
  const int len = active ? static_cast<int>(min<int64_t>(a.span0, a.n - first)) : 0;
  constexpr double sgn = INC ? 1.0 : -1.0;
  // Ragged rows (MAP, a.map): the lane's row in the packed arrays, and rlim, the span's elements
  // that are the row's own; from rlim on the span holds the pad (weight 1), made in registers: a
  // block wholly past rlim is never read (its loads take an offset past the buffer's end, which
  // returns zeros without a memory access).
  constexpr bool mapped = MAP;
  int64_t mfirst = 0, mlen = a.n;
  if constexpr (MAP) map_row(a.map, active ? row : 0, a.n, mfirst, mlen);
  const int rlim = MAP ? static_cast<int>(max<int64_t>(mlen - first, 0)) : 0x7FFFFFFF;
  const T tpad = static_cast<T>(a.map.pad);
  // The wave's spans are consecutive elements (of one row, or of its rows), so one buffer
  // resource based at the first of them serves every lane.
  // (from the wave's own indices only, and read from the first lane: the compiler then keeps
  // the buffer resources in scalar registers, where a per-lane value would put every load in a
  // loop over the lanes' distinct resources)
  // (ragged rows: one resource over the whole packed arrays, under 2 GB)
  const int64_t wrow = static_cast<int64_t>(blockIdx.x) / a.gpr;  // (one row a wave: its row)
  const int64_t base = wave_uniform(mapped  ? int64_t{0}
                                    : packed ? static_cast<int64_t>(blockIdx.x) * kSpanLanes * a.n
                                    : multi  ? static_cast<int64_t>(blockIdx.x) * a.rpw * a.n
                                             : wrow * a.n + (blockIdx.x - wrow * a.gpr) * kSpanLanes * a.span0);
  const int64_t total = mapped ? a.map.total : batch * a.n;  // elements of the arrays
  const __amdgpu_buffer_rsrc_t ry = make_rsrc(static_cast<const T*>(a.y) + base, (total - base) * sizeof(T));
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(W ? static_cast<const T*>(a.w) + base : a.y, (total - base) * sizeof(T));
  // this lane's span (packed: its row) as an element index in the wave's sequence of elements,
  // and its place in memory, an element offset from base
  const int64_t lel = packed ? lane * a.n : multi ? (lane / kl) * a.n + first : lane * a.span0;
  const int64_t lmem = mapped ? mfirst + first : lel;
  // block b's byte offset (a block wholly past rlim: past the resource, never read)
  auto boff = [&](int b) -> uint32_t {
    if constexpr (!MAP) return static_cast<uint32_t>((lmem + b) * static_cast<int64_t>(sizeof(T)));
    return b < rlim ? static_cast<uint32_t>((lmem + b) * static_cast<int64_t>(sizeof(T))) : 0x80000000u;
  };
  const NodeOut o = node_out(a.hulls, W, node);

  auto ring_put = [&](int q, const HPt& p) {
    const int r = q & (R - 1);
    L.ri[r][lane] = p.i;
    L.rs[r][lane] = p.s;
    if constexpr (PR) L.rsl[r][lane] = p.sl;
    if constexpr (W) L.rw[r][lane] = p.w;
    if constexpr (W && PR) L.rwl[r][lane] = p.wl;
  };
  auto ring_get = [&](int q) -> HPt {
    const int r = q & (R - 1);
    HPt p;
    p.i = L.ri[r][lane];
    p.s = L.rs[r][lane];
    p.sl = PR ? L.rsl[PR ? r : 0][lane] : 0.0;
    p.w = W ? L.rw[W ? r : 0][lane] : 0.0;
    p.wl = (W && PR) ? L.rwl[(W && PR) ? r : 0][lane] : 0.0;
    return p;
  };
  // node arrays hold double-double sums; float32 data has no rounding errors to carry (lo = 0)
  auto node_put = [&](int q, const HPt& p) {
    o.idx[q] = p.i;
    put_dd(o.shi, o.slo, q, p.s, p.sl);
    if constexpr (W) put_dd(o.whi, o.wlo, q, p.w, p.wl);
  };
  auto node_get = [&](int q) -> HPt {
    HPt p;
    p.i = o.idx[q];
    p.s = o.shi[q];
    p.sl = PR ? lo_at(o.slo, q) : 0.0;
    p.w = W ? o.whi[q] : 0.0;
    p.wl = (W && PR) ? lo_at(o.wlo, q) : 0.0;
    return p;
  };

  auto q_put = [&](int q, const HPt& p) {
    const int r = q & (Q - 1);
    L.qi[r][lane] = p.i;
    L.qs[r][lane] = p.s;
    if constexpr (PR) L.qsl[r][lane] = p.sl;
    if constexpr (W) L.qw[r][lane] = p.w;
    if constexpr (W && PR) L.qwl[r][lane] = p.wl;
  };
  auto q_get = [&](int q) -> HPt {
    const int r = q & (Q - 1);
    HPt p;
    p.i = L.qi[r][lane];
    p.s = L.qs[r][lane];
    p.sl = PR ? L.qsl[PR ? r : 0][lane] : 0.0;
    p.w = W ? L.qw[W ? r : 0][lane] : 0.0;
    p.wl = (W && PR) ? L.qwl[(W && PR) ? r : 0][lane] : 0.0;
    return p;
  };

  // The stack holds positions [0, depth): [r0, depth) in the ring (1 <= depth - r0 <= R), [0, r0)
  // in the node array. The queue holds the candidates [qh, qt).
  int depth = 1, r0 = 0;
  ring_put(0, HPt{0, 0.0, 0.0, 0.0, 0.0});
  int qh = 0, qt = 0;

  double S = 0.0, SL = 0.0, P = 0.0, PL = 0.0;
  bool bad = false, wbad = false;
  // 2. one stack operation per lane and iteration - pop the top vertex B, or push the first
  // queued candidate c - until every lane holds at most `limit` queued candidates. An iteration's
  // reads depend on the previous iteration's depth and queue position only, and its one ring
  // write needs no branch: a push writes c above B, any other lane writes B back into its own
  // slot (a pop frees it next). The loop touches LDS only (and stores spills), so the next loads
  // stay in flight; a lane whose second vertex went to the node array makes the wave leave it,
  // refill that lane's ring from the node array, and come back (rare).
  // (at a raised issue priority: a wave in its chain wins the SIMD over the other wave's uniform
  // chunk work, so the chains, the kernel's bound, wait less; C4 forward 0.522 -> 0.517 ms, C5
  // 0.321 -> 0.318 ms)
  auto run = [&](int limit) {
    __builtin_amdgcn_s_setprio(1);
    for (;;) {
      while (__any(qt - qh > limit)) {
        const bool act = qt != qh;
        const bool two = act && depth >= 2;
        if (__any(two && depth - 2 < r0)) break;
        const HPt c = q_get(qh);
        const HPt A = ring_get(depth - 2), B = ring_get(depth - 1);
        // pools(A, B, c): a filtered fma test, exact where it cannot decide (see pools<true>)
        double dS1 = B.s - A.s, dS2 = c.s - B.s, dW1, dW2;
        if constexpr (PR) {
          dS1 += B.sl - A.sl;
          dS2 += c.sl - B.sl;
        }
        if constexpr (W) {
          dW1 = B.w - A.w;
          dW2 = c.w - B.w;
          if constexpr (PR) {
            dW1 += B.wl - A.wl;
            dW2 += c.wl - B.wl;
          }
        } else {
          dW1 = static_cast<double>(B.i - A.i);
          dW2 = static_cast<double>(c.i - B.i);
        }
        const double qq = dS2 * dW1;
        const double dd = __builtin_fma(dS1, dW2, -qq);
        const bool close = !(__builtin_fabs(dd) > 0x1p-52 * __builtin_fabs(qq));
        bool pop = two && dd > 0.0;
        if (__any(two && close)) {
          // (an empty statement with side effects: it keeps this rare path a branch, where the
          // compiler would otherwise compute the exact test in every iteration and select)
          asm volatile("");
          if (two && close) pop = cross_sign(dS1, dW2, dS2, dW1) >= 0;
        }
        const bool push = act && !pop;
        if (__any(push && depth - r0 == R)) {
          // a full ring: its oldest position leaves for the node array
          asm volatile("");
          if (push && depth - r0 == R) {
            node_put(r0, ring_get(r0));
            ++r0;
          }
        }
        ring_put(push ? depth : depth - 1, hsel(push, c, B));
        depth += push ? 1 : (pop ? -1 : 0);
        qh += push ? 1 : 0;
      }
      if (!__any(qt - qh > limit)) break;
      if (qt != qh && depth >= 2 && depth - 2 < r0) {
        // only the top is in the ring (depth - 1 == r0): bring back up to R / 2 positions below
        const int lo = r0 > R / 2 ? r0 - R / 2 : 0;
        for (int q = lo; q < r0; ++q) ring_put(q, node_get(q));
        r0 = lo;
      }
    }
    __builtin_amdgcn_s_setprio(0);
  };

  // loads come in blocks of LC elements (the next block in flight while this one is processed),
  // processed in chunks of C: before a chunk, the loop makes room in every queue for its
  // candidates
  T yc[LC], yn[LC];
  T wc[W ? LC : 1], wn[W ? LC : 1];
  load_block<T, LC>(ry, boff(0), yc);
  if constexpr (W) load_block<T, LC>(rw, boff(0), wc);
  // FILT: a point is queued one element late, for the stronger test below, which needs the
  // element after it. Carried from element to element: the last three elements' terms (t1 the
  // newest), their weights and signed values, the running sum of |term| (the rounding margin's
  // scale), and the sums of the point waiting to be queued.
  double t1 = 0.0, t2 = 0.0, t3 = 0.0, w1 = 1.0, w2 = 1.0, w3 = 1.0, v1 = 0.0, v2 = 0.0, A = 0.0;
  HPt pend{0, 0.0, 0.0, 0.0, 0.0};
  // (FILT) Point e - 1 (between elements e - 2 and e - 1; e the element just summed, its term t0
  // and weight w0) is a candidate where the data rises into it (v2 < v1) and it does not lie
  // above the chord from point e - 3 to point e (b, from e >= 3) or from point e - 2 to point
  // e + 1 (c, where e is in the span). Such a point is no vertex of the exact hull; it is dropped
  // only where its height above the chord exceeds 2^-39 x A x the chord's width, which bounds
  // what the rounding of the span's sums (and of this test) can move, so that near-ties stay
  // candidates and the event loop decides them as without the test.
  auto keep = [&](bool use_b, bool use_c, double t0, double w0) {
    const double thr = A * 0x1p-39;
    bool k = v2 < v1;
    if constexpr (W) {
      const double d3 = w3 + w2;
      const double db = __builtin_fma(t3 + t2, w1, -(t1 * d3));
      const double wc1 = w1 + w0;
      const double dc = __builtin_fma(t2, wc1, -((t1 + t0) * w2));
      k &= !(use_b && db > thr * (d3 + w1));
      k &= !(use_c && dc > thr * (w2 + wc1));
    } else {
      const double db = (t3 + t2) - 2.0 * t1;
      const double dc = 2.0 * t2 - (t1 + t0);
      k &= !(use_b && db > 3.0 * thr);
      k &= !(use_c && dc > 3.0 * thr);
    }
    return k;
  };
  for (int b0 = 0; b0 < len; b0 += LC) {
    // the next block, whole, whether or not the span reaches it
    load_block<T, LC>(ry, boff(b0 + LC), yn);
    if constexpr (W) load_block<T, LC>(rw, boff(b0 + LC), wn);
    // (ragged rows: the pad past the row's end, in the one block a lane's row ends in or after)
    if (MAP && __any(b0 + LC > rlim)) {
#pragma unroll
      for (int k = 0; k < LC; ++k) {
        if (b0 + k >= rlim) {
          yc[k] = tpad;
          if constexpr (W) wc[W ? k : 0] = T(1);
        }
      }
    }
    // the element after the block: the next block's first, or the pad
    auto after_block = [&]() { return MAP && b0 + LC >= rlim ? tpad : yn[0]; };
#pragma unroll
    for (int sub = 0; sub < LC; sub += C) {
      const int c0 = b0 + sub;
      run(Q - C);
      // 1. sums at every point of the chunk; each point goes to the queue's next free slot,
      // which it keeps if it is a candidate (so the stores need no branch). Without FILT, point
      // e + 1 as element e is summed, a candidate where y rises into element e + 1 (or at the
      // span's end); with FILT, point e - 1.
      auto element = [&](int k, bool cand) {
        const int e = c0 + k;
        const double ye = sgn * static_cast<double>(yc[sub + k]);
        bad |= ye != ye;
        double term = ye, we = 1.0;
        if constexpr (W) {
          we = static_cast<double>(wc[W ? sub + k : 0]);
          wbad |= !(we > 0.0);
          term = we * ye;
        }
        if constexpr (FILT) {
          A += __builtin_fabs(term);
          const bool kept = e >= 2 && keep(e >= 3, true, term, we);
          q_put(qt, pend);
          qt += kept ? 1 : 0;
          pend = HPt{e, S, PR ? SL : 0.0, W ? P : 0.0, (W && PR) ? PL : 0.0};
        }
        if constexpr (W) {
          if constexpr (PR) {
            const DD t = two_sum(P, we);
            P = t.hi;
            PL += t.lo;
          } else {
            P += we;
          }
        }
        if constexpr (PR) {
          const DD t = two_sum(S, term);
          S = t.hi;
          SL += t.lo;
        } else {
          S += term;
        }
        if constexpr (FILT) {
          t3 = t2;
          t2 = t1;
          t1 = term;
          w3 = w2;
          w2 = w1;
          w1 = we;
          v2 = v1;
          v1 = ye;
        } else {
          q_put(qt, HPt{e + 1, S, PR ? SL : 0.0, W ? P : 0.0, (W && PR) ? PL : 0.0});
          qt += cand ? 1 : 0;
        }
      };
      // the point after element e is a candidate where y rises into e + 1, or at the span's end
      auto rises = [&](T u, T v) { return INC ? u < v : v < u; };
      if (__all(c0 + C <= len)) {
        // whole chunks (all but a row's last span): no per-element bounds
#pragma unroll
        for (int k = 0; k < C; ++k) {
          if constexpr (FILT) {
            element(k, false);
          } else {
            const int kk = sub + k;
            const T ynext = kk + 1 < LC ? yc[kk + 1 < LC ? kk + 1 : 0] : after_block();
            // (the span can end only after a chunk's last element here)
            element(k, k + 1 < C ? rises(yc[kk], ynext) : ((c0 + C == len) | rises(yc[kk], ynext)));
          }
        }
      } else {
#pragma unroll
        for (int k = 0; k < C; ++k) {
          const int e = c0 + k;
          if (e < len) {
            if constexpr (FILT) {
              element(k, false);
            } else {
              const int kk = sub + k;
              const T ynext = kk + 1 < LC ? yc[kk + 1 < LC ? kk + 1 : 0] : after_block();
              element(k, (e + 1 == len) | (e + 1 < len && rises(yc[kk], ynext)));
            }
          }
        }
      }
    }
#pragma unroll
    for (int k = 0; k < LC; ++k) {
      yc[k] = yn[k];
      if constexpr (W) wc[W ? k : 0] = wn[W ? k : 0];
    }
  }
  if constexpr (FILT) {
    // the span's last two points: point len - 1 (tests a and b: there is no point len + 1), and
    // the span's end, always a vertex
    run(Q - 2);
    if (len >= 1) {
      const bool kept = len >= 2 && keep(len >= 3, false, 0.0, 1.0);
      q_put(qt, pend);
      qt += kept ? 1 : 0;
      q_put(qt, HPt{len, S, PR ? SL : 0.0, W ? P : 0.0, (W && PR) ? PL : 0.0});
      ++qt;
    }
  }
  // the last candidates
  run(0);
  if (W && wbad && a.bad_weight != nullptr) *a.bad_weight = 1u;

  // The span's hull, whole, to the span array (for the merge kernel, or as the row's final hull)
  auto write_span_hull = [&]() {
    if (active) {
      for (int q = r0; q < depth; ++q) node_put(q, ring_get(q));
      *o.count = depth;
      *o.bad = bad ? 1 : 0;
      o.tot[0] = W ? P : static_cast<double>(len);
      o.tot[1] = W ? PL : 0.0;
      o.tot[2] = S;
      o.tot[3] = SL;
    }
  };
  if (packed) {  // the row's hull is final
    write_span_hull();
    return;
  }
  // A final hull of float32 data convex in its stored values (a.fix): once every lane has
  // written it, the wave checks it and, where a vertex lies on or above its neighbours' chord,
  // repairs it in place, with the wave's LDS (free by then) for the repair's staging.
  auto fold = [&](const NodeOut& h, bool row_bad) {
    if constexpr (!PR) {
      if (a.fix != 0 && !row_bad) {
        __syncthreads();  // the hull written by every lane, the LDS read
        VPt* tile = reinterpret_cast<VPt*>(&L);
        int* wcount = reinterpret_cast<int*>(tile + kSpanLanes + 2);
        repair_row<W, kSpanLanes>(h, tile, wcount, wcount[kSpanLanes / kWave], a.fix - 1);
      }
    }
  };
  // The row's final hull h expanded by the wave (a.expand; one row a wave, the group the whole
  // row), in place of the rank and expansion launches, with the wave's LDS (free by then).
  // (rows of one group: n <= 64 spans of kSpanMax, so the bitmap and the word counts take at
  // most 4 KB, and the table holds thousands of edges, past the 1024 a pass can need)
  static_assert(expand_lds_min(kGroup * kSpanMax, kSpanLanes, sizeof(T)) <= static_cast<int>(sizeof(SpanLds<T, W, Q, R>)),
                "bitmap, counts and a pass's edges fit the wave's LDS");
  auto expand = [&](const NodeOut& h, bool row_bad) {
    RowExpand x = a.xp;
    x.lds_bytes = static_cast<int>(sizeof(L));
    expand_row<T, W, MAP, kSpanLanes>(x, h, row_bad, row, reinterpret_cast<char*>(&L));
  };

  // The group's merge (the first merge level), in the wave's own LDS when the spans' hulls fit:
  // lane c's hull is child c, positions [0, depth), its first point shared with lane c - 1 - but
  // a row's first lane (multi: every kl-th) stores its first point itself. Each row has a frame
  // of its own, from its first point: one shared by the wave's rows would hold a row's sums
  // beside all earlier rows' totals, whose rounding (up to half an ulp of the largest)
  // double-double cannot keep apart from the row's own sums where magnitudes differ by 2^50 or
  // more.
  const bool rfirst = (lane & (kl - 1)) == 0;
  const int own = active ? (rfirst ? depth : depth - 1) : 0;
  // (a row holding a NaN: its fit is NaN whatever its hull, and the backward needs only its
  // weights; its sums are taken as 0, its weights kept)
  bool zero_s = false;
  if (multi) {
    const uint64_t bm = __ballot(active && bad);
    const uint64_t kmask = kl == 64 ? ~uint64_t{0} : ((uint64_t{1} << kl) - 1);
    zero_s = ((bm >> ((lane / kl) * kl)) & kmask) != 0;
  }
  const DD vw = active ? DD{W ? P : static_cast<double>(len), W ? PL : 0.0} : DD{0.0, 0.0};
  const DD vs = active && !zero_s ? DD{S, SL} : DD{0.0, 0.0};
  const DD iw = multi ? seg_incl_dd(vw, kl) : wave_incl_dd(vw);
  const DD is = multi ? seg_incl_dd(vs, kl) : wave_incl_dd(vs);
  const int islot = wave_incl_i32(own);
  const int nslots = __builtin_amdgcn_readlane(islot, kSpanLanes - 1);
  // (the round state first, then the slots, in the wave's LDS)
  constexpr size_t kRoundBytes = (sizeof(MergeRounds) + 63) & ~size_t(63);
  constexpr int kCap =
      static_cast<int>((sizeof(SpanLds<T, W, Q, R>) - kRoundBytes) / slot_bytes<W, true>());
  static_assert(kCap >= 256, "the wave's LDS holds a group's noisy hulls");
  static_assert(!(W && !PR) || sizeof(SpanLds<T, W, Q, R>) == 20480, "weighted float32: 20 KB a wave");
  if (nslots > kCap) {
    // Too many vertices for the wave's LDS: the spans' hulls go to the span array, and (one row
    // a wave) the group merges them there by reference to them (merge_global, its round state in
    // the wave's LDS, free now), so that no merge launch is needed for the first level; a
    // multi-row wave's spans are merged by the merge kernel.
    write_span_hull();
    if (multi) return;
    const DD pw = wave_shr1_dd(iw), ps = wave_shr1_dd(is);
    const bool gbad = __any(active && bad);
    __syncthreads();  // (every lane's hull written, and its ring read, before the LDS is reused)
    char* const gm = reinterpret_cast<char*>(&L);
    MergeSmall& sm = *reinterpret_cast<MergeSmall*>(gm);
    MergeRanges& mr = *reinterpret_cast<MergeRanges*>(gm + ((sizeof(MergeSmall) + 63) & ~size_t(63)));
    static_assert(((sizeof(MergeSmall) + 63) & ~size_t(63)) + sizeof(MergeRanges) <= sizeof(SpanLds<T, W, Q, R>),
                  "the global merge's round state fits the wave's LDS");
    if (lane < nch) {
      sm.cnt[lane] = depth;
      sm.tot[0][lane] = lane == 0 ? 0.0 : pw.hi;
      sm.tot[1][lane] = lane == 0 ? 0.0 : pw.lo;
      sm.tot[2][lane] = lane == 0 ? 0.0 : ps.hi;
      sm.tot[3][lane] = lane == 0 ? 0.0 : ps.lo;
    }
    if (lane == nch - 1) {
      sm.tot[0][nch] = iw.hi;
      sm.tot[1][nch] = iw.lo;
      sm.tot[2][nch] = is.hi;
      sm.tot[3][nch] = is.lo;
    }
    __syncthreads();
    MergeArgs ma;
    ma.in = a.hulls;
    ma.out = a.hulls1;
    ma.child_elems = a.span0;
    const NodeOut gout = node_out(a.hulls1, W, blockIdx.x);
    merge_global<W, true, kSpanLanes>(ma, sm, mr.rlo, mr.rhi, mr.pre, row, grp * kSpanLanes, nch, gout);
    if (lane == 0) {
      *gout.bad = gbad ? 1 : 0;
      gout.tot[0] = sm.tot[0][nch];
      gout.tot[1] = sm.tot[1][nch];
      gout.tot[2] = sm.tot[2][nch];
      gout.tot[3] = sm.tot[3][nch];
      *o.count = -1;  // (the group is merged: its first span's count says so to the merge kernel)
    }
    fold(gout, gbad);
    if (a.expand) expand(gout, gbad);
    return;
  }
  // offsets of this lane's span within its row (the group's, or multi: its row's)
  // (the shifts in every lane first: a cross-lane read inside the select would run with the
  // row-first lanes switched off, and their right neighbours would read nothing from them)
  const DD zero{0.0, 0.0}, pw_all = wave_shr1_dd(iw), ps_all = wave_shr1_dd(is);
  const DD ew = rfirst ? zero : pw_all, es = rfirst ? zero : ps_all;
  const int off = islot - own;
  // (indices: positions in the wave's elements, each row's rebased from its first point below)
  const int lidx = static_cast<int>(lel);
  const bool anybad = __any(active && bad);
  auto to_group = [&](HPt p) {
    p.i += lidx;
    const DD Sd = dd_add(es, zero_s ? DD{0.0, 0.0} : DD{p.s, p.sl});
    p.s = Sd.hi;
    p.sl = Sd.lo;
    if constexpr (W) {
      const DD Wd = dd_add(ew, DD{p.w, p.wl});
      p.w = Wd.hi;
      p.wl = Wd.lo;
    }
    return p;
  };
  // the ring into registers first: the slots take over the wave's LDS
  HPt rv[R];
#pragma unroll
  for (int k = 0; k < R; ++k) rv[k] = ring_get(r0 + k);
  char* const mem = reinterpret_cast<char*>(&L);
  MergeRounds& rs = *reinterpret_cast<MergeRounds*>(mem);
  const Slots<W, true> v = slots_carve<W, true>(mem + kRoundBytes, kCap);
  const int q0 = rfirst ? 0 : 1;  // the first point of a later span is its left neighbour's last
  if (active) {
    for (int q = q0; q < r0; ++q) {
      const int sl = off + q - q0;
      sput(v, sl, to_group(node_get(q)));
      v.cid[sl] = static_cast<uint8_t>(lane);
    }
#pragma unroll
    for (int k = 0; k < R; ++k) {
      const int q = r0 + k;
      if (q >= q0 && q < depth) {
        const int sl = off + q - q0;
        sput(v, sl, to_group(rv[k]));
        v.cid[sl] = static_cast<uint8_t>(lane);
      }
    }
    rs.seg[0][lane] = off + own - 1;
  }
  __syncthreads();
  if (multi) {
    // log2(kl) rounds merge each row's spans and no further: segment r is then row r's hull,
    // slots [seg[r - 1] + 1, seg[r]] (slot 0 for row 0), in the row's own frame
    const int lgk = __builtin_ctz(kl);
    merge_rounds<W, true, kSpanLanes, 2>(v, rs, nslots, nch, lgk, lgk);
    const int* se = rs.seg[lgk & 1];
    const uint64_t badm = __ballot(active && bad);
    const uint64_t kmask = kl == 64 ? ~uint64_t{0} : ((uint64_t{1} << kl) - 1);
    for (int r = 0; r < nch / kl; ++r) {
      const int f = r == 0 ? 0 : se[r - 1] + 1;
      const int cnt = se[r] - f + 1;
      const NodeOut pout = node_out(a.hulls1, W, static_cast<int64_t>(blockIdx.x) * a.rpw + r);
      const HPt x0 = sget(v, f);
      auto rebase = [&](HPt x) {
        x.i -= x0.i;
        const DD Sd = dd_add(DD{x.s, x.sl}, DD{-x0.s, -x0.sl});
        x.s = Sd.hi;
        x.sl = Sd.lo;
        if constexpr (W) {
          const DD Wd = dd_add(DD{x.w, x.wl}, DD{-x0.w, -x0.wl});
          x.w = Wd.hi;
          x.wl = Wd.lo;
        }
        return x;
      };
      for (int q = lane; q < cnt; q += kSpanLanes) {
        const HPt x = q == 0 ? HPt{0, 0.0, 0.0, 0.0, 0.0} : rebase(sget(v, f + q));
        pout.idx[q] = x.i;
        put_dd(pout.shi, pout.slo, q, x.s, x.sl);
        if constexpr (W) put_dd(pout.whi, pout.wlo, q, x.w, x.wl);
      }
      if (lane == 0) {
        const HPt e = rebase(sget(v, se[r]));  // the row's end point: its totals
        *pout.count = cnt;
        *pout.bad = ((badm >> (r * kl)) & kmask) != 0 ? 1 : 0;
        pout.tot[0] = W ? e.w : static_cast<double>(e.i);
        pout.tot[1] = W ? e.wl : 0.0;
        pout.tot[2] = e.s;
        pout.tot[3] = e.sl;
      }
    }
    for (int r = 0; r < nch / kl; ++r)
      fold(node_out(a.hulls1, W, static_cast<int64_t>(blockIdx.x) * a.rpw + r), ((badm >> (r * kl)) & kmask) != 0);
    // every row merged: its first span's count says so to the merge kernel
    if (active && span == 0) *o.count = -1;
    return;
  }
  const int count = merge_rounds<W, true, kSpanLanes, 2>(v, rs, nslots, nch);
  const NodeOut pout = node_out(a.hulls1, W, blockIdx.x);
  for (int k = lane; k < count; k += kSpanLanes) {
    const HPt x = sget(v, k);
    pout.idx[k] = x.i;
    put_dd(pout.shi, pout.slo, k, x.s, x.sl);
    if constexpr (W) put_dd(pout.whi, pout.wlo, k, x.w, x.wl);
  }
  if (lane == nch - 1) {
    *pout.count = count;
    *pout.bad = anybad ? 1 : 0;
    pout.tot[0] = iw.hi;
    pout.tot[1] = iw.lo;
    pout.tot[2] = is.hi;
    pout.tot[3] = is.lo;
  }
  // the group is merged: its first span's count says so to the merge kernel
  if (lane == 0) *o.count = -1;
  fold(pout, anybad);
  if (a.expand) expand(pout, anybad);
}

// SIMDs of the current device (four a CU), read once per device
int simd_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 1024;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    v = 4 * cus;
    cache[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

}  // namespace

hipError_t span_run(const TileArgs& t, const NodeLevel& hulls, int64_t span0, const NodeLevel& hulls1,
                     int rows_per_wave, int fix, TileRec* tiles) {
  const int64_t spr = hulls.npr;
  SpanArgs a;
  a.y = t.y;
  a.w = t.w;
  a.bad_weight = t.bad_weight;
  a.n = t.n;
  a.spr = spr;
  a.nodes = t.batch * spr;
  a.flags = t.flags;
  a.hulls = hulls;
  a.span0 = span0;
  a.gpr = (spr + kSpanLanes - 1) / kSpanLanes;
  a.rpw = rows_per_wave;
  a.hulls1 = hulls1;
  a.map = t.map;
  a.fix = fix;
  a.expand = tiles != nullptr;
  a.xp.n = t.n;
  a.xp.out = t.out;
  a.xp.starts = t.starts;
  a.xp.tiles = tiles;
  a.xp.tile_n = static_cast<int>(tile_elems(t.w != nullptr));
  a.xp.tpr = (t.n + a.xp.tile_n - 1) / a.xp.tile_n;
  a.xp.flags = t.flags;
  a.xp.lo = t.lo;
  a.xp.hi = t.hi;
  a.xp.map = t.map;
  a.xp.lds_bytes = 0;  // (the kernel's: its wave's LDS)
  a.mark = t.start_mark;
  a.mark_value = t.mark_value;
  // (rows of one span: one row per lane, and no first merge level to write; several rows a wave:
  // rows_per_wave of them)
  const unsigned grid = static_cast<unsigned>(spr == 1 ? (t.batch + kSpanLanes - 1) / kSpanLanes
                                              : rows_per_wave > 1 ? (t.batch + rows_per_wave - 1) / rows_per_wave
                                                                  : t.batch * a.gpr);
  const bool W = t.w != nullptr;
  const bool inc = (t.flags & TI_INCREASING) != 0;
  // A grid the GPU holds in one round at two waves a SIMD or fewer is latency-bound: each wave's
  // event loop sets the time, and the stronger candidate test (FILT: fewer loop iterations for
  // more arithmetic per element) pays (1000 rows of 5000: 67 -> 61.5 us; 2000: 79.8 -> 75.2 us);
  // over several rounds it costs more than it saves (C4-shaped rows 519 -> 547 us).
  const bool filt = t.map.rows == nullptr && grid <= 2u * static_cast<unsigned>(simd_count());
  auto go = [&](auto k_inc, auto k_dec) {
    if (inc) k_inc<<<dim3(grid), dim3(kSpanLanes), 0, t.stream>>>(a);
    else k_dec<<<dim3(grid), dim3(kSpanLanes), 0, t.stream>>>(a);
  };
  if (t.dtype == TI_F32) {
    if (t.map.rows != nullptr) {  // (ragged rows of a block: float32 only)
      if (W) go(span_kernel<float, true, 4, 8, 8, 32, true, true>, span_kernel<float, true, 4, 8, 8, 32, false, true>);
      else go(span_kernel<float, false, 4, 8, 16, 32, true, true>, span_kernel<float, false, 4, 8, 16, 32, false, true>);
    } else if (W) {
      if (filt) go(span_kernel<float, true, 4, 8, 8, 32, true, false, true>, span_kernel<float, true, 4, 8, 8, 32, false, false, true>);
      else go(span_kernel<float, true, 4, 8, 8, 32, true>, span_kernel<float, true, 4, 8, 8, 32, false>);
    } else {
      if (filt) go(span_kernel<float, false, 4, 8, 16, 32, true, false, true>, span_kernel<float, false, 4, 8, 16, 32, false, false, true>);
      else go(span_kernel<float, false, 4, 8, 16, 32, true>, span_kernel<float, false, 4, 8, 16, 32, false>);
    }
  } else {
    if (W) {
      if (filt) go(span_kernel<double, true, 4, 8, 8, 8, true, false, true>, span_kernel<double, true, 4, 8, 8, 8, false, false, true>);
      else go(span_kernel<double, true, 4, 8, 8, 8, true>, span_kernel<double, true, 4, 8, 8, 8, false>);
    } else {
      if (filt) go(span_kernel<double, false, 4, 8, 16, 8, true, false, true>, span_kernel<double, false, 4, 8, 16, 8, false, false, true>);
      else go(span_kernel<double, false, 4, 8, 16, 8, true>, span_kernel<double, false, 4, 8, 16, 8, false>);
    }
  }
  return hipGetLastError();
}

}  // namespace ti
