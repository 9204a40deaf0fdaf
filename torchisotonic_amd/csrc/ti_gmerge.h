// The merge of child hulls in the parent's global array (merge_global), shared by the merge
// kernel and the span kernel's group merge, with the vertex accessors and the bridge it uses.
#pragma once

#include "ti_common.h"
#include "ti_slots.h"
#include "ti_tile.h"

namespace ti {
namespace {

// A vertex array: index (relative to the node's first element) and double-double sums.
struct VArr {
  int* idx;
  double *shi, *slo, *whi, *wlo;
};

struct VPt {
  int i;
  DD s, w;
};

template <bool W>
__device__ __forceinline__ VPt vload(const VArr& a, int k) {
  VPt p;
  p.i = a.idx[k];
  p.s = DD{a.shi[k], lo_at(a.slo, k)};
  if constexpr (W) p.w = DD{a.whi[k], lo_at(a.wlo, k)};
  else p.w = DD{static_cast<double>(p.i), 0.0};
  return p;
}

template <bool W>
__device__ __forceinline__ void vstore(const VArr& a, int k, const VPt& p) {
  a.idx[k] = p.i;
  put_dd(a.shi, a.slo, k, p.s.hi, p.s.lo);
  if constexpr (W) put_dd(a.whi, a.wlo, k, p.w.hi, p.w.lo);
}

template <bool W>
__device__ __forceinline__ void vdiff(const VPt& a, const VPt& b, double& dW, double& dS) {
  dS = dd_diff(b.s, a.s);
  if constexpr (W) dW = dd_diff(b.w, a.w);
  else dW = static_cast<double>(b.i - a.i);
}

template <bool W>
__device__ __forceinline__ bool vpools(const VPt& a, const VPt& b, const VPt& c) {
  double dW1, dS1, dW2, dS2;
  vdiff<W>(a, b, dW1, dS1);
  vdiff<W>(b, c, dW2, dS2);
  return pools<true>(dS1, dW1, dS2, dW2);
}

// The vertex of B[1 .. cB) touched by the lower tangent from p (the last of equal slopes);
// getB(j) is B's vertex j.
template <bool W, class GB>
__device__ int vtangent(const VPt& p, GB getB, int cB) {
  int lo = 1, hi = cB - 1;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (!vpools<W>(p, getB(mid), getB(mid + 1))) hi = mid;
    else lo = mid + 1;
  }
  return lo;
}

// Bridge of hulls A (cA vertices, getA(i) its vertex i) and B (cB, getB(j)) sharing their
// boundary point (A's last is B's first); the merged hull is A[0 .. keep) ++ B[from .. cB).
// (Same method as the tile kernel's.)
template <bool W, class GA, class GB>
__device__ void vbridge(GA getA, int cA, GB getB, int cB, int& keep, int& from) {
  if (cB <= 1) {
    keep = cA;
    from = cB;
    return;
  }
  if (cA <= 1) {
    keep = 0;
    from = 0;
    return;
  }
  VPt a = getA(cA - 2);
  const VPt x = getA(cA - 1);
  VPt b = getB(1);
  if (!vpools<W>(a, x, b)) {
    keep = cA;
    from = 1;
    return;
  }
  int i = cA - 2, j = 1;
  bool done = false;
  VPt ap = i > 0 ? getA(i - 1) : a;
  VPt bn = j + 1 < cB ? getB(j + 1) : b;
  for (int steps = 0; steps < 24; ++steps) {
    if (i > 0 && vpools<W>(ap, a, b)) {
      --i;
      a = ap;
      if (i > 0) ap = getA(i - 1);
    } else if (j + 1 < cB && vpools<W>(a, b, bn)) {
      ++j;
      b = bn;
      if (j + 1 < cB) bn = getB(j + 1);
    } else {
      done = true;
      break;
    }
  }
  if (!done) {
    int lo = 0, hi = cA - 2;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      const VPt am = getA(mid);
      const int t = vtangent<W>(am, getB, cB);
      if (vpools<W>(am, getA(mid + 1), getB(t))) hi = mid;
      else lo = mid + 1;
    }
    i = lo;
    j = vtangent<W>(getA(lo), getB, cB);
  }
  keep = i + 1;
  from = j;
}

__device__ VArr dvarr_of(const NodeOut& o) { return VArr{o.idx, o.shi, o.slo, o.whi, o.wlo}; }

// (field by field, and without the weights of unweighted rows, which vpools takes from the
// indices: whole-struct copies between LDS and registers went through scratch memory)
template <bool W>
__device__ __forceinline__ void vput(VPt& d, const VPt& x) {
  d.i = x.i;
  d.s.hi = x.s.hi;
  d.s.lo = x.s.lo;
  if constexpr (W) {
    d.w.hi = x.w.hi;
    d.w.lo = x.w.lo;
  }
}

// Parallel removal passes before the repair finishes a row with chain_row instead. Each pass
// removes every vertex then on or above the chord between its neighbours, so it removes one at
// least, but a removal can expose its neighbours in turn: a long near-collinear run can need a
// cascade of passes, each a read of the whole hull.
constexpr int kRepairPasses = 64;

// The lower hull of the row's `cnt` stored vertices by one monotone chain (the same predicate
// as the passes, so the same hull: a vertex on or above a chord between two others is on no
// lower hull, and a convex chain through every lower-hull vertex holds no other). Thread 0
// pushes and pops in place, writing a vertex at or below its own position, while the workgroup
// stages the next NT vertices into `tile` (NT + 2 slots); returns the count (in thread 0).
template <bool W, int NT>
__device__ int chain_row(const VArr& v, int cnt, VPt* tile) {
  const int tid = threadIdx.x;
  int top = 0;  // stack entries, at v[0, top); a and b the two at its top
  VPt a, b;
  for (int c0 = 0; c0 < cnt; c0 += NT) {
    const int i = c0 + tid;
    if (i < cnt) vput<W>(tile[tid], vload<W>(v, i));
    __syncthreads();
    if (tid == 0) {
      const int e = min(NT, cnt - c0);
      for (int k = 0; k < e; ++k) {
        VPt p;
        vput<W>(p, tile[k]);
        while (top >= 2 && vpools<W>(a, b, p)) {
          --top;
          vput<W>(b, a);
          if (top >= 2) vput<W>(a, vload<W>(v, top - 2));  // (written by this thread before)
        }
        vstore<W>(v, top, p);
        ++top;
        vput<W>(a, b);
        vput<W>(b, p);
      }
    }
    __syncthreads();  // (the tile read before it is filled again)
  }
  return top;
}

// A workgroup of NT threads removes, pass after pass, every vertex of the row's hull `o` on or
// above the chord between its neighbours, until none is (the first pass is the check); after
// `passes` removal passes the row is finished by chain_row. LDS: tile[NT + 2], wcount[NT / 64],
// any.
template <bool W, int NT>
__device__ void repair_row(const NodeOut& o, VPt* tile, int* wcount, int& any, int passes) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const VArr v = dvarr_of(o);
  int cnt = *o.count;
  bool convex = false;
  for (int pass = 0; pass <= passes; ++pass) {
    if (tid == 0) any = 0;
    __syncthreads();
    // (four vertices a thread at a time, all their reads in flight together: a row's hull can
    // have as many vertices as elements)
    bool found = false;
    for (int i0 = 1 + tid; i0 < cnt - 1; i0 += 4 * NT) {
      VPt a[4], b[4], c[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = min(i0 + u * NT, cnt - 2);
        a[u] = vload<W>(v, i - 1);
        b[u] = vload<W>(v, i);
        c[u] = vload<W>(v, i + 1);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) found |= vpools<W>(a[u], b[u], c[u]);
    }
    if (__any(found) && lane == 0) any = 1;
    __syncthreads();
    if (any == 0) {
      convex = true;
      break;
    }
    if (pass == passes) break;  // (still not convex: chain_row below)
    int base = 0;
    VPt last;  // (thread NT - 1: the previous chunk's last original vertex)
    for (int c0 = 0; c0 < cnt; c0 += NT) {
      const int i = c0 + tid;
      if (i < cnt) vput<W>(tile[tid + 1], vload<W>(v, i));
      if (tid == NT - 1) {
        if (c0 > 0) vput<W>(tile[0], last);
        if (c0 + NT < cnt) vput<W>(tile[NT + 1], vload<W>(v, c0 + NT));
      }
      __syncthreads();
      const bool keep = i < cnt && (i == 0 || i == cnt - 1 || !vpools<W>(tile[tid], tile[tid + 1], tile[tid + 2]));
      const uint64_t m = __ballot(keep);
      if (lane == 0) wcount[wave] = __popcll(m);
      __syncthreads();
      int before = base, all = 0;
      for (int k = 0; k < NT / kWave; ++k) {
        before += k < wave ? wcount[k] : 0;
        all += wcount[k];
      }
      VPt x;
      vput<W>(x, tile[tid + 1]);
      if (tid == NT - 1) vput<W>(last, x);
      __syncthreads();  // every read of this chunk's slots is done
      if (keep) vstore<W>(v, before + __popcll(m & ((uint64_t{1} << lane) - 1)), x);
      base += all;
    }
    cnt = base;
    __syncthreads();
  }
  if (!convex) cnt = chain_row<W, NT>(v, cnt, tile);
  if (tid == 0) *o.count = cnt;
}

struct MergeSmall {
  int cnt[kGroup], off[kGroup];
  double tot[4][kGroup + 1];  // child offsets (W hi, lo, S hi, lo); [nch]: the parent's total
  int keep[kGroup / 2], from[kGroup / 2];
  int total, bad, rounds_max;
};

// Slot s of the children laid end to end (each child's first vertex is the previous child's
// last, stored once): the child holding it, i.e. the last child whose first slot is below s
// (child 0 for s = 0).
__device__ __forceinline__ int child_of_slot(const MergeSmall& sm, int nch, int s) {
  int lo = 0, hi = nch - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (sm.off[mid] < s) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// Vertex k of child c in the parent's coordinates, double-double: the child's offset added
// to its coordinates without re-rounding them, so the parent sees the child's hull exactly as
// the child built it (re-rounded into the parent's larger coordinates, a convex child could
// turn non-convex where sums cancel).
template <bool W, bool PR>
__device__ __forceinline__ HPt child_vertex(const MergeArgs& a, const MergeSmall& sm, int64_t row,
                                            int64_t c0, int c, int k) {
  const NodeOut ci = node_out(a.in, W, row * a.in.npr + c0 + c);
  HPt p;
  p.i = ci.idx[k] + static_cast<int>(c * a.child_elems);
  const DD S = dd_add(DD{sm.tot[2][c], sm.tot[3][c]}, DD{ci.shi[k], PR ? lo_at(ci.slo, k) : 0.0});
  p.s = S.hi;
  p.sl = PR ? S.lo : 0.0;
  p.w = 0.0;
  p.wl = 0.0;
  if constexpr (W) {
    const DD Wd = dd_add(DD{sm.tot[0][c], sm.tot[1][c]}, DD{ci.whi[k], PR ? lo_at(ci.wlo, k) : 0.0});
    p.w = Wd.hi;
    p.wl = PR ? Wd.lo : 0.0;
  }
  return p;
}

// The merge in the parent's global array, for children with more vertices than LDS holds
// (hulls of trend-like data, where few vertices drop), by reference to the children's own
// vertices: child c keeps a range [rlo[c], rhi[c]) of its vertices (without its first for
// c > 0: that is child c - 1's last), pairwise rounds find each bridge (one lane a pair) on the
// concatenations of those ranges and only shorten the ranges, and one pass then writes the
// survivors into the parent's array. A merge of segments A and B (runs of children) bridges A
// with its first point in front (for a segment after the first: the previous segment keeps
// that point) and B with A's last point in front, so both are whole convex chains. The pass
// writes in increasing slot order, a chunk read before any of it is written: child c lies at
// a fixed offset in the parent's range, c times a child's capacity, and the survivors laid
// end to end never take a slot above their vertex's own, so no write lands on a vertex still
// to be read. (Copying the children end to end and moving each right part's survivors down,
// round after round, moved every vertex several times through one workgroup.)
// DF (parents whose hull lies in the other store than their children's): more than kDeferMin
// survivors are left to survivors_kernel, their ranges and offsets in *tab.
template <bool W, bool PR, int NT, bool DF = false>
__device__ void merge_global(const MergeArgs& a, MergeSmall& sm, int* rlo, int* rhi, int* pre, int64_t row,
                             int64_t c0, int nch, const NodeOut& pout, DeferTab* tab = nullptr) {
  const int tid = threadIdx.x;
  const VArr v = dvarr_of(pout);
  for (int c = tid; c < nch; c += NT) {
    rlo[c] = c == 0 ? 0 : 1;
    rhi[c] = sm.cnt[c];
  }
  __syncthreads();
  auto vertex = [&](int c, int k) -> VPt {
    const HPt h = child_vertex<W, PR>(a, sm, row, c0, c, k);
    VPt p;
    p.i = h.i;
    p.s = DD{h.s, h.sl};
    p.w = W ? DD{h.w, h.wl} : DD{static_cast<double>(h.i), 0.0};
    return p;
  };
  // vertex i of the concatenation of children [c_lo, c_hi)'s ranges (pre[]: the kept vertices
  // before each child within it): the last child whose count before it is at most i
  auto kept = [&](int c_lo, int c_hi, int i) -> VPt {
    int lo = c_lo, hi = c_hi - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (pre[mid] <= i) lo = mid;
      else hi = mid - 1;
    }
    return vertex(lo, rlo[lo] + (i - pre[lo]));
  };
#pragma unroll 1
  for (int span = 1; span < nch; span <<= 1) {
    const int nm = (nch + 2 * span - 1) / (2 * span);  // merges this round
    for (int m = tid; m < nm; m += NT) {
      const int pa = m * 2 * span, pb = pa + span;
      if (pb >= nch) continue;
      const int pe = min(pb + span, nch);
      int nA = 0, nB = 0;
      for (int c = pa; c < pb; ++c) {
        pre[c] = nA;
        nA += rhi[c] - rlo[c];
      }
      for (int c = pb; c < pe; ++c) {
        pre[c] = nB;
        nB += rhi[c] - rlo[c];
      }
      const int s0 = pa > 0 ? 1 : 0;  // A's first point in front
      const VPt first = vertex(pa, 0);
      const int cA = s0 + nA, cB = 1 + nB;
      auto getA = [&](int i) -> VPt { return (s0 != 0 && i == 0) ? first : kept(pa, pb, i - s0); };
      auto getB = [&](int j) -> VPt { return j == 0 ? getA(cA - 1) : kept(pb, pe, j - 1); };
      int keep = cA, from = 1;
      vbridge<W>(getA, cA, getB, cB, keep, from);
      // A keeps its first a_keep kept vertices, B drops its first b_drop
      int left = from == 0 ? nA : keep - s0;
      for (int c = pa; c < pb; ++c) {
        const int k = rhi[c] - rlo[c];
        if (left >= k) {
          left -= k;
        } else {
          rhi[c] = rlo[c] + max(left, 0);
          left = 0;
        }
      }
      int drop = from > 1 ? from - 1 : 0;
      for (int c = pb; c < pe; ++c) {
        const int k = rhi[c] - rlo[c];
        if (drop >= k) {
          rlo[c] = rhi[c];
          drop -= k;
        } else {
          rlo[c] += drop;
          drop = 0;
        }
      }
    }
    __syncthreads();
  }
  // the survivors, in slot order
  if (tid == 0) {
    int t = 0;
    for (int c = 0; c < nch; ++c) {
      pre[c] = t;
      t += rhi[c] - rlo[c];
    }
    sm.total = t;
  }
  __syncthreads();
  const int total = sm.total;
  if (DF && total > kDeferMin) {
    for (int c = tid; c < nch; c += NT) {
      tab->rlo[c] = rlo[c];
      tab->pre[c] = pre[c];
#pragma unroll
      for (int q = 0; q < 4; ++q) tab->tot[q][c] = sm.tot[q][c];
    }
    if (tid == 0) {
      tab->total = total;
      tab->deferred = 1;
      *pout.count = total;
    }
    return;
  }
  // Batches of NT * B slots: batch k's slots lie below every source of batch k + 1 (a survivor's
  // slot is never above its vertex's own), so batch k + 1 is read while batch k is written; a
  // batch is read by every thread (the barrier) before any of its slots is written.
  constexpr int B = (W || PR) ? 4 : 8;
  auto load = [&](int s0, VPt (&p)[B]) {
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int s = s0 + u * NT + tid;
      if (s < total) p[u] = kept(0, nch, s);
    }
  };
  auto store = [&](int s0, const VPt (&p)[B]) {
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int s = s0 + u * NT + tid;
      if (s < total) vstore<W>(v, s, p[u]);
    }
  };
  VPt pa[B], pb[B];
  load(0, pa);
  __syncthreads();
  for (int s0 = 0; s0 < total;) {
    load(s0 + NT * B, pb);
    store(s0, pa);
    __syncthreads();
    s0 += NT * B;
    if (s0 >= total) break;
    load(s0 + NT * B, pa);
    store(s0, pb);
    __syncthreads();
    s0 += NT * B;
  }
  if (tid == 0) *pout.count = total;
}

// The round state merge_global keeps in LDS: kGroup ranges and counts.
struct MergeRanges {
  int rlo[kGroup], rhi[kGroup], pre[kGroup];
};

}  // namespace
}  // namespace ti
