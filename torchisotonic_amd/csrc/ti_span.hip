// Rows longer than one tile, first stage: one lane per span of kSpan elements.
//
// Replaces the reference's chunk stage for long rows (reference src/torchisotonic/csrc/
// tiles.cuh:665-913, chunk_kernel, which builds small lane hulls and merges them across the
// block in rounds). A lane instead runs the monotone chain over its whole span by itself,
// streaming the elements through registers kChunk at a time (the next chunk loading while the
// current one is processed): no block-wide scans, no merge rounds, no barriers, every lane
// busy. The lane's cumulative sums are float64 relative to the span start; float64 data also
// carries their rounding errors (two-sum), so the difference of neighbouring points keeps the
// precision of the difference. The hull stack keeps its top three vertices in registers and
// its positions in a ring of kRing LDS slots per lane; positions that fall out of the ring go
// to the span's hull array in global memory, where the finished hull ends anyway (noisy data
// seldom gets that deep).
//
// A point is a candidate only where the data rises into it (y_{k-1} < y_k): elsewhere the slope
// into it is at least the slope out of it, and equal slopes pool, so it is never a vertex.
//
// Output: the span hulls as the first node array of the cross-span merge (ti_merge.hip).
#include "ti_common.h"
#include "ti_kernels.h"
#include "ti_tile.h"

namespace ti {

namespace {

constexpr int kSpanLanes = 64;
constexpr int kChunk = 16;

struct SpanArgs {
  const void* y;
  const void* w;
  uint32_t* bad_weight;
  int64_t n, spr, nodes;  // row length, spans per row, spans in total
  unsigned flags;
  void* hulls;            // node array of the spans
  int64_t cap;
};

template <typename T, bool W>
struct SpanOps {
  static constexpr bool PR = sizeof(T) == 8;
  static constexpr int kRing = W ? 8 : 16;

  struct Ring {
    int idx[kRing][kSpanLanes];
    double s[kRing][kSpanLanes];
    double sl[PR ? kRing : 1][kSpanLanes];
    double w[W ? kRing : 1][kSpanLanes];
    double wl[W && PR ? kRing : 1][kSpanLanes];
  };

  __device__ static void put(Ring& r, int slot, int lane, const HPt& p) {
    r.idx[slot][lane] = p.i;
    r.s[slot][lane] = p.s;
    if constexpr (PR) r.sl[slot][lane] = p.sl;
    if constexpr (W) r.w[slot][lane] = p.w;
    if constexpr (W && PR) r.wl[slot][lane] = p.wl;
  }

  __device__ static HPt get(const Ring& r, int slot, int lane) {
    HPt p;
    p.i = r.idx[slot][lane];
    p.s = r.s[slot][lane];
    p.sl = PR ? r.sl[PR ? slot : 0][lane] : 0.0;
    p.w = W ? r.w[W ? slot : 0][lane] : 0.0;
    p.wl = (W && PR) ? r.wl[(W && PR) ? slot : 0][lane] : 0.0;
    return p;
  }

  // Node arrays hold double-double sums; float32 data has no rounding errors to carry (lo = 0).
  __device__ static void node_put(const NodeOut& o, int q, const HPt& p) {
    o.idx[q] = p.i;
    o.shi[q] = p.s;
    o.slo[q] = p.sl;
    if constexpr (W) {
      o.whi[q] = p.w;
      o.wlo[q] = p.wl;
    }
  }

  __device__ static HPt node_get(const NodeOut& o, int q) {
    HPt p;
    p.i = o.idx[q];
    p.s = o.shi[q];
    p.sl = PR ? o.slo[q] : 0.0;
    p.w = W ? o.whi[q] : 0.0;
    p.wl = (W && PR) ? o.wlo[q] : 0.0;
    return p;
  }

};

template <typename T, int N>
__device__ __forceinline__ void load_chunk(const T* __restrict__ p, int count, T (&v)[N]) {
  constexpr int V = 16 / sizeof(T);
  using VT = T __attribute__((ext_vector_type(V)));
  if (count >= N && (reinterpret_cast<uintptr_t>(p) & 15) == 0) {
    const VT* q = reinterpret_cast<const VT*>(p);
#pragma unroll
    for (int j = 0; j < N / V; ++j) {
      const VT x = __builtin_nontemporal_load(q + j);
#pragma unroll
      for (int t = 0; t < V; ++t) v[j * V + t] = x[t];
    }
  } else {
#pragma unroll
    for (int k = 0; k < N; ++k) v[k] = k < count ? p[k] : T(0);
  }
}

template <typename T, bool W>
__global__ __launch_bounds__(kSpanLanes) void span_kernel(SpanArgs a) {
  using Ops = SpanOps<T, W>;
  constexpr bool PR = Ops::PR;
  constexpr int kRing = Ops::kRing;
  __shared__ typename Ops::Ring ring;
  const int lane = threadIdx.x;
  const int64_t node = static_cast<int64_t>(blockIdx.x) * kSpanLanes + lane;
  if (node >= a.nodes) return;  // no barriers below: the lanes are independent
  const int64_t row = node / a.spr;
  const int64_t span = node - row * a.spr;
  const int64_t first = span * kSpan;
  const int len = static_cast<int>(min<int64_t>(kSpan, a.n - first));
  const bool inc = (a.flags & TI_INCREASING) != 0;
  const double sgn = inc ? 1.0 : -1.0;
  const T* y = static_cast<const T*>(a.y) + row * a.n + first;
  const T* w = W ? static_cast<const T*>(a.w) + row * a.n + first : nullptr;
  const NodeOut o = node_out(a.hulls, a.nodes, a.cap, W, node);

  // The stack holds positions [0, depth): [r0, depth) in the ring (position q in slot q % kRing),
  // [0, r0) in the node array. t1, t2, t3: positions depth-1, depth-2, depth-3.
  int depth = 1, r0 = 0;
  HPt t1{0, 0.0, 0.0, 0.0, 0.0}, t2 = t1, t3 = t1;
  Ops::put(ring, 0, lane, t1);

  double S = 0.0, SL = 0.0, P = 0.0, PL = 0.0;
  bool bad = false, wbad = false;
  T yc[kChunk], yn[kChunk];
  T wc[W ? kChunk : 1], wn[W ? kChunk : 1];
  load_chunk<T, kChunk>(y, len, yc);
  if constexpr (W) load_chunk<T, kChunk>(w, len, wc);
  for (int c0 = 0; c0 < len; c0 += kChunk) {
    const int rest = len - (c0 + kChunk);
    if (rest > 0) {
      load_chunk<T, kChunk>(y + c0 + kChunk, rest, yn);
      if constexpr (W) load_chunk<T, kChunk>(w + c0 + kChunk, rest, wn);
    }
#pragma unroll
    for (int k = 0; k < kChunk; ++k) {
      const int e = c0 + k;  // the element; the point after it is e + 1
      if (e < len) {
        const double ye = sgn * static_cast<double>(yc[k]);
        bad |= ye != ye;
        double term = ye;
        if constexpr (W) {
          const double we = static_cast<double>(wc[k]);
          wbad |= !(we > 0.0);
          term = we * ye;
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
        // the point after e is a candidate at the span's end or where y rises into e + 1
        bool cand = e + 1 == len;
        if (!cand) {
          const T ynext = k + 1 < kChunk ? yc[k + 1 < kChunk ? k + 1 : 0] : yn[0];
          cand = inc ? yc[k] < ynext : ynext < yc[k];
        }
        if (cand) {
          const HPt c{e + 1, S, SL, P, PL};
          while (depth >= 2 && hpools<W, PR>(t2, t1, c)) {
            --depth;
            t1 = t2;
            t2 = t3;
            if (depth >= 3) {
              const int q = depth - 3;
              t3 = q >= r0 ? Ops::get(ring, q % kRing, lane) : Ops::node_get(o, q);
            }
          }
          const int q = depth;
          if (q < r0) r0 = q;  // popped below the ring: it restarts at q
          if (q >= r0 + kRing) {  // the ring's oldest position leaves for the node array
            const int old = q - kRing;
            Ops::node_put(o, old, Ops::get(ring, old % kRing, lane));
            r0 = old + 1;
          }
          Ops::put(ring, q % kRing, lane, c);
          ++depth;
          t3 = t2;
          t2 = t1;
          t1 = c;
        }
      }
    }
#pragma unroll
    for (int k = 0; k < kChunk; ++k) {
      yc[k] = yn[k];
      if constexpr (W) wc[W ? k : 0] = wn[W ? k : 0];
    }
  }
  // the finished hull: positions [0, depth) of the span's array
  for (int q = r0; q < depth; ++q) Ops::node_put(o, q, Ops::get(ring, q % kRing, lane));
  *o.count = depth;
  *o.bad = bad ? 1 : 0;
  o.tot[0] = W ? P : static_cast<double>(len);
  o.tot[1] = W ? PL : 0.0;
  o.tot[2] = S;
  o.tot[3] = SL;
  if (W && wbad && a.bad_weight != nullptr) *a.bad_weight = 1u;
}

}  // namespace

hipError_t span_run(const TileArgs& t, void* hulls, int64_t spr, int64_t cap) {
  SpanArgs a;
  a.y = t.y;
  a.w = t.w;
  a.bad_weight = t.bad_weight;
  a.n = t.n;
  a.spr = spr;
  a.nodes = t.batch * spr;
  a.flags = t.flags;
  a.hulls = hulls;
  a.cap = cap;
  const unsigned grid = static_cast<unsigned>((a.nodes + kSpanLanes - 1) / kSpanLanes);
  const bool W = t.w != nullptr;
  if (t.dtype == TI_F32) {
    if (W) span_kernel<float, true><<<dim3(grid), dim3(kSpanLanes), 0, t.stream>>>(a);
    else span_kernel<float, false><<<dim3(grid), dim3(kSpanLanes), 0, t.stream>>>(a);
  } else {
    if (W) span_kernel<double, true><<<dim3(grid), dim3(kSpanLanes), 0, t.stream>>>(a);
    else span_kernel<double, false><<<dim3(grid), dim3(kSpanLanes), 0, t.stream>>>(a);
  }
  return hipGetLastError();
}

}  // namespace ti
