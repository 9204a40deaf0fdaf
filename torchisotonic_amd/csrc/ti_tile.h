// Shared definitions of the long-row kernels: tile geometry, launch arguments and the layout of
// the hull arrays that tiles and merged nodes leave in the workspace.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "ti_common.h"
#include "ti_kernels.h"

namespace ti {

constexpr int kWaves256 = 4;

// The tiles of the expansion and of the long-row backward: 256 threads x E elements, E = 16
// unweighted (4096-element tiles), 8 weighted (2048).
template <bool W>
struct TileCfg {
  static constexpr int kThreads = 256;
  static constexpr int kLogE = W ? 3 : 4;
  static constexpr int kE = 1 << kLogE;
  static constexpr int kN = kThreads * kE;
};

// Ragged rows taken as the rows of a [batch, n] block (n at least every length): row r's
// elements are at rows[2 r] + i of the packed arrays for i < rows[2 r + 1] (clamped to the
// packed array and to n), and past its length the row holds `pad` with weight 1 (and g = 0 in a
// backward), made in registers, never read. Fits and gradients are stored at the packed
// places of the row's own elements only. rows null: the dense layout, row r at r * n. The
// kernels address the packed arrays through one buffer resource, so total * sizeof(T) stays
// below kRowMapBytes.
struct RowMap {
  const int64_t* rows = nullptr;
  int64_t total = 0;  // elements of the packed arrays
  double pad = 0.0;
};
constexpr int64_t kRowMapBytes = int64_t{0x7FFF0000};

// Row r's first element and length (the dense layout without a map).
__device__ __forceinline__ void map_row(const RowMap& m, int64_t r, int64_t n, int64_t& first, int64_t& len) {
  if (m.rows == nullptr) {
    first = r * n;
    len = n;
    return;
  }
  first = m.rows[2 * r];
  first = first < 0 ? 0 : (first > m.total ? m.total : first);
  len = m.rows[2 * r + 1];
  len = len < 0 ? 0 : len;
  len = len > m.total - first ? m.total - first : len;
  len = len > n ? n : len;
}

struct TileArgs {
  const void* y;
  const void* w;
  void* out;
  uint32_t* starts;
  uint32_t* bad_weight;
  int64_t batch, n;
  int dtype;
  unsigned flags;
  double lo, hi;
  hipStream_t stream;
  hipEvent_t weights_read = nullptr;  // recorded once every weight has been read, if given
  // Where given: mark_value written to *weights_mark (a word of host memory that the host polls)
  // once every weight has been read, with no event between kernels: at the start of the first
  // merge launch after the span kernel, or by a kernel of one thread where none follows it
  uint32_t* weights_mark = nullptr;
  uint32_t mark_value = 0;
  // Where given (the weights read by a kernel before the fit): mark_value written to *start_mark
  // by the span kernel's first thread as it starts, all of that kernel's reads being done
  uint32_t* start_mark = nullptr;
  // Where given (rows over 32 elements): a bound on the final hulls' vertex counts (at least the
  // largest, at most n + 1) is written here (a device-visible word) and hulls_ready recorded once
  // it is, before the last merges and the expansion run.
  int64_t* max_vertices = nullptr;
  hipEvent_t hulls_ready = nullptr;
  RowMap map;  // ragged rows of one block (see RowMap)
};

// One node's hull: vertex indices relative to the node's first element, cumulative sums
// relative to the node's first point, the vertex count, a NaN flag and the node totals (W hi,
// W lo, S hi, S lo). Float64 data keeps the sums double-double; float32 data keeps them rounded
// to float64 (slo, wlo null), which halves the store (the merges still work in double-double in
// LDS, and the final hulls are made convex in the stored values: see repair_kernel).
struct NodeOut {
  int* count;
  int* bad;
  double* tot;
  int* idx;
  double *shi, *slo, *whi, *wlo;
};

// The sums of vertex k of a node, whichever way they are stored.
__device__ __forceinline__ double lo_at(const double* lo, int64_t k) { return lo != nullptr ? lo[k] : 0.0; }
// Stores a double-double value: hi and lo, or, without a low array, their sum rounded once.
__device__ __forceinline__ void put_dd(double* hi, double* lo, int64_t k, double h, double l) {
  if (lo != nullptr) {
    hi[k] = h;
    lo[k] = l;
  } else {
    hi[k] = h + l;
  }
}

__host__ __device__ inline size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

// One level of node hulls. Every level keeps its vertices in one shared store: a row's spans
// take r0 = span0 + 1 slots each, one after another, and a node's vertices start at the slot of
// the first span it covers. A node never has more vertices than its spans have slots (a hull of
// e elements has at most e + 1), so a parent's hull is written where its children's were, and
// the levels need no second store. Per level only the counts, NaN flags and totals are apart.
struct NodeLevel {
  char* meta;     // count[K], bad[K], tot[K][4]
  char* store;    // the shared vertex arrays: idx, shi, slo (and whi, wlo weighted), `slots` each
  int64_t K;      // nodes of the level
  int64_t npr;    // nodes per row
  int64_t spn;    // spans per node (its first span: j * spn of its row)
  int64_t npr0;   // spans per row
  int64_t r0;     // slots per span
  int64_t slots;  // slots of the store
  bool lo;        // the store keeps low parts (float64 data)
};

__host__ __device__ inline size_t node_meta_bytes(int64_t K) {
  const size_t k = static_cast<size_t>(K);
  return align256(k * 4) * 2 + align256(k * 32);
}

__host__ __device__ inline size_t vertex_store_bytes(int64_t slots, bool weighted, bool lo) {
  const size_t c = static_cast<size_t>(slots);
  return align256(c * 4) + align256(c * 8) * ((weighted ? 2 : 1) * (lo ? 2 : 1));
}

__host__ __device__ inline NodeOut node_out(const NodeLevel& L, bool weighted, int64_t k) {
  NodeOut o;
  char* p = L.meta;
  const size_t kk = static_cast<size_t>(L.K), c = static_cast<size_t>(L.slots);
  o.count = reinterpret_cast<int*>(p) + k;
  p += align256(kk * 4);
  o.bad = reinterpret_cast<int*>(p) + k;
  p += align256(kk * 4);
  o.tot = reinterpret_cast<double*>(p) + 4 * k;
  const int64_t row = k / L.npr, j = k - row * L.npr;
  const int64_t v0 = (row * L.npr0 + j * L.spn) * L.r0;
  char* q = L.store;
  o.idx = reinterpret_cast<int*>(q) + v0;
  q += align256(c * 4);
  o.shi = reinterpret_cast<double*>(q) + v0;
  q += align256(c * 8);
  o.slo = o.whi = o.wlo = nullptr;
  if (L.lo) {
    o.slo = reinterpret_cast<double*>(q) + v0;
    q += align256(c * 8);
  }
  if (weighted) {
    o.whi = reinterpret_cast<double*>(q) + v0;
    q += align256(c * 8);
    if (L.lo) o.wlo = reinterpret_cast<double*>(q) + v0;
  }
  return o;
}

// The stateless gradient (ti_grad): every element's block sums of g and w from the partition.
struct SegGradArgs {
  const void* fit;  // needed with y
  const uint32_t* starts;
  const void* g;
  const void* w;  // null: weights of one
  const void* y;  // null: no weight gradient
  void* gy;
  void* gw;
  int64_t batch, n;
  int dtype;
  hipStream_t stream;
};
size_t seg_grad_bytes(int64_t batch, int64_t n);
int64_t seg_grad_tiles(int64_t batch, int64_t n);
hipError_t seg_grad(const SegGradArgs& a, void* ws);

// E consecutive elements of one thread (count of them valid): 16-byte loads when whole and
// aligned, element by element otherwise.
template <typename T, int E>
__device__ __forceinline__ void load_elems_any(const T* __restrict__ p, int count, T (&v)[E]) {
  constexpr int V = 16 / sizeof(T);
  using VT = T __attribute__((ext_vector_type(V)));
  if (count == E && (reinterpret_cast<uintptr_t>(p) & 15) == 0) {
    const VT* q = reinterpret_cast<const VT*>(p);
    VT buf[E / V];
#pragma unroll
    for (int j = 0; j < E / V; ++j) buf[j] = q[j];
#pragma unroll
    for (int j = 0; j < E / V; ++j) {
#pragma unroll
      for (int t = 0; t < V; ++t) v[j * V + t] = buf[j][t];
    }
  } else {
#pragma unroll
    for (int k = 0; k < E; ++k) {
      if (k < count) v[k] = p[k];
    }
  }
}

// The same, the elements past count zero (so sums over all E need no per-element checks).
template <typename T, int E>
__device__ __forceinline__ void load_elems_zero(const T* __restrict__ p, int count, T (&v)[E]) {
  constexpr int V = 16 / sizeof(T);
  using VT = T __attribute__((ext_vector_type(V)));
  if (count == E && (reinterpret_cast<uintptr_t>(p) & 15) == 0) {
    const VT* q = reinterpret_cast<const VT*>(p);
    VT buf[E / V];
#pragma unroll
    for (int j = 0; j < E / V; ++j) buf[j] = q[j];
#pragma unroll
    for (int j = 0; j < E / V; ++j) {
#pragma unroll
      for (int t = 0; t < V; ++t) v[j * V + t] = buf[j][t];
    }
  } else {
#pragma unroll
    for (int k = 0; k < E; ++k) v[k] = k < count ? p[k] : T(0);
  }
}

// (NTS: non-temporal 16-byte stores, whose lines leave the caches as they are written)
template <typename T, int E, bool NTS = false>
__device__ __forceinline__ void store_elems_any(T* __restrict__ p, int count, const T (&v)[E]) {
  constexpr int V = 16 / sizeof(T);
  using VT = T __attribute__((ext_vector_type(V)));
  if (count == E && (reinterpret_cast<uintptr_t>(p) & 15) == 0) {
    VT* q = reinterpret_cast<VT*>(p);
#pragma unroll
    for (int j = 0; j < E / V; ++j) {
      VT x;
#pragma unroll
      for (int t = 0; t < V; ++t) x[t] = v[j * V + t];
      if constexpr (NTS) __builtin_nontemporal_store(x, q + j);
      else q[j] = x;
    }
  } else {
#pragma unroll
    for (int k = 0; k < E; ++k) {
      if (k < count) p[k] = v[k];
    }
  }
}

// Fills p[0, len) with f from the NT threads of a workgroup, each store instruction of a wave on
// one contiguous run of 16-byte pieces (len <= NT * E). The elements before the first 16-byte
// boundary are written singly.
template <typename T, int E, int NT, bool NTS = false>
__device__ __forceinline__ void fill_elems(T* __restrict__ p, int len, int tid, T f) {
  constexpr int V = 16 / sizeof(T);
  using VT = T __attribute__((ext_vector_type(V)));
  const int head = min(len, static_cast<int>(((16 - (reinterpret_cast<uintptr_t>(p) & 15)) & 15) / sizeof(T)));
  if (tid < head) p[tid] = f;
  T* __restrict__ q = p + head;
  const int rest = len - head;
  VT x;
#pragma unroll
  for (int t = 0; t < V; ++t) x[t] = f;
#pragma unroll
  for (int j = 0; j < E / V; ++j) {
    const int k = (j * NT + tid) * V;
    if (k + V <= rest) {
      if constexpr (NTS) __builtin_nontemporal_store(x, reinterpret_cast<VT*>(q + k));
      else *reinterpret_cast<VT*>(q + k) = x;
    } else {
#pragma unroll
      for (int t = 0; t < V; ++t)
        if (k + t < rest) q[k + t] = f;
    }
  }
}

// A hull point of the long-row kernels: index (relative to its node's first element), and
// cumulative w*y (s) and w (w; unweighted rows use the index) relative to the node's first point.
// Float64 data also carries the sums' rounding errors (sl, wl), zero for float32 data.
struct HPt {
  int i;
  double s, sl, w, wl;
};

// The vertex b leaves the hull through a, b, c (equal slopes pool); PR: the points carry
// rounding errors.
template <bool W, bool PR>
__device__ __forceinline__ bool hpools(const HPt& a, const HPt& b, const HPt& c) {
  double dS1 = b.s - a.s, dS2 = c.s - b.s;
  if constexpr (PR) {
    dS1 += b.sl - a.sl;
    dS2 += c.sl - b.sl;
  }
  double dW1, dW2;
  if constexpr (W) {
    dW1 = b.w - a.w;
    dW2 = c.w - b.w;
    if constexpr (PR) {
      dW1 += b.wl - a.wl;
      dW2 += c.wl - b.wl;
    }
  } else {
    dW1 = static_cast<double>(b.i - a.i);
    dW2 = static_cast<double>(c.i - b.i);
  }
  return pools<true>(dS1, dW1, dS2, dW2);
}

// Rows longer than 32 elements: one lane builds the hull of each span of span0 elements
// (kSpanMin..kSpanMax, a multiple of 4, chosen per call so that the span kernel has enough
// lanes), then
// workgroups merge G neighbouring hulls at a time until one hull per row remains.
constexpr int kSpanMin = 32;
constexpr int kSpanMax = 256;
constexpr int kGroup = 64;
constexpr int kMaxLevels = 8;

struct MergeArgs {
  NodeLevel in, out;    // the children's level and the parents'
  int64_t child_elems;  // elements per child node
  // (where given) mark_value stored to *mark by the launch's first thread as it starts: the
  // caller's mark that the kernels before have read every weight
  uint32_t* mark = nullptr;
  uint32_t mark_value = 0;
};

// Merge levels 2 and up with fewer than kDeferParents parents, each over kDeferSpan elements or
// more (a small batch's upper levels), write their hulls into the other vertex store than their
// children's, so that a parent's survivors need not move in order: a parent with more than
// kDeferMin of them leaves its children's kept ranges in its DeferTab, and survivors_kernel's
// workgroups, many a parent, write them (one workgroup moving the survivors in place took
// about 1.1 ns a vertex: 11 ms for 1e7).
constexpr int64_t kDeferParents = 256;
constexpr int64_t kDeferSpan = int64_t{1} << 16;
constexpr int kDeferMin = 4096;
struct DeferTab {
  int deferred;  // 1: survivors_kernel writes this parent's hull
  int total;     // the parent's vertices
  int unused[2];
  int rlo[kGroup];       // child c keeps its vertices rlo[c] ..
  int pre[kGroup];       // .. as the parent's vertices pre[c] .. (pre[c + 1] or total)
  double tot[4][kGroup];  // child c's offsets in the parent (W hi, lo, S hi, lo)
};

// Per tile of a long row, written by rank_kernel once the row's final hull is known: the hull's
// vertex ranks around the tile and, for the common case of one hull edge over the whole tile
// (rb == ra + 1 on a row without NaN), that edge's slope, so that the expansion and the
// backward start from one 32-byte read per tile.
struct alignas(32) TileRec {
  int ra;        // the last vertex at or before the tile's first element
  int rb;        // the first vertex at or after the tile's end
  int flags;     // kTileBad | kTileHead
  int last;      // the row's last vertex (vertex count - 1)
  double slope;  // dS / dW of the edge ra -> ra + 1, float64 from the double-double sums
  double unused;
};
constexpr int kTileBad = 1;   // the row holds a NaN (its fit is NaN throughout)
constexpr int kTileHead = 2;  // a block starts at the tile's first element: a vertex sits there
                              // (on a NaN row: the tile is the row's first)

struct ExpandArgs {
  NodeLevel hulls;  // the final level: one node per row
  int64_t batch, n, tiles_per_row;
  void* out;
  uint32_t* starts;
  const TileRec* tiles;  // per tile (rank_kernel's)
  unsigned flags;
  double lo, hi;
  RowMap map;  // out in the packed layout (starts stay in the block's)
};

// Workspace of a long-row fit: the shared vertex store of every level (span0 + 1 slots per span),
// each level's counts, NaN flags and totals, and the per-tile records of the expansion.
struct LongPlan {
  int64_t tiles_per_row;  // expansion (and backward) tiles
  int64_t span0;          // elements per span (the first node level)
  int rows_per_wave;      // > 1: the span kernel's wave holds that many short rows, 64 / it lanes each
  int levels;
  int keep_level;  // the level whose vertex counts bound the final hulls' (see long_fit)
  int64_t batch;
  int64_t npr[kMaxLevels + 1], spn[kMaxLevels + 1], span[kMaxLevels + 1];
  int64_t slots;  // of the store: batch * npr[0] * (span0 + 1)
  // defer[l]: level l's merges may leave survivors to survivors_kernel (see DeferTab); alt[l]:
  // level l's hulls lie in the second store (each deferring level writes the other store than
  // its children's)
  bool defer[kMaxLevels + 1], alt[kMaxLevels + 1];
  size_t off_meta[kMaxLevels + 1], off_store, off_store2, off_defer, off_rank, off_maxc, off_rflag, bytes;
  bool weighted;
  bool lo;  // the vertex store keeps low parts (float64 data)

  NodeLevel level(void* ws, int l) const {
    char* base = static_cast<char*>(ws);
    return NodeLevel{base + off_meta[l], base + (alt[l] ? off_store2 : off_store), batch * npr[l], npr[l], spn[l],
                     npr[0], span0 + 1, slots, lo};
  }
};

// lo: float64 data (its vertex store keeps double-double sums)
LongPlan long_plan(int64_t batch, int64_t n, bool weighted, bool lo);
hipError_t long_fit(const TileArgs& t, const LongPlan& p, void* ws);

// The part of a long-row forward's workspace that its backward reads, kept on its own
// (ti_keep): the final hulls, each row's in a stretch of maxc slots (maxc: a bound on the final
// hulls' vertex counts), and the per-tile records.
struct KeepPlan {
  int64_t batch, maxc, tiles;
  size_t off_meta, off_store, off_tiles, bytes;
  bool lo;
  NodeLevel level(void* kept) const {
    char* b = static_cast<char*>(kept);
    return NodeLevel{b + off_meta, b + off_store, batch, 1, 1, 1, maxc, batch * maxc, lo};
  }
};
KeepPlan keep_plan(int64_t batch, int64_t n, bool weighted, bool lo, int64_t maxc);
hipError_t long_keep(const LongPlan& p, const void* ws, const KeepPlan& k, void* kept, hipStream_t stream);

// Level 0 (span hulls) and, fused, level 1: a group whose hulls fit the wave's LDS is merged in
// place into its level-1 node of `hulls1` and its first span's count set to -1. With
// rows_per_wave > 1, each wave holds that many rows of spans_per_row spans (a power of two) and
// merges each row's spans into the row's hull. fix > 0: those hulls are the rows' final hulls of
// float32 data, made convex in their stored values by the same waves (fix - 1 removal passes).
// tiles given (rows of one merge level, one row a wave): each wave also writes its row's fit,
// start bits and tile records (into tiles), in place of the rank and expansion launches.
hipError_t span_run(const TileArgs& t, const NodeLevel& hulls, int64_t span0, const NodeLevel& hulls1,
                    int rows_per_wave, int fix, TileRec* tiles);

// Backward of long rows, from the forward's final hulls and tile ranks (its workspace).
struct LongGradArgs {
  const uint32_t* starts;
  const void* g;
  const void* w;
  const void* y;
  void* gy;
  void* gw;
  int64_t batch, n;
  int dtype;
  unsigned flags;
  double lo, hi;
  const void* fwd_ws;  // the forward's workspace, or
  const void* kept;    // what ti_keep kept of it (fwd_ws null)
  int64_t kept_maxc;   // the kept hulls' slots a row
  hipStream_t stream;
  RowMap map;  // g, w, y, gy, gw in the packed layout (starts in the block's)
};
// kept_maxc > 0: the workspace of a backward from a kept state (its vertex prefixes sized for
// hulls of that many vertices instead of a row's every slot)
size_t long_grad_bytes(int64_t batch, int64_t n, bool weighted, bool lo, int64_t kept_maxc = 0);
hipError_t long_grad(const LongGradArgs& a, const LongPlan& p, void* ws);

inline int64_t tile_elems(bool weighted) { return weighted ? TileCfg<true>::kN : TileCfg<false>::kN; }

}  // namespace ti
