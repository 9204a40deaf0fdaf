// The expansion of one row's final hull by the workgroup that made it (the span kernel's wave
// for rows of one merge level, the last merge launch's workgroup for rows of several): the
// row's tile records, start bits and fit, in place of the rank and expansion launches.
#pragma once

#include "ti_common.h"
#include "ti_gmerge.h"
#include "ti_tile.h"

namespace ti {
namespace {

// What the expansion writes, and where.
struct RowExpand {
  int64_t n;         // row length (ragged rows: the block's length L)
  void* out;         // the fit
  uint32_t* starts;  // start bits (or null)
  TileRec* tiles;    // per row: tpr tile records of tile_n elements each
  int64_t tpr;
  int tile_n;
  unsigned flags;    // TI_INCREASING, TI_CLIP_MIN / TI_CLIP_MAX, TI_STREAM_OUT
  double lo, hi;
  RowMap map;        // ragged rows (with MAP)
  int lds_bytes;     // LDS the expansion may use
};

// LDS an expansion of rows of n elements needs at least, NT threads (the table then holds a
// pass's edges).
__host__ __device__ constexpr int expand_lds_min(int64_t n, int nt, int tbytes) {
  return 64 + 2 * static_cast<int>(((n + 31) / 32 + 3) & ~int64_t{3}) * 4 + 16 * nt * tbytes;
}

// Exclusive scan of one int per thread over NT threads (wsum: NT / 64 ints of LDS; NT = 64: a
// wave scan, no LDS and no barrier). A barrier must come before wsum is written again.
template <int NT>
__device__ __forceinline__ int block_excl_i32(int v, int* wsum) {
  const int incl = wave_incl_i32(v);
  if constexpr (NT == kWave) {
    return incl - v;
  } else {
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    if (lane == kWave - 1) wsum[wave] = incl;
    __syncthreads();
    int before = 0;
    for (int w2 = 0; w2 < wave; ++w2) before += wsum[w2];
    return before + incl - v;
  }
}

// The row's final hull h (row_bad: a NaN row) expanded by NT threads, with x.lds_bytes of LDS
// at lds (at least expand_lds_min). The hull's vertices become a bitmap of the row's elements in
// LDS, and per bitmap word the vertices before it (one scan), from which an element's edge (the
// vertices at or before it, less one) and a tile's records (its first and last edges, as
// rank_kernel's searches find them) follow without a search; the start bits are the bitmap; the
// fit, 16 * NT elements a pass, is each edge's slope rounded once, signed and clamped as the
// expansion kernels form it, from a table of the edges' values in LDS, restaged where a pass needs
// edges past the table (a row's hull can have a vertex every element). Each thread stores pieces
// of 16 bytes, every store instruction of a wave on one contiguous 1 KiB.
template <typename T, bool W, bool MAP, int NT>
__device__ void expand_row(const RowExpand& x, const NodeOut& h, bool row_bad, int64_t row, char* lds) {
  constexpr int E = 16;              // elements a thread a pass
  constexpr int V = 16 / sizeof(T);  // elements a 16-byte store
  constexpr int G = E / V;           // stores a thread a pass
  constexpr int kStep = E * NT;      // elements a pass
  const int tid = threadIdx.x;
  __syncthreads();  // the hull written (and repaired) by every thread, the LDS read
  const int n = static_cast<int>(x.n);
  const int cnt = *h.count;
  const VArr hv = dvarr_of(h);
  const int words = (n + 31) / 32;
  const int words4 = (words + 3) & ~3;
  int* wsum = reinterpret_cast<int*>(lds);  // (16 ints)
  uint32_t* vbits = reinterpret_cast<uint32_t*>(lds + 64);
  int* wpre = reinterpret_cast<int*>(vbits + words4);
  T* tab = reinterpret_cast<T*>(wpre + words4);
  const int cap = (x.lds_bytes - 64 - 2 * words4 * static_cast<int>(sizeof(uint32_t))) / static_cast<int>(sizeof(T));
  // the bitmap (a NaN row's too: its records come from its hull as any row's)
  for (int k = tid; k < words; k += NT) vbits[k] = 0u;
  __syncthreads();
  for (int e = tid; e < cnt - 1; e += NT) {
    const int p = hv.idx[e];
    atomicOr(&vbits[p >> 5], 1u << (p & 31));
  }
  __syncthreads();
  // vertices before each word: thread t counts words [t * wl, t * wl + wl)
  {
    const int wl = (words + NT - 1) / NT;
    const int k0 = min(tid * wl, words), k1 = min(k0 + wl, words);
    int c = 0;
    for (int k = k0; k < k1; ++k) c += __popc(vbits[k]);
    int ex = block_excl_i32<NT>(c, wsum);
    for (int k = k0; k < k1; ++k) {
      wpre[k] = ex;
      ex += __popc(vbits[k]);
    }
  }
  __syncthreads();
  // vertices at positions below i (i < n)
  auto below = [&](int i) { return wpre[i >> 5] + __popc(vbits[i >> 5] & ((1u << (i & 31)) - 1u)); };
  // the start bits (a NaN row: its first element only)
  if (x.starts != nullptr)
    for (int k = tid; k < words; k += NT) x.starts[row * words + k] = row_bad ? (k == 0 ? 1u : 0u) : vbits[k];
  // tile records: ra, the last vertex at or before the tile's first element; rb, the first at or
  // after its end (the row's end vertex, cnt - 1, for the last tile)
  for (int64_t t = tid; t < x.tpr; t += NT) {
    const int ta = static_cast<int>(t * x.tile_n);
    const int tb = min(ta + x.tile_n, n);
    const bool at_vertex = (vbits[ta >> 5] >> (ta & 31)) & 1u;
    TileRec r;
    r.ra = below(ta) + (at_vertex ? 1 : 0) - 1;
    r.rb = tb == n ? cnt - 1 : below(tb);
    r.last = cnt - 1;
    const bool head = row_bad ? ta == 0 : at_vertex;
    r.flags = (row_bad ? kTileBad : 0) | (head ? kTileHead : 0);
    r.slope = 0.0;
    r.unused = 0.0;
    if (!row_bad && r.rb == r.ra + 1) {
      double dW, dS;
      vdiff<W>(vload<W>(hv, r.ra), vload<W>(hv, r.ra + 1), dW, dS);
      r.slope = slope_div(dS, dW);
    }
    x.tiles[row * x.tpr + t] = r;
  }
  // the fit (ragged rows: the row's own elements, at their packed place)
  int64_t xfirst = row * x.n, xlen = x.n;
  if constexpr (MAP) map_row(x.map, row, x.n, xfirst, xlen);
  T* const out = static_cast<T*>(x.out) + xfirst;
  const int lim = static_cast<int>(xlen);
  if (row_bad) {
    const T nanv = quiet_nan<T>();
    for (int i = tid; i < lim; i += NT) out[i] = nanv;
    return;
  }
  const T tsgn = static_cast<T>((x.flags & TI_INCREASING) ? 1.0 : -1.0);
  const bool use_lo = x.flags & TI_CLIP_MIN, use_hi = x.flags & TI_CLIP_MAX;
  const bool nts = x.flags & TI_STREAM_OUT;
  const T lo = static_cast<T>(x.lo), hi = static_cast<T>(x.hi);
  auto stage = [&](int e0) {  // edges [e0, e0 + cap) of the row's cnt - 1
    const int e1 = min(cnt - 1, e0 + cap);
    for (int e = e0 + tid; e < e1; e += NT) {
      double dW, dS;
      vdiff<W>(vload<W>(hv, e), vload<W>(hv, e + 1), dW, dS);
      tab[e - e0] = clip(tsgn * static_cast<T>(slope_div(dS, dW)), use_lo, lo, use_hi, hi);
    }
  };
  int e0 = 0;
  stage(0);
  __syncthreads();
  const bool aligned = (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  for (int c = 0; c < n; c += kStep) {
    if (cnt - 1 > cap) {
      // the pass's edges: from its first element's, f, to at most f + kStep - 1 (and cnt - 2);
      // the table restaged from f where it ends short of them
      const int f = below(c) + static_cast<int>((vbits[c >> 5] >> (c & 31)) & 1u) - 1;
      if (min(f + kStep, cnt - 1) > e0 + cap) {
        __syncthreads();
        e0 = f;
        stage(e0);
        __syncthreads();
      }
    }
    // every piece's bitmap word and count read at once, then every element's table entry (a
    // piece past n reads the pass's first element's, in the table, and stores nothing); a
    // piece's V elements lie in one bitmap word (c is a multiple of kStep)
    int g0[G];
    uint32_t wb[G];
    int cum[G];
#pragma unroll
    for (int j = 0; j < G; ++j) {
      g0[j] = c + j * (NT * V) + tid * V;
      const int ii = g0[j] < n ? g0[j] : c;
      wb[j] = vbits[ii >> 5] >> (ii & 31);
      cum[j] = wpre[ii >> 5] + __popc(vbits[ii >> 5] & ((1u << (ii & 31)) - 1u));
    }
    T fit[G][V];
#pragma unroll
    for (int j = 0; j < G; ++j) {
#pragma unroll
      for (int k = 0; k < V; ++k) {
        cum[j] += (wb[j] >> k) & 1u;  // (zero past n: the last edge again)
        fit[j][k] = tab[cum[j] - 1 - e0];
      }
    }
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const int m = lim - g0[j];
      if (m >= V && aligned) {
        using VT = T __attribute__((ext_vector_type(V)));
        VT v;
#pragma unroll
        for (int k = 0; k < V; ++k) v[k] = fit[j][k];
        if (nts) __builtin_nontemporal_store(v, reinterpret_cast<VT*>(out + g0[j]));
        else *reinterpret_cast<VT*>(out + g0[j]) = v;
      } else {
#pragma unroll
        for (int k = 0; k < V; ++k)
          if (k < m) out[g0[j] + k] = fit[j][k];
      }
    }
  }
}

}  // namespace
}  // namespace ti
