// Rows longer than one tile: the cross-span merge and the expansion.
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
//   expand_kernel  per tile of the row: the final hull's vertices around the tile (a 256-ary
//                  search), edge slopes in float64 rounded once, every element the slope of its
//                  edge with the clamp fused, and the start bits. y is not read again.
#include "ti_common.h"
#include "ti_kernels.h"
#include "ti_tile.h"

namespace ti {

namespace {

constexpr int kMergeThreads = 256;
constexpr int kLdsVerts = 2048;  // vertices a merge keeps in LDS

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
  p.s = DD{a.shi[k], a.slo[k]};
  if constexpr (W) p.w = DD{a.whi[k], a.wlo[k]};
  else p.w = DD{static_cast<double>(p.i), 0.0};
  return p;
}

template <bool W>
__device__ __forceinline__ void vstore(const VArr& a, int k, const VPt& p) {
  a.idx[k] = p.i;
  a.shi[k] = p.s.hi;
  a.slo[k] = p.s.lo;
  if constexpr (W) {
    a.whi[k] = p.w.hi;
    a.wlo[k] = p.w.lo;
  }
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

// The vertex of B[1 .. cB) touched by the lower tangent from p (the last of equal slopes).
template <bool W>
__device__ int vtangent(const VArr& v, const VPt& p, int bb, int cB) {
  int lo = 1, hi = cB - 1;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (!vpools<W>(p, vload<W>(v, bb + mid), vload<W>(v, bb + mid + 1))) hi = mid;
    else lo = mid + 1;
  }
  return lo;
}

// Bridge of hulls A = [ba, ba + cA) and B = [bb, bb + cB) sharing their boundary point; the
// merged hull is A[0 .. keep) ++ B[from .. cB). (Same method as the tile kernel's.)
template <bool W>
__device__ void vbridge(const VArr& v, int ba, int cA, int bb, int cB, int& keep, int& from) {
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
  VPt a = vload<W>(v, ba + cA - 2);
  const VPt x = vload<W>(v, ba + cA - 1);
  VPt b = vload<W>(v, bb + 1);
  if (!vpools<W>(a, x, b)) {
    keep = cA;
    from = 1;
    return;
  }
  int i = cA - 2, j = 1;
  bool done = false;
  VPt ap = i > 0 ? vload<W>(v, ba + i - 1) : a;
  VPt bn = j + 1 < cB ? vload<W>(v, bb + j + 1) : b;
  for (int steps = 0; steps < 24; ++steps) {
    if (i > 0 && vpools<W>(ap, a, b)) {
      --i;
      a = ap;
      if (i > 0) ap = vload<W>(v, ba + i - 1);
    } else if (j + 1 < cB && vpools<W>(a, b, bn)) {
      ++j;
      b = bn;
      if (j + 1 < cB) bn = vload<W>(v, bb + j + 1);
    } else {
      done = true;
      break;
    }
  }
  if (!done) {
    int lo = 0, hi = cA - 2;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      const VPt am = vload<W>(v, ba + mid);
      const int t = vtangent<W>(v, am, bb, cB);
      if (vpools<W>(am, vload<W>(v, ba + mid + 1), vload<W>(v, bb + t))) hi = mid;
      else lo = mid + 1;
    }
    i = lo;
    j = vtangent<W>(v, vload<W>(v, ba + lo), bb, cB);
  }
  keep = i + 1;
  from = j;
}

__device__ VArr dvarr_of(const NodeOut& o) { return VArr{o.idx, o.shi, o.slo, o.whi, o.wlo}; }

template <bool W>
struct MergeShared {
  int idx[kLdsVerts];
  double shi[kLdsVerts], slo[kLdsVerts];
  double whi[W ? kLdsVerts : 1], wlo[W ? kLdsVerts : 1];
  int cnt[kGroup], off[kGroup];       // per child: vertex count, first slot
  double tot[4][kGroup + 1];          // per child offsets (W hi, lo, S hi, lo); [nch]: total
  int keep[kGroup / 2], from[kGroup / 2];
  int maxlen;
  int bad;
};

template <bool W>
__global__ __launch_bounds__(kMergeThreads) void merge_kernel(MergeArgs a) {
  __shared__ MergeShared<W> sh;
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x / a.npr_out;
  const int64_t j = blockIdx.x - row * a.npr_out;
  const int64_t c0 = j * kGroup;  // first child within the row
  const int nch = static_cast<int>(min<int64_t>(kGroup, a.npr_in - c0));
  const NodeOut pout = node_out(a.out, a.k_out, a.cap_out, W, row * a.npr_out + j);

  // Children: counts, NaN flags, and offsets within the parent (double-double scan).
  if (tid < kWave) {
    int cnt = 0, bad = 0;
    DD tw{0.0, 0.0}, ts{0.0, 0.0};
    if (tid < nch) {
      const NodeOut ci = node_out(const_cast<void*>(a.in), a.k_in, a.cap_in, W, row * a.npr_in + c0 + tid);
      cnt = *ci.count;
      bad = *ci.bad;
      tw = DD{ci.tot[0], ci.tot[1]};
      ts = DD{ci.tot[2], ci.tot[3]};
    }
    // inclusive scans: totals (dd) and slots (count - 1, the shared point stored once)
    DD iw = tw, is = ts;
    int islot = max(cnt - 1, 0);
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      DD ow{__shfl_up(iw.hi, d, kWave), __shfl_up(iw.lo, d, kWave)};
      DD os{__shfl_up(is.hi, d, kWave), __shfl_up(is.lo, d, kWave)};
      const int oslot = __shfl_up(islot, d, kWave);
      if (tid >= d) {
        iw = dd_add(ow, iw);
        is = dd_add(os, is);
        islot += oslot;
      }
    }
    const int anybad = __any(bad != 0);
    DD ew{__shfl_up(iw.hi, 1, kWave), __shfl_up(iw.lo, 1, kWave)};
    DD es{__shfl_up(is.hi, 1, kWave), __shfl_up(is.lo, 1, kWave)};
    if (tid == 0) ew = es = DD{0.0, 0.0};
    if (tid < nch) {
      sh.cnt[tid] = cnt;
      sh.off[tid] = islot - max(cnt - 1, 0);
      sh.tot[0][tid] = ew.hi;
      sh.tot[1][tid] = ew.lo;
      sh.tot[2][tid] = es.hi;
      sh.tot[3][tid] = es.lo;
    }
    if (tid == nch - 1) {
      sh.tot[0][nch] = iw.hi;
      sh.tot[1][nch] = iw.lo;
      sh.tot[2][nch] = is.hi;
      sh.tot[3][nch] = is.lo;
      sh.maxlen = islot + 1;  // total slots
    }
    if (tid == 0) sh.bad = anybad;
  }
  __syncthreads();
  const int total = sh.maxlen;
  const bool in_lds = total <= kLdsVerts;
  VArr v;
  if (in_lds) v = VArr{sh.idx, sh.shi, sh.slo, W ? sh.whi : nullptr, W ? sh.wlo : nullptr};
  else v = dvarr_of(pout);

  // Lay the children end to end (each child's first vertex is the previous child's last,
  // stored once), in coordinates relative to the parent: one thread per slot, its child found
  // by a binary search over the children's first slots.
  for (int s = tid; s < total; s += kMergeThreads) {
    int lo = 0, hi = nch - 1;  // the last child whose first slot is below s (child 0 for s = 0)
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (sh.off[mid] < s) lo = mid;
      else hi = mid - 1;
    }
    const int c = lo, k = s - sh.off[c];
    const NodeOut ci = node_out(const_cast<void*>(a.in), a.k_in, a.cap_in, W, row * a.npr_in + c0 + c);
    const DD ow{sh.tot[0][c], sh.tot[1][c]}, os{sh.tot[2][c], sh.tot[3][c]};
    VPt p;
    p.i = ci.idx[k] + static_cast<int>(c * a.child_elems);
    p.s = dd_add(os, DD{ci.shi[k], ci.slo[k]});
    if constexpr (W) p.w = dd_add(ow, DD{ci.whi[k], ci.wlo[k]});
    vstore<W>(v, s, p);
  }
  __syncthreads();

  // Pairwise rounds.
#pragma unroll 1
  for (int span = 1; span < nch; span <<= 1) {
    const int nm = (nch + 2 * span - 1) / (2 * span);  // merges this round
    if (tid < nm) {
      const int pa = tid * 2 * span, pb = pa + span;
      int keep = sh.cnt[pa], from = 0;
      if (pb < nch) {
        vbridge<W>(v, sh.off[pa], sh.cnt[pa], sh.off[pb], sh.cnt[pb], keep, from);
      }
      sh.keep[tid] = keep;
      sh.from[tid] = from;
    }
    __syncthreads();
    // Move each right part's kept suffix next to its left part's kept prefix.
    const int gsz = kMergeThreads / nm >= 1 ? kMergeThreads / nm : 1;
    const int m = tid / gsz;
    const int r = tid - m * gsz;
    int len = 0, src = 0, dst = 0;
    if (m < nm) {
      const int pa = m * 2 * span, pb = pa + span;
      if (pb < nch) {
        len = sh.cnt[pb] - sh.from[m];
        src = sh.off[pb] + sh.from[m];
        dst = sh.off[pa] + sh.keep[m];
        if (src == dst) len = 0;
      }
    }
    // rounds: every thread reads its share into registers, then writes (src is never below dst)
    __shared__ int rounds_max;
    if (tid == 0) rounds_max = 0;
    __syncthreads();
    constexpr int R = 4;
    const int my_rounds = (len + gsz * R - 1) / (gsz * R);
    if (my_rounds > 0) atomicMax(&rounds_max, my_rounds);
    __syncthreads();
    const int rounds = rounds_max;
    for (int rd = 0; rd < rounds; ++rd) {
      VPt buf[R];
#pragma unroll
      for (int q = 0; q < R; ++q) {
        const int jj = rd * gsz * R + q * gsz + r;
        if (jj < len) buf[q] = vload<W>(v, src + jj);
      }
      __syncthreads();
#pragma unroll
      for (int q = 0; q < R; ++q) {
        const int jj = rd * gsz * R + q * gsz + r;
        if (jj < len) vstore<W>(v, dst + jj, buf[q]);
      }
      __syncthreads();
    }
    if (tid < nm) {
      const int pa = tid * 2 * span, pb = pa + span;
      if (pb < nch) sh.cnt[pa] = sh.keep[tid] + (sh.cnt[pb] - sh.from[tid]);
    }
    __syncthreads();
  }

  // The parent's hull.
  const int hull = sh.cnt[0];
  if (in_lds) {
    for (int k = tid; k < hull; k += kMergeThreads) vstore<W>(dvarr_of(pout), k, vload<W>(v, k));
  }
  if (tid == 0) {
    *pout.count = hull;
    *pout.bad = sh.bad;
    pout.tot[0] = sh.tot[0][nch];
    pout.tot[1] = sh.tot[1][nch];
    pout.tot[2] = sh.tot[2][nch];
    pout.tot[3] = sh.tot[3][nch];
  }
}

// Per tile: the fit from the row's final hull.
template <typename T, bool W>
__global__ __launch_bounds__(256) void expand_kernel(ExpandArgs a) {
  using C = TileCfg<W>;
  constexpr int E = C::kE;
  constexpr int NT = C::kThreads;
  __shared__ double sl[C::kN + 2];
  __shared__ uint32_t bits[C::kN / 32];
  __shared__ int lo_s, hi_s, rank_scan[kWaves256];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int64_t row = blockIdx.x / a.tiles_per_row;
  const int64_t tile = blockIdx.x - row * a.tiles_per_row;
  const int64_t first = tile * C::kN;
  const int len = static_cast<int>(min<int64_t>(C::kN, a.n - first));
  const NodeOut fin = node_out(const_cast<void*>(a.hulls), a.batch, a.cap, W, row);
  const VArr v = dvarr_of(fin);
  const int count = *fin.count;
  const bool row_bad = *fin.bad != 0;
  const int ta = static_cast<int>(first), tb = static_cast<int>(first + len);

  // rA: the last vertex at or before the tile's first element; rB: the first at or after its
  // end. 256-ary search over the final hull's indices.
  if (tid == 0) {
    lo_s = 0;
    hi_s = count - 1;
  }
  __syncthreads();
  // (the indices strictly increase, so one sub-range always brackets ta; at most
  // ceil(log_256(count)) rounds, bounded by 8 in any case)
  for (int it = 0; it < 8; ++it) {
    const int lo = lo_s, hi = hi_s;  // invariant: idx[lo] <= ta < idx[hi] (or lo == hi)
    __syncthreads();
    if (hi - lo <= 1) break;
    const int64_t span = hi - lo;
    const int p = lo + static_cast<int>((span * tid) / NT);
    const int q = lo + static_cast<int>((span * (tid + 1)) / NT);
    if (p < q) {
      const int ip = v.idx[p];
      const int iq = v.idx[q];
      if (ip <= ta && ta < iq) {
        lo_s = p;
        hi_s = q;
      }
    }
    __syncthreads();
  }
  const int rA = lo_s;
  // rB: first vertex with idx >= tb, searching from rA
  __syncthreads();
  if (tid == 0) {
    lo_s = rA;
    hi_s = count - 1;
  }
  __syncthreads();
  for (int it = 0; it < 8; ++it) {
    const int lo = lo_s, hi = hi_s;  // invariant: idx[lo] < tb <= idx[hi] (or lo == hi)
    __syncthreads();
    if (hi - lo <= 1) break;
    const int64_t span = hi - lo;
    const int p = lo + static_cast<int>((span * tid) / NT);
    const int q = lo + static_cast<int>((span * (tid + 1)) / NT);
    if (p < q) {
      const int ip = v.idx[p];
      const int iq = v.idx[q];
      if (ip < tb && tb <= iq) {
        lo_s = p;
        hi_s = q;
      }
    }
    __syncthreads();
  }
  int rB = v.idx[lo_s] >= tb ? lo_s : hi_s;
  rB = min(rB, rA + C::kN + 1);  // holds for any well-formed hull; keeps sl[] in bounds regardless
  if (a.tile_rank != nullptr && tid == 0) {
    a.tile_rank[2 * blockIdx.x] = rA;
    a.tile_rank[2 * blockIdx.x + 1] = rB;
  }

  // Edge slopes rA .. rB-1 and the vertex bits of the tile.
  for (int wd = tid; wd < C::kN / 32; wd += NT) bits[wd] = 0u;
  __syncthreads();
  for (int e = rA + tid; e < rB; e += NT) {
    const VPt p = vload<W>(v, e), q = vload<W>(v, e + 1);
    double dW, dS;
    vdiff<W>(p, q, dW, dS);
    sl[e - rA] = slope_div(dS, dW);
    if (p.i >= ta) atomicOr(&bits[(p.i - ta) >> 5], 1u << ((p.i - ta) & 31));
  }
  __syncthreads();
  const int t0 = tid * E;
  const int ecount = max(0, min(E, len - t0));
  uint32_t mybits;
  if constexpr (E == 16) mybits = (bits[t0 >> 5] >> (t0 & 31)) & 0xFFFFu;
  else mybits = (bits[t0 >> 5] >> (t0 & 31)) & 0xFFu;
  const int pc = __builtin_popcount(mybits);
  int incl = pc;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int o = __shfl_up(incl, d, kWave);
    if (lane >= d) incl += o;
  }
  if (lane == kWave - 1) rank_scan[wave] = incl;
  __syncthreads();
  int before = incl - pc;
  for (int w2 = 0; w2 < wave; ++w2) before += rank_scan[w2];
  const int at_start = (v.idx[rA] == ta) ? 1 : 0;
  int jj = before + static_cast<int>(mybits & 1u) - at_start;
  const bool use_lo = a.flags & TI_CLIP_MIN, use_hi = a.flags & TI_CLIP_MAX;
  const T lo = static_cast<T>(a.lo), hi = static_cast<T>(a.hi);
  const T tsgn = static_cast<T>((a.flags & TI_INCREASING) ? 1.0 : -1.0);
  T fit[E];
#pragma unroll
  for (int k = 0; k < E; ++k) {
    if (k > 0) jj += (mybits >> k) & 1u;
    const T val = row_bad ? quiet_nan<T>() : tsgn * static_cast<T>(sl[jj]);
    fit[k] = clip(val, use_lo, lo, use_hi, hi);
  }
  T* out = static_cast<T*>(a.out) + row * a.n + first;
  store_elems_any<T, E>(out + t0, ecount, fit);
  if (a.starts != nullptr && ecount > 0) {
    uint32_t sb = row_bad ? ((first + t0) == 0 ? 1u : 0u) : mybits;
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
}

}  // namespace

LongPlan long_plan(int64_t batch, int64_t n, bool weighted) {
  LongPlan p{};
  const int64_t tn = tile_elems(weighted);
  p.tiles_per_row = (n + tn - 1) / tn;
  int64_t npr = (n + kSpan - 1) / kSpan;
  int64_t span = kSpan;  // elements per node at this level
  size_t buf[2] = {0, 0};
  int level = 0;
  for (;;) {
    const int64_t cap = (span < n ? span : n) + 1;
    p.npr[level] = npr;
    p.cap[level] = cap;
    p.span[level] = span;
    const size_t bytes = node_array_bytes(batch * npr, cap, weighted);
    buf[level & 1] = buf[level & 1] > bytes ? buf[level & 1] : bytes;
    if (npr == 1) break;
    npr = (npr + kGroup - 1) / kGroup;
    span *= kGroup;
    ++level;
  }
  p.levels = level;  // merge launches; the final hulls are at level p.levels
  p.off_buf[0] = 0;
  p.off_buf[1] = align256(buf[0]);
  p.off_rank = p.off_buf[1] + align256(buf[1]);
  p.bytes = p.off_rank + align256(static_cast<size_t>(batch * p.tiles_per_row) * 8);
  return p;
}

hipError_t long_fit(const TileArgs& t, const LongPlan& p, void* ws) {
  const bool W = t.w != nullptr;
  char* base = static_cast<char*>(ws);
  // level 0: span hulls
  hipError_t e = span_run(t, base + p.off_buf[0], p.npr[0], p.cap[0]);
  if (e != hipSuccess) return e;
  for (int l = 1; l <= p.levels; ++l) {
    MergeArgs m;
    m.in = base + p.off_buf[(l - 1) & 1];
    m.k_in = t.batch * p.npr[l - 1];
    m.cap_in = p.cap[l - 1];
    m.npr_in = p.npr[l - 1];
    m.out = base + p.off_buf[l & 1];
    m.k_out = t.batch * p.npr[l];
    m.cap_out = p.cap[l];
    m.npr_out = p.npr[l];
    m.child_elems = p.span[l - 1];
    const unsigned grid = static_cast<unsigned>(t.batch * p.npr[l]);
    if (W) merge_kernel<true><<<dim3(grid), dim3(kMergeThreads), 0, t.stream>>>(m);
    else merge_kernel<false><<<dim3(grid), dim3(kMergeThreads), 0, t.stream>>>(m);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  ExpandArgs x;
  x.hulls = base + p.off_buf[p.levels & 1];
  x.batch = t.batch;
  x.cap = p.cap[p.levels];
  x.n = t.n;
  x.tiles_per_row = p.tiles_per_row;
  x.out = t.out;
  x.starts = t.starts;
  x.tile_rank = reinterpret_cast<int*>(base + p.off_rank);
  x.flags = t.flags;
  x.lo = t.lo;
  x.hi = t.hi;
  const unsigned grid = static_cast<unsigned>(t.batch * p.tiles_per_row);
  if (t.dtype == TI_F32) {
    if (W) expand_kernel<float, true><<<dim3(grid), dim3(256), 0, t.stream>>>(x);
    else expand_kernel<float, false><<<dim3(grid), dim3(256), 0, t.stream>>>(x);
  } else {
    if (W) expand_kernel<double, true><<<dim3(grid), dim3(256), 0, t.stream>>>(x);
    else expand_kernel<double, false><<<dim3(grid), dim3(256), 0, t.stream>>>(x);
  }
  return hipGetLastError();
}

}  // namespace ti
