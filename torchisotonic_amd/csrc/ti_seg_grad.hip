// The reference's stateless gradient operator (ti_grad): gradients of a fit from the fit, its
// partition and the upstream gradient alone, for rows of any length.
//
// Replaces torchisotonic::isotonic_grad (reference src/torchisotonic/csrc/grad.cuh:304-413:
// tile-end summaries, an ATen scan over tiles, a fill kernel). Every element needs G and W, the
// sums of g and w over its block. The [batch, n] problem set is taken as ONE sequence of
// batch * n elements with a block start forced at every row's first element (a block never
// crosses a row), cut into tiles of 2048 elements, 8 consecutive elements a thread:
//
//   seg_ends_kernel    per tile: its "head" (the sums over the elements before its first start;
//                      the whole tile if it holds none), its "tail" (from its last start to its
//                      end) and whether it holds a start. Only the threads that overlap the
//                      head or the tail read g and w; where blocks are short the kernel reads
//                      little beyond the start bits, and a tile without a start is summed
//                      plainly.
//   seg_scan_kernel    per group of 256 tiles: segmented scans of the tile summaries, forward
//                      (a block's sum before a tile: the previous tile's tail, plus the heads of
//                      start-free tiles before it) and backward (after a tile: the following
//                      heads up to the first tile with a start); the group's aggregates.
//   seg_groups_kernel  one workgroup: the same scans over the groups.
//   seg_fill_kernel    per tile: within each thread, the sum over each block's elements there;
//                      across the workgroup, the same segmented scans over the threads (seeded
//                      with the tile's carries from both sides); then gy = w G / W and
//                      gw = (y - fit) G / W. A tile without a start lies inside one block whose
//                      sums the carries and its total give: it reads w (and y, fit) only.
// A problem set of one tile runs seg_fill_kernel alone. Sums are float64 within a thread and
// double-double across threads, tiles and groups.
#include <type_traits>

#include "ti_common.h"
#include "ti_kernels.h"
#include "ti_tile.h"

namespace ti {

namespace {

constexpr int kSegE = 8;                            // elements a thread
constexpr int kSegThreads = 256;                    // threads a tile
constexpr int kSegTile = kSegE * kSegThreads;       // elements a tile
constexpr int kSegGroup = 256;                      // tiles a scan group
constexpr int kSegWaves = kSegThreads / kWave;

// Segmented state over a stretch of elements for two quantities (g and w), double-double:
// f = the stretch holds a block start. Forward states carry the sums after the stretch's last
// start (the whole stretch if none); backward states the sums before its first start.
struct SegSt {
  int f;
  DD v[2];
};

__device__ __forceinline__ SegSt seg_zero() { return SegSt{0, {DD{0.0, 0.0}, DD{0.0, 0.0}}}; }

// a is earlier, b later: the forward state of the two stretches together
__device__ __forceinline__ SegSt comb_fwd(const SegSt& a, const SegSt& b) {
  SegSt r;
  r.f = a.f | b.f;
#pragma unroll
  for (int q = 0; q < 2; ++q) r.v[q] = b.f ? b.v[q] : dd_add(a.v[q], b.v[q]);
  return r;
}

// a is earlier, b later: the backward state of the two stretches together
__device__ __forceinline__ SegSt comb_bwd(const SegSt& a, const SegSt& b) {
  SegSt r;
  r.f = a.f | b.f;
#pragma unroll
  for (int q = 0; q < 2; ++q) r.v[q] = a.f ? a.v[q] : dd_add(a.v[q], b.v[q]);
  return r;
}

__device__ __forceinline__ SegSt shfl_up_st(const SegSt& s, int d) {
  SegSt r;
  r.f = __shfl_up(s.f, d, kWave);
#pragma unroll
  for (int q = 0; q < 2; ++q) r.v[q] = DD{__shfl_up(s.v[q].hi, d, kWave), __shfl_up(s.v[q].lo, d, kWave)};
  return r;
}

__device__ __forceinline__ SegSt shfl_down_st(const SegSt& s, int d) {
  SegSt r;
  r.f = __shfl_down(s.f, d, kWave);
#pragma unroll
  for (int q = 0; q < 2; ++q) r.v[q] = DD{__shfl_down(s.v[q].hi, d, kWave), __shfl_down(s.v[q].lo, d, kWave)};
  return r;
}

struct SegArgs {
  const void* fit;
  const uint32_t* starts;
  const void* g;
  const void* w;  // null: weights of one
  const void* y;  // null: no weight gradient
  void* gy;
  void* gw;
  int64_t n, total, ntiles, ngroups;
  bool flat;  // one row, or rows of a multiple of 32 elements: bit e of the set is bit e % 32 of word e / 32
  // workspace (null for a problem set of one tile)
  SegSt* tfwd;   // [ntiles] per tile: forward state (tail, or the whole tile)
  SegSt* tbwd;   // [ntiles] per tile: backward state (head)
  SegSt* cfwd;   // [ntiles] per tile: forward state of the tiles before it in its group
  SegSt* cbwd;   // [ntiles] per tile: backward state of the tiles after it in its group
  SegSt* gfwd;   // [ngroups] per group: its forward aggregate, then the carry into it from the left
  SegSt* gbwd;   // [ngroups] per group: its backward aggregate, then the carry into it from the right
};

// The start bits of a thread's kSegE elements from flat index e0 (bit k: element e0 + k starts a
// block; row starts included), and how many of them exist.
__device__ __forceinline__ uint32_t thread_starts(const SegArgs& a, int64_t e0, int& count) {
  count = static_cast<int>(max<int64_t>(0, min<int64_t>(kSegE, a.total - e0)));
  if (count == 0) return 0u;
  if (a.flat) {
    // one word holds the thread's bits (e0 is a multiple of kSegE, which divides 32), and a row
    // start can fall only on e0 (rows are one, or a multiple of 32 elements long)
    static_assert(32 % kSegE == 0, "a thread's start bits lie in one word");
    uint32_t sb = (a.starts[e0 >> 5] >> (e0 & 31)) & ((1u << kSegE) - 1u);
    if (count < kSegE) sb &= (1u << count) - 1u;
    // e0 % n without a 64-bit division: the quotient from float64 (exact to one either way)
    int64_t q = static_cast<int64_t>(static_cast<double>(e0) / static_cast<double>(a.n));
    int64_t r = e0 - q * a.n;
    r = r < 0 ? r + a.n : (r >= a.n ? r - a.n : r);
    return sb | (r == 0 ? 1u : 0u);
  }
  const int64_t wpr = (a.n + 31) / 32;
  int64_t row = e0 / a.n;
  int64_t i = e0 - row * a.n;
  uint32_t sb = 0;
#pragma unroll
  for (int k = 0; k < kSegE; ++k) {
    if (k < count) {
      const uint32_t bit = i == 0 ? 1u : (a.starts[row * wpr + (i >> 5)] >> (i & 31)) & 1u;
      sb |= bit << k;
      if (++i == a.n) {
        i = 0;
        ++row;
      }
    }
  }
  return sb;
}

template <typename T, bool W>
__device__ __forceinline__ void load_gw(const SegArgs& a, int64_t e0, int count, double (&v)[2][kSegE]) {
  T gv[kSegE], wv[W ? kSegE : 1];
  load_elems_any<T, kSegE>(static_cast<const T*>(a.g) + e0, count, gv);
  if constexpr (W) load_elems_any<T, kSegE>(static_cast<const T*>(a.w) + e0, count, wv);
#pragma unroll
  for (int k = 0; k < kSegE; ++k) {
    const bool ok = k < count;
    v[0][k] = ok ? static_cast<double>(gv[k]) : 0.0;
    v[1][k] = ok ? (W ? static_cast<double>(wv[W ? k : 0]) : 1.0) : 0.0;
  }
}

// Sum over the workgroup (double-double), for thread 0. `red` holds kSegWaves entries.
__device__ __forceinline__ void block_sum2(DD (&v)[2], DD (*red)[2]) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
#pragma unroll
  for (int d = kWave / 2; d >= 1; d >>= 1) {
#pragma unroll
    for (int q = 0; q < 2; ++q)
      v[q] = dd_add(v[q], DD{__shfl_xor(v[q].hi, d, kWave), __shfl_xor(v[q].lo, d, kWave)});
  }
  if (lane == 0) {
    red[wave][0] = v[0];
    red[wave][1] = v[1];
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w2 = 1; w2 < kSegWaves; ++w2) {
      v[0] = dd_add(v[0], red[w2][0]);
      v[1] = dd_add(v[1], red[w2][1]);
    }
  }
}

template <typename T, bool W>
__global__ __launch_bounds__(kSegThreads) void seg_ends_kernel(SegArgs a) {
  __shared__ int first_start, last_start;
  __shared__ DD red[2][kSegWaves][2];
  const int tid = threadIdx.x;
  const int64_t tile = blockIdx.x;
  const int64_t base = tile * kSegTile;
  const int len = static_cast<int>(min<int64_t>(kSegTile, a.total - base));
  const int64_t e0 = base + tid * kSegE;
  if (tid == 0) {
    first_start = len;
    last_start = -1;
  }
  __syncthreads();
  int count;
  const uint32_t sb = thread_starts(a, e0, count);
  if (sb != 0) {
    atomicMin(&first_start, tid * kSegE + __builtin_ctz(sb));
    atomicMax(&last_start, tid * kSegE + 31 - __builtin_clz(sb));
  }
  __syncthreads();
  const int fs = first_start, ls = last_start;
  const int p0 = tid * kSegE;
  DD head[2] = {DD{0.0, 0.0}, DD{0.0, 0.0}}, tail[2] = {DD{0.0, 0.0}, DD{0.0, 0.0}};
  if (ls < 0) {
    // no start in the tile (long blocks: most tiles): its total, each thread's part summed in
    // float64 (double-double for float64 data)
    if (count > 0) {
      double v[2][kSegE];
      load_gw<T, W>(a, e0, count, v);
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        if constexpr (sizeof(T) == 8) {
#pragma unroll
          for (int k = 0; k < kSegE; ++k) head[q] = dd_add(head[q], v[q][k]);
        } else {
          double t = 0.0;
#pragma unroll
          for (int k = 0; k < kSegE; ++k) t += v[q][k];
          head[q] = DD{t, 0.0};
        }
      }
    }
    block_sum2(head, red[0]);
    if (tid == 0) a.tbwd[tile] = a.tfwd[tile] = SegSt{0, {head[0], head[1]}};
    return;
  }
  // (threads with nothing before the first start or after the last one read nothing)
  const bool need = count > 0 && (p0 < fs || p0 + count > ls);
  if (need) {
    double v[2][kSegE];
    load_gw<T, W>(a, e0, count, v);
#pragma unroll
    for (int k = 0; k < kSegE; ++k) {
      const int p = p0 + k;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        if (p < fs) head[q] = dd_add(head[q], v[q][k]);
        if (p >= ls) tail[q] = dd_add(tail[q], v[q][k]);
      }
    }
  }
  block_sum2(head, red[0]);
  block_sum2(tail, red[1]);
  if (tid == 0) {
    a.tbwd[tile] = SegSt{1, {head[0], head[1]}};
    a.tfwd[tile] = SegSt{1, {tail[0], tail[1]}};
  }
}

// Exclusive forward and backward scans of `count` states over a 256-thread workgroup, in order:
// for thread t, the forward state of entries [0, t) and the backward state of (t, count); the
// aggregates of all. `sh` holds 2 * kSegWaves states.
__device__ __forceinline__ void block_scan_st(const SegSt& mine_f, const SegSt& mine_b, SegSt (*sh)[kSegWaves],
                                              SegSt& ex_f, SegSt& ex_b, SegSt& all_f, SegSt& all_b) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  SegSt inc_f = mine_f, inc_b = mine_b;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const SegSt of = shfl_up_st(inc_f, d);
    if (lane >= d) inc_f = comb_fwd(of, inc_f);
    const SegSt ob = shfl_down_st(inc_b, d);
    if (lane + d < kWave) inc_b = comb_bwd(inc_b, ob);
  }
  if (lane == kWave - 1) sh[0][wave] = inc_f;
  if (lane == 0) sh[1][wave] = inc_b;
  __syncthreads();
  SegSt xf = shfl_up_st(inc_f, 1);
  if (lane == 0) xf = seg_zero();
  SegSt xb = shfl_down_st(inc_b, 1);
  if (lane == kWave - 1) xb = seg_zero();
  SegSt pf = seg_zero(), pb = seg_zero();
  for (int w2 = 0; w2 < wave; ++w2) pf = comb_fwd(pf, sh[0][w2]);
  for (int w2 = kSegWaves - 1; w2 > wave; --w2) pb = comb_bwd(sh[1][w2], pb);
  ex_f = comb_fwd(pf, xf);
  ex_b = comb_bwd(xb, pb);
  all_f = seg_zero();
  all_b = seg_zero();
  for (int w2 = 0; w2 < kSegWaves; ++w2) all_f = comb_fwd(all_f, sh[0][w2]);
  for (int w2 = kSegWaves - 1; w2 >= 0; --w2) all_b = comb_bwd(sh[1][w2], all_b);
  __syncthreads();  // sh is reused
}

__global__ __launch_bounds__(kSegThreads) void seg_scan_kernel(SegArgs a) {
  __shared__ SegSt sh[2][kSegWaves];
  const int64_t grp = blockIdx.x;
  const int64_t t = grp * kSegGroup + threadIdx.x;
  const bool ok = t < a.ntiles;
  const SegSt f = ok ? a.tfwd[t] : seg_zero();
  const SegSt b = ok ? a.tbwd[t] : seg_zero();
  SegSt ex_f, ex_b, all_f, all_b;
  block_scan_st(f, b, sh, ex_f, ex_b, all_f, all_b);
  if (ok) {
    a.cfwd[t] = ex_f;
    a.cbwd[t] = ex_b;
  }
  if (threadIdx.x == 0 && a.ngroups > 1) {
    a.gfwd[grp] = all_f;
    a.gbwd[grp] = all_b;
  }
}

// The groups' carries, in place of their aggregates: chunks of 256 groups, forward from the
// first and backward from the last.
__global__ __launch_bounds__(kSegThreads) void seg_groups_kernel(SegArgs a) {
  __shared__ SegSt sh[2][kSegWaves];
  const int tid = threadIdx.x;
  const int64_t chunks = (a.ngroups + kSegThreads - 1) / kSegThreads;
  SegSt carry = seg_zero();
  for (int64_t c = 0; c < chunks; ++c) {
    const int64_t gi = c * kSegThreads + tid;
    const SegSt f = gi < a.ngroups ? a.gfwd[gi] : seg_zero();
    SegSt ex_f, ex_b, all_f, all_b;
    block_scan_st(f, seg_zero(), sh, ex_f, ex_b, all_f, all_b);
    if (gi < a.ngroups) a.gfwd[gi] = comb_fwd(carry, ex_f);
    carry = comb_fwd(carry, all_f);
  }
  carry = seg_zero();
  for (int64_t c = chunks - 1; c >= 0; --c) {
    const int64_t gi = c * kSegThreads + tid;
    const SegSt b = gi < a.ngroups ? a.gbwd[gi] : seg_zero();
    SegSt ex_f, ex_b, all_f, all_b;
    block_scan_st(seg_zero(), b, sh, ex_f, ex_b, all_f, all_b);
    if (gi < a.ngroups) a.gbwd[gi] = comb_bwd(ex_b, carry);
    carry = comb_bwd(all_b, carry);
  }
}

template <typename T, bool W, bool WANT_W>
__global__ __launch_bounds__(kSegThreads) void seg_fill_kernel(SegArgs a) {
  __shared__ SegSt sh[2][kSegWaves];
  const int tid = threadIdx.x;
  const int64_t tile = blockIdx.x;
  const int64_t e0 = tile * kSegTile + tid * kSegE;
  if (a.cfwd != nullptr && a.tbwd[tile].f == 0) {
    // a tile inside one block: its block sums are the carry from the left, the tile's total and
    // the carry from the right, the same for every element, so g is not read again
    const int64_t grp = tile / kSegGroup;
    SegSt cf = a.cfwd[tile], cb = a.cbwd[tile];
    if (a.ngroups > 1) {
      cf = comb_fwd(a.gfwd[grp], cf);
      cb = comb_bwd(cb, a.gbwd[grp]);
    }
    const SegSt tt = a.tbwd[tile];
    const DD G = dd_add(dd_add(cf.v[0], tt.v[0]), cb.v[0]);
    const DD Wt = dd_add(dd_add(cf.v[1], tt.v[1]), cb.v[1]);
    const double q = (G.hi + G.lo) / (Wt.hi + Wt.lo);
    const int count = static_cast<int>(max<int64_t>(0, min<int64_t>(kSegE, a.total - e0)));
    if (count == 0) return;
    T wv[W ? kSegE : 1], yv[WANT_W ? kSegE : 1], fv[WANT_W ? kSegE : 1];
    if constexpr (W) load_elems_any<T, kSegE>(static_cast<const T*>(a.w) + e0, count, wv);
    if constexpr (WANT_W) {
      load_elems_any<T, kSegE>(static_cast<const T*>(a.y) + e0, count, yv);
      load_elems_any<T, kSegE>(static_cast<const T*>(a.fit) + e0, count, fv);
    }
    T oy[kSegE], ow[kSegE];
#pragma unroll
    for (int k = 0; k < kSegE; ++k) {
      oy[k] = static_cast<T>((W ? static_cast<double>(wv[W ? k : 0]) : 1.0) * q);
      if constexpr (WANT_W) ow[k] = static_cast<T>((static_cast<double>(yv[k]) - static_cast<double>(fv[k])) * q);
    }
    store_elems_any<T, kSegE>(static_cast<T*>(a.gy) + e0, count, oy);
    if constexpr (WANT_W) store_elems_any<T, kSegE>(static_cast<T*>(a.gw) + e0, count, ow);
    return;
  }
  int count;
  const uint32_t sb = thread_starts(a, e0, count);
  double v[2][kSegE];
  load_gw<T, W>(a, e0, count, v);
  T yv[WANT_W ? kSegE : 1], fv[WANT_W ? kSegE : 1];
  if constexpr (WANT_W) {
    load_elems_any<T, kSegE>(static_cast<const T*>(a.y) + e0, count, yv);
    load_elems_any<T, kSegE>(static_cast<const T*>(a.fit) + e0, count, fv);
  }
  // within the thread: the running sums (reset at starts), the head and the tail
  double run[2][kSegE];
  SegSt mine_f = seg_zero(), mine_b = seg_zero();
  mine_f.f = mine_b.f = sb != 0 ? 1 : 0;
  {
    double r0 = 0.0, r1 = 0.0;
#pragma unroll
    for (int k = 0; k < kSegE; ++k) {
      if ((sb >> k) & 1u) {
        if ((sb & ((1u << k) - 1u)) == 0) {  // the thread's first start: what came before is its head
          mine_b.v[0] = DD{r0, 0.0};
          mine_b.v[1] = DD{r1, 0.0};
        }
        r0 = 0.0;
        r1 = 0.0;
      }
      r0 += v[0][k];
      r1 += v[1][k];
      run[0][k] = r0;
      run[1][k] = r1;
    }
    mine_f.v[0] = DD{r0, 0.0};
    mine_f.v[1] = DD{r1, 0.0};
    if (sb == 0) mine_b = mine_f;
  }
  SegSt ex_f, ex_b, all_f, all_b;
  block_scan_st(mine_f, mine_b, sh, ex_f, ex_b, all_f, all_b);
  // the tile's own carries, from the tiles before and after it
  if (a.cfwd != nullptr) {
    const int64_t grp = tile / kSegGroup;
    SegSt cf = a.cfwd[tile], cb = a.cbwd[tile];
    if (a.ngroups > 1) {
      cf = comb_fwd(a.gfwd[grp], cf);
      cb = comb_bwd(cb, a.gbwd[grp]);
    }
    ex_f = comb_fwd(cf, ex_f);
    ex_b = comb_bwd(ex_b, cb);
  }
  // each element's block sums: its sum within the thread (the running sum at the block's last
  // element here), plus the carry from the left if the block began before the thread, plus the
  // carry from the right if it goes on after it
  T oy[kSegE], ow[kSegE];
  double blk0 = run[0][kSegE - 1], blk1 = run[1][kSegE - 1];
#pragma unroll
  for (int k = kSegE - 1; k >= 0; --k) {
    if (k + 1 < kSegE && ((sb >> (k + 1)) & 1u)) {
      blk0 = run[0][k];
      blk1 = run[1][k];
    }
    const bool from_left = (sb & ((2u << k) - 1u)) == 0;
    const bool to_right = (sb >> (k + 1)) == 0;
    DD G{blk0, 0.0}, Wt{blk1, 0.0};
    if (from_left) {
      G = dd_add(ex_f.v[0], G);
      Wt = dd_add(ex_f.v[1], Wt);
    }
    if (to_right) {
      G = dd_add(G, ex_b.v[0]);
      Wt = dd_add(Wt, ex_b.v[1]);
    }
    const double q = (G.hi + G.lo) / (Wt.hi + Wt.lo);
    oy[k] = static_cast<T>(v[1][k] * q);
    if constexpr (WANT_W) ow[k] = static_cast<T>((static_cast<double>(yv[k]) - static_cast<double>(fv[k])) * q);
  }
  store_elems_any<T, kSegE>(static_cast<T*>(a.gy) + e0, count, oy);
  if constexpr (WANT_W) store_elems_any<T, kSegE>(static_cast<T*>(a.gw) + e0, count, ow);
}

struct SegPlan {
  int64_t ntiles, ngroups;
  size_t off_tfwd, off_tbwd, off_cfwd, off_cbwd, off_gfwd, off_gbwd, bytes;
};

SegPlan seg_plan(int64_t batch, int64_t n) {
  SegPlan p{};
  const int64_t total = batch * n;
  p.ntiles = (total + kSegTile - 1) / kSegTile;
  p.ngroups = (p.ntiles + kSegGroup - 1) / kSegGroup;
  if (p.ntiles <= 1) return p;  // one tile: no workspace
  const size_t st = sizeof(SegSt);
  size_t off = 0;
  p.off_tfwd = off;
  off += align256(p.ntiles * st);
  p.off_tbwd = off;
  off += align256(p.ntiles * st);
  p.off_cfwd = off;
  off += align256(p.ntiles * st);
  p.off_cbwd = off;
  off += align256(p.ntiles * st);
  p.off_gfwd = off;
  off += align256(p.ngroups * st);
  p.off_gbwd = off;
  off += align256(p.ngroups * st);
  p.bytes = off;
  return p;
}

template <typename T, bool W>
hipError_t seg_launch(const SegArgs& a, hipStream_t s) {
  if (a.cfwd != nullptr) {
    seg_ends_kernel<T, W><<<dim3(static_cast<unsigned>(a.ntiles)), dim3(kSegThreads), 0, s>>>(a);
    seg_scan_kernel<<<dim3(static_cast<unsigned>(a.ngroups)), dim3(kSegThreads), 0, s>>>(a);
    if (a.ngroups > 1) seg_groups_kernel<<<dim3(1), dim3(kSegThreads), 0, s>>>(a);
  }
  if (a.y != nullptr) seg_fill_kernel<T, W, true><<<dim3(static_cast<unsigned>(a.ntiles)), dim3(kSegThreads), 0, s>>>(a);
  else seg_fill_kernel<T, W, false><<<dim3(static_cast<unsigned>(a.ntiles)), dim3(kSegThreads), 0, s>>>(a);
  return hipGetLastError();
}

}  // namespace

size_t seg_grad_bytes(int64_t batch, int64_t n) { return seg_plan(batch, n).bytes; }

int64_t seg_grad_tiles(int64_t batch, int64_t n) { return seg_plan(batch, n).ntiles; }

hipError_t seg_grad(const SegGradArgs& in, void* ws) {
  const SegPlan p = seg_plan(in.batch, in.n);
  SegArgs a{};
  a.fit = in.fit;
  a.starts = in.starts;
  a.g = in.g;
  a.w = in.w;
  a.y = in.y;
  a.gy = in.gy;
  a.gw = in.gw;
  a.n = in.n;
  a.total = in.batch * in.n;
  a.flat = in.batch == 1 || in.n % 32 == 0;
  a.ntiles = p.ntiles;
  a.ngroups = p.ngroups;
  if (p.bytes > 0) {
    char* b = static_cast<char*>(ws);
    a.tfwd = reinterpret_cast<SegSt*>(b + p.off_tfwd);
    a.tbwd = reinterpret_cast<SegSt*>(b + p.off_tbwd);
    a.cfwd = reinterpret_cast<SegSt*>(b + p.off_cfwd);
    a.cbwd = reinterpret_cast<SegSt*>(b + p.off_cbwd);
    a.gfwd = reinterpret_cast<SegSt*>(b + p.off_gfwd);
    a.gbwd = reinterpret_cast<SegSt*>(b + p.off_gbwd);
  }
  const bool W = in.w != nullptr;
  if (in.dtype == TI_F32) return W ? seg_launch<float, true>(a, in.stream) : seg_launch<float, false>(a, in.stream);
  return W ? seg_launch<double, true>(a, in.stream) : seg_launch<double, false>(a, in.stream);
}

}  // namespace ti
