// Backward of rows that fit one tile (33 .. 4096 elements unweighted, .. 2048 weighted) for a
// caller without the forward's workspace (the reference-named isotonic_grad, which gets only the
// partition): one workgroup per row, the blocks' sums recomputed from y and w.
//
// Replaces the reference's short-row gradient (reference src/torchisotonic/csrc/
// grad.cuh:200-290, grad_fill_kernel with SINGLE) for these lengths. Every element needs the
// sums of g, w (and w*y, for the clamp mask and the weight gradient) over its block. Two
// segmented scans give them without storing anything per element: a forward scan (restarting
// at block starts) gives the sum from the block's start to the element, a reverse scan
// (restarting after block ends) the sum from the element to the block's end; their sum minus
// the element itself is the block total. Each scan runs per thread over its E elements, then
// across the workgroup on (flag, value) pairs (wave64 shuffles, then the four waves' totals).
#include "ti_common.h"
#include "ti_kernels.h"
#include "ti_tile.h"

namespace ti {

namespace {

constexpr int kQ = 3;  // scanned quantities: g, w, w*y

struct Seg {
  bool f;
  double v[kQ];
};

// Forward: a earlier, b later. Reverse: a is left of b, aggregating towards the left.
__device__ __forceinline__ Seg comb_fwd(const Seg& a, const Seg& b, int nq) {
  Seg r;
  r.f = a.f || b.f;
#pragma unroll
  for (int q = 0; q < kQ; ++q)
    if (q < nq) r.v[q] = b.f ? b.v[q] : a.v[q] + b.v[q];
  return r;
}

__device__ __forceinline__ Seg comb_rev(const Seg& a, const Seg& b, int nq) {
  Seg r;
  r.f = a.f || b.f;
#pragma unroll
  for (int q = 0; q < kQ; ++q)
    if (q < nq) r.v[q] = a.f ? a.v[q] : a.v[q] + b.v[q];
  return r;
}

__device__ __forceinline__ Seg shfl_seg(const Seg& s, int src_lane, int nq) {
  Seg r;
  r.f = __shfl(static_cast<int>(s.f), src_lane, kWave) != 0;
#pragma unroll
  for (int q = 0; q < kQ; ++q)
    if (q < nq) r.v[q] = __shfl(s.v[q], src_lane, kWave);
  return r;
}

struct GradShared {
  bool f[2][kWaves256];
  double v[2][kWaves256][kQ];
};

template <typename T, bool W>
__global__ __launch_bounds__(256) void tile_grad_kernel(TileGradArgs a) {
  using C = TileCfg<W>;
  constexpr int E = C::kE;
  __shared__ GradShared sh;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int64_t row = blockIdx.x;
  const int len = static_cast<int>(a.n);
  const int t0 = tid * E;
  const int ecount = max(0, min(E, len - t0));
  const bool use_lo = a.flags & TI_CLIP_MIN, use_hi = a.flags & TI_CLIP_MAX;
  const bool need_mean = a.gw != nullptr || use_lo || use_hi;
  const int nq = need_mean ? 3 : (W ? 2 : 2);  // g, w (or count) [, w*y]

  const T* g = static_cast<const T*>(a.g) + row * a.n;
  T gv[E], wv[W ? E : 1], yv[E];
  load_elems_any<T, E>(g + t0, ecount, gv);
  if constexpr (W) load_elems_any<T, E>(static_cast<const T*>(a.w) + row * a.n + t0, ecount, wv);
  if (need_mean) load_elems_any<T, E>(static_cast<const T*>(a.y) + row * a.n + t0, ecount, yv);

  // Block starts of my elements (element 0 of the row always starts one) and ends (the next
  // element starts a block, or the row ends).
  const int64_t wpr = (a.n + 31) / 32;
  const uint32_t* srow = a.starts + row * wpr;
  uint32_t sbits = 0;
  if (ecount > 0) {
    sbits = (srow[t0 >> 5] >> (t0 & 31)) & ((E == 32) ? 0xFFFFFFFFu : ((1u << E) - 1u));
    if (t0 == 0) sbits |= 1u;
    if (ecount < E) sbits &= (1u << ecount) - 1u;
  }
  const int tn = t0 + E;
  const bool next_start = tn >= len ? true : ((srow[tn >> 5] >> (tn & 31)) & 1u) != 0;
  uint32_t ebits = (sbits >> 1);
  if (ecount > 0) {
    if (ecount == E) ebits |= (next_start ? 1u : 0u) << (E - 1);
    else ebits |= 1u << (ecount - 1);
  }

  double v[E][kQ];
#pragma unroll
  for (int k = 0; k < E; ++k) {
    const bool ok = k < ecount;
    v[k][0] = ok ? static_cast<double>(gv[k]) : 0.0;
    double wk = 1.0;
    if constexpr (W) wk = ok ? static_cast<double>(wv[k]) : 0.0;
    else wk = ok ? 1.0 : 0.0;
    v[k][1] = wk;
    v[k][2] = (need_mean && ok) ? wk * static_cast<double>(yv[k]) : 0.0;
  }

  // Local scans.
  double F[E][kQ], R[E][kQ];
  {
    double acc[kQ] = {0.0, 0.0, 0.0};
#pragma unroll
    for (int k = 0; k < E; ++k) {
      const bool st = (sbits >> k) & 1u;
#pragma unroll
      for (int q = 0; q < kQ; ++q) {
        acc[q] = (st ? 0.0 : acc[q]) + v[k][q];
        F[k][q] = acc[q];
      }
    }
    double racc[kQ] = {0.0, 0.0, 0.0};
#pragma unroll
    for (int k = E - 1; k >= 0; --k) {
      const bool en = (ebits >> k) & 1u;
#pragma unroll
      for (int q = 0; q < kQ; ++q) {
        racc[q] = (en ? 0.0 : racc[q]) + v[k][q];
        R[k][q] = racc[q];
      }
    }
  }
  Seg fs, rs;
  fs.f = sbits != 0;
  rs.f = ebits != 0;
#pragma unroll
  for (int q = 0; q < kQ; ++q) {
    fs.v[q] = F[E - 1][q];
    rs.v[q] = R[0][q];
  }
  // Inclusive scans across the wave, forward and reverse.
  Seg fi = fs, ri = rs;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const Seg o = shfl_seg(fi, lane - d, nq);
    if (lane >= d) fi = comb_fwd(o, fi, nq);
    const Seg p = shfl_seg(ri, lane + d, nq);
    if (lane + d < kWave) ri = comb_rev(ri, p, nq);
  }
  if (lane == kWave - 1) {
    sh.f[0][wave] = fi.f;
    for (int q = 0; q < kQ; ++q) sh.v[0][wave][q] = fi.v[q];
  }
  if (lane == 0) {
    sh.f[1][wave] = ri.f;
    for (int q = 0; q < kQ; ++q) sh.v[1][wave][q] = ri.v[q];
  }
  __syncthreads();
  // Exclusive carries: forward from the earlier lanes and waves, reverse from the later ones.
  Seg cf = shfl_seg(fi, lane - 1, nq);
  if (lane == 0) {
    cf.f = false;
    for (int q = 0; q < kQ; ++q) cf.v[q] = 0.0;
  }
  for (int wv2 = wave - 1; wv2 >= 0; --wv2) {
    Seg o;
    o.f = sh.f[0][wv2];
    for (int q = 0; q < kQ; ++q) o.v[q] = sh.v[0][wv2][q];
    cf = comb_fwd(o, cf, nq);
  }
  Seg cr = shfl_seg(ri, lane + 1, nq);
  if (lane == kWave - 1) {
    cr.f = false;
    for (int q = 0; q < kQ; ++q) cr.v[q] = 0.0;
  }
  for (int wv2 = wave + 1; wv2 < kWaves256; ++wv2) {
    Seg o;
    o.f = sh.f[1][wv2];
    for (int q = 0; q < kQ; ++q) o.v[q] = sh.v[1][wv2][q];
    cr = comb_rev(cr, o, nq);
  }

  // Block totals per element, then the gradients.
  const T lo = static_cast<T>(a.lo), hi = static_cast<T>(a.hi);
  T oy[E], ow[E];
  const int first_start = sbits ? __builtin_ctz(sbits) : E;
  const int last_end = ebits ? 31 - __builtin_clz(ebits) : -1;
#pragma unroll
  for (int k = 0; k < E; ++k) {
    double tot[kQ];
#pragma unroll
    for (int q = 0; q < kQ; ++q) {
      const double fwd = F[k][q] + (k < first_start ? cf.v[q] : 0.0);
      const double rev = R[k][q] + (k > last_end ? cr.v[q] : 0.0);
      tot[q] = (fwd + rev) - v[k][q];
    }
    double qv = tot[0] / tot[1];
    T mean = T(0);
    if (need_mean) {
      mean = static_cast<T>(slope_div(tot[2], tot[1]));
      if ((use_lo || use_hi) && !clip_passes(mean, use_lo, lo, use_hi, hi)) qv = 0.0;
    }
    oy[k] = static_cast<T>(v[k][1] * qv);
    ow[k] = need_mean ? static_cast<T>((static_cast<double>(yv[k]) - static_cast<double>(mean)) * qv) : T(0);
  }
  if (a.gy != nullptr) store_elems_any<T, E>(static_cast<T*>(a.gy) + row * a.n + t0, ecount, oy);
  if (a.gw != nullptr) store_elems_any<T, E>(static_cast<T*>(a.gw) + row * a.n + t0, ecount, ow);
}

template <typename T, bool W>
hipError_t launch(const TileGradArgs& a) {
  tile_grad_kernel<T, W><<<dim3(static_cast<unsigned>(a.batch)), dim3(256), 0, a.stream>>>(a);
  return hipGetLastError();
}

}  // namespace

hipError_t tile_grad_single(const TileGradArgs& a) {
  const bool weighted = a.w != nullptr;
  if (a.dtype == TI_F32) return weighted ? launch<float, true>(a) : launch<float, false>(a);
  return weighted ? launch<double, true>(a) : launch<double, false>(a);
}

}  // namespace ti
