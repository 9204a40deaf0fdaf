// The calibration step after an isotonic fit: piecewise-linear interpolation of a fitted curve
// (xp, fp) at new points, constant beyond its ends (np.interp's semantics).
//
// Replaces the reference's interp (reference examples/ctr_calibration/calibrate.py:163-168),
// five tensor operations and their launches (searchsorted, four gathers, then the arithmetic),
// with one kernel: per point, a binary search over xp (the first knot at or above x, clamped to
// [1, m - 1]) and the same arithmetic in the same order, each operation rounded once
// (contraction off), so the result is the reference's bit for bit:
//
//   t = clamp((x - x0) / max(x1 - x0, 1e-300), 0, 1),   out = f0 + t * (f1 - f0).
//
// A NaN x gives NaN (the clamp keeps it); one knot gives fp[0] everywhere.
#include <hip/hip_runtime.h>

#include "ti_kernels.h"

namespace ti {

namespace {

template <typename T>
__global__ __launch_bounds__(256) void interp_kernel(const T* __restrict__ x, const T* __restrict__ xp,
                                                     const T* __restrict__ fp, T* __restrict__ out,
                                                     int64_t n, int64_t m) {
#pragma clang fp contract(off)
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < n; e += stride) {
    const T v = x[e];
    if (m == 1) {
      out[e] = v == v ? fp[0] : v;
      continue;
    }
    // the first i in [0, m) with !(xp[i] < v) (m if none), as searchsorted(side="left")
    int64_t lo = 0, hi = m;
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if (xp[mid] < v) lo = mid + 1;
      else hi = mid;
    }
    const int64_t i = lo < 1 ? 1 : (lo > m - 1 ? m - 1 : lo);
    const T x0 = xp[i - 1], x1 = xp[i], f0 = fp[i - 1], f1 = fp[i];
    T dx = x1 - x0;
    dx = dx < T(1e-300) ? T(1e-300) : dx;
    T t = (v - x0) / dx;
    t = t < T(0) ? T(0) : (t > T(1) ? T(1) : t);
    out[e] = f0 + t * (f1 - f0);
  }
}

}  // namespace

hipError_t interp(const void* x, const void* xp, const void* fp, void* out, int64_t n, int64_t m, int dtype,
                  hipStream_t stream) {
  const int64_t blocks64 = (n + 255) / 256;
  const unsigned blocks = static_cast<unsigned>(blocks64 < 65536 ? blocks64 : 65536);
  if (dtype == TI_F32)
    interp_kernel<float><<<dim3(blocks), dim3(256), 0, stream>>>(
        static_cast<const float*>(x), static_cast<const float*>(xp), static_cast<const float*>(fp),
        static_cast<float*>(out), n, m);
  else
    interp_kernel<double><<<dim3(blocks), dim3(256), 0, stream>>>(
        static_cast<const double*>(x), static_cast<const double*>(xp), static_cast<const double*>(fp),
        static_cast<double*>(out), n, m);
  return hipGetLastError();
}

}  // namespace ti
