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
//
// A search over millions of knots is a chain of ~23 dependent reads a query, most of them
// misses. The knot index (interp_index) cuts it to about three: buckets of equal width over
// [xp[0], xp[m - 1]], about kKnotsPerBucket knots each,
//
//   bucket(v) = clamp(floor((v - xp[0]) * scale), 0, B - 1),   scale = B / (xp[m - 1] - xp[0]),
//   first[b]  = the first knot i with bucket(xp[i]) >= b        (first[B] = m).
//
// bucket() is monotone in v (a subtraction, a product with scale >= 0, a clamp and a floor, each
// rounding a monotone function), so xp[i] < v gives bucket(xp[i]) <= bucket(v) and xp[i] >= v
// gives bucket(xp[i]) >= bucket(v): the first knot at or above v lies in [first[b], first[b + 1]]
// for b = bucket(v), and only those knots are searched - the same index as the full search, so
// the output is ti_interp's bit for bit. Knot ranges that are not finite and positive (an
// infinite or NaN end, all knots equal) give scale 0, and every query then searches all knots.
#include <hip/hip_runtime.h>

#include <cmath>

#include "ti_kernels.h"

namespace ti {

namespace {

// The reference formula at the first knot i at or above v (m after the last), i clamped to
// [1, m - 1]; each operation rounded once.
template <typename T>
__device__ __forceinline__ T interp_at(const T* __restrict__ xp, const T* __restrict__ fp, int64_t i, int64_t m,
                                       T v) {
#pragma clang fp contract(off)
  i = i < 1 ? 1 : (i > m - 1 ? m - 1 : i);
  const T x0 = xp[i - 1], x1 = xp[i], f0 = fp[i - 1], f1 = fp[i];
  T dx = x1 - x0;
  dx = dx < T(1e-300) ? T(1e-300) : dx;
  T t = (v - x0) / dx;
  t = t < T(0) ? T(0) : (t > T(1) ? T(1) : t);
  return f0 + t * (f1 - f0);
}

// The first i in [lo, hi) with !(xp[i] < v) (hi if none), as searchsorted(side="left").
template <typename T>
__device__ __forceinline__ int64_t lower_bound(const T* __restrict__ xp, int64_t lo, int64_t hi, T v) {
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (xp[mid] < v) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

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
    out[e] = interp_at(xp, fp, lower_bound(xp, int64_t{0}, m, v), m, v);
  }
}

// The index's header, then first[0..B] (uint32). m and dtype name the knots it was built from:
// a search through an index of another knot count or dtype would narrow to the wrong buckets.
struct InterpIndex {
  double lo, scale;
  int64_t buckets, m, dtype;
};

template <typename T>
constexpr int64_t dtype_code() {
  return sizeof(T) == 4 ? TI_F32 : TI_F64;
}
constexpr size_t kIndexHead = 256;
constexpr int64_t kKnotsPerBucket = 4;
constexpr int kCountMax = 8;  // buckets of at most this many knots are counted, not searched

__device__ __forceinline__ int64_t bucket_of(double v, double lo, double scale, int64_t buckets) {
#pragma clang fp contract(off)
  double d = (v - lo) * scale;
  d = d >= 0.0 ? d : 0.0;  // NaN and below the first knot: bucket 0
  const double top = static_cast<double>(buckets - 1);
  d = d < top ? d : top;
  return static_cast<int64_t>(d);
}

// One thread a bucket b in [0, B]: first[b] by a search over the knots' buckets.
template <typename T>
__global__ __launch_bounds__(256) void interp_index_kernel(const T* __restrict__ xp, int64_t m, int64_t buckets,
                                                           InterpIndex* __restrict__ head,
                                                           uint32_t* __restrict__ first) {
  const double lo = static_cast<double>(xp[0]);
  const double range = static_cast<double>(xp[m - 1]) - lo;
  double scale = range > 0.0 && range < INFINITY ? static_cast<double>(buckets) / range : 0.0;
  scale = scale < INFINITY ? scale : 0.0;
  const int64_t b = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b == 0) {
    head->lo = lo;
    head->scale = scale;
    head->buckets = buckets;
    head->m = m;
    head->dtype = dtype_code<T>();
  }
  if (b > buckets) return;
  int64_t l = 0, h = b == 0 ? 0 : m;
  while (l < h) {
    const int64_t mid = (l + h) >> 1;
    if (bucket_of(static_cast<double>(xp[mid]), lo, scale, buckets) < b) l = mid + 1;
    else h = mid;
  }
  first[b] = static_cast<uint32_t>(l);
}

// interp_kernel through the index: the bucket's knots [a, c) are counted (at most kCountMax) or
// searched. The header is read as stored, with the bucket count capped at what the buffer holds
// (cap) and the bounds clamped to [0, m], so every read stays in the buffers whatever they hold;
// an index built from another knot count or dtype is not used (every query searches all knots).
template <typename T>
__global__ __launch_bounds__(256) void interp_indexed_kernel(const T* __restrict__ x, const T* __restrict__ xp,
                                                             const T* __restrict__ fp,
                                                             const InterpIndex* __restrict__ head,
                                                             const uint32_t* __restrict__ first, int64_t cap,
                                                             T* __restrict__ out, int64_t n, int64_t m) {
  const double lo = head->lo, scale = head->scale;
  int64_t buckets = head->buckets;
  buckets = buckets < cap ? buckets : cap;
  const bool indexed = scale > 0.0 && buckets >= 1 && head->m == m && head->dtype == dtype_code<T>();
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < n; e += stride) {
    const T v = x[e];
    if (m == 1) {
      out[e] = v == v ? fp[0] : v;
      continue;
    }
    int64_t i;
    if (indexed) {
      const int64_t b = bucket_of(static_cast<double>(v), lo, scale, buckets);
      int64_t c = first[b + 1];
      c = c < m ? c : m;
      int64_t a = first[b];
      a = a < c ? a : c;
      if (c - a <= kCountMax) {
        int cnt = 0;
#pragma unroll
        for (int j = 0; j < kCountMax; ++j)
          if (j < c - a) cnt += xp[a + j] < v ? 1 : 0;
        i = a + cnt;
      } else {
        i = lower_bound(xp, a, c, v);
      }
    } else {
      i = lower_bound(xp, int64_t{0}, m, v);
    }
    out[e] = interp_at(xp, fp, i, m, v);
  }
}

unsigned grid_for(int64_t n) {
  const int64_t blocks64 = (n + 255) / 256;
  return static_cast<unsigned>(blocks64 < 65536 ? blocks64 : 65536);
}

}  // namespace

int64_t interp_buckets(int64_t m) {
  const int64_t b = (m + kKnotsPerBucket - 1) / kKnotsPerBucket;
  return b < 1 ? 1 : b;
}

size_t interp_index_bytes(int64_t m) {
  return (kIndexHead + 4 * static_cast<size_t>(interp_buckets(m) + 1) + 255) & ~size_t{255};
}

hipError_t interp_index(const void* xp, int64_t m, int dtype, void* index, hipStream_t stream) {
  const int64_t buckets = interp_buckets(m);
  auto* head = static_cast<InterpIndex*>(index);
  auto* first = reinterpret_cast<uint32_t*>(static_cast<char*>(index) + kIndexHead);
  const unsigned blocks = static_cast<unsigned>((buckets + 1 + 255) / 256);
  if (dtype == TI_F32)
    interp_index_kernel<float><<<dim3(blocks), dim3(256), 0, stream>>>(static_cast<const float*>(xp), m, buckets,
                                                                        head, first);
  else
    interp_index_kernel<double><<<dim3(blocks), dim3(256), 0, stream>>>(static_cast<const double*>(xp), m, buckets,
                                                                         head, first);
  return hipGetLastError();
}

hipError_t interp_indexed(const void* x, const void* xp, const void* fp, const void* index, size_t index_bytes,
                          void* out, int64_t n, int64_t m, int dtype, hipStream_t stream) {
  const auto* head = static_cast<const InterpIndex*>(index);
  const auto* first = reinterpret_cast<const uint32_t*>(static_cast<const char*>(index) + kIndexHead);
  const int64_t cap = static_cast<int64_t>((index_bytes - kIndexHead) / 4) - 1;
  const unsigned blocks = grid_for(n);
  if (dtype == TI_F32)
    interp_indexed_kernel<float><<<dim3(blocks), dim3(256), 0, stream>>>(
        static_cast<const float*>(x), static_cast<const float*>(xp), static_cast<const float*>(fp), head, first, cap,
        static_cast<float*>(out), n, m);
  else
    interp_indexed_kernel<double><<<dim3(blocks), dim3(256), 0, stream>>>(
        static_cast<const double*>(x), static_cast<const double*>(xp), static_cast<const double*>(fp), head, first,
        cap, static_cast<double*>(out), n, m);
  return hipGetLastError();
}

hipError_t interp(const void* x, const void* xp, const void* fp, void* out, int64_t n, int64_t m, int dtype,
                  hipStream_t stream) {
  const unsigned blocks = grid_for(n);
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
