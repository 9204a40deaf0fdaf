// Ragged rows longer than 32 elements: the rows of a length bucket gathered into one dense
// [k, L] block, fitted (and differentiated) by the regular long-row kernels in one call, and
// scattered back into the packed arrays.
//
// The reference has no ragged input: its callers pad rows to a common length with tail values
// that never pool into the data - above the row's maximum for an increasing fit, below its
// minimum for a decreasing one (reference README.md:100-103). The bucket's block uses the same
// rule per row: pad = m + max(1, |m|) for an increasing fit, m the row's largest value (NaN
// skipped), and the mirror image for a decreasing one, with weight 1. Every real block's mean
// is at most m < pad, so the pad elements pool with each other only and the row's own elements
// keep their fit, their partition and their gradients. (A row whose largest value is +inf, or
// so large that m + max(1, |m|) is not finite in the row's dtype, pads with that infinity or
// the largest finite value; a row holding a NaN is NaN throughout whatever its pad.)
//
// Those rows (a NaN row, or one whose extreme the pad cannot exceed) may have their last block
// reach into the pad: the fit of the row's own elements is still the row's, since a block that
// pools with the pad has a mean equal to the pad's, but the block's weight in the backward holds
// the pad's weight too. The unpack of a gradient block therefore checks each row's start bit at
// its length and, where it is clear, scales the gradients over that last block by (W + P) / W,
// W the row's own weight over the block and P the pad elements in it (weight 1 each: up to the
// next start bit, which need not be the row's end, since a long run of equal pads need not stay
// one block where their sums round), which takes the pad back out.
//
// float32 rows may skip the extreme: their pad is the largest finite float32 (its negative for a
// decreasing fit), beyond every finite value of any row; a row holding that value or an infinity
// is one whose pad may join its last block, as above.
//
// Row descriptors: int64 pairs (first element in the packed array, length), k of them; the
// block is row-major [k, L], L at least every length. ragged_rows gathers them from the offsets
// in the order the caller gives (rows sorted by length bucket). Every kernel clamps a row to [0, total) of
// the packed array and to L, so no access leaves the buffers whatever the descriptors hold.
#include "ti_common.h"
#include "ti_kernels.h"

namespace ti {

namespace {

constexpr int kRagThreads = 256;
constexpr int kRagE = 8;                             // elements a thread
constexpr int64_t kRagChunk = kRagThreads * kRagE;  // elements a workgroup

// An order-preserving map of doubles to unsigned 64-bit keys (larger doubles, larger keys);
// key 0 is below every double and decodes to NaN ("no value").
__device__ __forceinline__ unsigned long long key_of(double x) {
  const unsigned long long u = __builtin_bit_cast(unsigned long long, x);
  return (u >> 63) ? ~u : (u | 0x8000000000000000ull);
}

__device__ __forceinline__ double value_of(unsigned long long k) {
  if (k == 0) return __builtin_nan("");
  const unsigned long long u = (k >> 63) ? (k & 0x7FFFFFFFFFFFFFFFull) : ~k;
  return __builtin_bit_cast(double, u);
}

// Row r's first element and length, clamped to the packed array (total) and the block (L).
__device__ __forceinline__ void row_of(const int64_t* __restrict__ rows, int64_t r, int64_t total, int64_t L,
                                       int64_t& first, int64_t& len) {
  first = rows[2 * r];
  first = first < 0 ? 0 : (first > total ? total : first);
  len = rows[2 * r + 1];
  len = len < 0 ? 0 : len;
  len = len > total - first ? total - first : len;
  len = len > L ? L : len;
}

// The row's pad from its extreme key (the key of the largest sgn * y).
template <typename T>
__device__ __forceinline__ T pad_of(unsigned long long key, double sgn) {
  const double m = value_of(key);
  const double a = m < 0.0 ? -m : m;
  double p = m + (a > 1.0 ? a : 1.0);  // (NaN stays NaN; +inf stays +inf)
  const double big = static_cast<double>(sizeof(T) == 4 ? 3.4028234663852886e38 : 1.7976931348623157e308);
  if (p > big && m <= big) p = big;  // (m finite: the largest finite value, not an overflow)
  return static_cast<T>(sgn * p);
}

// Per (row, chunk of kRagChunk of its elements): the largest sgn * y of the chunk, NaN skipped,
// into the row's key (an atomic max).
template <typename T>
__global__ __launch_bounds__(kRagThreads) void ragged_extreme_kernel(const T* __restrict__ y,
                                                                     const int64_t* __restrict__ rows, int64_t k,
                                                                     int64_t total, int64_t L, int64_t cpr, double sgn,
                                                                     unsigned long long* __restrict__ keys) {
  __shared__ unsigned long long wmax[kRagThreads / kWave];
  const int64_t b = blockIdx.x;
  const int64_t r = b / cpr, c = b - r * cpr;
  int64_t first, len;
  row_of(rows, r, total, L, first, len);
  unsigned long long best = 0;
  const int64_t e0 = c * kRagChunk;
#pragma unroll
  for (int u = 0; u < kRagE; ++u) {
    const int64_t e = e0 + u * kRagThreads + threadIdx.x;
    if (e < len) {
      const double v = sgn * static_cast<double>(y[first + e]);
      if (v == v) {
        const unsigned long long kv = key_of(v);
        best = kv > best ? kv : best;
      }
    }
  }
#pragma unroll
  for (int d = kWave / 2; d >= 1; d >>= 1) {
    const unsigned long long o = __shfl_xor(best, d, kWave);
    best = o > best ? o : best;
  }
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  if (lane == 0) wmax[wave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long m = wmax[0];
    for (int w = 1; w < kRagThreads / kWave; ++w) m = wmax[w] > m ? wmax[w] : m;
    if (m != 0 && r < k) atomicMax(&keys[r], m);
  }
}

// Per (row, chunk of kRagChunk of the block's L): dst[r][j] = src[first + j] for j < len, else the
// row's pad (from its key, or the constant pad without keys); wdst likewise from w, with weight 1
// past the row.
template <typename T>
__global__ __launch_bounds__(kRagThreads) void ragged_pack_kernel(const T* __restrict__ src, const T* __restrict__ w,
                                                                  const int64_t* __restrict__ rows,
                                                                  const unsigned long long* __restrict__ keys,
                                                                  T cpad, int64_t total, int64_t L, int64_t cpr,
                                                                  double sgn, T* __restrict__ dst,
                                                                  T* __restrict__ wdst) {
  const int64_t b = blockIdx.x;
  const int64_t r = b / cpr, c = b - r * cpr;
  int64_t first, len;
  row_of(rows, r, total, L, first, len);
  const T pad = keys != nullptr ? pad_of<T>(keys[r], sgn) : cpad;
  const int64_t e0 = c * kRagChunk;
#pragma unroll
  for (int u = 0; u < kRagE; ++u) {
    const int64_t e = e0 + u * kRagThreads + threadIdx.x;
    if (e < L) {
      const bool in = e < len;
      dst[r * L + e] = in ? src[first + e] : pad;
      if (wdst != nullptr) wdst[r * L + e] = in ? w[first + e] : T(1);
    }
  }
}

// dst[first + j] = src[r][j] for j < len (dst2 from src2 likewise, where given).
template <typename T>
__global__ __launch_bounds__(kRagThreads) void ragged_unpack_kernel(const T* __restrict__ src,
                                                                    const T* __restrict__ src2,
                                                                    const int64_t* __restrict__ rows, int64_t total,
                                                                    int64_t L, int64_t cpr, T* __restrict__ dst,
                                                                    T* __restrict__ dst2) {
  const int64_t b = blockIdx.x;
  const int64_t r = b / cpr, c = b - r * cpr;
  int64_t first, len;
  row_of(rows, r, total, L, first, len);
  const int64_t e0 = c * kRagChunk;
#pragma unroll
  for (int u = 0; u < kRagE; ++u) {
    const int64_t e = e0 + u * kRagThreads + threadIdx.x;
    if (e < len) {
      dst[first + e] = src[r * L + e];
      if (dst2 != nullptr) dst2[first + e] = src2[r * L + e];
    }
  }
}

// rows[i] = (offsets[o], offsets[o + 1] - offsets[o]) for o = order[i] (clamped into the rows).
__global__ __launch_bounds__(kRagThreads) void ragged_rows_kernel(const int64_t* __restrict__ offsets, int64_t nrows,
                                                                  const int64_t* __restrict__ order, int64_t n,
                                                                  int64_t* __restrict__ rows) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kRagThreads + threadIdx.x;
  if (i >= n) return;
  int64_t o = order[i];
  o = o < 0 ? 0 : (o >= nrows ? nrows - 1 : o);
  const int64_t a = offsets[o];
  rows[2 * i] = a;
  rows[2 * i + 1] = offsets[o + 1] - a;
}

// One wave per row: a row whose last block reaches into its pad (start bit len clear, len < L)
// has gy (and gw) over that block scaled by (W + P) / W, W its own weight over the block and P
// the pad elements in it, those before the next start bit (or L).
template <typename T>
__global__ __launch_bounds__(kRagThreads) void ragged_grad_fix_kernel(const uint32_t* __restrict__ starts,
                                                                      const T* __restrict__ w,
                                                                      const int64_t* __restrict__ rows, int64_t k,
                                                                      int64_t total, int64_t L, T* __restrict__ gy,
                                                                      T* __restrict__ gw) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t r = static_cast<int64_t>(blockIdx.x) * (kRagThreads / kWave) + threadIdx.x / kWave;
  if (r >= k) return;
  int64_t first, len;
  row_of(rows, r, total, L, first, len);
  if (len == 0 || len >= L) return;
  const uint32_t* srow = starts + r * ((L + 31) / 32);
  if ((srow[len >> 5] >> (len & 31)) & 1u) return;  // the pad starts a block of its own
  // the block's first element: the last start bit below len (bit 0 always counts)
  const int64_t top = (len - 1) >> 5;
  const uint32_t top_mask = (len & 31) ? ((1u << (len & 31)) - 1u) : ~0u;
  int64_t s = -1;
  for (int64_t base = top; s < 0; base -= kWave) {
    const int64_t j = base - lane;
    int64_t pos = -1;
    if (j >= 0) {
      uint32_t bits = srow[j];
      if (j == top) bits &= top_mask;
      if (j == 0) bits |= 1u;
      if (bits != 0) pos = j * 32 + 31 - __builtin_clz(bits);
    }
#pragma unroll
    for (int d = kWave / 2; d >= 1; d >>= 1) {
      const int64_t o = __shfl_xor(pos, d, kWave);
      pos = o > pos ? o : pos;
    }
    s = pos;  // (word 0 holds bit 0: the loop ends there at the latest)
  }
  // the block's end: the first start bit past len (bits at L or beyond count as L)
  const int64_t words = (L + 31) / 32, w0 = (len + 1) >> 5;
  int64_t e = L;
  for (int64_t base = w0; base < words; base += kWave) {
    const int64_t j = base + lane;
    int64_t pos = L;
    if (j < words) {
      uint32_t bits = srow[j];
      if (j == w0) bits &= ~0u << ((len + 1) & 31);
      if (bits != 0) pos = j * 32 + __builtin_ctz(bits);
    }
#pragma unroll
    for (int d = kWave / 2; d >= 1; d >>= 1) {
      const int64_t o = __shfl_xor(pos, d, kWave);
      pos = o < pos ? o : pos;
    }
    if (pos < L) {  // (the same in every lane)
      e = pos;
      break;
    }
  }
  double wsum = 0.0;
  for (int64_t i = s + lane; i < len; i += kWave) wsum += w != nullptr ? static_cast<double>(w[first + i]) : 1.0;
#pragma unroll
  for (int d = kWave / 2; d >= 1; d >>= 1) wsum += __shfl_xor(wsum, d, kWave);
  const double f = (wsum + static_cast<double>(e - len)) / wsum;
  for (int64_t i = s + lane; i < len; i += kWave) {
    if (gy != nullptr) gy[first + i] = static_cast<T>(static_cast<double>(gy[first + i]) * f);
    if (gw != nullptr) gw[first + i] = static_cast<T>(static_cast<double>(gw[first + i]) * f);
  }
}

}  // namespace

int64_t ragged_chunks(int64_t len) { return (len + kRagChunk - 1) / kRagChunk; }

hipError_t ragged_extreme(const void* y, int64_t total, const int64_t* rows, int64_t k, int64_t L, int dtype,
                          bool increasing, unsigned long long* keys, hipStream_t stream) {
  const int64_t cpr = ragged_chunks(L);
  const dim3 grid(static_cast<unsigned>(k * cpr));
  const double sgn = increasing ? 1.0 : -1.0;
  if (dtype == TI_F32)
    ragged_extreme_kernel<float><<<grid, dim3(kRagThreads), 0, stream>>>(static_cast<const float*>(y), rows, k, total,
                                                                         L, cpr, sgn, keys);
  else
    ragged_extreme_kernel<double><<<grid, dim3(kRagThreads), 0, stream>>>(static_cast<const double*>(y), rows, k,
                                                                          total, L, cpr, sgn, keys);
  return hipGetLastError();
}

hipError_t ragged_pack(const void* src, const void* w, int64_t total, const int64_t* rows,
                       const unsigned long long* keys, double pad, int64_t k, int64_t L, int dtype, bool increasing,
                       void* dst, void* wdst, hipStream_t stream) {
  const int64_t cpr = ragged_chunks(L);
  const dim3 grid(static_cast<unsigned>(k * cpr));
  const double sgn = increasing ? 1.0 : -1.0;
  if (dtype == TI_F32)
    ragged_pack_kernel<float><<<grid, dim3(kRagThreads), 0, stream>>>(
        static_cast<const float*>(src), static_cast<const float*>(w), rows, keys, static_cast<float>(pad), total, L,
        cpr, sgn, static_cast<float*>(dst), static_cast<float*>(wdst));
  else
    ragged_pack_kernel<double><<<grid, dim3(kRagThreads), 0, stream>>>(
        static_cast<const double*>(src), static_cast<const double*>(w), rows, keys, pad, total, L, cpr, sgn,
        static_cast<double*>(dst), static_cast<double*>(wdst));
  return hipGetLastError();
}

hipError_t ragged_rows(const int64_t* offsets, int64_t nrows, const int64_t* order, int64_t n, int64_t* rows,
                       hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>((n + kRagThreads - 1) / kRagThreads));
  ragged_rows_kernel<<<grid, dim3(kRagThreads), 0, stream>>>(offsets, nrows, order, n, rows);
  return hipGetLastError();
}

hipError_t ragged_unpack(const void* src, const void* src2, const int64_t* rows, int64_t k, int64_t L, int dtype,
                         void* dst, void* dst2, int64_t total, const uint32_t* starts, const void* w,
                         hipStream_t stream) {
  const int64_t cpr = ragged_chunks(L);
  const dim3 grid(static_cast<unsigned>(k * cpr));
  if (dtype == TI_F32) {
    ragged_unpack_kernel<float><<<grid, dim3(kRagThreads), 0, stream>>>(
        static_cast<const float*>(src), static_cast<const float*>(src2), rows, total, L, cpr, static_cast<float*>(dst),
        static_cast<float*>(dst2));
  } else {
    ragged_unpack_kernel<double><<<grid, dim3(kRagThreads), 0, stream>>>(
        static_cast<const double*>(src), static_cast<const double*>(src2), rows, total, L, cpr,
        static_cast<double*>(dst), static_cast<double*>(dst2));
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess || starts == nullptr) return e;
  return ragged_grad_fix(starts, w, rows, k, L, dtype, dst, dst2, total, stream);
}

hipError_t ragged_grad_fix(const uint32_t* starts, const void* w, const int64_t* rows, int64_t k, int64_t L, int dtype,
                           void* gy, void* gw, int64_t total, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>((k + kRagThreads / kWave - 1) / (kRagThreads / kWave)));
  if (dtype == TI_F32)
    ragged_grad_fix_kernel<float><<<grid, dim3(kRagThreads), 0, stream>>>(
        starts, static_cast<const float*>(w), rows, k, total, L, static_cast<float*>(gy), static_cast<float*>(gw));
  else
    ragged_grad_fix_kernel<double><<<grid, dim3(kRagThreads), 0, stream>>>(
        starts, static_cast<const double*>(w), rows, k, total, L, static_cast<double*>(gy), static_cast<double*>(gw));
  return hipGetLastError();
}

}  // namespace ti
