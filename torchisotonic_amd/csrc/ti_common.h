// Device helpers shared by the isotonic kernels (gfx950, wave64).
//
// The fit of a row is the slope of the greatest convex minorant (lower convex hull) of its
// cumulative sum diagram P_k = (W_k, S_k), W_k = sum_{j<k} w_j, S_k = sum_{j<k} w_j y_j: element
// i takes the slope of the hull edge over [W_i, W_{i+1}], and blocks start at hull vertices.
// Pool-adjacent-violators (reference src/torchisotonic/csrc/pava.h:16-69) pools a block into its
// predecessor while mean(prev) >= mean(cur); in the diagram that is: drop the vertex B between
// A and C while slope(A, B) >= slope(B, C). Equal means pool, so collinear points are not
// vertices.
//
// All sums and predicates run in float64 whatever the data's dtype: on CDNA3/4 a float64 add,
// mul or fma issues at the float32 rate, and the path is bound by HBM bandwidth.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ti {

constexpr int kWave = 64;

// Sign of a*b - c*d, exact whenever a, b, c, d are exact: each product is split into its
// rounded value and its exact rounding error with an fma (two-product, Dekker / Ogita-Rump-
// Oishi). The rounded products' difference is exact when they are within a factor of two of
// each other (Sterbenz), and otherwise too large for the errors to change its sign; the
// errors' difference only decides when the rounded products tie.
__device__ __forceinline__ int cross_sign(double a, double b, double c, double d) {
  // (no contraction: fused into an fma, p - q would become a*b - q exactly and count the
  // product's rounding error twice)
#pragma clang fp contract(off)
  const double p = a * b;
  const double q = c * d;
  const double ep = __builtin_fma(a, b, -p);
  const double eq = __builtin_fma(c, d, -q);
  const double r = (p - q) + (ep - eq);
  return (r > 0.0) - (r < 0.0);
}

// True when vertex B (between A and C) must leave a lower hull built for PAVA semantics:
// slope(A,B) >= slope(B,C), i.e. dS1 * dW2 >= dS2 * dW1 with dS1 = S_B - S_A, dW1 = W_B - W_A,
// dS2 = S_C - S_B, dW2 = W_C - W_B (weights positive). Mirrors reference pava.h:46-55:
// merge unless total_a * weight_b < total_b * weight_a.
//
// EXACT: the decision is exact for the given (exact) differences. A single fma forms
// dS1*dW2 - fl(dS2*dW1) with one rounding; its sign is right unless it is within
// 2^-52 |dS2*dW1| of zero (the second product's rounding error plus its own), and only then
// does the two-product test run. Without EXACT the products are compared as rounded, which
// is exact whenever they fit 53 bits (unweighted float32 rows: sums of at most 32 float32
// values times counts of at most 32).
template <bool EXACT>
__device__ __forceinline__ bool pools(double dS1, double dW1, double dS2, double dW2) {
  if constexpr (EXACT) {
    const double q = dS2 * dW1;
    const double d = __builtin_fma(dS1, dW2, -q);
    if (__builtin_fabs(d) > 0x1p-52 * __builtin_fabs(q)) return d > 0.0;
    return cross_sign(dS1, dW2, dS2, dW1) >= 0;
  } else {
    return dS1 * dW2 >= dS2 * dW1;
  }
}

// pools<true> as straight-line code: both the filtered test and the exact one are formed and
// one is selected, for loops that keep several tests in flight.
__device__ __forceinline__ bool pools_nb(double dS1, double dW1, double dS2, double dW2) {
  const double q = dS2 * dW1;
  const double d = __builtin_fma(dS1, dW2, -q);
  const bool sure = __builtin_fabs(d) > 0x1p-52 * __builtin_fabs(q);
  const bool exact = cross_sign(dS1, dW2, dS2, dW1) >= 0;
  return sure ? d > 0.0 : exact;
}

// num / den for den > 0, within an ulp or so of the correctly rounded quotient: a hardware
// reciprocal refined by two Newton steps, then one residual correction of the quotient
// (Markstein). Used wherever a block's mean (a hull slope) is formed, so the forward and the
// backward get bit-identical means from the same sums.
__device__ __forceinline__ double slope_div(double num, double den) {
  double r = __builtin_amdgcn_rcp(den);
  r = __builtin_fma(__builtin_fma(-den, r, 1.0), r, r);
  r = __builtin_fma(__builtin_fma(-den, r, 1.0), r, r);
  const double q = num * r;
  return __builtin_fma(__builtin_fma(-den, q, num), r, q);
}

// Double-double numbers (hi + lo, |lo| <= ulp(hi)/2): cumulative sums across threads, tiles and
// rows, so that the difference of two nearby points keeps the precision of the difference
// (Knuth's two-sum, Dekker's fast two-sum).
struct DD {
  double hi, lo;
};

// Error-free transformations hold only for separately rounded operations: contraction (an
// fma formed from a product passed in and the sum here) is off in each of them.
__device__ __forceinline__ DD two_sum(double a, double b) {
#pragma clang fp contract(off)
  const double s = a + b;
  const double bb = s - a;
  const double e = (a - (s - bb)) + (b - bb);
  return {s, e};
}

__device__ __forceinline__ DD dd_add(DD a, DD b) {
#pragma clang fp contract(off)
  DD s = two_sum(a.hi, b.hi);
  const double e = s.lo + (a.lo + b.lo);
  const double hi = s.hi + e;
  return {hi, e - (hi - s.hi)};
}

__device__ __forceinline__ DD dd_add(DD a, double b) {
#pragma clang fp contract(off)
  DD s = two_sum(a.hi, b);
  const double e = s.lo + a.lo;
  const double hi = s.hi + e;
  return {hi, e - (hi - s.hi)};
}

// a - b, rounded once to a double.
__device__ __forceinline__ double dd_diff(DD a, DD b) {
#pragma clang fp contract(off)
  return (a.hi - b.hi) + (a.lo - b.lo);
}

// v, taken from the wave's first lane (for values the same in every lane).
__device__ __forceinline__ int64_t wave_uniform(int64_t v) {
  const uint64_t u = static_cast<uint64_t>(v);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// A buffer resource over [base, base + bytes) (bytes clamped to the 32-bit range field). Loads
// past its end return zero and stores past it are dropped, without a fault.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  const int nrec = static_cast<int>(bytes > 0x7FFFFFFF ? 0x7FFFFFFF : bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), nrec, 0x00020000);
}

template <typename T>
__device__ __forceinline__ T quiet_nan();
template <>
__device__ __forceinline__ float quiet_nan<float>() {
  return __builtin_nanf("");
}
template <>
__device__ __forceinline__ double quiet_nan<double>() {
  return __builtin_nan("");
}

// torch.clamp on the fit's dtype: NaN stays NaN (both comparisons are false), and with
// lo > hi everything becomes hi (the upper bound is applied last).
template <typename T>
__device__ __forceinline__ T clip(T v, bool use_lo, T lo, bool use_hi, T hi) {
  if (use_lo) v = v < lo ? lo : v;
  if (use_hi) v = v > hi ? hi : v;
  return v;
}

// torch.clamp's backward mask for the fit value v: passes where lo <= v <= hi (equality
// included); a NaN fit passes nothing.
template <typename T>
__device__ __forceinline__ bool clip_passes(T v, bool use_lo, T lo, bool use_hi, T hi) {
  bool ok = v == v;
  if (use_lo) ok = ok && v >= lo;
  if (use_hi) ok = ok && v <= hi;
  return ok;
}

// Wavefront scans through DPP: every cross-lane step is a VALU move with a lane-shift modifier,
// not an LDS permute, so a scan's steps wait on no memory pipe. Inclusive scans run row_shr 1,
// 2, 4, 8 within each 16-lane row, then row_bcast:15 (the last lane of rows 0 and 2 into rows 1
// and 3) and row_bcast:31 (lane 31 into rows 2 and 3); lanes without a source keep the
// identity (zero). Controls as in the GFX9 DPP encoding: row_shr:k 0x110 + k, wave_shr:1 0x138,
// row_bcast:15 0x142, row_bcast:31 0x143.
template <int CTRL, int ROWS>
__device__ __forceinline__ int dpp_i32(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, ROWS, 0xF, false);
}

template <int CTRL, int ROWS>
__device__ __forceinline__ double dpp_f64(double x) {
  const uint64_t b = __builtin_bit_cast(uint64_t, x);
  const uint32_t lo = static_cast<uint32_t>(dpp_i32<CTRL, ROWS>(static_cast<int>(static_cast<uint32_t>(b))));
  const uint32_t hi = static_cast<uint32_t>(dpp_i32<CTRL, ROWS>(static_cast<int>(static_cast<uint32_t>(b >> 32))));
  return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}

template <int CTRL, int ROWS>
__device__ __forceinline__ DD dpp_dd(DD x) {
  return DD{dpp_f64<CTRL, ROWS>(x.hi), dpp_f64<CTRL, ROWS>(x.lo)};
}

// Inclusive sum over lanes 0..lane of the wave (all 64 lanes active).
__device__ __forceinline__ int wave_incl_i32(int v) {
  v += dpp_i32<0x111, 0xF>(v);
  v += dpp_i32<0x112, 0xF>(v);
  v += dpp_i32<0x114, 0xF>(v);
  v += dpp_i32<0x118, 0xF>(v);
  v += dpp_i32<0x142, 0xA>(v);
  v += dpp_i32<0x143, 0xC>(v);
  return v;
}

// The same in float64.
__device__ __forceinline__ double wave_incl_f64(double v) {
  v = dpp_f64<0x111, 0xF>(v) + v;
  v = dpp_f64<0x112, 0xF>(v) + v;
  v = dpp_f64<0x114, 0xF>(v) + v;
  v = dpp_f64<0x118, 0xF>(v) + v;
  v = dpp_f64<0x142, 0xA>(v) + v;
  v = dpp_f64<0x143, 0xC>(v) + v;
  return v;
}

// The same in double-double, each step adding the lower lanes' part on the left.
__device__ __forceinline__ DD wave_incl_dd(DD v) {
  v = dd_add(dpp_dd<0x111, 0xF>(v), v);
  v = dd_add(dpp_dd<0x112, 0xF>(v), v);
  v = dd_add(dpp_dd<0x114, 0xF>(v), v);
  v = dd_add(dpp_dd<0x118, 0xF>(v), v);
  v = dd_add(dpp_dd<0x142, 0xA>(v), v);
  v = dd_add(dpp_dd<0x143, 0xC>(v), v);
  return v;
}

// Inclusive scan of double-double values over aligned segments of `seg` lanes (a power of two,
// the same in every lane), each segment on its own: lane l sums lanes l & ~(seg - 1) .. l.
__device__ __forceinline__ DD seg_incl_dd(DD v, int seg) {
  const int lane = threadIdx.x & (kWave - 1);
  for (int d = 1; d < seg; d <<= 1) {
    const DD o{__shfl_up(v.hi, d, kWave), __shfl_up(v.lo, d, kWave)};
    if ((lane & (seg - 1)) >= d) v = dd_add(o, v);
  }
  return v;
}

// Lane - 1's value (zero in lane 0): an inclusive scan made exclusive.
__device__ __forceinline__ int wave_shr1_i32(int v) { return dpp_i32<0x138, 0xF>(v); }
__device__ __forceinline__ DD wave_shr1_dd(DD v) { return dpp_dd<0x138, 0xF>(v); }

// Lane 63's value, in every lane.
__device__ __forceinline__ double wave_last_f64(double x) {
  const uint64_t b = __builtin_bit_cast(uint64_t, x);
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(b)), 63));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(b >> 32)), 63));
  return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}
__device__ __forceinline__ DD wave_last_dd(DD v) { return DD{wave_last_f64(v.hi), wave_last_f64(v.lo)}; }

// floor(e / n) for e * n < 2^32 (e >= 0, n >= 1): the high word of e * ceil(2^32 / n), exact
// there since e * (ceil(2^32/n) - 2^32/n) < e < 2^32 / n. n = 1 has no 32-bit multiplier and is
// passed through.
struct DivBy {
  uint32_t n, magic;
  __device__ __forceinline__ explicit DivBy(uint32_t d) : n(d), magic(d > 1 ? 0xFFFFFFFFu / d + 1u : 0u) {}
  __device__ __forceinline__ uint32_t operator()(uint32_t e) const {
    return n > 1 ? __umulhi(e, magic) : e;
  }
};

}  // namespace ti
