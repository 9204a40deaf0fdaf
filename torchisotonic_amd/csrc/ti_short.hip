// Short rows (n <= 32): one thread per row, many rows per wavefront.
//
// Replaces the reference's packed regime (reference src/torchisotonic/csrc/tiles.cuh:920-1112,
// packed_kernel; grad.cuh:200-290 with E=1 for the backward) with a design for wave64:
//   - rows that are a whole number of 16-byte chunks (n * sizeof(T) % 16 == 0, aligned: the
//     headline [1e6, 16] float32 case) take short_rows_kernel / short_grad_rows_kernel: a
//     persistent grid whose workgroups walk blocks of rows with the next block's loads in
//     flight, each wave moving its 64 rows through LDS with coalesced 16-byte accesses and
//     transposing them to one row per lane; other rows take short_fit_kernel /
//     short_grad_kernel, one block of THREADS consecutive rows a workgroup, the block's span
//     moved with coalesced 16-byte accesses through LDS, rows padded to n + 1 entries;
//   - each thread builds its row's cumulative sums in float64 registers and runs the monotone
//     chain (Andrew) for the lower hull of the n + 1 points, keeping the hull as a bit mask
//     and the points in a per-thread LDS column for the chain's random access (unweighted
//     rows: the mask alone is the stack; weighted rows carry the top two vertices and read
//     both possible successors before each choice);
//   - the fit is one float64 slope per block, rounded once, with the clamp fused; the
//     partition is one 32-bit word of start bits per row.
// The backward moves g (and w, y) the same way; block sums of g (and w) and the block mean
// for the clamp mask and the weight gradient are formed per thread, in registers.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "ti_common.h"
#include "ti_kernels.h"

namespace ti {

namespace {

// Threads per workgroup: the pops' point columns take (NMAX + 1) * THREADS float64 values per
// coordinate; keep them at or under 36 KB, four workgroups per CU.
template <int NMAX, bool W>
constexpr int short_threads() {
  constexpr int per_thread = (NMAX + 1) * 8 * (W ? 2 : 1);
  return per_thread * 256 <= 36 * 1024 ? 256 : per_thread * 128 <= 36 * 1024 ? 128 : 64;
}

template <int NMAX, bool W>
constexpr int short_lds_doubles() {
  return (NMAX + 1) * short_threads<NMAX, W>() * (W ? 2 : 1);
}

template <typename T>
struct Vec16 {
  static constexpr int kN = 16 / sizeof(T);
  using type = T __attribute__((ext_vector_type(kN)));
};

// The staged path: this workgroup's span of `count` = rows * n elements, read with coalesced
// 16-byte loads (all issued before any is used), into registers; then written to LDS row r at
// stg[r * (n + 1) + c]. A span that does not start on a 16-byte boundary is read per element.
template <typename T, int THREADS, int NMAX>
struct Span {
  static constexpr int V = Vec16<T>::kN;
  static constexpr int kIters = (NMAX + V - 1) / V;
  using VT = typename Vec16<T>::type;
  VT buf[kIters];
  T tailv;  // the span's last (count % V) elements, one per thread, in the vector path

  __device__ __forceinline__ void load(const T* __restrict__ src, int count) {
    const int tid = threadIdx.x;
    if ((reinterpret_cast<uintptr_t>(src) & 15) == 0) {
      const VT* s = reinterpret_cast<const VT*>(src);
      const int nvec = count / V;
#pragma unroll
      for (int j = 0; j < kIters; ++j) {
        const int idx = tid + j * THREADS;
        if (idx < nvec) buf[j] = s[idx];
      }
      const int tail = count - nvec * V;
      if (tid < tail) tailv = src[nvec * V + tid];
    } else {
#pragma unroll
      for (int j = 0; j < kIters; ++j) {
#pragma unroll
        for (int t = 0; t < V; ++t) {
          const int e = (tid + j * THREADS) * V + t;
          if (e < count) buf[j][t] = src[e];
        }
      }
    }
  }

  __device__ __forceinline__ void to_lds(const T* __restrict__ src, T* stg, int count,
                                         DivBy div) const {
    const int tid = threadIdx.x;
    const bool vec = (reinterpret_cast<uintptr_t>(src) & 15) == 0;
    const int nvec = vec ? count / V : (count + V - 1) / V;
#pragma unroll
    for (int j = 0; j < kIters; ++j) {
      const int idx = tid + j * THREADS;
      if (idx < nvec) {
#pragma unroll
        for (int t = 0; t < V; ++t) {
          const int e = idx * V + t;
          if (e < count) stg[e + div(e)] = buf[j][t];
        }
      }
    }
    if (vec) {
      const int tail = count - (count / V) * V;
      if (tid < tail) {
        const int e = (count / V) * V + tid;
        stg[e + div(e)] = tailv;
      }
    }
  }
};

template <typename T, int THREADS>
__device__ __forceinline__ void stage_out(T* __restrict__ dst, const T* stg, int count, DivBy div) {
  constexpr int V = Vec16<T>::kN;
  using VT = typename Vec16<T>::type;
  const int tid = threadIdx.x;
  if ((reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
    const int nvec = count / V;
    VT* d = reinterpret_cast<VT*>(dst);
    for (int idx = tid; idx < nvec; idx += THREADS) {
      VT x;
#pragma unroll
      for (int t = 0; t < V; ++t) {
        const int e = idx * V + t;
        x[t] = stg[e + div(e)];
      }
      d[idx] = x;
    }
    for (int e = nvec * V + tid; e < count; e += THREADS) dst[e] = stg[e + div(e)];
  } else {
    for (int e = tid; e < count; e += THREADS) dst[e] = stg[e + div(e)];
  }
}

// Vertex masks over the n + 1 points of a row.
template <int NMAX>
struct MaskOf {
  using type = typename std::conditional<(NMAX < 32), uint32_t, uint64_t>::type;
};

__device__ __forceinline__ int lowest_bit(uint32_t v) { return __builtin_ctz(v); }
__device__ __forceinline__ int lowest_bit(uint64_t v) { return __builtin_ctzll(v); }
__device__ __forceinline__ int highest_bit(uint32_t v) { return 31 - __builtin_clz(v); }
__device__ __forceinline__ int highest_bit(uint64_t v) { return 63 - __builtin_clzll(v); }

// Unweighted rows (block weights are element counts, at most 32): a block's mean is its sum
// times the correctly rounded reciprocal of its length, in the forward and the backward alike.
constexpr int kRcpN = 33;

// 1/d for d = 1 .. kRcpN - 1, rounded once (by the compiler), so no kernel divides to build it.
struct RcpTable {
  double v[kRcpN];
};

constexpr RcpTable make_rcp_table() {
  RcpTable t{};
  for (int d = 1; d < kRcpN; ++d) t.v[d] = 1.0 / static_cast<double>(d);
  return t;
}

__constant__ RcpTable kRcp = make_rcp_table();

// The fit of one row per thread from its values in registers: float64 cumulative sums, the
// candidate points, the monotone chain (the vertex mask), the block means, NaN rows and the
// clamp. Every thread of the workgroup calls it (RCP_BARRIER: it meets a barrier before the
// chain, once the reciprocal table is in LDS). colS / colW: the workgroup's point columns,
// [NMAX + 1][THREADS] each; rcp: the reciprocal table (unweighted rows).
template <typename T, int NMAX, bool W, bool INC, bool RCP_BARRIER>
__device__ __forceinline__ void row_fit(const T (&yv)[NMAX], const T (&wv)[W ? NMAX : 1], const int nn,
                                        const bool active, double* colS, double* colW, const double* rcp,
                                        uint32_t* __restrict__ bad_weight, unsigned flags, T lo, T hi,
                                        T (&fit)[NMAX], typename MaskOf<NMAX>::type& m_out, bool& bad_out) {
  constexpr int THREADS = short_threads<NMAX, W>();
  constexpr bool EXACT = W || sizeof(T) == 8;
  constexpr double sgn = INC ? 1.0 : -1.0;
  const int tid = threadIdx.x;
  // Cumulative sums in float64 (of sgn * y: a decreasing fit is minus the increasing fit of -y).
  double S[NMAX + 1];
  double P[W ? NMAX + 1 : 1];
  bool bad = false;
  bool wbad = false;
  S[0] = 0.0;
  if constexpr (W) P[0] = 0.0;
#pragma unroll
  for (int c = 0; c < NMAX; ++c) {
    if (c < nn) {
      const double yc = sgn * static_cast<double>(yv[c]);
      if (nn != NMAX) bad |= yc != yc;
      if constexpr (W) {
        const double wc = static_cast<double>(wv[c]);
        wbad |= !(wc > 0.0);
        S[c + 1] = S[c] + wc * yc;
        P[c + 1] = P[c] + wc;
      } else {
        S[c + 1] = S[c] + yc;
      }
    }
  }
  if (nn == NMAX) {
    // (whole rows: a NaN anywhere makes the row's total NaN; so do +inf and -inf together, so a
    // NaN total sends the wave to the elements themselves)
    bad = S[NMAX] != S[NMAX];
    if (__any(bad)) {
      bad = false;
#pragma unroll
      for (int c = 0; c < NMAX; ++c) bad |= yv[c] != yv[c];
    }
  }
  if constexpr (W) {
    if (active && wbad && bad_weight != nullptr) *bad_weight = 1u;
  }
  if (active) {
#pragma unroll
    for (int k = 0; k <= NMAX; ++k) {
      if (k <= nn) {
        colS[k * THREADS + tid] = S[k];
        if constexpr (W) colW[k * THREADS + tid] = P[k];
      }
    }
  }
  if constexpr (RCP_BARRIER) __syncthreads();  // the reciprocals (staged rows met barriers already)

  // Lower hull of P_0..P_n by the monotone chain, run as an event loop: every iteration either
  // pops the last vertex or pushes the next candidate, so a wave iterates max over its lanes of
  // (pushes + pops) rather than, step by step, the most pops any lane needs.
  //
  // Candidates: a point k (0 < k < n) with y_{k-1} >= y_k lies on or above the segment between
  // its neighbours (the slopes into and out of it are y_{k-1} and y_k, weighted or not), so it
  // is never a vertex of the hull with equal means pooled; dropping those first is exact and
  // removes about half the work on noisy rows.
  using Mask = typename MaskOf<NMAX>::type;
  Mask m = 1;
  if (active) {
    Mask cand = Mask(1) | (Mask(1) << nn);
#pragma unroll
    for (int k = 1; k < NMAX; ++k) {
      if (k < nn) {
        bool keep = INC ? yv[k - 1] < yv[k] : yv[k] < yv[k - 1];
        if constexpr (!W) {
          // Unweighted rows: two more necessary conditions for a vertex. The slope into k from
          // k - 2 must be below the slope out of it to k + 1, and the slope from k - 1 below
          // the slope to k + 2 (equal slopes pool). Both compare the differences of the same
          // sums the chain reads, times counts of 1 and 2, so exactly: a point that fails
          // either is no vertex of the hull, and dropping it first only spares the chain its
          // iterations (a wave's iterations on noisy rows of 16: 17 -> 12.7).
          if (k >= 2 && k + 1 <= nn) keep = keep && !(S[k] - S[k - 2] >= 2.0 * (S[k + 1] - S[k]));
          if (k + 2 <= nn) keep = keep && !(2.0 * (S[k] - S[k - 1]) >= S[k + 2] - S[k]);
        }
        if (keep) cand |= Mask(1) << k;
      }
    }
    if constexpr (!W) {
      // Unweighted rows: the stack is the mask m alone (its highest bit t1 the top vertex), the
      // candidates still to push are `rest`. Each iteration takes the vertex t2 below the top
      // and the next candidate k by bit scans, reads the three sums from the point column
      // (independent reads; a point's weight is its index) and pops t1 or pushes k: two masks
      // and one index are the whole state, so the loop carries no sums from one iteration to
      // the next (about 26 VALU instructions an iteration, where carrying the top two vertices
      // and the next candidate in registers took about 40 in selects and moves).
      // The first candidate goes on the stack at once (with only point 0 below it there is
      // nothing to test), which spares every lane the loop's first iteration.
      Mask rest = cand & ~Mask(1);
      int t1 = lowest_bit(rest);  // point nn is always a candidate
      rest &= rest - 1;
      m |= Mask(1) << t1;
      while (rest) {
        // (point 0 never leaves the bottom; with it alone on the stack there is nothing to pop,
        // and the bit scan below then reads point 0 again)
        const Mask below = m & ~(Mask(1) << t1);
        const int t2 = highest_bit(below | Mask(1));
        const int k = lowest_bit(rest);
        const double sA = colS[t2 * THREADS + tid];
        const double sB = colS[t1 * THREADS + tid];
        const double sk = colS[k * THREADS + tid];
        // (t1 > 0 means something lies below the top, point 0 at least: the test of both, not a
        // short circuit, which would put the test behind a branch)
        const bool pop =
            (t1 != 0) & pools<EXACT>(sB - sA, static_cast<double>(t1 - t2), sk - sB, static_cast<double>(k - t1));
        // (selects, not branches: a wave whose lanes differ would run both)
        m = pop ? below : (m | (Mask(1) << k));
        t1 = pop ? t2 : k;
        rest = pop ? rest : (rest & (rest - 1));
      }
    } else {
      // stack: t1 (last vertex) and t2 (< 0: none) with their sums and weights; the stack itself
      // is the mask m. The candidate being pushed is k; rest holds the candidates after it.
      // The first candidate goes on the stack at once (with only point 0 below it there is
      // nothing to test), which spares every lane the loop's first iteration.
      Mask rest = cand & ~Mask(1);
      int t1 = lowest_bit(rest);  // point nn is always a candidate
      rest &= rest - 1;
      int t2 = 0;
      double s1 = colS[t1 * THREADS + tid], s2 = 0.0;
      double w1 = W ? colW[W ? t1 * THREADS + tid : 0] : static_cast<double>(t1), w2 = 0.0;
      m |= Mask(1) << t1;
      int k = rest ? lowest_bit(rest) : -1;
      rest &= rest - 1;
      double sk = colS[(k > 0 ? k : 0) * THREADS + tid];
      double wk = W ? colW[W ? (k > 0 ? k : 0) * THREADS + tid : 0] : static_cast<double>(k);
      while (k >= 0) {
        bool pop = false;
        if constexpr (W) {
          pop = t2 >= 0 && pools<EXACT>(s1 - s2, w1 - w2, sk - s1, wk - w1);
        } else {
          pop = t2 >= 0 && pools<EXACT>(s1 - s2, static_cast<double>(t1 - t2), sk - s1,
                                        static_cast<double>(k - t1));
        }
        // Both possible successors are read before the choice: the vertex below t2 (a pop makes
        // it the second vertex) and the candidate after k (a push makes it the next candidate).
        const Mask below = t2 > 0 ? (m & ((Mask(1) << t2) - Mask(1))) : Mask(0);
        const int t3 = below ? highest_bit(below) : -1;
        const int kn = rest ? lowest_bit(rest) : -1;
        const double s3 = colS[(t3 > 0 ? t3 : 0) * THREADS + tid];
        const double skn = colS[(kn > 0 ? kn : 0) * THREADS + tid];
        double w3 = 0.0, wkn = 0.0;
        if constexpr (W) {
          w3 = colW[(t3 > 0 ? t3 : 0) * THREADS + tid];
          wkn = colW[(kn > 0 ? kn : 0) * THREADS + tid];
        } else {
          wkn = static_cast<double>(kn);
        }
        // (selects, not branches: a wave whose lanes differ would run both)
        m = pop ? (m & ~(Mask(1) << t1)) : (m | (Mask(1) << k));
        const int nt1 = pop ? t2 : k, nt2 = pop ? t3 : t1;
        const double ns1 = pop ? s2 : sk, ns2 = pop ? s3 : s1;
        const double nw1 = pop ? w2 : wk, nw2 = pop ? w3 : w1;
        t1 = nt1;
        t2 = nt2;
        s1 = ns1;
        s2 = ns2;
        w1 = nw1;
        w2 = nw2;
        k = pop ? k : kn;
        sk = pop ? sk : skn;
        wk = pop ? wk : wkn;
        rest = pop ? rest : (rest & (rest - 1));
      }
    }
  }

  const bool use_lo = flags & TI_CLIP_MIN, use_hi = flags & TI_CLIP_MAX;
  if constexpr (!W) {
    // Left to right: at a vertex i the block runs to the next vertex v (found from the mask, so
    // every element's reads are independent), with mean (S_v - S_i) / (v - i); the others keep
    // the mean of the block they are in.
    const Mask mv = m | (Mask(1) << nn);  // (point nn is a vertex; idle threads set it here)
    T cur = T(0);  // (rounded before the select: one register to carry, not two)
#pragma unroll
    for (int i = 0; i < NMAX; ++i) {
      if (i < nn) {
        const int v = i + 1 + lowest_bit(static_cast<Mask>(mv >> (i + 1)));
        const double mean = (colS[v * THREADS + tid] - colS[i * THREADS + tid]) * rcp[v - i];
        cur = ((m >> i) & 1u) ? static_cast<T>(sgn * mean) : cur;
        fit[i] = cur;
      }
    }
  } else {
    // Slopes, one per hull edge, from the last vertex down: each edge's slope replaces the sum
    // at its first vertex in the point column (that sum is kept in a register for the next
    // edge), then every element takes the slope of the last vertex at or before it.
    if (active) {
      double sh = colS[nn * THREADS + tid];
      double wh = colW[nn * THREADS + tid];
      Mask rem = m & ((Mask(1) << nn) - Mask(1));  // vertices below nn (point 0 among them)
      while (rem) {
        const int vl = highest_bit(rem);
        rem &= ~(Mask(1) << vl);
        const double sl = colS[vl * THREADS + tid];
        const double wl = colW[vl * THREADS + tid];
        colS[vl * THREADS + tid] = slope_div(sh - sl, wh - wl);
        sh = sl;
        wh = wl;
      }
    }
    double cur = 0.0;
#pragma unroll
    for (int i = 0; i < NMAX; ++i) {
      if (i < nn) {
        if ((m >> i) & 1ull) cur = colS[i * THREADS + tid];
        fit[i] = static_cast<T>(sgn * cur);
      }
    }
  }
  // NaN rows and the clamp, each behind a test of the whole wave (most waves skip both)
  if (__any(bad)) {
#pragma unroll
    for (int i = 0; i < NMAX; ++i) fit[i] = bad ? quiet_nan<T>() : fit[i];
  }
  if (use_lo || use_hi) {
#pragma unroll
    for (int i = 0; i < NMAX; ++i) fit[i] = clip(fit[i], use_lo, lo, use_hi, hi);
  }

  m_out = m;
  bad_out = bad;
}

template <typename T, int NMAX, bool W, bool INC>
__global__ __launch_bounds__((short_threads<NMAX, W>())) void short_fit_kernel(
    const T* __restrict__ y, const T* __restrict__ w, T* __restrict__ out,
    uint32_t* __restrict__ starts, uint32_t* __restrict__ bad_weight, int64_t batch, int n,
    unsigned flags, T lo, T hi) {
  constexpr int THREADS = short_threads<NMAX, W>();
  __shared__ double lds[short_lds_doubles<NMAX, W>()];
  T* stg = reinterpret_cast<T*>(lds);
  double* colS = lds;                        // [NMAX + 1][THREADS]
  double* colW = lds + (NMAX + 1) * THREADS;  // weighted only

  const int tid = threadIdx.x;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * THREADS;
  const int rows = static_cast<int>(min<int64_t>(THREADS, batch - row0));
  const int count = rows * n;
  const DivBy div(static_cast<uint32_t>(n));
  const bool active = tid < rows;
  __shared__ double rcp[W ? 1 : kRcpN];
  if constexpr (!W) {
    if (tid < kRcpN) rcp[tid] = kRcp.v[tid];
  }

  T yv[NMAX];
  T wv[W ? NMAX : 1];
  Span<T, THREADS, NMAX> sy;
  Span<T, THREADS, NMAX> sw;
  sy.load(y + row0 * n, count);
  if constexpr (W) sw.load(w + row0 * n, count);
  sy.to_lds(y + row0 * n, stg, count, div);
  __syncthreads();
#pragma unroll
  for (int c = 0; c < NMAX; ++c) {
    if (c < n) yv[c] = stg[tid * (n + 1) + c];
  }
  if constexpr (W) {
    __syncthreads();
    sw.to_lds(w + row0 * n, stg, count, div);
    __syncthreads();
#pragma unroll
    for (int c = 0; c < NMAX; ++c) {
      if (c < n) wv[c] = stg[tid * (n + 1) + c];
    }
  }
  __syncthreads();  // staging is dead from here: the area becomes the point columns

  T fit[NMAX];
  typename MaskOf<NMAX>::type m;
  bool bad;
  row_fit<T, NMAX, W, INC, false>(yv, wv, n, active, colS, colW, rcp, bad_weight, flags, lo, hi, fit, m, bad);

  if (starts != nullptr && active) {
    const uint32_t low = n >= 32 ? 0xFFFFFFFFu : ((1u << n) - 1u);
    starts[row0 + tid] = bad ? 1u : static_cast<uint32_t>(m) & low;
  }

  __syncthreads();  // every thread is done with the point columns
#pragma unroll
  for (int c = 0; c < NMAX; ++c) {
    if (c < n && active) stg[tid * (n + 1) + c] = fit[c];
  }
  __syncthreads();
  stage_out<T, THREADS>(out + row0 * n, stg, count, div);
}

__device__ __forceinline__ int64_t clamp64(int64_t v, int64_t lo, int64_t hi) { return v < lo ? lo : (v > hi ? hi : v); }

// Ragged rows: row r is y[offsets[r], offsets[r + 1]) of a packed array, one thread per row as
// above. A workgroup whose rows lie within THREADS * NMAX elements stages them through LDS:
// 16-byte loads and stores of the aligned chunks that cover its range (element by element in
// the two partial end chunks, or throughout if a base pointer is not 16-byte aligned). A row
// longer than NMAX is not fitted (its elements of out are not written: a workgroup holding one
// stores through an ownership bitmap) and gets its first start bit only, which keeps it apart
// from its neighbours in a segmented pass over the packed array. A workgroup whose range is
// longer than THREADS * NMAX holds such a row; each thread then reads and writes its own row.
// The start bits are flat (bit e of the packed array, word e / 32) in a zeroed array: a
// workgroup's first and last words are shared with its neighbours' (OR-ed in with atomics),
// the words between hold its elements only (stored).
template <typename T, int NMAX, bool W, bool INC>
__global__ __launch_bounds__((short_threads<NMAX, W>())) void ragged_fit_kernel(
    const T* __restrict__ y, const T* __restrict__ w, T* __restrict__ out, uint32_t* __restrict__ starts,
    uint32_t* __restrict__ bad_weight, const int64_t* __restrict__ offsets, int64_t nrows, int64_t n_all,
    unsigned flags, T lo,
    T hi) {
  constexpr int THREADS = short_threads<NMAX, W>();
  constexpr int CAP = THREADS * NMAX;        // elements a workgroup stages
  constexpr int V = Vec16<T>::kN;            // elements per 16-byte chunk
  using VT = typename Vec16<T>::type;
  constexpr int KI = (CAP / V + 2 + THREADS - 1) / THREADS;  // chunks per thread (two partial)
  constexpr int WORDS = CAP / 32 + 2;        // start-bit (or ownership) words of the range
  __shared__ __align__(16) double lds[short_lds_doubles<NMAX, W>()];
  __shared__ uint32_t own[WORDS];            // staged elements that belong to a fitted row
  __shared__ uint32_t sbits[WORDS];          // start bits of the staged range, from bit e0 % 32
  __shared__ double rcp[W ? 1 : kRcpN];
  static_assert(short_lds_doubles<NMAX, W>() * 8 >= (CAP + 2 * V) * static_cast<int>(sizeof(T)), "staging fits");
  T* stg = reinterpret_cast<T*>(lds);
  double* colS = lds;
  double* colW = lds + (NMAX + 1) * THREADS;
  const int tid = threadIdx.x;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * THREADS;
  const int rows = static_cast<int>(min<int64_t>(THREADS, nrows - row0));
  const bool active = tid < rows;
  if constexpr (!W) {
    if (tid < kRcpN) rcp[tid] = kRcp.v[tid];
  }
  // (every offset clamped: to [0, n_all], a row's to its workgroup's range, a row's end to at
  // least its start, so that no access leaves the buffers even on offsets not yet validated)
  const int64_t e0 = clamp64(offsets[row0], 0, n_all), e1 = clamp64(offsets[row0 + rows], e0, n_all);
  const int64_t my0 = active ? clamp64(offsets[row0 + tid], e0, e1) : e1;
  const int64_t my1 = active ? clamp64(offsets[row0 + tid + 1], my0, e1) : e1;
  const bool fits = active && my1 > my0 && my1 - my0 <= NMAX;  // (empty rows: nothing to fit)
  const int len = fits ? static_cast<int>(my1 - my0) : 0;
  const int64_t total = e1 - e0;
  const bool staged = total <= CAP;  // (the same in every thread)
  const int b0 = static_cast<int>(e0 & 31);    // bit of e0 within its word
  const int rel = static_cast<int>(my0 - e0);  // (staged: this row's first element in the range)
  // staged: the range as 16-byte chunks from a0 (LDS element k is y[a0 + k])
  const int64_t a0 = e0 - e0 % V;
  const int sh = static_cast<int>(e0 - a0);
  const int nch = staged ? static_cast<int>((e1 - a0 + V - 1) / V) : 0;
  const uintptr_t bases = reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(out) |
                          (W ? reinterpret_cast<uintptr_t>(w) : uintptr_t{0});
  const bool vec = (bases & 15) == 0;

  auto stage_in = [&](const T* __restrict__ src) {
    VT buf[KI];
#pragma unroll
    for (int j = 0; j < KI; ++j) {
      const int k = tid + j * THREADS;
      const int64_t g = a0 + static_cast<int64_t>(k) * V;
      buf[j] = VT{};
      if (k < nch) {
        if (vec && g >= e0 && g + V <= e1) {
          buf[j] = *reinterpret_cast<const VT*>(src + g);
        } else {
#pragma unroll
          for (int t = 0; t < V; ++t) {
            if (g + t >= e0 && g + t < e1) buf[j][t] = src[g + t];
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < KI; ++j) {
      const int k = tid + j * THREADS;
      if (k < nch) *reinterpret_cast<VT*>(stg + k * V) = buf[j];
    }
  };

  T yv[NMAX];
  T wv[W ? NMAX : 1];
  bool has_long = false;
  if (staged) {
    has_long = __syncthreads_or(active && my1 - my0 > NMAX);
    for (int k = tid; k < WORDS; k += THREADS) {
      own[k] = 0u;
      sbits[k] = 0u;
    }
    stage_in(y);
    __syncthreads();
#pragma unroll
    for (int c = 0; c < NMAX; ++c) {
      if (c < len) yv[c] = stg[sh + rel + c];
    }
    if (has_long && len > 0) {  // mark this row's elements as fitted (at most two words)
      const uint32_t mask = len >= 32 ? 0xFFFFFFFFu : ((1u << len) - 1u);
      const int bit = rel + b0;
      atomicOr(&own[bit >> 5], mask << (bit & 31));
      if ((bit & 31) + len > 32) atomicOr(&own[(bit >> 5) + 1], mask >> (32 - (bit & 31)));
    }
    if constexpr (W) {
      __syncthreads();
      stage_in(w);
      __syncthreads();
#pragma unroll
      for (int c = 0; c < NMAX; ++c) {
        if (c < len) wv[c] = stg[sh + rel + c];
      }
    }
    __syncthreads();  // staging is dead from here: the area becomes the point columns
  } else {
#pragma unroll
    for (int c = 0; c < NMAX; ++c) {
      if (c < len) {
        yv[c] = y[my0 + c];
        if constexpr (W) wv[c] = w[my0 + c];
      }
    }
  }

  T fit[NMAX];
  typename MaskOf<NMAX>::type m;
  bool bad;
  row_fit<T, NMAX, W, INC, !W>(yv, wv, len, fits, colS, colW, rcp, bad_weight, flags, lo, hi, fit, m, bad);
  // this row's start bits (a long row: its first element only)
  const uint32_t rbits = !active ? 0u : (!fits || bad) ? 1u : static_cast<uint32_t>(m) & (len >= 32 ? 0xFFFFFFFFu : ((1u << len) - 1u));

  if (staged) {
    __syncthreads();  // every thread is done with the point columns
#pragma unroll
    for (int c = 0; c < NMAX; ++c) {
      if (c < len) stg[sh + rel + c] = fit[c];
    }
    if (active && my1 > my0) {
      const int bit = rel + b0;
      atomicOr(&sbits[bit >> 5], rbits << (bit & 31));
      if ((bit & 31) != 0 && (rbits >> (32 - (bit & 31))) != 0) atomicOr(&sbits[(bit >> 5) + 1], rbits >> (32 - (bit & 31)));
    }
    __syncthreads();
    if (!has_long) {  // every element of the range is a fitted row's
#pragma unroll
      for (int j = 0; j < KI; ++j) {
        const int k = tid + j * THREADS;
        const int64_t g = a0 + static_cast<int64_t>(k) * V;
        if (k < nch) {
          if (vec && g >= e0 && g + V <= e1) {
            *reinterpret_cast<VT*>(out + g) = *reinterpret_cast<const VT*>(stg + k * V);
          } else {
#pragma unroll
            for (int t = 0; t < V; ++t) {
              if (g + t >= e0 && g + t < e1) out[g + t] = stg[k * V + t];
            }
          }
        }
      }
    } else {
      for (int e = tid; e < total; e += THREADS) {
        const int bit = e + b0;
        if ((own[bit >> 5] >> (bit & 31)) & 1u) out[e0 + e] = stg[sh + e];
      }
    }
    if (starts != nullptr) {
      const int nwords = static_cast<int>((total + b0 + 31) >> 5);
      for (int k = tid; k < nwords; k += THREADS) {
        const uint32_t v = sbits[k];
        if (k == 0 || k == nwords - 1) {
          if (v != 0u) atomicOr(&starts[(e0 >> 5) + k], v);
        } else {
          starts[(e0 >> 5) + k] = v;
        }
      }
    }
  } else {
#pragma unroll
    for (int c = 0; c < NMAX; ++c) {
      if (c < len) out[my0 + c] = fit[c];
    }
    if (starts != nullptr && active && my1 > my0) {
      const int64_t bit = my0;
      atomicOr(&starts[bit >> 5], rbits << (bit & 31));
      if ((bit & 31) != 0 && (rbits >> (32 - (bit & 31))) != 0) atomicOr(&starts[(bit >> 5) + 1], rbits >> (32 - (bit & 31)));
    }
  }
}

// The plan of a ragged set, one pass over its offsets: plan[0] bit 0 set if offsets[0] != 0,
// bit 1 if offsets[nrows] != total, bit 2 if some row has a negative length; plan[1] the longest
// row of at most kShortMax elements, plan[2] the number of longer rows, plan[3] the longest
// row; plan[4 + b] the number of rows of length bucket b (lengths in (2^(b-1), 2^b], b >= 6:
// the rows past kShortMax) and plan[68 + b] the longest of them. plan: kRaggedPlanWords zeroed
// words. keys (optional): per row its bucket, 0 for a row of at most kShortMax elements. A
// workgroup's bucket counts and longest rows gather in LDS (atomics there), then one thread per
// nonempty bucket folds them into plan. Each thread reads kPlanRows rows at a time (their loads in
// flight together), each workgroup reduces its rows through its waves and LDS, then one thread
// folds the result into plan. The grid stays at kPlanBlocks: the folds are atomics on the same
// four words, about 12 ns each on MI355X, so 256 workgroups take 10.7 us at 1e6 rows where 977
// take 25 us (their partial results written apart would take 4.9 us before a fold of their own).
constexpr int kPlanThreads = 256;
constexpr int kPlanRows = 4;
constexpr int kPlanBlocks = 256;

// the length bucket of a row longer than kShortMax: ceil(log2(len))
__device__ __forceinline__ int ragged_bucket(unsigned long long len) { return 64 - __builtin_clzll(len - 1); }

__device__ __forceinline__ void plan_fold(unsigned long long v[4], unsigned long long o[4]) {
  v[0] |= o[0];
  v[1] = o[1] > v[1] ? o[1] : v[1];
  v[2] += o[2];
  v[3] = o[3] > v[3] ? o[3] : v[3];
}

__global__ __launch_bounds__(kPlanThreads) void ragged_plan_kernel(const int64_t* __restrict__ offsets,
                                                                  int64_t nrows, int64_t total,
                                                                  unsigned long long* __restrict__ plan,
                                                                  uint8_t* __restrict__ keys) {
  __shared__ unsigned long long part[kPlanThreads / 64][4];
  __shared__ unsigned long long hcnt[64], hmax[64];
  if (threadIdx.x < 64) {
    hcnt[threadIdx.x] = 0;
    hmax[threadIdx.x] = 0;
  }
  __syncthreads();
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kPlanThreads;
  unsigned long long v[4] = {0, 0, 0, 0};  // errors, longest short row, long rows, longest row
  for (int64_t r0 = static_cast<int64_t>(blockIdx.x) * kPlanThreads + threadIdx.x; r0 < nrows;
       r0 += kPlanRows * stride) {
    int64_t len[kPlanRows];
#pragma unroll
    for (int u = 0; u < kPlanRows; ++u) {
      const int64_t r = r0 + u * stride;
      len[u] = r < nrows ? offsets[r + 1] - offsets[r] : 0;
    }
#pragma unroll
    for (int u = 0; u < kPlanRows; ++u) {
      int key = 0;
      if (len[u] < 0) {
        v[0] |= 4u;
      } else {
        const unsigned long long l = static_cast<unsigned long long>(len[u]);
        if (len[u] <= kShortMax) {
          v[1] = l > v[1] ? l : v[1];
        } else {
          v[2] += 1;
          key = ragged_bucket(l);
          atomicAdd(&hcnt[key], 1ull);
          atomicMax(&hmax[key], l);
        }
        v[3] = l > v[3] ? l : v[3];
      }
      const int64_t r = r0 + u * stride;
      if (keys != nullptr && r < nrows) keys[r] = static_cast<uint8_t>(key);
    }
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    if (offsets[0] != 0) v[0] |= 1u;
    if (offsets[nrows] != total) v[0] |= 2u;
  }
#pragma unroll
  for (int s = 32; s > 0; s >>= 1) {
    unsigned long long o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = __shfl_xor(v[k], s);
    plan_fold(v, o);
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
#pragma unroll
    for (int k = 0; k < 4; ++k) part[wave][k] = v[k];
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int q = 1; q < kPlanThreads / 64; ++q) plan_fold(v, part[q]);
    if (v[0] != 0) atomicOr(&plan[0], v[0]);
    if (v[1] != 0) atomicMax(&plan[1], v[1]);
    if (v[2] != 0) atomicAdd(&plan[2], v[2]);
    if (v[3] != 0) atomicMax(&plan[3], v[3]);
  }
  if (threadIdx.x < 64 && hcnt[threadIdx.x] != 0) {  // (the barrier above ordered the LDS atomics)
    atomicAdd(&plan[4 + threadIdx.x], hcnt[threadIdx.x]);
    atomicMax(&plan[68 + threadIdx.x], hmax[threadIdx.x]);
  }
}

// One row's backward (block sums of g, and w; the block's fit as the forward formed it for the
// clamp mask and gw): gy = w * mask * G / W into oy, gw = (y - fit) * mask * G / W into ow
// (need_mean: gw or a clamp asks for the fit). bits: the row's start bits, bit 0 set.
template <typename T, int NMAX, bool W>
__device__ __forceinline__ void row_grad(const T (&gv)[NMAX], const T (&wv)[W ? NMAX : 1], const T (&yv)[NMAX],
                                         uint32_t bits, int n, bool need_mean, bool use_lo, T lo, bool use_hi, T hi,
                                         T (&oy)[NMAX], T (&ow)[NMAX]) {
  // Cumulative sums of w*y and w exactly as the forward forms them (increasing sign).
  double S[NMAX + 1];
  double P[W ? NMAX + 1 : 1];
  S[0] = 0.0;
  if constexpr (W) P[0] = 0.0;
  if (need_mean) {
#pragma unroll
    for (int c = 0; c < NMAX; ++c) {
      if (c < n) {
        const double yc = static_cast<double>(yv[c]);
        if constexpr (W) {
          const double wc = static_cast<double>(wv[c]);
          S[c + 1] = S[c] + wc * yc;
          P[c + 1] = P[c] + wc;
        } else {
          S[c + 1] = S[c] + yc;
        }
      }
    }
  }
  auto Wk = [&](int k) -> double {
    if constexpr (W) return P[k];
    else return static_cast<double>(k);
  };

  // Backwards: per block start i, q[i] = mask * G / W and fitv[i] = the block's fit.
  double q[NMAX];
  T fitv[NMAX];
  {
    double ga = 0.0, wa = 0.0, se = 0.0, we = 0.0;
    int end = n;
#pragma unroll
    for (int i = NMAX - 1; i >= 0; --i) {
      if (i < n) {
        if (i == n - 1 && need_mean) {
          se = S[i + 1];
          we = Wk(i + 1);
        }
        ga += static_cast<double>(gv[i]);
        if constexpr (W) wa += static_cast<double>(wv[i]);
        if ((bits >> i) & 1u) {
          const double wsum = W ? wa : static_cast<double>(end - i);
          bool pass = true;
          if (need_mean) {
            // the forward's block mean, bit for bit
            const T f = W ? static_cast<T>(slope_div(se - S[i], we - Wk(i)))
                          : static_cast<T>((se - S[i]) * (1.0 / static_cast<double>(end - i)));
            fitv[i] = f;
            pass = !(use_lo || use_hi) || clip_passes(f, use_lo, lo, use_hi, hi);
            se = S[i];
            we = Wk(i);
          }
          q[i] = pass ? ga / wsum : 0.0;
          ga = 0.0;
          wa = 0.0;
          end = i;
        }
      }
    }
  }
  {
    double cq = 0.0;
    T cf = T(0);
#pragma unroll
    for (int i = 0; i < NMAX; ++i) {
      if (i < n) {
        if ((bits >> i) & 1u) {
          cq = q[i];
          if (need_mean) cf = fitv[i];
        }
        const double wi = W ? static_cast<double>(wv[W ? i : 0]) : 1.0;
        oy[i] = static_cast<T>(wi * cq);
        if (need_mean) {
          ow[i] = static_cast<T>((static_cast<double>(yv[i]) - static_cast<double>(cf)) * cq);
        }
      }
    }
  }
}

// Ragged rows' backward: row r is [offsets[r], offsets[r + 1]) of the packed array. One wave per
// 64 consecutive rows, one lane per row of at most NMAX elements (no workgroup barriers: each
// wave has its own LDS slice). Where the packed arrays are 16-byte aligned and none of the wave's
// rows is longer than NMAX, the wave's range moves through its slice: 16-byte loads of the
// chunks covering it (from the range's start rounded down to a chunk; past the array's end a
// buffer load reads zeros), each lane then reading its row; the results go back the same way,
// whole chunks inside the range as 16-byte stores and the at most two partial chunks at its ends
// element by element, so no store touches a neighbouring wave's elements. Otherwise each lane
// reads and writes its own row. Each row's start bits come from the forward's flat bits.
// gy = w * mask * G / W and gw = (y - fit) * mask * G / W over each block (row_grad, with the
// forward's clamp). A row longer than NMAX is left alone (its elements of gy and gw are not
// written: its backward is its own forward's). Every offset is clamped into [0, n_all].
template <typename T, int NMAX, bool W>
__global__ __launch_bounds__(256) void ragged_grad_kernel(
    const uint32_t* __restrict__ starts, const T* __restrict__ g, const T* __restrict__ w, const T* __restrict__ y,
    T* __restrict__ gy, T* __restrict__ gw, const int64_t* __restrict__ offsets, int64_t nrows, int64_t n_all,
    unsigned flags, T lo, T hi) {
  constexpr int V = Vec16<T>::kN;
  constexpr int CH = NMAX / V + 1;                          // chunks a lane moves (the range + a partial one)
  constexpr int SLICE = (kWave * NMAX + V) * sizeof(T);     // bytes of a wave's slice
  static_assert((NMAX * sizeof(T)) % 16 == 0, "rows of whole chunks bound the range");
  using IT = unsigned __attribute__((ext_vector_type(4)));
  __shared__ __align__(16) char stg[4][SLICE];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int64_t r0 = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * kWave;
  if (r0 >= nrows) return;  // (the whole wave)
  char* const sl = stg[wave];
  const int rows = static_cast<int>(min<int64_t>(kWave, nrows - r0));
  const bool active = lane < rows;
  const int64_t e0 = wave_uniform(clamp64(offsets[r0], 0, n_all));
  const int64_t e1 = wave_uniform(clamp64(offsets[r0 + rows], e0, n_all));
  const int64_t my0 = active ? clamp64(offsets[r0 + lane], e0, e1) : e1;
  const int64_t my1 = active ? clamp64(offsets[r0 + lane + 1], my0, e1) : e1;
  const int64_t raw = my1 - my0;
  const bool fits = raw > 0 && raw <= NMAX;
  const int len = fits ? static_cast<int>(raw) : 0;
  const bool use_lo = flags & TI_CLIP_MIN, use_hi = flags & TI_CLIP_MAX;
  const bool need_mean = gw != nullptr || use_lo || use_hi;
  const uintptr_t bases = reinterpret_cast<uintptr_t>(g) | reinterpret_cast<uintptr_t>(gy) |
                          reinterpret_cast<uintptr_t>(gw) | (W ? reinterpret_cast<uintptr_t>(w) : uintptr_t{0}) |
                          reinterpret_cast<uintptr_t>(y);
  // (the range's length is checked as well as its rows': clamped offsets that do not increase
  // can leave short rows in a longer range, which the slice would not hold)
  const bool staged = (bases & 15) == 0 && !__any(raw > NMAX) && e1 - e0 <= int64_t{kWave} * NMAX;
  const int64_t a0 = e0 - e0 % V;                // the range's first chunk
  const int sh = static_cast<int>(e0 - a0);       // elements of that chunk before the range
  const int rel = static_cast<int>(my0 - e0);     // this row's first element within the range
  const int nch = static_cast<int>((e1 - a0 + V - 1) / V);
  uint32_t bits = 1u;
  if (len > 0) {
    const int64_t wd = my0 >> 5;
    const int sb = static_cast<int>(my0 & 31);
    uint32_t bw = starts[wd] >> sb;
    if (sb != 0 && sb + len > 32) bw |= starts[wd + 1] << (32 - sb);
    bits |= bw & (len >= 32 ? 0xFFFFFFFFu : ((1u << len) - 1u));
  }
  auto sync = [] {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  // the range of src into the slice (element a0 + x at byte x * sizeof(T)), then this lane's row
  auto row_in = [&](const T* __restrict__ src, T (&v)[NMAX]) {
    const __amdgpu_buffer_rsrc_t r = make_rsrc(src + a0, (n_all - a0) * static_cast<int64_t>(sizeof(T)));
    IT c[CH];
#pragma unroll
    for (int j = 0; j < CH; ++j) c[j] = __builtin_amdgcn_raw_buffer_load_b128(r, (lane + j * kWave) * 16, 0, 0);
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int k = lane + j * kWave;
      if (k < nch) *reinterpret_cast<IT*>(sl + k * 16) = c[j];
    }
    sync();
    const T* sv = reinterpret_cast<const T*>(sl) + sh + rel;
#pragma unroll
    for (int c2 = 0; c2 < NMAX; ++c2) {
      if (c2 < len) v[c2] = sv[c2];
    }
    sync();
  };
  // this lane's row into the slice, then the range out to dst
  auto row_out = [&](T* __restrict__ dst, const T (&v)[NMAX]) {
    T* sv = reinterpret_cast<T*>(sl) + sh + rel;
#pragma unroll
    for (int c2 = 0; c2 < NMAX; ++c2) {
      if (c2 < len) sv[c2] = v[c2];
    }
    sync();
    // whole chunks [kf, kl) inside [e0, e1); the partial ones element by element
    const int kf = sh == 0 ? 0 : 1;
    const int kl = max(kf, static_cast<int>((e1 - a0) / V));
    const int64_t fs = min(a0 + static_cast<int64_t>(kf) * V, e1);
    const int64_t fe = max(a0 + static_cast<int64_t>((e1 - a0) / V) * V, fs);
    const __amdgpu_buffer_rsrc_t r = make_rsrc(dst + a0, (e1 - a0) * static_cast<int64_t>(sizeof(T)));
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int k = lane + j * kWave;
      if (k >= kf && k < kl) __builtin_amdgcn_raw_buffer_store_b128(*reinterpret_cast<const IT*>(sl + k * 16), r, k * 16, 0, 0);
    }
    const T* sr = reinterpret_cast<const T*>(sl);
    if (lane < V) {
      const int64_t e = e0 + lane;  // the head [e0, fs)
      if (e < fs) dst[e] = sr[e - a0];
    } else if (lane < 2 * V) {
      const int64_t e = fe + (lane - V);  // the tail [fe, e1)
      if (e < e1) dst[e] = sr[e - a0];
    }
    sync();
  };

  T gv[NMAX];
  T wv[W ? NMAX : 1];
  T yv[NMAX];
  if (staged) {
    row_in(g, gv);
    if constexpr (W) row_in(w, wv);
    if (need_mean) row_in(y, yv);
  } else {
#pragma unroll
    for (int c2 = 0; c2 < NMAX; ++c2) {
      if (c2 < len) {
        gv[c2] = g[my0 + c2];
        if constexpr (W) wv[c2] = w[my0 + c2];
        if (need_mean) yv[c2] = y[my0 + c2];
      }
    }
  }
  T oy[NMAX], ow[NMAX];
  row_grad<T, NMAX, W>(gv, wv, yv, bits, len, need_mean, use_lo, lo, use_hi, hi, oy, ow);
  if (staged) {
    if (gy != nullptr) row_out(gy, oy);
    if (gw != nullptr) row_out(gw, ow);
  } else {
#pragma unroll
    for (int c2 = 0; c2 < NMAX; ++c2) {
      if (c2 < len) {
        if (gy != nullptr) gy[my0 + c2] = oy[c2];
        if (gw != nullptr) gw[my0 + c2] = ow[c2];
      }
    }
  }
}

// Backward: gy = w * mask * G / W, gw = (y - fit) * mask * G / W over each block, the block's
// fit recomputed from the same float64 cumulative sums and division the forward used (so
// bit-identical to it).
template <typename T, int NMAX, bool W>
__global__ __launch_bounds__((short_threads<NMAX, W>())) void short_grad_kernel(
    const uint32_t* __restrict__ starts, const T* __restrict__ g, const T* __restrict__ w,
    const T* __restrict__ y, T* __restrict__ gy, T* __restrict__ gw, int64_t batch, int n,
    unsigned flags, T lo, T hi) {
  constexpr int THREADS = short_threads<NMAX, W>();
  // staging only (no point columns), one array of T at a time
  __shared__ T stg[(NMAX + 1) * THREADS];

  const int tid = threadIdx.x;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * THREADS;
  const int rows = static_cast<int>(min<int64_t>(THREADS, batch - row0));
  const int count = rows * n;
  const DivBy div(static_cast<uint32_t>(n));
  const bool active = tid < rows;
  const bool use_lo = flags & TI_CLIP_MIN, use_hi = flags & TI_CLIP_MAX;
  const bool need_mean = (gw != nullptr) || use_lo || use_hi;

  T gv[NMAX];
  T wv[W ? NMAX : 1];
  T yv[NMAX];
  const uint32_t bits = (active ? starts[row0 + tid] : 0u) | 1u;
  Span<T, THREADS, NMAX> sg, sw, sy;
  sg.load(g + row0 * n, count);
  if constexpr (W) sw.load(w + row0 * n, count);
  if (need_mean) sy.load(y + row0 * n, count);
  sg.to_lds(g + row0 * n, stg, count, div);
  __syncthreads();
#pragma unroll
  for (int c = 0; c < NMAX; ++c) {
    if (c < n) gv[c] = stg[tid * (n + 1) + c];
  }
  if constexpr (W) {
    __syncthreads();
    sw.to_lds(w + row0 * n, stg, count, div);
    __syncthreads();
#pragma unroll
    for (int c = 0; c < NMAX; ++c) {
      if (c < n) wv[c] = stg[tid * (n + 1) + c];
    }
  }
  if (need_mean) {
    __syncthreads();
    sy.to_lds(y + row0 * n, stg, count, div);
    __syncthreads();
#pragma unroll
    for (int c = 0; c < NMAX; ++c) {
      if (c < n) yv[c] = stg[tid * (n + 1) + c];
    }
  }

  T oy[NMAX], ow[NMAX];
  row_grad<T, NMAX, W>(gv, wv, yv, bits, n, need_mean, use_lo, lo, use_hi, hi, oy, ow);
  if (gy != nullptr) {
    __syncthreads();
#pragma unroll
    for (int c = 0; c < NMAX; ++c) {
      if (c < n && active) stg[tid * (n + 1) + c] = oy[c];
    }
    __syncthreads();
    stage_out<T, THREADS>(gy + row0 * n, stg, count, div);
  }
  if (gw != nullptr) {
    __syncthreads();
#pragma unroll
    for (int c = 0; c < NMAX; ++c) {
      if (c < n && active) stg[tid * (n + 1) + c] = ow[c];
    }
    __syncthreads();
    stage_out<T, THREADS>(gw + row0 * n, stg, count, div);
  }
}

// A wave's 64 consecutive rows of NMAX values (a whole number of 16-byte chunks each), moved
// between memory and one row per lane through LDS: memory sees coalesced 16-byte accesses (lane l
// takes chunks l, l + 64, ...) and each lane gets its whole row. (Each lane reading its own row
// with 16-byte accesses 64 bytes apart moved C2's 128 MB in 25 us where a coalesced copy takes
// 19.) `at(o)` maps byte o of the wave's 64 * NMAX * sizeof(T) bytes to its LDS address; LDS
// operations of a wave complete in order, so a wave-scope fence between the writes and the reads
// is all the ordering the exchange needs. Chunk q is kept at chunk position q ^ ((q >> 4) & 15)
// (within its own 256 bytes): in row order lanes 4 apart would otherwise hit the same banks.
template <typename T, int NMAX>
struct WaveRows {
  static constexpr int kRowBytes = NMAX * sizeof(T);
  static constexpr int kChunks = kRowBytes / 16;  // 16-byte chunks per lane
  static constexpr int V = Vec16<T>::kN;
  using VT = typename Vec16<T>::type;
  using IT = unsigned __attribute__((ext_vector_type(4)));
  static_assert(kRowBytes % 16 == 0, "whole 16-byte chunks");

  IT c[kChunks];

  __device__ __forceinline__ static int pos(int q) { return (q ^ ((q >> 4) & 15)) * 16; }

  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t r, int lane) {
#pragma unroll
    for (int j = 0; j < kChunks; ++j) c[j] = __builtin_amdgcn_raw_buffer_load_b128(r, (lane + j * kWave) * 16, 0, 0);
  }

  template <class At>
  __device__ __forceinline__ void to_row(At at, int lane, T (&v)[NMAX]) const {
#pragma unroll
    for (int j = 0; j < kChunks; ++j) *reinterpret_cast<IT*>(at(pos(lane + j * kWave))) = c[j];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const VT x = *reinterpret_cast<const VT*>(at(pos(lane * kChunks + j)));
#pragma unroll
      for (int t = 0; t < V; ++t) v[j * V + t] = x[t];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // NT: the global stores non-temporal (the forward's fit, which no later kernel of the call
  // reads: its lines leave the caches as they are written, so no write-back of them waits at the
  // kernel's end; C2 forward 31.6 -> 30.2 us a launch, 32.2 -> 30.4 us a call; the backward's
  // outputs so stored took 0.6 us longer, and keep ordinary stores)
  template <bool NT = false, class At>
  __device__ __forceinline__ static void store(At at, int lane, const T (&v)[NMAX], __amdgpu_buffer_rsrc_t r) {
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      VT x;
#pragma unroll
      for (int t = 0; t < V; ++t) x[t] = v[j * V + t];
      *reinterpret_cast<VT*>(at(pos(lane * kChunks + j))) = x;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const IT x = *reinterpret_cast<const IT*>(at(pos(lane + j * kWave)));
      // (cache policy operand: bit 1 is the non-temporal hint)
      __builtin_amdgcn_raw_buffer_store_b128(x, r, (lane + j * kWave) * 16, 0, NT ? 2 : 0);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
};

// Whole rows of NMAX values that are a whole number of 16-byte chunks (n == NMAX, aligned): one
// row per lane, moved by WaveRows through the wave's own slice of the point columns (free while
// the rows move in and out). A workgroup walks blocks of THREADS rows (its own index, then every
// gridDim.x-th block after it), the next block's loads in flight while it fits the current one:
// two register buffers in turn (a copy from one to the other would make the compiler wait for the
// loads at the copy). Loads and stores go through buffer resources based at each wave's rows, so
// rows past the batch's end (the last block's) read zeros and store nothing, and every memory
// instruction is unconditional.
template <typename T, int NMAX, bool W, bool INC>
__global__ __launch_bounds__((short_threads<NMAX, W>())) void short_rows_kernel(
    const T* __restrict__ y, const T* __restrict__ w, T* __restrict__ out,
    uint32_t* __restrict__ starts, uint32_t* __restrict__ bad_weight, int64_t batch, unsigned flags,
    T lo, T hi) {
  constexpr int THREADS = short_threads<NMAX, W>();
  using WR = WaveRows<T, NMAX>;
  constexpr int64_t kRowBytes = WR::kRowBytes;
  __shared__ double lds[(NMAX + 1) * THREADS * (W ? 2 : 1)];
  double* colS = lds;                        // [NMAX + 1][THREADS]
  double* colW = lds + (NMAX + 1) * THREADS;  // weighted only
  __shared__ double rcp[W ? 1 : kRcpN];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  if constexpr (!W) {
    if (tid < kRcpN) rcp[tid] = kRcp.v[tid];
    __syncthreads();
  }
  // the wave's staging: byte o of its 64 rows in row o / 512 of a point-column array, at the
  // wave's 512 bytes of that row (64 * NMAX * sizeof(T) <= 512 * NMAX bytes: the array has NMAX + 1
  // rows)
  auto at_s = [&](int o) { return reinterpret_cast<char*>(colS) + (o >> 9) * (THREADS * 8) + wave * 512 + (o & 511); };
  auto at_w = [&](int o) { return reinterpret_cast<char*>(colW) + (o >> 9) * (THREADS * 8) + wave * 512 + (o & 511); };
  const int64_t nblk = (batch + THREADS - 1) / THREADS;
  const int64_t stride = gridDim.x;
  // (every resource from the block index alone, so it stays in scalar registers)
  auto rsrc = [&](const void* base, int64_t b, int64_t row_bytes) {
    const int64_t first = wave_uniform(b * THREADS + wave * kWave);
    const int64_t left = first < batch ? (batch - first) * row_bytes : 0;
    return make_rsrc(static_cast<const char*>(base) + (first < batch ? first : 0) * row_bytes, left);
  };
  struct Buf {
    WR y, w;
  };
  auto load = [&](int64_t b, Buf& bf) {
    bf.y.load(rsrc(y, b, kRowBytes), lane);
    if constexpr (W) bf.w.load(rsrc(w, b, kRowBytes), lane);
  };
  auto fit_block = [&](int64_t b, const Buf& bf) {
    const bool active = b * THREADS + tid < batch;
    T yv[NMAX], wv[W ? NMAX : 1];
    bf.y.to_row(at_s, lane, yv);
    if constexpr (W) bf.w.to_row(at_w, lane, wv);
    T fit[NMAX];
    typename MaskOf<NMAX>::type m;
    bool bad;
    // (the hull chain at a raised issue priority: a wave in it wins the SIMD over waves that are
    // staging rows in or out, so the chains, the kernel's bound, wait less; C2 forward
    // 29.2 -> 28.5 us a launch)
    __builtin_amdgcn_s_setprio(1);
    row_fit<T, NMAX, W, INC, false>(yv, wv, NMAX, active, colS, colW, rcp, bad_weight, flags, lo, hi, fit, m, bad);
    __builtin_amdgcn_s_setprio(0);
    WR::template store<true>(at_s, lane, fit, rsrc(out, b, kRowBytes));
    if (starts != nullptr) {
      const uint32_t low = NMAX >= 32 ? 0xFFFFFFFFu : ((1u << NMAX) - 1u);
      const uint32_t bits = bad ? 1u : static_cast<uint32_t>(m) & low;
      __builtin_amdgcn_raw_buffer_store_b32(bits, rsrc(starts, b, 4), lane * 4, 0, 0);
    }
  };
  Buf ba, bb;
  int64_t blk = blockIdx.x;
  load(blk, ba);
  while (blk < nblk) {
    load(blk + stride, bb);
    fit_block(blk, ba);
    blk += stride;
    if (blk >= nblk) break;
    load(blk + stride, ba);
    fit_block(blk, bb);
    blk += stride;
  }
}

// Workgroups for a kernel that walks `blocks` blocks: as many as the GPU holds at once (per CU,
// the lesser of what LDS and threads allow), or fewer where there are fewer blocks.
unsigned resident_grid(int64_t blocks, size_t lds_bytes, int threads) {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int cu = cus[dev].load(std::memory_order_relaxed);
  if (cu <= 0) {
    if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cu <= 0) cu = 256;
    cus[dev].store(cu, std::memory_order_relaxed);
  }
  const int by_lds = static_cast<int>((160 * 1024) / (lds_bytes > 0 ? lds_bytes : 1));
  const int by_threads = 2048 / threads;
  const int64_t per_cu = std::max(1, std::min(by_lds, by_threads));
  return static_cast<unsigned>(std::min<int64_t>(blocks, per_cu * cu));
}

// The backward of whole 16-byte-chunk rows (n == NMAX, aligned), laid out like short_rows_kernel:
// a persistent grid, the next block's loads in flight, coalesced accesses through a per-wave LDS
// staging area (64 rows of one array at a time). NEEDY: y is read (gw, or a clamp's mask, needs
// the block's fit).
template <typename T, int NMAX, bool W, bool NEEDY>
__global__ __launch_bounds__((short_threads<NMAX, W>())) void short_grad_rows_kernel(
    const uint32_t* __restrict__ starts, const T* __restrict__ g, const T* __restrict__ w,
    const T* __restrict__ y, T* __restrict__ gy, T* __restrict__ gw, int64_t batch, unsigned flags, T lo,
    T hi) {
  constexpr int THREADS = short_threads<NMAX, W>();
  using WR = WaveRows<T, NMAX>;
  constexpr int kRowBytes = WR::kRowBytes;
  __shared__ __align__(16) char stg[THREADS * kRowBytes];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  auto at = [&](int o) { return stg + wave * (kWave * kRowBytes) + o; };
  const bool use_lo = flags & TI_CLIP_MIN, use_hi = flags & TI_CLIP_MAX;
  const int64_t nblk = (batch + THREADS - 1) / THREADS;
  const int64_t stride = gridDim.x;
  auto rsrc = [&](const void* base, int64_t b, int64_t row_bytes) {
    const int64_t first = wave_uniform(b * THREADS + wave * kWave);
    const int64_t left = first < batch ? (batch - first) * row_bytes : 0;
    return make_rsrc(static_cast<const char*>(base) + (first < batch ? first : 0) * row_bytes, left);
  };
  struct Buf {
    WR g, w, y;
    uint32_t bits;
  };
  auto load = [&](int64_t b, Buf& bf) {
    bf.bits = __builtin_amdgcn_raw_buffer_load_b32(rsrc(starts, b, 4), lane * 4, 0, 0);
    bf.g.load(rsrc(g, b, kRowBytes), lane);
    if constexpr (W) bf.w.load(rsrc(w, b, kRowBytes), lane);
    if constexpr (NEEDY) bf.y.load(rsrc(y, b, kRowBytes), lane);
  };
  auto grad_block = [&](int64_t b, const Buf& bf) {
    T gv[NMAX], wv[W ? NMAX : 1], yv[NMAX];
    bf.g.to_row(at, lane, gv);
    if constexpr (W) bf.w.to_row(at, lane, wv);
    if constexpr (NEEDY) bf.y.to_row(at, lane, yv);
    T oy[NMAX], ow[NMAX];
    row_grad<T, NMAX, W>(gv, wv, yv, bf.bits | 1u, NMAX, NEEDY, use_lo, lo, use_hi, hi, oy, ow);
    if (gy != nullptr) WR::store(at, lane, oy, rsrc(gy, b, kRowBytes));
    if constexpr (NEEDY) {
      if (gw != nullptr) WR::store(at, lane, ow, rsrc(gw, b, kRowBytes));
    }
  };
  Buf ba, bb;
  int64_t blk = blockIdx.x;
  load(blk, ba);
  while (blk < nblk) {
    load(blk + stride, bb);
    grad_block(blk, ba);
    blk += stride;
    if (blk >= nblk) break;
    load(blk + stride, ba);
    grad_block(blk, bb);
    blk += stride;
  }
}

bool aligned16(const void* p) {
  return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15) == 0;
}

template <typename T, int NMAX, bool W>
hipError_t launch_fit(const ShortArgs& a) {
  constexpr int THREADS = short_threads<NMAX, W>();
  const unsigned blocks = static_cast<unsigned>((a.batch + THREADS - 1) / THREADS);
  auto run = [&](auto kernel) {
    kernel<<<dim3(blocks), dim3(THREADS), 0, a.stream>>>(
        static_cast<const T*>(a.y), static_cast<const T*>(a.w), static_cast<T*>(a.out),
        a.starts, a.bad_weight, a.batch, static_cast<int>(a.n), a.flags, static_cast<T>(a.lo),
        static_cast<T>(a.hi));
    return hipGetLastError();
  };
  const bool inc = (a.flags & TI_INCREASING) != 0;
  if constexpr ((NMAX * sizeof(T)) % 16 == 0) {
    if (a.n == NMAX && aligned16(a.y) && aligned16(a.w) && aligned16(a.out)) {
      const size_t lds = (static_cast<size_t>(NMAX + 1) * THREADS * (W ? 2 : 1) + (W ? 1 : kRcpN)) * sizeof(double);
      const unsigned grid = resident_grid(blocks, lds, THREADS);
      auto rows = [&](auto kernel) {
        kernel<<<dim3(grid), dim3(THREADS), 0, a.stream>>>(static_cast<const T*>(a.y), static_cast<const T*>(a.w),
                                                          static_cast<T*>(a.out), a.starts, a.bad_weight, a.batch,
                                                          a.flags, static_cast<T>(a.lo), static_cast<T>(a.hi));
        return hipGetLastError();
      };
      return inc ? rows(short_rows_kernel<T, NMAX, W, true>) : rows(short_rows_kernel<T, NMAX, W, false>);
    }
  }
  return inc ? run(short_fit_kernel<T, NMAX, W, true>) : run(short_fit_kernel<T, NMAX, W, false>);
}

template <typename T, int NMAX, bool W>
hipError_t launch_grad(const ShortGradArgs& a) {
  constexpr int THREADS = short_threads<NMAX, W>();
  const unsigned blocks = static_cast<unsigned>((a.batch + THREADS - 1) / THREADS);
  auto run = [&](auto kernel) {
    kernel<<<dim3(blocks), dim3(THREADS), 0, a.stream>>>(
        a.starts, static_cast<const T*>(a.g), static_cast<const T*>(a.w),
        static_cast<const T*>(a.y), static_cast<T*>(a.gy), static_cast<T*>(a.gw), a.batch,
        static_cast<int>(a.n), a.flags, static_cast<T>(a.lo), static_cast<T>(a.hi));
    return hipGetLastError();
  };
  if constexpr ((NMAX * sizeof(T)) % 16 == 0) {
    if (a.n == NMAX && aligned16(a.g) && aligned16(a.w) && aligned16(a.y) && aligned16(a.gy) &&
        aligned16(a.gw)) {
      const bool needy = a.gw != nullptr || (a.flags & (TI_CLIP_MIN | TI_CLIP_MAX)) != 0;
      const unsigned grid = resident_grid(blocks, static_cast<size_t>(THREADS) * NMAX * sizeof(T), THREADS);
      auto rows = [&](auto kernel) {
        kernel<<<dim3(grid), dim3(THREADS), 0, a.stream>>>(
            a.starts, static_cast<const T*>(a.g), static_cast<const T*>(a.w), static_cast<const T*>(a.y),
            static_cast<T*>(a.gy), static_cast<T*>(a.gw), a.batch, a.flags, static_cast<T>(a.lo),
            static_cast<T>(a.hi));
        return hipGetLastError();
      };
      return needy ? rows(short_grad_rows_kernel<T, NMAX, W, true>) : rows(short_grad_rows_kernel<T, NMAX, W, false>);
    }
  }
  return run(short_grad_kernel<T, NMAX, W>);
}

template <typename T, bool W>
hipError_t fit_by_n(const ShortArgs& a) {
  if (a.n <= 4) return launch_fit<T, 4, W>(a);
  if (a.n <= 8) return launch_fit<T, 8, W>(a);
  if (a.n <= 16) return launch_fit<T, 16, W>(a);
  return launch_fit<T, 32, W>(a);
}

template <typename T, bool W>
hipError_t grad_by_n(const ShortGradArgs& a) {
  if (a.n <= 4) return launch_grad<T, 4, W>(a);
  if (a.n <= 8) return launch_grad<T, 8, W>(a);
  if (a.n <= 16) return launch_grad<T, 16, W>(a);
  return launch_grad<T, 32, W>(a);
}

}  // namespace

int64_t short_grid(int64_t batch, int64_t n, bool weighted) {
  int threads = 0;
  if (n <= 4) threads = weighted ? short_threads<4, true>() : short_threads<4, false>();
  else if (n <= 8) threads = weighted ? short_threads<8, true>() : short_threads<8, false>();
  else if (n <= 16) threads = weighted ? short_threads<16, true>() : short_threads<16, false>();
  else threads = weighted ? short_threads<32, true>() : short_threads<32, false>();
  return (batch + threads - 1) / threads;
}

template <typename T, bool W>
hipError_t ragged_by_len(const RaggedArgs& a) {
  const T lo = static_cast<T>(a.lo), hi = static_cast<T>(a.hi);
  const bool inc = (a.flags & TI_INCREASING) != 0;
  auto go = [&](auto nmax) -> hipError_t {
    constexpr int NMAX = decltype(nmax)::value;
    constexpr int TH = short_threads<NMAX, W>();
    const dim3 grid(static_cast<unsigned>((a.nrows + TH - 1) / TH));
    const T* y = static_cast<const T*>(a.y);
    const T* w = static_cast<const T*>(a.w);
    T* out = static_cast<T*>(a.out);
    if (inc)
      ragged_fit_kernel<T, NMAX, W, true><<<grid, dim3(TH), 0, a.stream>>>(y, w, out, a.starts, a.bad_weight, a.offsets,
                                                                          a.nrows, a.total, a.flags, lo, hi);
    else
      ragged_fit_kernel<T, NMAX, W, false><<<grid, dim3(TH), 0, a.stream>>>(y, w, out, a.starts, a.bad_weight, a.offsets,
                                                                           a.nrows, a.total, a.flags, lo, hi);
    return hipGetLastError();
  };
  if (a.max_len <= 4) return go(std::integral_constant<int, 4>{});
  if (a.max_len <= 8) return go(std::integral_constant<int, 8>{});
  if (a.max_len <= 16) return go(std::integral_constant<int, 16>{});
  return go(std::integral_constant<int, 32>{});
}

template <typename T, bool W>
hipError_t ragged_grad_by_len(const RaggedGradArgs& a) {
  auto go = [&](auto nmax) -> hipError_t {
    constexpr int NMAX = decltype(nmax)::value;
    const dim3 grid(static_cast<unsigned>((a.nrows + 4 * kWave - 1) / (4 * kWave)));
    ragged_grad_kernel<T, NMAX, W><<<grid, dim3(4 * kWave), 0, a.stream>>>(
        a.starts, static_cast<const T*>(a.g), static_cast<const T*>(a.w), static_cast<const T*>(a.y),
        static_cast<T*>(a.gy), static_cast<T*>(a.gw), a.offsets, a.nrows, a.total, a.flags, static_cast<T>(a.lo),
        static_cast<T>(a.hi));
    return hipGetLastError();
  };
  if (a.max_len <= 4) return go(std::integral_constant<int, 4>{});
  if (a.max_len <= 8) return go(std::integral_constant<int, 8>{});
  if (a.max_len <= 16) return go(std::integral_constant<int, 16>{});
  return go(std::integral_constant<int, 32>{});
}

int64_t ragged_grid(int64_t nrows, int64_t max_len, bool weighted) { return short_grid(nrows, max_len, weighted); }

hipError_t ragged_grad(const RaggedGradArgs& a) {
  const bool weighted = a.w != nullptr;
  if (a.dtype == TI_F32) return weighted ? ragged_grad_by_len<float, true>(a) : ragged_grad_by_len<float, false>(a);
  return weighted ? ragged_grad_by_len<double, true>(a) : ragged_grad_by_len<double, false>(a);
}

hipError_t ragged_plan(const int64_t* offsets, int64_t nrows, int64_t total, unsigned long long* plan,
                       uint8_t* keys, hipStream_t stream) {
  const int64_t per_block = int64_t{kPlanThreads} * kPlanRows;
  const int64_t blocks = std::min<int64_t>(std::max<int64_t>((nrows + per_block - 1) / per_block, 1), kPlanBlocks);
  ragged_plan_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(kPlanThreads), 0, stream>>>(offsets, nrows, total,
                                                                                            plan, keys);
  return hipGetLastError();
}

hipError_t ragged_fit(const RaggedArgs& a) {
  const bool weighted = a.w != nullptr;
  if (a.dtype == TI_F32) return weighted ? ragged_by_len<float, true>(a) : ragged_by_len<float, false>(a);
  return weighted ? ragged_by_len<double, true>(a) : ragged_by_len<double, false>(a);
}

hipError_t short_fit(const ShortArgs& a) {
  const bool weighted = a.w != nullptr;
  if (a.dtype == TI_F32) return weighted ? fit_by_n<float, true>(a) : fit_by_n<float, false>(a);
  return weighted ? fit_by_n<double, true>(a) : fit_by_n<double, false>(a);
}

hipError_t short_grad(const ShortGradArgs& a) {
  const bool weighted = a.w != nullptr;
  if (a.dtype == TI_F32) return weighted ? grad_by_n<float, true>(a) : grad_by_n<float, false>(a);
  return weighted ? grad_by_n<double, true>(a) : grad_by_n<double, false>(a);
}

}  // namespace ti
