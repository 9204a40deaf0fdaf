/*
 * TEST INFRASTRUCTURE ONLY. The CPU oracle for the batched isotonic-regression path.
 *
 * Nothing in the product (torchisotonic_amd/) links, loads or calls this file. It is the checker
 * that tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg compare the HIP kernels
 * against, and it is the CPU baseline ("port") that bench.py times.
 *
 * It restates the reference's CPU path in plain C:
 *   - pool adjacent violators for one weighted increasing problem:
 *     reference src/torchisotonic/csrc/pava.h:16-69 (stack of blocks, merge while the previous
 *     block's mean is not below the current one's, NaN row -> all NaN with starts [1,0,...]);
 *   - the row-parallel driver, accumulating in the input dtype:
 *     reference src/torchisotonic/csrc/ops.cpp:17-41 (pava<scalar_t, scalar_t, int64_t>);
 *   - decreasing fits as minus the increasing fit of -y, unweighted as weights of one:
 *     reference src/torchisotonic/_api.py:131-134;
 *   - the backward, sums of g (and w) over each block:
 *     reference src/torchisotonic/_api.py:92-115.
 *
 * Three accumulation types are offered. "f32"/"f64" accumulate in the input dtype, as the
 * reference does. "f64x" runs float64 data with long double (x87, 64-bit significand)
 * block sums and products: exact on integer-valued data whose sums stay below 2^63 and whose
 * cross products stay below 2^64 (the calibration-shaped 0/1-label, integer-count rows), so
 * that block partitions there are the mathematically exact ones.
 *
 * Pinned by: tests/test_oracle.py (scipy/sklearn golden vectors under tests/golden/, brute
 * force on small rows, closed forms, KKT certificates, and bit-for-bit agreement with the
 * reference's own pava.h compiled under oracle/_ref/ when that library is present).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define TI_ORACLE_ABI 1

int ti_oracle_abi_version(void) { return TI_ORACLE_ABI; }

/* One problem: y, w of length n (unit stride), increasing fit into out, block starts into
 * starts (may be NULL). Scratch: start/weight/total stacks of n entries. Follows
 * reference pava.h:16-69 statement by statement. */
#define DEFINE_PAVA(NAME, SCALAR, ACC)                                                        \
  static void NAME(const SCALAR* y, const SCALAR* w, SCALAR* out, uint8_t* starts, int64_t n, \
                   int64_t* start, ACC* weight, ACC* total) {                                 \
    int64_t top = -1;                                                                         \
    for (int64_t i = 0; i < n; ++i) {                                                         \
      ACC yi = (ACC)y[i];                                                                     \
      if (yi != yi) { /* NaN: the whole row is NaN, one block */                              \
        for (int64_t j = 0; j < n; ++j) {                                                     \
          out[j] = (SCALAR)yi;                                                                \
          if (starts) starts[j] = (uint8_t)(j == 0);                                          \
        }                                                                                     \
        return;                                                                               \
      }                                                                                       \
      ACC wi = (ACC)w[i];                                                                     \
      ++top;                                                                                  \
      start[top] = i;                                                                         \
      weight[top] = wi;                                                                       \
      total[top] = wi * yi;                                                                   \
      while (top > 0) { /* pool while mean(prev) >= mean(cur), compared without dividing */   \
        ACC wa = weight[top - 1], ta = total[top - 1];                                        \
        ACC wb = weight[top], tb = total[top];                                                \
        if (ta * wb < tb * wa) break;                                                         \
        weight[top - 1] = wa + wb;                                                            \
        total[top - 1] = ta + tb;                                                             \
        --top;                                                                                \
      }                                                                                       \
    }                                                                                         \
    for (int64_t k = top; k >= 0; --k) { /* every element takes its block's mean */           \
      int64_t first = start[k];                                                               \
      int64_t last = k == top ? n : start[k + 1];                                             \
      SCALAR mean = (SCALAR)(total[k] / weight[k]);                                           \
      for (int64_t j = first; j < last; ++j) {                                                \
        out[j] = mean;                                                                        \
        if (starts) starts[j] = (uint8_t)(j == first);                                        \
      }                                                                                       \
    }                                                                                         \
  }

DEFINE_PAVA(pava_f32, float, float)
DEFINE_PAVA(pava_f64, double, double)
DEFINE_PAVA(pava_f64x, double, long double)

/* [batch, n] driver, rows in parallel (reference ops.cpp:30 parallelises over rows). A
 * decreasing problem runs on -y and negates the fit (reference _api.py:132-134); w == NULL
 * means weights of one (reference _api.py:131). Returns 0, or -1 on a failed allocation. */
#define DEFINE_DRIVER(NAME, PAVA, SCALAR, ACC)                                                 \
  int NAME(const SCALAR* y, const SCALAR* w, SCALAR* out, uint8_t* starts, int64_t batch,      \
           int64_t n, int increasing, int threads) {                                           \
    if (batch <= 0 || n <= 0) return 0;                                                        \
    int failed = 0;                                                                            \
    _Pragma("omp parallel num_threads(threads > 0 ? threads : 1) reduction(|| : failed)")      \
    {                                                                                          \
      int64_t* start = (int64_t*)malloc(sizeof(int64_t) * (size_t)n);                          \
      ACC* weight = (ACC*)malloc(sizeof(ACC) * (size_t)n);                                     \
      ACC* total = (ACC*)malloc(sizeof(ACC) * (size_t)n);                                      \
      SCALAR* yy = (SCALAR*)malloc(sizeof(SCALAR) * (size_t)n);                                \
      SCALAR* ww = (SCALAR*)malloc(sizeof(SCALAR) * (size_t)n);                                \
      if (!start || !weight || !total || !yy || !ww) {                                         \
        failed = 1;                                                                            \
      } else {                                                                                 \
        _Pragma("omp for schedule(static)")                                                    \
        for (int64_t b = 0; b < batch; ++b) {                                                  \
          const SCALAR* yr = y + b * n;                                                        \
          for (int64_t j = 0; j < n; ++j) {                                                    \
            yy[j] = increasing ? yr[j] : -yr[j];                                               \
            ww[j] = w ? w[b * n + j] : (SCALAR)1;                                              \
          }                                                                                    \
          SCALAR* o = out + b * n;                                                             \
          PAVA(yy, ww, o, starts ? starts + b * n : NULL, n, start, weight, total);            \
          if (!increasing)                                                                     \
            for (int64_t j = 0; j < n; ++j) o[j] = -o[j];                                      \
        }                                                                                      \
      }                                                                                        \
      free(start); free(weight); free(total); free(yy); free(ww);                              \
    }                                                                                          \
    return failed ? -1 : 0;                                                                    \
  }

DEFINE_DRIVER(ti_oracle_pava_f32, pava_f32, float, float)
DEFINE_DRIVER(ti_oracle_pava_f64, pava_f64, double, double)
DEFINE_DRIVER(ti_oracle_pava_f64x, pava_f64x, double, long double)

/* Backward of the fit over its blocks (reference _api.py:92-115): with G and W the sums of g
 * and w over an element's block (W = element count when w == NULL),
 *   gy_i = w_i * G / W,   gw_i = (y_i - fit_i) * G / W.
 * Element 0 of a row always starts a block (reference _api.py:108). Sums run in order, in the
 * dtype of the data (as index_add_ does). Any of gy / gw may be NULL; gw needs y and fit. */
#define DEFINE_GRAD(NAME, SCALAR)                                                              \
  int NAME(const uint8_t* starts, const SCALAR* g, const SCALAR* w, const SCALAR* y,           \
           const SCALAR* fit, SCALAR* gy, SCALAR* gw, int64_t batch, int64_t n, int threads) { \
    if (batch <= 0 || n <= 0) return 0;                                                        \
    if (gw && (!y || !fit)) return -2;                                                         \
    _Pragma("omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)")        \
    for (int64_t b = 0; b < batch; ++b) {                                                      \
      const int64_t base = b * n;                                                              \
      int64_t i = 0;                                                                           \
      while (i < n) {                                                                          \
        int64_t e = i + 1;                                                                     \
        while (e < n && !starts[base + e]) ++e;                                                \
        SCALAR gs = 0, ws = 0;                                                                 \
        for (int64_t j = i; j < e; ++j) {                                                      \
          gs += g[base + j];                                                                   \
          ws += w ? w[base + j] : (SCALAR)1;                                                   \
        }                                                                                      \
        SCALAR mean_grad = gs / ws;                                                            \
        for (int64_t j = i; j < e; ++j) {                                                      \
          if (gy) gy[base + j] = (w ? w[base + j] : (SCALAR)1) * mean_grad;                    \
          if (gw) gw[base + j] = (y[base + j] - fit[base + j]) * mean_grad;                    \
        }                                                                                      \
        i = e;                                                                                 \
      }                                                                                        \
    }                                                                                          \
    return 0;                                                                                  \
  }

DEFINE_GRAD(ti_oracle_grad_f32, float)
DEFINE_GRAD(ti_oracle_grad_f64, double)
