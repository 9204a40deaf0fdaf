// TEST INFRASTRUCTURE ONLY. A thin C-ABI driver around the reference's own CPU solver,
// compiled (by oracle/Makefile) from the reference's header where it lies:
//   /root/reference/src/torchisotonic/csrc/pava.h   (included by path, never copied)
// into oracle/_ref/libti_ref.so. It takes the place of the reference's ATen driver
// (reference src/torchisotonic/csrc/ops.cpp:17-41, which needs torch's headers and ATen's
// parallel_for): the same per-row call pava<scalar_t, scalar_t, int64_t>(..., stride 1, ...)
// with per-thread scratch of n entries, rows split over OpenMP threads instead of ATen's.
// Decreasing problems are negated around the call as reference _api.py:132-134 does.
//
// Used to pin oracle/ti_oracle.c bit for bit and, in bench.py, as the CPU baseline
// (kind "reference"). The product never loads it.
#include <cstdint>
#include <vector>

#include "pava.h"

namespace {

template <typename scalar_t>
int drive(const scalar_t* y, const scalar_t* w, scalar_t* out, uint8_t* starts, int64_t batch,
          int64_t n, int increasing, int threads) {
  if (batch <= 0 || n <= 0) return 0;
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
  {
    std::vector<int64_t> start(n);
    std::vector<scalar_t> weight(n), total(n), yy(n), ww(n);
#pragma omp for schedule(static)
    for (int64_t b = 0; b < batch; ++b) {
      for (int64_t j = 0; j < n; ++j) {
        yy[j] = increasing ? y[b * n + j] : -y[b * n + j];
        ww[j] = w ? w[b * n + j] : scalar_t(1);
      }
      scalar_t* o = out + b * n;
      torchisotonic::pava<scalar_t, scalar_t, int64_t>(yy.data(), ww.data(), o,
                                                       starts ? starts + b * n : nullptr, n, 1,
                                                       start.data(), weight.data(), total.data());
      if (!increasing)
        for (int64_t j = 0; j < n; ++j) o[j] = -o[j];
    }
  }
  return 0;
}

}  // namespace

extern "C" {

int ti_ref_pava_f32(const float* y, const float* w, float* out, uint8_t* starts, int64_t batch,
                    int64_t n, int increasing, int threads) {
  return drive<float>(y, w, out, starts, batch, n, increasing, threads);
}

int ti_ref_pava_f64(const double* y, const double* w, double* out, uint8_t* starts,
                    int64_t batch, int64_t n, int increasing, int threads) {
  return drive<double>(y, w, out, starts, batch, n, increasing, threads);
}

}  // extern "C"
