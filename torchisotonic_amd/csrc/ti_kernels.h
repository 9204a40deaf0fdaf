// Internal interface between the C ABI (ti_abi.hip) and the kernel families.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/torchisotonic_amd.h"

namespace ti {

// Rows up to this length take the short-row kernels (one thread per row).
constexpr int64_t kShortMax = 32;

// v written to *word (a word of host memory the host polls) by a kernel of one thread, with a
// store that reaches host memory directly: the stream's earlier kernels have finished by then, so
// whatever they wrote to host memory (a weight flag) is there before it.
hipError_t mark_run(uint32_t* word, uint32_t v, hipStream_t stream);

struct ShortArgs {
  const void* y;
  const void* w;  // null: unweighted
  void* out;
  uint32_t* starts;      // null: not wanted
  uint32_t* bad_weight;  // null: not checked
  int64_t batch, n;
  int dtype;
  unsigned flags;
  double lo, hi;
  hipStream_t stream;
};

struct ShortGradArgs {
  const uint32_t* starts;
  const void* g;
  const void* w;  // null: unweighted
  const void* y;  // needed for gw and for the clamp mask
  void* gy;
  void* gw;
  int64_t batch, n;
  int dtype;
  unsigned flags;
  double lo, hi;
  hipStream_t stream;
};

// Calibration: piecewise-linear interpolation of (xp, fp) (m knots, xp sorted) at n points.
hipError_t interp(const void* x, const void* xp, const void* fp, void* out, int64_t n, int64_t m, int dtype,
                  hipStream_t stream);
// The knot index that narrows each query's search to a bucket of about four knots: its size
// for m knots, its build from xp, and interp through it (the same output bit for bit).
size_t interp_index_bytes(int64_t m);
hipError_t interp_index(const void* xp, int64_t m, int dtype, void* index, hipStream_t stream);
hipError_t interp_indexed(const void* x, const void* xp, const void* fp, const void* index, size_t index_bytes,
                          void* out, int64_t n, int64_t m, int dtype, hipStream_t stream);

// Ragged rows of at most max_len (<= kShortMax) elements: row r is y[offsets[r], offsets[r + 1]).
struct RaggedArgs {
  const void* y;
  const void* w;  // null: unweighted
  void* out;
  uint32_t* starts;      // flat bits of the packed array (zeroed by the caller), or null
  uint32_t* bad_weight;  // null: not checked
  const int64_t* offsets;
  int64_t nrows, total, max_len;  // total: the packed array's elements (offsets are clamped to it)
  int dtype;
  unsigned flags;
  double lo, hi;
  hipStream_t stream;
};
int64_t ragged_grid(int64_t nrows, int64_t max_len, bool weighted);
hipError_t ragged_fit(const RaggedArgs& a);
// The backward of the ragged rows of at most max_len (<= kShortMax) elements, from the
// forward's flat start bits; longer rows' elements are not written.
struct RaggedGradArgs {
  const uint32_t* starts;  // the forward's flat bits
  const void* g;
  const void* w;  // null: unweighted
  const void* y;  // needed for gw and for the clamp mask
  void* gy;       // null: not wanted
  void* gw;       // null: not wanted
  const int64_t* offsets;
  int64_t nrows, total, max_len;
  int dtype;
  unsigned flags;  // the forward's (its clamp)
  double lo, hi;
  hipStream_t stream;
};
hipError_t ragged_grad(const RaggedGradArgs& a);
// plan: kRaggedPlanWords zeroed device words; keys: one byte per row, or null (see
// ragged_plan_kernel)
constexpr int kRaggedPlanWords = 132;
hipError_t ragged_plan(const int64_t* offsets, int64_t nrows, int64_t total, unsigned long long* plan,
                       uint8_t* keys, hipStream_t stream);

// Ragged rows of a length bucket as a dense [k, L] block (ti_ragged.hip): each row's extreme
// (keys: k zeroed device words), the block with each row's pad (or 0 without keys), and back
// (a gradient block with its forward's starts, and w: the rows whose pad joined their last block
// have that block's gradients scaled back to the row's own weight).
int64_t ragged_chunks(int64_t len);
hipError_t ragged_extreme(const void* y, int64_t total, const int64_t* rows, int64_t k, int64_t L, int dtype,
                          bool increasing, unsigned long long* keys, hipStream_t stream);
hipError_t ragged_pack(const void* src, const void* w, int64_t total, const int64_t* rows,
                       const unsigned long long* keys, double pad, int64_t k, int64_t L, int dtype, bool increasing,
                       void* dst, void* wdst, hipStream_t stream);
hipError_t ragged_rows(const int64_t* offsets, int64_t nrows, const int64_t* order, int64_t n, int64_t* rows,
                       hipStream_t stream);
// the gradients of rows whose pad joined their last block scaled back to the row's own weight
hipError_t ragged_grad_fix(const uint32_t* starts, const void* w, const int64_t* rows, int64_t k, int64_t L, int dtype,
                           void* gy, void* gw, int64_t total, hipStream_t stream);
hipError_t ragged_unpack(const void* src, const void* src2, const int64_t* rows, int64_t k, int64_t L, int dtype,
                         void* dst, void* dst2, int64_t total, const uint32_t* starts, const void* w,
                         hipStream_t stream);

int64_t short_grid(int64_t batch, int64_t n, bool weighted);
hipError_t short_fit(const ShortArgs& a);
hipError_t short_grad(const ShortGradArgs& a);

}  // namespace ti
