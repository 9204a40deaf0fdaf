// The C ABI of libtorchisotonic_amd.so (declared in include/torchisotonic_amd.h): argument
// checks, regime dispatch and launch-error reporting. Preconditions mirror the reference's
// TORCH_CHECKs (reference src/torchisotonic/csrc/tiles.cuh:1926-1934, grad.cuh:389-394) as
// status codes with a thread-local message instead of exceptions.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

#include "ti_kernels.h"
#include "ti_tile.h"

namespace {

thread_local std::string g_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int ok() {
  g_error.clear();
  return TI_OK;
}

int launched(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(TI_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

// The largest row the kernels index with 32-bit element offsets within a row (the reference
// limits n the same way, tiles.cuh:1933-1934).
constexpr int64_t kMaxN = (int64_t(1) << 31) - 2;

int check_shape(int64_t batch, int64_t n, int dtype) {
  if (dtype != TI_F32 && dtype != TI_F64) return fail(TI_EDTYPE, "dtype must be TI_F32 or TI_F64, got %d", dtype);
  if (batch < 0 || n < 1) return fail(TI_EINVAL, "need batch >= 0 and n >= 1, got batch=%lld n=%lld", (long long)batch, (long long)n);
  if (n > kMaxN) return fail(TI_ESIZE, "rows of %lld elements exceed the limit of 2^31 - 2", (long long)n);
  return TI_OK;
}

__global__ void starts_to_bool_kernel(const uint32_t* __restrict__ starts, uint8_t* __restrict__ out,
                                      int64_t batch, int64_t n, int64_t wpr) {
  const int64_t total = batch * n;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = e / n, i = e - b * n;
    out[e] = (starts[b * wpr + (i >> 5)] >> (i & 31)) & 1u;
  }
}

// The call's mark (see ti::mark_run): a system-scope store, which goes to host memory directly.
__global__ __launch_bounds__(64) void mark_kernel(uint32_t* word, uint32_t v) {
  if (threadIdx.x == 0) __hip_atomic_store(word, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Sets *bad to 1 if any of w[0, count) is not positive (or is NaN). A lane that finds one
// stores the word itself.
template <typename T>
__global__ __launch_bounds__(256) void check_weights_kernel(const T* __restrict__ w, int64_t count,
                                                            uint32_t* __restrict__ bad) {
  bool found = false;
  for (int64_t e = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; e < count;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x)
    found |= !(w[e] > T(0));
  if (found) *bad = 1u;
}

// A weighted fit of at most this many elements whose caller waits for the weights to be read
// (ti_fwd_ev) reads them in a kernel of their own first: the caller's wait then ends before the
// fit starts, and its next calls queue while the fit runs. Without it the wait ends after the
// fit's first kernel, and where the fit's remaining kernels take less time than the caller's
// own work between calls the GPU idles (1000 x 5000 float32 weighted: 105 -> 96 us a call through
// torch, forward and backward 161 -> 133 us). Beyond it the second read of w costs more than that
// gap (1e8 elements: 400 MB).
constexpr int64_t kEarlyCheckElems = int64_t{1} << 24;

// ti_fwd_noalloc's workspace: one array per device, held from the library's first use on that
// device until the process ends. In host code its name is only a host-side stand-in; its
// device address comes from hipGetSymbolAddress (scratch_ptr) and only that address is used.
static __device__ __align__(256) unsigned char scratch[TI_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's scratch address, looked up once per device (that device current).
int scratch_ptr(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(TI_ELAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(TI_EINVAL, "device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(TI_ELAUNCH, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return TI_OK;
}

}  // namespace

namespace ti {
hipError_t mark_run(uint32_t* word, uint32_t v, hipStream_t stream) {
  mark_kernel<<<dim3(1), dim3(64), 0, stream>>>(word, v);
  return hipGetLastError();
}
}  // namespace ti

extern "C" {

int ti_abi_version(void) { return TI_ABI_VERSION; }

const char* ti_last_error(void) { return g_error.c_str(); }

int64_t ti_starts_words(int64_t batch, int64_t n) {
  if (batch < 0 || n < 0) return 0;
  return batch * ((n + 31) / 32);
}

int ti_fwd_workspace(int64_t batch, int64_t n, int dtype, int weighted, size_t* bytes) {
  (void)weighted;
  if (bytes == nullptr) return fail(TI_EINVAL, "bytes is null");
  if (int rc = check_shape(batch, n, dtype)) return rc;
  *bytes = 0;
  if (n <= ti::kShortMax) return ok();
  *bytes = ti::long_plan(batch, n, weighted != 0, dtype == TI_F64).bytes;
  return ok();
}

int ti_fwd_geometry(int64_t batch, int64_t n, int weighted, int64_t* span0, int* levels, int* rows_per_wave) {
  if (span0 == nullptr || levels == nullptr || rows_per_wave == nullptr) return fail(TI_EINVAL, "null output");
  if (int rc = check_shape(batch, n, TI_F32)) return rc;
  *span0 = 0;
  *levels = 0;
  *rows_per_wave = 0;
  if (n <= ti::kShortMax) return ok();
  const ti::LongPlan p = ti::long_plan(batch, n, weighted != 0, false);  // (the geometry is the dtype's either way)
  *span0 = p.span0;
  *levels = p.levels;
  *rows_per_wave = p.rows_per_wave;
  return ok();
}

}  // extern "C"

namespace {

// ti_fwd, recording weights_read (when given) on the stream once every weight has been read,
// and for rows over 32 elements writing the final hulls' largest vertex count to *max_vertices
// (when given) and recording hulls_ready (when given) once it is written.
int fwd_impl(const void* y, const void* w, void* out, uint32_t* starts, uint32_t* bad_weight,
             int64_t batch, int64_t n, int dtype, unsigned flags, double y_min, double y_max,
             void* workspace, size_t workspace_bytes, void* stream, hipEvent_t weights_read,
             hipEvent_t hulls_ready = nullptr, int64_t* max_vertices = nullptr, const ti::RowMap* map = nullptr,
             uint32_t* weights_mark = nullptr, uint32_t mark_value = 0) {
  const hipStream_t hs = static_cast<hipStream_t>(stream);
  // the one-kernel paths read the weights in their only kernel (and have no hulls to keep)
  auto then_record = [&](int rc) -> int {
    if (rc == TI_OK && weights_read != nullptr) rc = launched(hipEventRecord(weights_read, hs), "weights-read event");
    if (rc == TI_OK && weights_mark != nullptr) rc = launched(ti::mark_run(weights_mark, mark_value, hs), "weights mark");
    if (rc == TI_OK && hulls_ready != nullptr) rc = launched(hipEventRecord(hulls_ready, hs), "hulls-ready event");
    return rc;
  };
  if (int rc = check_shape(batch, n, dtype)) return rc;
  if (batch == 0) return then_record(ok());
  if (y == nullptr || out == nullptr) return fail(TI_EINVAL, "y and out must not be null");
  if (out == y || (w != nullptr && out == w)) return fail(TI_EINVAL, "out must not alias y or w");
  uint32_t* start_mark = nullptr;
  if ((weights_read != nullptr || weights_mark != nullptr) && w != nullptr && bad_weight != nullptr &&
      batch * n <= kEarlyCheckElems) {
    const int64_t count = batch * n;
    const unsigned blocks = static_cast<unsigned>((count + 1023) / 1024 < 2048 ? (count + 1023) / 1024 : 2048);
    if (dtype == TI_F32)
      check_weights_kernel<float><<<dim3(blocks), dim3(256), 0, hs>>>(static_cast<const float*>(w), count, bad_weight);
    else
      check_weights_kernel<double><<<dim3(blocks), dim3(256), 0, hs>>>(static_cast<const double*>(w), count, bad_weight);
    if (int rc = launched(hipGetLastError(), "weight check")) return rc;
    if (weights_read != nullptr)
      if (int rc = launched(hipEventRecord(weights_read, hs), "weights-read event")) return rc;
    // (rows over 32 elements: the span kernel's first thread stores the mark as it starts, one
    // launch fewer)
    if (weights_mark != nullptr && n > ti::kShortMax) start_mark = weights_mark;
    else if (weights_mark != nullptr)
      if (int rc = launched(ti::mark_run(weights_mark, mark_value, hs), "weights mark")) return rc;
    bad_weight = nullptr;  // (checked: the fit need not)
    weights_read = nullptr;
    weights_mark = nullptr;
  }
  if (n <= ti::kShortMax) {
    if (map != nullptr) return fail(TI_EINVAL, "ragged rows of a block need a block longer than 32");
    if (ti::short_grid(batch, n, w != nullptr) > 0x7FFFFFFF) return fail(TI_ESIZE, "batch too large");
    ti::ShortArgs a{y, w, out, starts, bad_weight, batch, n, dtype, flags, y_min, y_max, hs};
    return then_record(launched(ti::short_fit(a), "short-row fit"));
  }
  const ti::LongPlan plan = ti::long_plan(batch, n, w != nullptr, dtype == TI_F64);
  if (workspace == nullptr || workspace_bytes < plan.bytes)
    return fail(TI_EWORKSPACE, "workspace of %zu bytes needed, %zu given", plan.bytes, workspace_bytes);
  if ((reinterpret_cast<uintptr_t>(workspace) & 255) != 0) return fail(TI_EINVAL, "workspace must be 256-byte aligned");
  if (batch * plan.tiles_per_row > 0x7FFFFFFF) return fail(TI_ESIZE, "too many tiles");
  ti::TileArgs a{y, w, out, starts, bad_weight, batch, n, dtype, flags, y_min, y_max, hs};
  a.weights_read = weights_read;  // after the span kernel, the first of several
  a.weights_mark = weights_mark;  // likewise
  a.start_mark = start_mark;
  a.mark_value = mark_value;
  a.hulls_ready = hulls_ready;    // after the merges
  a.max_vertices = max_vertices;
  if (map != nullptr) a.map = *map;
  return launched(ti::long_fit(a, plan, workspace), "multi-tile fit");
}

// ti_bwd from the forward's workspace (fwd_ws) or from what ti_keep kept of it (kept).
int bwd_impl(const uint32_t* starts, const void* fwd_ws, size_t fwd_ws_bytes, const void* kept,
             size_t kept_bytes, int64_t kept_maxc, const void* g, const void* w, const void* y, void* gy,
             void* gw, int64_t batch, int64_t n, int dtype, unsigned flags, double y_min, double y_max,
             void* workspace, size_t workspace_bytes, void* stream, const ti::RowMap* map = nullptr) {
  if (int rc = check_shape(batch, n, dtype)) return rc;
  if (batch == 0) return ok();
  if (starts == nullptr || g == nullptr) return fail(TI_EINVAL, "starts and g must not be null");
  const bool clipping = (flags & (TI_CLIP_MIN | TI_CLIP_MAX)) != 0;
  if ((gw != nullptr || clipping) && y == nullptr)
    return fail(TI_EINVAL, "y is needed for the weight gradient and for the clamp's mask");
  if (gy == nullptr && gw == nullptr) return ok();
  if (n <= ti::kShortMax) {
    if (map != nullptr) return fail(TI_EINVAL, "ragged rows of a block need a block longer than 32");
    if (ti::short_grid(batch, n, w != nullptr) > 0x7FFFFFFF) return fail(TI_ESIZE, "batch too large");
    ti::ShortGradArgs a{starts, g, w, y, gy, gw, batch, n, dtype, flags, y_min, y_max,
                        static_cast<hipStream_t>(stream)};
    return launched(ti::short_grad(a), "short-row gradient");
  }
  const bool W = w != nullptr;
  const ti::LongPlan plan = ti::long_plan(batch, n, W, dtype == TI_F64);
  if (kept != nullptr || kept_bytes > 0 || kept_maxc != 0) {
    if (kept_maxc < 1 || kept_maxc > n + 1)
      return fail(TI_EINVAL, "max_vertices must be in [1, n + 1], got %lld", (long long)kept_maxc);
    const size_t kneed = ti::keep_plan(batch, n, W, dtype == TI_F64, kept_maxc).bytes;
    if (kept == nullptr || kept_bytes < kneed)
      return fail(TI_EWORKSPACE, "the kept state (%zu bytes) is needed, %zu given", kneed, kept_bytes);
    if ((reinterpret_cast<uintptr_t>(kept) & 255) != 0) return fail(TI_EINVAL, "the kept state must be 256-byte aligned");
  } else {
    if (fwd_ws == nullptr || fwd_ws_bytes < plan.bytes)
      return fail(TI_EWORKSPACE,
                  "the forward's workspace (%zu bytes, rows of %lld elements) is needed, %zu given "
                  "(without it, ti_grad computes the gradients from the fit and the partition)",
                  plan.bytes, (long long)n, fwd_ws_bytes);
    if ((reinterpret_cast<uintptr_t>(fwd_ws) & 255) != 0) return fail(TI_EINVAL, "workspaces must be 256-byte aligned");
  }
  const size_t need = ti::long_grad_bytes(batch, n, W, dtype == TI_F64, kept != nullptr ? kept_maxc : 0);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(TI_EWORKSPACE, "workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  if ((reinterpret_cast<uintptr_t>(workspace) & 255) != 0) return fail(TI_EINVAL, "workspaces must be 256-byte aligned");
  ti::LongGradArgs a{starts, g, w, y, gy, gw, batch, n, dtype, flags, y_min, y_max,
                     kept != nullptr ? nullptr : fwd_ws, kept, kept != nullptr ? kept_maxc : 0,
                     static_cast<hipStream_t>(stream)};
  if (map != nullptr) a.map = *map;
  return launched(ti::long_grad(a, plan, workspace), "multi-tile gradient");
}

// The row map of a bucket of ragged rows (ti_fwd_rows, ti_bwd_rows): rows given, a block longer
// than 32, and packed arrays one buffer resource addresses.
int check_rows(const int64_t* rows, int64_t k, int64_t L, int64_t total, int dtype) {
  if (dtype != TI_F32)
    return fail(TI_EDTYPE, "ragged rows of a block are float32 only, got dtype %d (ti_ragged_pack serves float64)",
                dtype);
  if (k < 0 || total < 0) return fail(TI_EINVAL, "need k >= 0 and total >= 0");
  if (L <= ti::kShortMax) return fail(TI_EINVAL, "ragged rows of a block need a block longer than 32, got %lld",
                                      (long long)L);
  if (total > ti::kRowMapBytes / 4)
    return fail(TI_ESIZE, "the packed arrays must stay below %lld bytes (ti_ragged_pack serves larger ones)",
                (long long)ti::kRowMapBytes);
  if (k > 0 && rows == nullptr) return fail(TI_EINVAL, "rows must not be null");
  return TI_OK;
}

}  // namespace

extern "C" {

int ti_fwd(const void* y, const void* w, void* out, uint32_t* starts, uint32_t* bad_weight,
           int64_t batch, int64_t n, int dtype, unsigned flags, double y_min, double y_max,
           void* workspace, size_t workspace_bytes, void* stream) {
  return fwd_impl(y, w, out, starts, bad_weight, batch, n, dtype, flags, y_min, y_max, workspace,
                  workspace_bytes, stream, nullptr);
}

int ti_fwd_noalloc(const void* y, const void* w, void* out, uint32_t* starts, uint32_t* bad_weight,
                   int64_t batch, int64_t n, int dtype, unsigned flags, double y_min, double y_max, void* stream) {
  if (int rc = check_shape(batch, n, dtype)) return rc;
  const size_t need = n <= ti::kShortMax ? 0 : ti::long_plan(batch, n, w != nullptr, dtype == TI_F64).bytes;
  if (need > TI_NOALLOC_SCRATCH_BYTES)
    return fail(TI_EWORKSPACE,
                "ti_fwd_noalloc: this problem set needs %zu bytes of workspace, its scratch holds %zu "
                "(call ti_fwd with a workspace)",
                need, static_cast<size_t>(TI_NOALLOC_SCRATCH_BYTES));
  void* ws = nullptr;
  if (need > 0) {
    if (int rc = scratch_ptr(&ws)) return rc;
  }
  return fwd_impl(y, w, out, starts, bad_weight, batch, n, dtype, flags, y_min, y_max, ws, need, stream, nullptr);
}

int ti_fwd_ev(const void* y, const void* w, void* out, uint32_t* starts, uint32_t* bad_weight,
              int64_t batch, int64_t n, int dtype, unsigned flags, double y_min, double y_max,
              void* workspace, size_t workspace_bytes, void* stream, void* weights_read) {
  return fwd_impl(y, w, out, starts, bad_weight, batch, n, dtype, flags, y_min, y_max, workspace,
                  workspace_bytes, stream, static_cast<hipEvent_t>(weights_read));
}

int ti_bwd_workspace(int64_t batch, int64_t n, int dtype, int weighted, size_t* bytes) {
  if (bytes == nullptr) return fail(TI_EINVAL, "bytes is null");
  if (int rc = check_shape(batch, n, dtype)) return rc;
  *bytes = 0;
  if (n <= ti::kShortMax) return ok();
  *bytes = ti::long_grad_bytes(batch, n, weighted != 0, dtype == TI_F64);
  return ok();
}

int ti_bwd(const uint32_t* starts, const void* fwd_workspace, size_t fwd_workspace_bytes,
           const void* g, const void* w, const void* y, void* gy, void* gw, int64_t batch,
           int64_t n, int dtype, unsigned flags, double y_min, double y_max, void* workspace,
           size_t workspace_bytes, void* stream) {
  return bwd_impl(starts, fwd_workspace, fwd_workspace_bytes, nullptr, 0, 0, g, w, y, gy, gw, batch, n, dtype,
                  flags, y_min, y_max, workspace, workspace_bytes, stream);
}

int ti_fwd_rows(const void* y, const void* w, void* out, uint32_t* starts, uint32_t* bad_weight, const int64_t* rows,
                int64_t k, int64_t L, int64_t total, double pad, int dtype, unsigned flags, double y_min,
                double y_max, void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_rows(rows, k, L, total, dtype)) return rc;
  const ti::RowMap m{rows, total, pad};
  return fwd_impl(y, w, out, starts, bad_weight, k, L, dtype, flags, y_min, y_max, workspace, workspace_bytes, stream,
                  nullptr, nullptr, nullptr, &m);
}

int ti_bwd_rows(const uint32_t* starts, const void* fwd_workspace, size_t fwd_workspace_bytes, const void* g,
                const void* w, const void* y, void* gy, void* gw, const int64_t* rows, int64_t k, int64_t L,
                int64_t total, int dtype, unsigned flags, double y_min, double y_max, void* workspace,
                size_t workspace_bytes, void* stream) {
  if (int rc = check_rows(rows, k, L, total, dtype)) return rc;
  const ti::RowMap m{rows, total, 0.0};
  if (int rc = bwd_impl(starts, fwd_workspace, fwd_workspace_bytes, nullptr, 0, 0, g, w, y, gy, gw, k, L, dtype,
                        flags, y_min, y_max, workspace, workspace_bytes, stream, &m))
    return rc;
  if (k == 0 || (gy == nullptr && gw == nullptr)) return ok();
  return launched(ti::ragged_grad_fix(starts, w, rows, k, L, dtype, gy, gw, total, static_cast<hipStream_t>(stream)),
                  "ragged gradient correction");
}

int ti_fwd_ev_hulls(const void* y, const void* w, void* out, uint32_t* starts, uint32_t* bad_weight,
                    int64_t batch, int64_t n, int dtype, unsigned flags, double y_min, double y_max,
                    void* workspace, size_t workspace_bytes, void* stream, void* weights_read,
                    void* hulls_ready, int64_t* max_vertices) {
  return fwd_impl(y, w, out, starts, bad_weight, batch, n, dtype, flags, y_min, y_max, workspace,
                  workspace_bytes, stream, static_cast<hipEvent_t>(weights_read),
                  static_cast<hipEvent_t>(hulls_ready), max_vertices);
}

int ti_fwd_marked(const void* y, const void* w, void* out, uint32_t* starts, uint32_t* bad_weight,
                  int64_t batch, int64_t n, int dtype, unsigned flags, double y_min, double y_max,
                  void* workspace, size_t workspace_bytes, void* stream, uint32_t* weights_mark,
                  uint32_t mark_value, int64_t* max_vertices) {
  return fwd_impl(y, w, out, starts, bad_weight, batch, n, dtype, flags, y_min, y_max, workspace,
                  workspace_bytes, stream, nullptr, nullptr, max_vertices, nullptr, weights_mark, mark_value);
}

int ti_keep_bytes(int64_t batch, int64_t n, int dtype, int weighted, int64_t max_vertices, size_t* bytes) {
  if (bytes == nullptr) return fail(TI_EINVAL, "bytes is null");
  if (int rc = check_shape(batch, n, dtype)) return rc;
  *bytes = 0;
  if (n <= ti::kShortMax || batch == 0) return ok();
  if (max_vertices < 1 || max_vertices > n + 1)
    return fail(TI_EINVAL, "max_vertices must be in [1, n + 1], got %lld", (long long)max_vertices);
  *bytes = ti::keep_plan(batch, n, weighted != 0, dtype == TI_F64, max_vertices).bytes;
  return ok();
}

int ti_keep(const void* fwd_workspace, size_t fwd_workspace_bytes, void* kept, size_t kept_bytes,
            int64_t batch, int64_t n, int dtype, int weighted, int64_t max_vertices, void* stream) {
  if (int rc = check_shape(batch, n, dtype)) return rc;
  if (n <= ti::kShortMax || batch == 0) return ok();
  if (max_vertices < 1 || max_vertices > n + 1)
    return fail(TI_EINVAL, "max_vertices must be in [1, n + 1], got %lld", (long long)max_vertices);
  const ti::LongPlan plan = ti::long_plan(batch, n, weighted != 0, dtype == TI_F64);
  if (fwd_workspace == nullptr || fwd_workspace_bytes < plan.bytes)
    return fail(TI_EWORKSPACE, "the forward's workspace (%zu bytes) is needed, %zu given", plan.bytes,
                fwd_workspace_bytes);
  const ti::KeepPlan kp = ti::keep_plan(batch, n, weighted != 0, dtype == TI_F64, max_vertices);
  if (kept == nullptr || kept_bytes < kp.bytes)
    return fail(TI_EWORKSPACE, "a kept buffer of %zu bytes is needed, %zu given", kp.bytes, kept_bytes);
  if ((reinterpret_cast<uintptr_t>(kept) & 255) != 0 || (reinterpret_cast<uintptr_t>(fwd_workspace) & 255) != 0)
    return fail(TI_EINVAL, "the workspace and the kept buffer must be 256-byte aligned");
  if (batch > 0x7FFFFFFF) return fail(TI_ESIZE, "batch too large");
  return launched(ti::long_keep(plan, fwd_workspace, kp, kept, static_cast<hipStream_t>(stream)), "keep");
}

int ti_bwd_kept_workspace(int64_t batch, int64_t n, int dtype, int weighted, int64_t max_vertices, size_t* bytes) {
  if (bytes == nullptr) return fail(TI_EINVAL, "bytes is null");
  if (int rc = check_shape(batch, n, dtype)) return rc;
  *bytes = 0;
  if (n <= ti::kShortMax) return ok();
  if (max_vertices < 1 || max_vertices > n + 1)
    return fail(TI_EINVAL, "max_vertices must be in [1, n + 1], got %lld", (long long)max_vertices);
  *bytes = ti::long_grad_bytes(batch, n, weighted != 0, dtype == TI_F64, max_vertices);
  return ok();
}

int ti_bwd_kept(const uint32_t* starts, const void* kept, size_t kept_bytes, int64_t max_vertices,
                const void* g, const void* w, const void* y, void* gy, void* gw, int64_t batch,
                int64_t n, int dtype, unsigned flags, double y_min, double y_max, void* workspace,
                size_t workspace_bytes, void* stream) {
  if (n > ti::kShortMax && kept == nullptr) return fail(TI_EWORKSPACE, "the kept state is needed");
  return bwd_impl(starts, nullptr, 0, kept, kept_bytes, max_vertices, g, w, y, gy, gw, batch, n, dtype, flags,
                  y_min, y_max, workspace, workspace_bytes, stream);
}

int ti_grad_workspace(int64_t batch, int64_t n, int dtype, size_t* bytes) {
  if (bytes == nullptr) return fail(TI_EINVAL, "bytes is null");
  if (int rc = check_shape(batch, n, dtype)) return rc;
  *bytes = ti::seg_grad_bytes(batch, n);
  return ok();
}

int ti_grad(const void* out, const uint32_t* starts, const void* g, const void* w, const void* y, void* gy,
            void* gw, int64_t batch, int64_t n, int dtype, void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_shape(batch, n, dtype)) return rc;
  if (batch == 0) return ok();
  if (starts == nullptr || g == nullptr || gy == nullptr) return fail(TI_EINVAL, "starts, g and gy must not be null");
  if (y != nullptr && w == nullptr) return fail(TI_EINVAL, "y is only needed for the weights' gradient (give w)");
  if (y != nullptr && (out == nullptr || gw == nullptr))
    return fail(TI_EINVAL, "the weights' gradient needs the fit (out) and gw");
  if (ti::seg_grad_tiles(batch, n) > 0x7FFFFFFF) return fail(TI_ESIZE, "too many tiles");
  const size_t need = ti::seg_grad_bytes(batch, n);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail(TI_EWORKSPACE, "workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  if ((reinterpret_cast<uintptr_t>(workspace) & 255) != 0) return fail(TI_EINVAL, "workspace must be 256-byte aligned");
  ti::SegGradArgs a{out, starts, g, w, y, gy, y != nullptr ? gw : nullptr, batch, n, dtype,
                    static_cast<hipStream_t>(stream)};
  return launched(ti::seg_grad(a, workspace), "stateless gradient");
}

int ti_fwd_ragged(const void* y, const void* w, void* out, uint32_t* starts, uint32_t* bad_weight,
                  const int64_t* offsets, int64_t nrows, int64_t total, int64_t max_len, int dtype, unsigned flags,
                  double y_min, double y_max, void* stream) {
  if (dtype != TI_F32 && dtype != TI_F64) return fail(TI_EDTYPE, "dtype must be TI_F32 or TI_F64, got %d", dtype);
  if (nrows < 0 || total < 0) return fail(TI_EINVAL, "need nrows >= 0 and total >= 0");
  if (max_len < 1 || max_len > ti::kShortMax)
    return fail(TI_ESIZE, "max_len must be in [1, %lld], got %lld", (long long)ti::kShortMax, (long long)max_len);
  if (nrows == 0) return ok();
  if (y == nullptr || out == nullptr || offsets == nullptr) return fail(TI_EINVAL, "y, out and offsets must not be null");
  if (out == y || (w != nullptr && out == w)) return fail(TI_EINVAL, "out must not alias y or w");
  if (ti::ragged_grid(nrows, max_len, w != nullptr) > 0x7FFFFFFF) return fail(TI_ESIZE, "too many rows");
  ti::RaggedArgs a{y, w, out, starts, bad_weight, offsets, nrows, total, max_len, dtype, flags, y_min, y_max,
                   static_cast<hipStream_t>(stream)};
  return launched(ti::ragged_fit(a), "ragged fit");
}

int ti_bwd_ragged(const uint32_t* starts, const void* g, const void* w, const void* y, void* gy, void* gw,
                  const int64_t* offsets, int64_t nrows, int64_t total, int64_t max_len, int dtype, unsigned flags,
                  double y_min, double y_max, void* stream) {
  if (dtype != TI_F32 && dtype != TI_F64) return fail(TI_EDTYPE, "dtype must be TI_F32 or TI_F64, got %d", dtype);
  if (nrows < 0 || total < 0) return fail(TI_EINVAL, "need nrows >= 0 and total >= 0");
  if (max_len < 1 || max_len > ti::kShortMax)
    return fail(TI_ESIZE, "max_len must be in [1, %lld], got %lld", (long long)ti::kShortMax, (long long)max_len);
  if (gw != nullptr && (w == nullptr || y == nullptr)) return fail(TI_EINVAL, "gw needs w and y");
  if ((flags & (TI_CLIP_MIN | TI_CLIP_MAX)) != 0 && y == nullptr) return fail(TI_EINVAL, "the clamp mask needs y");
  if (nrows == 0) return ok();
  if (starts == nullptr || g == nullptr || offsets == nullptr) return fail(TI_EINVAL, "starts, g and offsets must not be null");
  if (gy == nullptr && gw == nullptr) return fail(TI_EINVAL, "gy and gw must not both be null");
  for (const void* o : {static_cast<const void*>(gy), static_cast<const void*>(gw)}) {
    if (o != nullptr && (o == g || o == w || o == y)) return fail(TI_EINVAL, "gy and gw must not alias g, w or y");
  }
  if (gy != nullptr && gy == gw) return fail(TI_EINVAL, "gy and gw must not alias each other");
  if (ti::ragged_grid(nrows, max_len, w != nullptr) > 0x7FFFFFFF) return fail(TI_ESIZE, "too many rows");
  ti::RaggedGradArgs a{starts, g,     w,     y,     gy,    gw, offsets, nrows, total, max_len, dtype, flags,
                       y_min,  y_max, static_cast<hipStream_t>(stream)};
  return launched(ti::ragged_grad(a), "ragged backward");
}

static_assert(ti::kRaggedPlanWords == TI_RAGGED_PLAN_WORDS, "the plan's size");

int ti_ragged_plan(const int64_t* offsets, int64_t nrows, int64_t total, int64_t* plan, uint8_t* keys,
                   void* stream) {
  if (nrows < 0 || total < 0) return fail(TI_EINVAL, "need nrows >= 0 and total >= 0");
  if (offsets == nullptr || plan == nullptr) return fail(TI_EINVAL, "offsets and plan must not be null");
  if ((reinterpret_cast<uintptr_t>(plan) & 7) != 0) return fail(TI_EINVAL, "plan must be 8-byte aligned");
  return launched(ti::ragged_plan(offsets, nrows, total, reinterpret_cast<unsigned long long*>(plan), keys,
                                  static_cast<hipStream_t>(stream)),
                  "ragged plan");
}

int ti_ragged_rows(const int64_t* offsets, int64_t nrows, const int64_t* order, int64_t n, int64_t* rows,
                   void* stream) {
  if (nrows < 0 || n < 0) return fail(TI_EINVAL, "need nrows >= 0 and n >= 0");
  if (n == 0) return ok();
  if (nrows == 0) return fail(TI_EINVAL, "no rows to describe");
  if (offsets == nullptr || order == nullptr || rows == nullptr)
    return fail(TI_EINVAL, "offsets, order and rows must not be null");
  if (n > int64_t{0x7FFFFFFF} * 256) return fail(TI_ESIZE, "too many rows");
  return launched(ti::ragged_rows(offsets, nrows, order, n, rows, static_cast<hipStream_t>(stream)), "ragged rows");
}

// (k rows of a bucket against its block [k, L]: the descriptors' grid must fit one launch)
int check_bucket(int64_t total, const int64_t* rows, int64_t k, int64_t L, int dtype) {
  if (dtype != TI_F32 && dtype != TI_F64) return fail(TI_EDTYPE, "dtype must be TI_F32 or TI_F64, got %d", dtype);
  if (total < 0 || k < 0 || L < 1) return fail(TI_EINVAL, "need total >= 0, k >= 0 and L >= 1");
  if (k > 0 && rows == nullptr) return fail(TI_EINVAL, "rows must not be null");
  if (k * ti::ragged_chunks(L) > 0x7FFFFFFF) return fail(TI_ESIZE, "k * ceil(L / 2048) must stay below 2^31");
  return TI_OK;
}

int ti_ragged_extreme(const void* y, int64_t total, const int64_t* rows, int64_t k, int64_t L, int dtype,
                      int increasing, uint64_t* keys, void* stream) {
  if (int rc = check_bucket(total, rows, k, L, dtype)) return rc;
  if (k == 0) return ok();
  if (y == nullptr || keys == nullptr) return fail(TI_EINVAL, "y and keys must not be null");
  return launched(ti::ragged_extreme(y, total, rows, k, L, dtype, increasing != 0,
                                     reinterpret_cast<unsigned long long*>(keys), static_cast<hipStream_t>(stream)),
                  "ragged extreme");
}

int ti_ragged_pack(const void* src, const void* w, int64_t total, const int64_t* rows, const uint64_t* keys,
                   double pad, int64_t k, int64_t L, int dtype, int increasing, void* dst, void* wdst, void* stream) {
  if (int rc = check_bucket(total, rows, k, L, dtype)) return rc;
  if (k == 0) return ok();
  if (src == nullptr || dst == nullptr) return fail(TI_EINVAL, "src and dst must not be null");
  if ((w == nullptr) != (wdst == nullptr)) return fail(TI_EINVAL, "w and wdst go together");
  return launched(ti::ragged_pack(src, w, total, rows, reinterpret_cast<const unsigned long long*>(keys), pad, k, L,
                                  dtype, increasing != 0, dst, wdst, static_cast<hipStream_t>(stream)),
                  "ragged pack");
}

int ti_ragged_unpack(const void* src, const void* src2, const int64_t* rows, int64_t k, int64_t L, int dtype,
                     void* dst, void* dst2, int64_t total, const uint32_t* starts, const void* w, void* stream) {
  if (int rc = check_bucket(total, rows, k, L, dtype)) return rc;
  if (k == 0) return ok();
  if (src == nullptr || dst == nullptr) return fail(TI_EINVAL, "src and dst must not be null");
  if ((src2 == nullptr) != (dst2 == nullptr)) return fail(TI_EINVAL, "src2 and dst2 go together");
  if (w != nullptr && starts == nullptr) return fail(TI_EINVAL, "w is read with starts only");
  return launched(
      ti::ragged_unpack(src, src2, rows, k, L, dtype, dst, dst2, total, starts, w, static_cast<hipStream_t>(stream)),
      "ragged unpack");
}

int ti_interp(const void* x, const void* xp, const void* fp, void* out, int64_t n, int64_t m, int dtype,
              void* stream) {
  if (dtype != TI_F32 && dtype != TI_F64) return fail(TI_EDTYPE, "dtype must be TI_F32 or TI_F64, got %d", dtype);
  if (n < 0 || m < 1) return fail(TI_EINVAL, "need n >= 0 and m >= 1 knots, got n=%lld m=%lld", (long long)n, (long long)m);
  if (n == 0) return ok();
  if (x == nullptr || xp == nullptr || fp == nullptr || out == nullptr) return fail(TI_EINVAL, "null pointer");
  return launched(ti::interp(x, xp, fp, out, n, m, dtype, static_cast<hipStream_t>(stream)), "interp");
}

int ti_interp_index_bytes(int64_t m, int dtype, size_t* bytes) {
  if (dtype != TI_F32 && dtype != TI_F64) return fail(TI_EDTYPE, "dtype must be TI_F32 or TI_F64, got %d", dtype);
  if (bytes == nullptr) return fail(TI_EINVAL, "null pointer");
  if (m < 1) return fail(TI_EINVAL, "need m >= 1 knots, got %lld", (long long)m);
  if (m >= (int64_t{1} << 32)) return fail(TI_ESIZE, "%lld knots exceed the index's limit of 2^32 - 1", (long long)m);
  *bytes = ti::interp_index_bytes(m);
  return ok();
}

int ti_interp_index(const void* xp, int64_t m, int dtype, void* index, size_t index_bytes, void* stream) {
  size_t need = 0;
  if (int rc = ti_interp_index_bytes(m, dtype, &need)) return rc;
  if (xp == nullptr || index == nullptr) return fail(TI_EINVAL, "null pointer");
  if (index_bytes < need)
    return fail(TI_EWORKSPACE, "index of %zu bytes, need %zu", index_bytes, need);
  if ((reinterpret_cast<uintptr_t>(index) & 255) != 0) return fail(TI_EINVAL, "index must be 256-byte aligned");
  return launched(ti::interp_index(xp, m, dtype, index, static_cast<hipStream_t>(stream)), "interp index");
}

int ti_interp_indexed(const void* x, const void* xp, const void* fp, const void* index, size_t index_bytes,
                      void* out, int64_t n, int64_t m, int dtype, void* stream) {
  size_t need = 0;
  if (int rc = ti_interp_index_bytes(m, dtype, &need)) return rc;
  if (n < 0) return fail(TI_EINVAL, "need n >= 0, got %lld", (long long)n);
  if (index == nullptr) return fail(TI_EINVAL, "null pointer");
  if (index_bytes < need)
    return fail(TI_EWORKSPACE, "index of %zu bytes, need %zu", index_bytes, need);
  if ((reinterpret_cast<uintptr_t>(index) & 255) != 0) return fail(TI_EINVAL, "index must be 256-byte aligned");
  if (n == 0) return ok();
  if (x == nullptr || xp == nullptr || fp == nullptr || out == nullptr) return fail(TI_EINVAL, "null pointer");
  return launched(ti::interp_indexed(x, xp, fp, index, index_bytes, out, n, m, dtype, static_cast<hipStream_t>(stream)),
                  "interp");
}

int ti_starts_to_bool(const uint32_t* starts, uint8_t* out, int64_t batch, int64_t n, void* stream) {
  if (batch < 0 || n < 0) return fail(TI_EINVAL, "negative size");
  if (batch == 0 || n == 0) return ok();
  if (starts == nullptr || out == nullptr) return fail(TI_EINVAL, "null pointer");
  const int64_t total = batch * n;
  const int64_t blocks = (total + 255) / 256 < 65536 ? (total + 255) / 256 : 65536;
  starts_to_bool_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                          static_cast<hipStream_t>(stream)>>>(starts, out, batch, n, (n + 31) / 32);
  return launched(hipGetLastError(), "starts_to_bool");
}

}  // extern "C"
