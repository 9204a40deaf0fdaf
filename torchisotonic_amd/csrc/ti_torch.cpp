// The fit as a torch operator with its backward in C++: torch.ops.torchisotonic_amd.isotonic_fit.
//
// Takes the place of the reference's torch extension (reference src/torchisotonic/csrc/ops.cpp,
// whose operators the Python autograd.Function in _api.py:73-97 wraps): here the autograd node
// itself is C++, so autograd runs the backward on its device thread without taking the Python
// interpreter lock, and a call costs a few microseconds of host time instead of tens. The
// operator holds no kernels: it allocates outputs and workspaces with torch, takes torch's
// current HIP stream, and calls the C ABI of libtorchisotonic_amd.so.
//
//   isotonic_fit(Tensor y, Tensor? w, bool increasing, float? y_min, float? y_max) -> Tensor
//
// y: [batch, n], float32 or float64, contiguous, on a ROCm device; w: like y, or None. The fit
// is clamped to [y_min, y_max] where given; non-positive weights raise ValueError (the
// reference's check, _api.py:60-61). Differentiable in y and w.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime_api.h>
#include <torch/csrc/autograd/custom_function.h>
#include <torch/library.h>

#include <optional>

#include "torchisotonic_amd.h"

namespace {

using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

void check(int rc, const char* what) {
  TORCH_CHECK(rc == TI_OK, "torchisotonic_amd.", what, ": ", ti_last_error(), " (status ", rc, ")");
}

void check_hip(hipError_t e, const char* what) {
  TORCH_CHECK(e == hipSuccess, "torchisotonic_amd: ", what, ": ", hipGetErrorString(e));
}

int dtype_code(const at::Tensor& t) {
  if (t.scalar_type() == at::kFloat) return TI_F32;
  if (t.scalar_type() == at::kDouble) return TI_F64;
  TORCH_CHECK(false, "torchisotonic_amd: kernels take float32 or float64, got ", t.scalar_type());
}

unsigned flags_of(bool increasing, std::optional<double> lo, std::optional<double> hi) {
  return (increasing ? TI_INCREASING : 0u) | TI_EXACT | (lo ? TI_CLIP_MIN : 0u) | (hi ? TI_CLIP_MAX : 0u);
}

void* ptr(const at::Tensor& t) { return t.defined() ? t.data_ptr() : nullptr; }

at::Tensor workspace(bool fwd, int64_t batch, int64_t n, int dtype, bool weighted, const at::Device& dev) {
  size_t bytes = 0;
  check(fwd ? ti_fwd_workspace(batch, n, dtype, weighted ? 1 : 0, &bytes)
            : ti_bwd_workspace(batch, n, dtype, weighted ? 1 : 0, &bytes),
        fwd ? "fwd_workspace" : "bwd_workspace");
  if (bytes == 0) return at::Tensor();
  return at::empty({static_cast<int64_t>(bytes)}, at::TensorOptions().dtype(at::kByte).device(dev));
}

// Per thread and device: the event a weighted fit records once it has read every weight, and
// the weight flag itself in pinned host memory, which the kernels write through the fabric. The
// host waits for that event only (the first of a long row's kernels) and reads the flag while
// the rest of the fit still runs on the stream. Likewise the event a long-row fit records once
// its final hulls are merged, with their largest vertex count (a second pinned word), for a
// node that keeps those hulls instead of the workspace. (Kept until the process ends.)
struct WeightCheck {
  hipEvent_t event = nullptr;
  uint32_t* host = nullptr;  // the host's view of the flag
  uint32_t* dev = nullptr;   // the kernels' view
  hipEvent_t hulls = nullptr;
  int64_t* maxv_host = nullptr;  // the final hulls' largest vertex count
  int64_t* maxv_dev = nullptr;
};

WeightCheck& weight_check(c10::DeviceIndex dev) {
  thread_local WeightCheck per_device[64];
  TORCH_CHECK(dev >= 0 && dev < 64, "torchisotonic_amd: device index ", static_cast<int>(dev), " out of range");
  WeightCheck& wc = per_device[dev];
  if (wc.event == nullptr) {
    check_hip(hipEventCreateWithFlags(&wc.event, hipEventDisableTiming), "hipEventCreateWithFlags");
    check_hip(hipEventCreateWithFlags(&wc.hulls, hipEventDisableTiming), "hipEventCreateWithFlags");
    void* p = nullptr;
    check_hip(hipHostMalloc(&p, 16, hipHostMallocDefault), "hipHostMalloc");
    wc.host = static_cast<uint32_t*>(p);
    wc.maxv_host = reinterpret_cast<int64_t*>(static_cast<char*>(p) + 8);
    void* d = nullptr;
    check_hip(hipHostGetDevicePointer(&d, p, 0), "hipHostGetDevicePointer");
    wc.dev = static_cast<uint32_t*>(d);
    wc.maxv_dev = reinterpret_cast<int64_t*>(static_cast<char*>(d) + 8);
  }
  return wc;
}

// A long-row fit under autograd whose workspace is at least this large keeps only the final hulls
// and tile records for its backward (ti_keep): waiting for the hulls costs the host the time of the
// merges, which smaller problems would not repay.
constexpr size_t kKeepMinBytes = size_t{256} << 20;

struct IsotonicFn : public torch::autograd::Function<IsotonicFn> {
  static at::Tensor forward(AutogradContext* ctx, const at::Tensor& y, const std::optional<at::Tensor>& w_opt,
                            bool increasing, std::optional<double> y_min, std::optional<double> y_max) {
    TORCH_CHECK(y.is_cuda(), "torchisotonic_amd runs on the GPU (HIP); y is on ", y.device());
    TORCH_CHECK(y.dim() == 2, "torchisotonic_amd.isotonic_fit: y must be [batch, n]");
    const at::Tensor yc = y.contiguous();
    const at::Tensor w = w_opt.has_value() ? w_opt->contiguous() : at::Tensor();
    if (w.defined()) {
      TORCH_CHECK(w.sizes() == yc.sizes() && w.scalar_type() == yc.scalar_type() && w.device() == yc.device(),
                  "torchisotonic_amd.isotonic_fit: w must match y in shape, dtype and device");
    }
    const int dtype = dtype_code(yc);
    const int64_t batch = yc.size(0), n = yc.size(1);
    const c10::DeviceGuard guard(yc.device());
    const hipStream_t stream = c10::hip::getCurrentHIPStream(yc.device().index()).stream();
    const bool want = y.requires_grad() || (w.defined() && w_opt->requires_grad());
    const unsigned flags = flags_of(increasing, y_min, y_max);

    at::Tensor out = at::empty_like(yc);
    at::Tensor starts;
    if (want) starts = at::empty({ti_starts_words(batch, n)}, yc.options().dtype(at::kInt));
    at::Tensor ws = workspace(true, batch, n, dtype, w.defined(), yc.device());
    const size_t ws_bytes = ws.defined() ? static_cast<size_t>(ws.numel()) : 0;
    const double lo = y_min.value_or(0.0), hi = y_max.value_or(0.0);
    const bool keep = want && ws_bytes >= kKeepMinBytes;
    int64_t maxv = 0;  // > 0: the backward reads `kept`, not the workspace
    at::Tensor kept;
    if (!w.defined() && !keep) {
      check(ti_fwd(ptr(yc), nullptr, ptr(out), static_cast<uint32_t*>(ptr(starts)), nullptr, batch, n, dtype,
                   flags, lo, hi, ptr(ws), ws_bytes, stream),
            "fit");
    } else {
      WeightCheck& wc = weight_check(yc.device().index());
      // (the previous call on this thread had read every weight, and its hull count, before it
      // returned, so nothing still running writes the words)
      *static_cast<volatile uint32_t*>(wc.host) = 0u;
      *static_cast<volatile int64_t*>(wc.maxv_host) = 0;
      // keeping the hulls: one wait, for the hulls (the weights were read before them)
      check(ti_fwd_ev_hulls(ptr(yc), ptr(w), ptr(out), static_cast<uint32_t*>(ptr(starts)),
                            w.defined() ? wc.dev : nullptr, batch, n, dtype, flags, lo, hi, ptr(ws), ws_bytes, stream,
                            keep ? nullptr : wc.event, keep ? wc.hulls : nullptr, keep ? wc.maxv_dev : nullptr),
            "fit");
      check_hip(hipEventSynchronize(keep ? wc.hulls : wc.event), "hipEventSynchronize");
      TORCH_CHECK_VALUE(!w.defined() || *static_cast<volatile uint32_t*>(wc.host) == 0u,
                        "weight must be strictly positive");
      if (keep) {
        const int64_t mv = *static_cast<volatile int64_t*>(wc.maxv_host);
        size_t kbytes = 0;
        check(ti_keep_bytes(batch, n, dtype, w.defined() ? 1 : 0, mv, &kbytes), "keep_bytes");
        // (hulls nearly as large as the workspace: keep the workspace itself)
        if (kbytes < ws_bytes / 2) {
          kept = at::empty({static_cast<int64_t>(kbytes)}, yc.options().dtype(at::kByte));
          check(ti_keep(ptr(ws), ws_bytes, ptr(kept), kbytes, batch, n, dtype, w.defined() ? 1 : 0, mv, stream),
                "keep");
          maxv = mv;
          ws = at::Tensor();  // (torch's allocator orders its reuse after the copy on this stream)
        }
      }
    }
    if (want) {
      // (the workspace or the kept hulls, when there are any, ride along as a fourth saved
      // tensor; the scalars in one entry: each saved_data entry is a hash-map insert and lookup
      // of host time per call)
      const at::Tensor& state = maxv > 0 ? kept : ws;
      if (state.defined()) ctx->save_for_backward({yc, w, starts, state});
      else ctx->save_for_backward({yc, w, starts});
      ctx->saved_data["p"] = c10::List<double>(
          {static_cast<double>(flags), lo, hi, w.defined() ? 1.0 : 0.0, static_cast<double>(maxv)});
    }
    return out;
  }

  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    const c10::List<double> prm = ctx->saved_data["p"].toDoubleList();
    const unsigned flags = static_cast<unsigned>(prm.get(0));
    const double lo = prm.get(1), hi = prm.get(2);
    // (a missing w is no input of the node: y's is its only gradient edge then)
    const bool has_w = prm.get(3) != 0.0;
    const int64_t maxv = static_cast<int64_t>(prm.get(4));  // > 0: saved[3] is a kept state
    const bool want_y = ctx->needs_input_grad(0), want_w = has_w && ctx->needs_input_grad(1);
    if (!want_y && !want_w) return {at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor()};
    const variable_list saved = ctx->get_saved_variables();
    const at::Tensor& y = saved[0];
    const at::Tensor& w = saved[1];
    const at::Tensor& starts = saved[2];
    const at::Tensor ws = saved.size() > 3 ? saved[3] : at::Tensor();
    const at::Tensor g = grads[0].contiguous();
    TORCH_CHECK(g.sizes() == y.sizes() && g.scalar_type() == y.scalar_type(),
                "torchisotonic_amd: the upstream gradient must match the fit");
    const int dtype = dtype_code(g);
    const int64_t batch = g.size(0), n = g.size(1);
    const c10::DeviceGuard guard(g.device());
    const hipStream_t stream = c10::hip::getCurrentHIPStream(g.device().index()).stream();
    const bool need_y = want_w || (flags & (TI_CLIP_MIN | TI_CLIP_MAX)) != 0;
    at::Tensor gy = want_y ? at::empty_like(g) : at::Tensor();
    at::Tensor gw = want_w ? at::empty_like(g) : at::Tensor();
    const size_t ws_bytes = ws.defined() ? static_cast<size_t>(ws.numel()) : 0;
    if (maxv > 0) {
      size_t bytes = 0;
      check(ti_bwd_kept_workspace(batch, n, dtype, w.defined() ? 1 : 0, maxv, &bytes), "bwd_kept_workspace");
      at::Tensor bws = bytes > 0 ? at::empty({static_cast<int64_t>(bytes)}, g.options().dtype(at::kByte)) : at::Tensor();
      check(ti_bwd_kept(static_cast<const uint32_t*>(ptr(starts)), ptr(ws), ws_bytes, maxv, ptr(g), ptr(w),
                        need_y ? ptr(y) : nullptr, ptr(gy), ptr(gw), batch, n, dtype, flags, lo, hi, ptr(bws), bytes,
                        stream),
            "grad");
      return {gy, gw, at::Tensor(), at::Tensor(), at::Tensor()};
    }
    at::Tensor bws = workspace(false, batch, n, dtype, w.defined(), g.device());
    check(ti_bwd(static_cast<const uint32_t*>(ptr(starts)), ptr(ws), ws_bytes, ptr(g), ptr(w),
                 need_y ? ptr(y) : nullptr, ptr(gy), ptr(gw), batch, n, dtype, flags, lo, hi, ptr(bws),
                 bws.defined() ? static_cast<size_t>(bws.numel()) : 0, stream),
          "grad");
    return {gy, gw, at::Tensor(), at::Tensor(), at::Tensor()};
  }
};

at::Tensor isotonic_fit(const at::Tensor& y, const std::optional<at::Tensor>& w, bool increasing,
                        std::optional<double> y_min, std::optional<double> y_max) {
  return IsotonicFn::apply(y, w, increasing, y_min, y_max);
}

}  // namespace

TORCH_LIBRARY(torchisotonic_amd, m) {
  m.def("isotonic_fit(Tensor y, Tensor? w, bool increasing, float? y_min, float? y_max) -> Tensor", &isotonic_fit);
}
