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

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <optional>
#include <vector>

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

// Per thread and device, in coherent pinned host memory (the kernels' stores reach it directly):
// the weight flag; the mark a weighted fit writes once it has read every weight (ti_fwd_marked:
// a kernel of one thread after the first of a long row's kernels), which the host polls before
// it reads the flag, while the rest of the fit still runs on the stream; and the final hulls'
// largest vertex count, which a long-row fit writes once they are merged and which the host
// polls for a node that keeps those hulls instead of the workspace. Polled words, not events: an
// event recorded between two kernels leaves the GPU idle for about 6 us. (Kept until the
// process ends.)
struct WeightCheck {
  uint32_t* host = nullptr;  // the host's view of the flag
  uint32_t* dev = nullptr;   // the kernels' view
  uint32_t* mark_host = nullptr;
  uint32_t* mark_dev = nullptr;
  uint32_t mark = 0;             // the last call's mark
  int64_t* maxv_host = nullptr;  // the final hulls' largest vertex count
  int64_t* maxv_dev = nullptr;
};

// Polls until done(); where a second passes first (a fit that never writes its word), waits for
// the stream instead.
template <class Done>
void poll_until(Done done, hipStream_t stream) {
  const auto t0 = std::chrono::steady_clock::now();
  for (unsigned it = 0;; ++it) {
    if (done()) return;
    if ((it & 4095) == 4095 && std::chrono::steady_clock::now() - t0 > std::chrono::seconds(1)) {
      check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
      return;
    }
  }
}

WeightCheck& weight_check(c10::DeviceIndex dev) {
  thread_local WeightCheck per_device[64];
  TORCH_CHECK(dev >= 0 && dev < 64, "torchisotonic_amd: device index ", static_cast<int>(dev), " out of range");
  WeightCheck& wc = per_device[dev];
  if (wc.host == nullptr) {
    void* p = nullptr;
    check_hip(hipHostMalloc(&p, 16, hipHostMallocCoherent), "hipHostMalloc");
    std::memset(p, 0, 16);  // (marks start at 1)
    void* d = nullptr;
    check_hip(hipHostGetDevicePointer(&d, p, 0), "hipHostGetDevicePointer");
    wc.host = static_cast<uint32_t*>(p);
    wc.mark_host = static_cast<uint32_t*>(p) + 1;
    wc.maxv_host = reinterpret_cast<int64_t*>(static_cast<char*>(p) + 8);
    wc.dev = static_cast<uint32_t*>(d);
    wc.mark_dev = static_cast<uint32_t*>(d) + 1;
    wc.maxv_dev = reinterpret_cast<int64_t*>(static_cast<char*>(d) + 8);
  }
  return wc;
}

// A long-row fit under autograd whose workspace is at least keep_min_bytes() keeps only the final
// hulls and tile records for its backward (ti_keep) and frees the workspace; a smaller one is held
// until the backward. The copy costs a step about 20 us (the hull-count bound's kernel and the
// copy; C5 forward + backward), the workspace costs its memory meanwhile: the threshold is 1/128 of
// the device's memory (2.25 GB on an MI355X: C5's 1.33 GB is held, C4's 4.06 GB copied), and never
// below 256 MB, under which waiting for the hulls costs the host the time of the merges. The
// environment's TI_KEEP_MIN_BYTES (bytes), read at each call, replaces it.
size_t keep_min_bytes(int dev) {
  if (const char* e = std::getenv("TI_KEEP_MIN_BYTES")) {
    char* end = nullptr;
    const unsigned long long v = std::strtoull(e, &end, 10);
    if (end != e && *end == '\0') return static_cast<size_t>(v);
  }
  static std::atomic<size_t> per_device[64];
  const int d = dev >= 0 && dev < 64 ? dev : 0;
  size_t v = per_device[d].load(std::memory_order_relaxed);
  if (v == 0) {
    size_t total = 0;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) == hipSuccess) total = prop.totalGlobalMem;
    v = std::max<size_t>(size_t{256} << 20, total / 128);
    per_device[d].store(v, std::memory_order_relaxed);
  }
  return v;
}

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
    // (a backward is expected: the fit streams out, so the backward's first reads do not wait
    // behind its write-back)
    const unsigned fit_flags = flags | (want ? TI_STREAM_OUT : 0u);

    at::Tensor out = at::empty_like(yc);
    at::Tensor starts;
    if (want) starts = at::empty({ti_starts_words(batch, n)}, yc.options().dtype(at::kInt));
    at::Tensor ws = workspace(true, batch, n, dtype, w.defined(), yc.device());
    const size_t ws_bytes = ws.defined() ? static_cast<size_t>(ws.numel()) : 0;
    const double lo = y_min.value_or(0.0), hi = y_max.value_or(0.0);
    const bool keep = want && ws_bytes >= keep_min_bytes(yc.device().index());
    int64_t maxv = 0;  // > 0: the backward reads `kept`, not the workspace
    at::Tensor kept;
    if (!w.defined() && !keep) {
      check(ti_fwd(ptr(yc), nullptr, ptr(out), static_cast<uint32_t*>(ptr(starts)), nullptr, batch, n, dtype,
                   fit_flags, lo, hi, ptr(ws), ws_bytes, stream),
            "fit");
    } else {
      WeightCheck& wc = weight_check(yc.device().index());
      // (the previous call on this thread had read every weight, and its hull count, before it
      // returned, so nothing still running writes the flag or the count; a mark it wrote late
      // would be its own, not this call's)
      *static_cast<volatile uint32_t*>(wc.host) = 0u;
      *static_cast<volatile int64_t*>(wc.maxv_host) = 0;
      const uint32_t mark = ++wc.mark == 0 ? ++wc.mark : wc.mark;
      // keeping the hulls: one wait, for the hull count (the weights were read before it)
      check(ti_fwd_marked(ptr(yc), ptr(w), ptr(out), static_cast<uint32_t*>(ptr(starts)),
                          w.defined() ? wc.dev : nullptr, batch, n, dtype, fit_flags, lo, hi, ptr(ws), ws_bytes, stream,
                          keep ? nullptr : wc.mark_dev, mark, keep ? wc.maxv_dev : nullptr),
            "fit");
      if (keep) poll_until([&] { return *static_cast<volatile int64_t*>(wc.maxv_host) != 0; }, stream);
      else poll_until([&] { return *static_cast<volatile uint32_t*>(wc.mark_host) == mark; }, stream);
      TORCH_CHECK_VALUE(!w.defined() || *static_cast<volatile uint32_t*>(wc.host) == 0u,
                        "weight must be strictly positive");
      const int64_t mv = keep ? *static_cast<volatile int64_t*>(wc.maxv_host) : 0;
      // (a bound not written, after the stream's wait: keep the workspace)
      if (mv >= 1) {
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

// Per thread and device: the pinned host words a ragged set's plan is copied into, and the event
// recorded once they are there. (Kept until the process ends.)
struct RaggedHost {
  hipEvent_t ready = nullptr;
  int64_t* words = nullptr;
};

RaggedHost& ragged_host(c10::DeviceIndex dev) {
  thread_local RaggedHost per_device[64];
  TORCH_CHECK(dev >= 0 && dev < 64, "torchisotonic_amd: device index ", static_cast<int>(dev), " out of range");
  RaggedHost& rh = per_device[dev];
  if (rh.ready == nullptr) {
    check_hip(hipEventCreateWithFlags(&rh.ready, hipEventDisableTiming), "hipEventCreateWithFlags");
    void* p = nullptr;
    check_hip(hipHostMalloc(&p, TI_RAGGED_PLAN_WORDS * sizeof(int64_t), hipHostMallocDefault), "hipHostMalloc");
    rh.words = static_cast<int64_t*>(p);
  }
  return rh;
}

constexpr int64_t kRaggedShort = 32;  // the longest rows ti_fwd_ragged fits
// the op's one zeroed buffer, in int32 words: the plan, the weight flag, the flat start bits
constexpr int64_t kRowMapBytes = 0x7FFF0000;  // (ti_fwd_rows' limit on the packed arrays)
constexpr int64_t kPlanAt = 0, kBadAt = 2 * TI_RAGGED_PLAN_WORDS, kBitsAt = kBadAt + 2;

// Length buckets of the longer rows, from the plan's counts and longest rows: (first descriptor,
// rows, block length) triples. A bucket joins the next longer one while that pads at most
// kBucketMerge more elements: a bucket's launches cost about as much as fitting that many (the
// span, merge and expansion kernels of a small block run for tens of microseconds).
constexpr int64_t kBucketMerge = int64_t{1} << 22;

std::vector<int64_t> ragged_buckets(const int64_t* words, int64_t n_long) {
  std::vector<int64_t> out;
  int64_t first = 0, k = 0, L = 0;
  for (int b = 6; b < 64; ++b) {
    const int64_t kb = words[4 + b], Lb = words[68 + b];
    if (kb <= 0) continue;
    if (k > 0 && k * (Lb - L) > kBucketMerge) {
      out.insert(out.end(), {first, k, L});
      first += k;
      k = 0;
    }
    k += kb;
    L = Lb;
  }
  if (k > 0) out.insert(out.end(), {first, k, L});
  TORCH_CHECK(first + k == n_long, "torchisotonic_amd: the plan's buckets hold ", first + k, " rows, not ", n_long);
  return out;
}

// Ragged rows (rows packed end to end, offsets on the device) with their backward in C++, the
// calls of ragged.py's steps in one operator: the offsets' plan (ti_ragged_plan) and the copy of
// its words to the host; given a bound max_len on the row lengths, the short rows' fit
// (ti_fwd_ragged, which clamps every offset it reads) launched right behind that copy, so that
// it runs while the host waits for the words; the wait and the offsets' errors; a second launch
// over every short row where rows past the bound are at most 32 long; the longer rows a length
// bucket at a time (lengths in (2^(b-1), 2^b], small buckets merged into the next): the rows
// in bucket order by a stable sort of the plan's keys on the device (ti_ragged_rows), the
// buckets sized by the plan's counts; per bucket the rows gathered into one dense block, each
// padded beyond its own extreme (float32: the largest finite value; float64: from
// ti_ragged_extreme) by ti_ragged_pack, one ti_fwd over the block, and its fits scattered back
// (ti_ragged_unpack). The backward is one launch for the
// short rows (ti_bwd_ragged) and, per bucket, g gathered into a block, one ti_bwd from the
// bucket's forward, and the gradients scattered back.
struct RaggedFn : public torch::autograd::Function<RaggedFn> {
  static at::Tensor forward(AutogradContext* ctx, const at::Tensor& values, const std::optional<at::Tensor>& w_opt,
                            const at::Tensor& offsets, bool increasing, int64_t max_len, bool from_lengths) {
    TORCH_CHECK(values.is_cuda() && values.dim() == 1 && values.is_contiguous(),
                "torchisotonic_amd.isotonic_ragged_fit: values must be 1-D, contiguous, on a ROCm device");
    TORCH_CHECK(offsets.dim() == 1 && offsets.numel() >= 1 && offsets.scalar_type() == at::kLong &&
                    offsets.is_contiguous() && offsets.device() == values.device(),
                "torchisotonic_amd.isotonic_ragged_fit: offsets must be 1-D int64, contiguous, on values' device");
    const at::Tensor w = w_opt.has_value() ? *w_opt : at::Tensor();
    if (w.defined()) {
      TORCH_CHECK(w.sizes() == values.sizes() && w.scalar_type() == values.scalar_type() &&
                      w.device() == values.device() && w.is_contiguous(),
                  "torchisotonic_amd.isotonic_ragged_fit: weight must match values");
    }
    const int dtype = dtype_code(values);
    const int64_t nrows = offsets.numel() - 1, total = values.numel();
    const c10::DeviceGuard guard(values.device());
    const hipStream_t stream = c10::hip::getCurrentHIPStream(values.device().index()).stream();
    const unsigned flags = (increasing ? TI_INCREASING : 0u) | TI_EXACT;

    // one zeroed buffer: the plan, the weight flag, the flat start bits
    at::Tensor zeros = at::zeros({kBitsAt + (total + 31) / 32}, values.options().dtype(at::kInt));
    int32_t* zp = zeros.data_ptr<int32_t>();
    int64_t* plan = reinterpret_cast<int64_t*>(zp + kPlanAt);
    uint32_t* bad = w.defined() ? reinterpret_cast<uint32_t*>(zp + kBadAt) : nullptr;
    uint32_t* bits = reinterpret_cast<uint32_t*>(zp + kBitsAt);
    RaggedHost& rh = ragged_host(values.device().index());
    // (the rows' bucket keys unless max_len rules longer rows out)
    const bool keyed = !(max_len > 0 && max_len <= kRaggedShort);
    at::Tensor keys = keyed ? at::empty({nrows}, offsets.options().dtype(at::kByte)) : at::Tensor();
    check(ti_ragged_plan(offsets.data_ptr<int64_t>(), nrows, total, plan,
                         keyed ? keys.data_ptr<uint8_t>() : nullptr, stream),
          "isotonic_ragged");
    check_hip(hipMemcpyAsync(rh.words, plan, TI_RAGGED_PLAN_WORDS * sizeof(int64_t), hipMemcpyDeviceToHost, stream),
              "hipMemcpyAsync");
    check_hip(hipEventRecord(rh.ready, stream), "hipEventRecord");
    at::Tensor out = at::empty_like(values);
    const int64_t nmax = max_len > 0 ? std::min(max_len, kRaggedShort) : 0;
    auto fit_short = [&](int64_t m) {
      check(ti_fwd_ragged(ptr(values), ptr(w), ptr(out), bits, bad, offsets.data_ptr<int64_t>(), nrows, total, m,
                          dtype, flags, 0.0, 0.0, stream),
            "isotonic_ragged");
    };
    if (nmax > 0 && total > 0 && nrows > 0) fit_short(nmax);
    check_hip(hipEventSynchronize(rh.ready), "hipEventSynchronize");
    const int64_t err = rh.words[0], short_max = rh.words[1], n_long = rh.words[2];
    TORCH_CHECK_VALUE((err & 4) == 0, from_lengths ? "lengths must be non-negative" : "offsets must not decrease");
    TORCH_CHECK_VALUE((err & 3) == 0, "offsets must run from 0 to values.numel() = ", total);
    if (short_max > nmax) fit_short(short_max);
    // the longer rows, a length bucket at a time
    const bool want = values.requires_grad() || (w.defined() && w.requires_grad());
    // float32 sets under 2 GB: each bucket fitted in place (ti_fwd_rows), else through a block
    const bool rows_mode = dtype == TI_F32 && total * 4 < kRowMapBytes;
    std::vector<int64_t> buckets;  // per bucket: its first descriptor, its rows, its block length
    std::vector<at::Tensor> keep;  // the descriptors, then per bucket: y, w blocks, starts, workspace
    if (n_long > 0) {
      buckets = ragged_buckets(rh.words, n_long);
      if (!keyed) {  // (max_len was wrong: the keys now)
        keys = at::empty({nrows}, offsets.options().dtype(at::kByte));
        check(ti_ragged_plan(offsets.data_ptr<int64_t>(), nrows, total,
                             at::zeros({TI_RAGGED_PLAN_WORDS}, offsets.options()).data_ptr<int64_t>(),
                             keys.data_ptr<uint8_t>(), stream),
              "isotonic_ragged");
      }
      // the longer rows in bucket order (the short rows, key 0, sort first)
      const at::Tensor order = std::get<1>(at::sort(keys, /*stable=*/true, 0, false)).slice(0, nrows - n_long);
      const at::Tensor rows = at::empty({n_long, 2}, offsets.options());
      check(ti_ragged_rows(offsets.data_ptr<int64_t>(), nrows, order.data_ptr<int64_t>(), n_long,
                           rows.data_ptr<int64_t>(), stream),
            "isotonic_ragged");
      keep.push_back(rows);
      const int64_t* rp = rows.data_ptr<int64_t>();
      // float32: every row padded with the largest finite value (no extreme needed)
      const bool f32 = dtype == TI_F32;
      const at::Tensor ext = f32 ? at::Tensor() : at::zeros({n_long}, offsets.options());
      uint64_t* kp = f32 ? nullptr : reinterpret_cast<uint64_t*>(ext.data_ptr<int64_t>());
      const double cpad = f32 ? (increasing ? 1.0 : -1.0) * static_cast<double>(std::numeric_limits<float>::max()) : 0.0;
      for (size_t i = 0; i < buckets.size(); i += 3) {
        const int64_t f = buckets[i], k = buckets[i + 1], L = buckets[i + 2];
        at::Tensor starts = at::empty({ti_starts_words(k, L)}, values.options().dtype(at::kInt));
        at::Tensor ws = workspace(true, k, L, dtype, w.defined(), values.device());
        if (rows_mode) {  // read and written in place: no block
          check(ti_fwd_rows(ptr(values), ptr(w), ptr(out), static_cast<uint32_t*>(starts.data_ptr()), bad, rp + 2 * f,
                            k, L, total, cpad, dtype, flags, 0.0, 0.0, ptr(ws),
                            ws.defined() ? static_cast<size_t>(ws.numel()) : 0, stream),
                "isotonic_ragged");
          if (want) keep.insert(keep.end(), {at::Tensor(), at::Tensor(), starts, ws});
          continue;
        }
        if (!f32) {
          check(ti_ragged_extreme(ptr(values), total, rp + 2 * f, k, L, dtype, increasing ? 1 : 0, kp + f, stream),
                "isotonic_ragged");
        }
        at::Tensor yb = at::empty({k, L}, values.options());
        at::Tensor wb = w.defined() ? at::empty({k, L}, values.options()) : at::Tensor();
        check(ti_ragged_pack(ptr(values), ptr(w), total, rp + 2 * f, f32 ? nullptr : kp + f, cpad, k, L, dtype,
                             increasing ? 1 : 0, ptr(yb), ptr(wb), stream),
              "isotonic_ragged");
        at::Tensor ob = at::empty({k, L}, values.options());
        check(ti_fwd(ptr(yb), ptr(wb), ptr(ob), static_cast<uint32_t*>(starts.data_ptr()), bad, k, L, dtype, flags, 0.0,
                     0.0, ptr(ws), ws.defined() ? static_cast<size_t>(ws.numel()) : 0, stream),
              "isotonic_ragged");
        check(ti_ragged_unpack(ptr(ob), nullptr, rp + 2 * f, k, L, dtype, ptr(out), nullptr, total, nullptr, nullptr,
                               stream),
              "isotonic_ragged");
        if (want) {
          keep.push_back(yb);
          keep.push_back(wb);
          keep.push_back(starts);
          keep.push_back(ws);
        }
      }
    }
    if (bad != nullptr && (short_max > 0 || n_long > 0)) {
      TORCH_CHECK_VALUE(zeros.slice(0, kBadAt, kBadAt + 1).item<int32_t>() == 0, "weight must be strictly positive");
    }
    if (want) {
      std::vector<at::Tensor> saved = {values, w, offsets, zeros};
      saved.insert(saved.end(), keep.begin(), keep.end());
      ctx->save_for_backward(saved);
      ctx->saved_data["buckets"] = c10::List<int64_t>(buckets);
      ctx->saved_data["p"] =
          c10::List<int64_t>({short_max, increasing ? 1 : 0, w.defined() ? 1 : 0, rows_mode ? 1 : 0});
    }
    return out;
  }

  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    const c10::List<int64_t> prm = ctx->saved_data["p"].toIntList();
    const int64_t short_max = prm.get(0);
    const unsigned flags = (prm.get(1) != 0 ? TI_INCREASING : 0u) | TI_EXACT;
    const bool has_w = prm.get(2) != 0;
    const bool rows_mode = prm.get(3) != 0;
    const c10::List<int64_t> buckets = ctx->saved_data["buckets"].toIntList();
    const bool want_y = ctx->needs_input_grad(0), want_w = has_w && ctx->needs_input_grad(1);
    variable_list none(6);
    if (!want_y && !want_w) return none;
    const variable_list saved = ctx->get_saved_variables();
    const at::Tensor& values = saved[0];
    const at::Tensor& w = saved[1];
    const at::Tensor& offsets = saved[2];
    const at::Tensor& zeros = saved[3];
    const at::Tensor g = grads[0].contiguous().to(values.scalar_type());
    const int dtype = dtype_code(values);
    const int64_t nrows = offsets.numel() - 1, total = values.numel();
    const c10::DeviceGuard guard(values.device());
    const hipStream_t stream = c10::hip::getCurrentHIPStream(values.device().index()).stream();
    // (every element belongs to a row: the short rows' elements are written by one launch, the
    // longer rows' by their own backward)
    at::Tensor gy = at::empty_like(g);
    at::Tensor gw = want_w ? at::empty_like(g) : at::Tensor();
    const uint32_t* bits = reinterpret_cast<const uint32_t*>(zeros.data_ptr<int32_t>() + kBitsAt);
    if (short_max > 0) {
      check(ti_bwd_ragged(bits, ptr(g), ptr(w), want_w ? ptr(values) : nullptr, ptr(gy), ptr(gw),
                          offsets.data_ptr<int64_t>(), nrows, total, short_max, dtype, 0u, 0.0, 0.0, stream),
            "isotonic_ragged backward");
    }
    if (!buckets.empty()) {
      // per bucket: g gathered into the bucket's block (0 past each row), the block's backward
      // from its forward, and the gradients scattered back (a row whose pad joined its last block
      // has that block's gradients scaled back to its own weight)
      const int64_t* rp = saved[4].data_ptr<int64_t>();
      for (size_t i = 0, j = 5; i < buckets.size(); i += 3, j += 4) {
        const int64_t f = buckets.get(i), k = buckets.get(i + 1), L = buckets.get(i + 2);
        const at::Tensor& yb = saved[j];
        const at::Tensor& wb = saved[j + 1];
        const at::Tensor& starts = saved[j + 2];
        const at::Tensor& ws = saved[j + 3];
        at::Tensor bws = workspace(false, k, L, dtype, w.defined(), values.device());
        if (rows_mode) {  // in place, the correction included
          check(ti_bwd_rows(static_cast<const uint32_t*>(starts.data_ptr()), ptr(ws),
                            ws.defined() ? static_cast<size_t>(ws.numel()) : 0, ptr(g), ptr(w),
                            want_w ? ptr(values) : nullptr, ptr(gy), ptr(gw), rp + 2 * f, k, L, total, dtype, flags, 0.0,
                            0.0, ptr(bws), bws.defined() ? static_cast<size_t>(bws.numel()) : 0, stream),
                "isotonic_ragged backward");
          continue;
        }
        at::Tensor gb = at::empty({k, L}, g.options());
        check(ti_ragged_pack(ptr(g), nullptr, total, rp + 2 * f, nullptr, 0.0, k, L, dtype, 0, ptr(gb), nullptr,
                             stream),
              "isotonic_ragged backward");
        at::Tensor gyb = at::empty({k, L}, g.options());
        at::Tensor gwb = want_w ? at::empty({k, L}, g.options()) : at::Tensor();
        check(ti_bwd(static_cast<const uint32_t*>(starts.data_ptr()), ptr(ws),
                     ws.defined() ? static_cast<size_t>(ws.numel()) : 0, ptr(gb), ptr(wb), want_w ? ptr(yb) : nullptr,
                     ptr(gyb), ptr(gwb), k, L, dtype, flags, 0.0, 0.0, ptr(bws),
                     bws.defined() ? static_cast<size_t>(bws.numel()) : 0, stream),
              "isotonic_ragged backward");
        check(ti_ragged_unpack(ptr(gyb), ptr(gwb), rp + 2 * f, k, L, dtype, ptr(gy), ptr(gw), total,
                               static_cast<const uint32_t*>(starts.data_ptr()), ptr(w), stream),
              "isotonic_ragged backward");
      }
    }
    none[0] = want_y ? gy : at::Tensor();
    none[1] = gw;
    return none;
  }
};

at::Tensor isotonic_ragged_fit(const at::Tensor& values, const std::optional<at::Tensor>& w, const at::Tensor& offsets,
                               bool increasing, int64_t max_len, bool from_lengths) {
  return RaggedFn::apply(values, w, offsets, increasing, max_len, from_lengths);
}

}  // namespace

TORCH_LIBRARY(torchisotonic_amd, m) {
  m.def("isotonic_fit(Tensor y, Tensor? w, bool increasing, float? y_min, float? y_max) -> Tensor", &isotonic_fit);
  m.def("isotonic_ragged_fit(Tensor values, Tensor? w, Tensor offsets, bool increasing, int max_len, "
        "bool from_lengths) -> Tensor",
        &isotonic_ragged_fit);
}
