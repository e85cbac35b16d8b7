// HipBackend::execute: the hip device's implementation of the reference
// backend contract (reference backends/cuda/cuda_backend.cpp:290-627 is the
// slot it fills; semantics follow the CPU reference, cpu_backend.cpp).

#include "tensorcx/backends/hip/hip_backend.h"
#include "tensorcx/backends/hip/hip_device_interval.h"

#include "tensorcx/core/predicate.h"
#include "tensorcx/core/profiling.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <mutex>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace tensorcx::hip {
namespace {

// Thrown for a missing or unusable device; mapped to kUnavailable.
struct Unavailable : std::runtime_error {
  using std::runtime_error::runtime_error;
};

void ok_or_throw(int code, const char* what) {
  if (code == TCX_OK) return;
  const std::string message = std::string(what) + ": " + tcx_hip_last_error();
  if (code == TCX_INVALID_ARGUMENT) throw std::invalid_argument(message);
  if (code == TCX_UNAVAILABLE) throw Unavailable(message);
  throw std::runtime_error(message);
}

Status status_from_code(int code, const std::string& what) {
  if (code == TCX_OK) return Status::Ok();
  const std::string message = what + ": " + tcx_hip_last_error();
  if (code == TCX_INVALID_ARGUMENT) return Status(StatusCode::kInvalidArgument, message);
  if (code == TCX_UNAVAILABLE) return Status(StatusCode::kUnavailable, message);
  return Status(StatusCode::kInternal, message);
}

tcx_stream_t stream() {
  tcx_stream_t s = nullptr;
  ok_or_throw(tcx_hip_stream(&s), "HIP stream");
  return s;
}

// The thread's stream, fetched at its first use: an execution validates its
// whole request (metadata, axes, shapes, dtypes) before it touches the
// device, so a malformed request is kInvalidArgument even where no device is
// present.
class Stream {
 public:
  operator tcx_stream_t() {  // NOLINT(google-explicit-constructor): used where a launcher takes one
    if (stream_ == nullptr) stream_ = stream();
    return stream_;
  }
  bool used() const { return stream_ != nullptr; }

 private:
  tcx_stream_t stream_{nullptr};
};

// Bytes of a contiguous tensor, rejecting sizes past size_t.
std::size_t byte_size(const Shape& shape, DType dtype) {
  const auto count = static_cast<std::size_t>(numel(shape));
  if (count > std::numeric_limits<std::size_t>::max() / dtype_size(dtype))
    throw std::invalid_argument("tensor byte size overflow");
  return count * dtype_size(dtype);
}

void synchronize(tcx_stream_t s) {
  ProfileScope span(ProfileCategory::kSynchronize, "stream_synchronize", "hip");
  ok_or_throw(tcx_hip_stream_synchronize(s), "HIP execution");
}

int tcx_dtype(DType dtype) {
  if (dtype == DType::kFloat32) return TCX_FLOAT32;
  if (dtype == DType::kInt32) return TCX_INT32;
  throw std::invalid_argument("HIP tensors support float32 and int32");
}

// Validates hip tensor metadata (the from_core_tensor checks of
// cuda_backend.cpp) and returns its device pointer.
void* device_ptr(const Tensor& t) {
  if (t.device.type != "hip") throw std::invalid_argument("HIP operations require HIP tensors");
  if (t.device.index != 0) throw std::invalid_argument("HIP tensor metadata requires device index 0");
  if (t.offset != 0) throw std::invalid_argument("HIP tensor metadata with non-zero offset is unsupported");
  if (t.strides != contiguous_strides(t.shape)) throw std::invalid_argument("HIP tensor metadata must be contiguous");
  const auto* buffer = dynamic_cast<const HipBuffer*>(t.buffer.get());
  if (buffer == nullptr) throw std::invalid_argument("HIP tensor metadata requires a HIP buffer");
  const auto bytes = byte_size(t.shape, t.dtype);
  if (buffer->nbytes() < bytes) throw std::invalid_argument("HIP tensor buffer is smaller than its shape");
  return buffer->data();
}

const float* f32(const Tensor& t) {
  if (t.dtype != DType::kFloat32) throw std::invalid_argument("operation requires float32 tensors");
  return static_cast<const float*>(device_ptr(t));
}

Tensor make_tensor(DType dtype, Shape shape) {
  auto created = empty(std::move(shape), dtype);
  if (!created) {
    const Status& s = created.status();
    if (s.code() == StatusCode::kUnavailable) throw Unavailable(s.message());
    if (s.code() == StatusCode::kInvalidArgument) throw std::invalid_argument(s.message());
    throw std::runtime_error(s.message());
  }
  return created.move_value();
}

// Fused kernels load 16 bytes at a time; borrowed storage may sit at any
// element-aligned address, and then takes the unfused route.
bool aligned16(const void* p) { return (reinterpret_cast<std::uintptr_t>(p) & 15U) == 0; }

void* out_ptr(const Tensor& t) { return static_cast<HipBuffer*>(t.buffer.get())->data(); }

// ------------------------------------------------------------ broadcast metadata
// A broadcast over `shape` with per-operand strides, compressed for the
// kernels' metadata (at most `max_rank` axes): size-1 axes are dropped and
// neighbouring axes that every operand walks contiguously are merged. The
// last `keep` axes stay as they are (the attention softmax reads its last
// two).
struct Strided {
  Shape shape;
  std::vector<Shape> strides;
};

Strided compress(const Shape& shape, const std::vector<Shape>& strides, std::size_t keep = 0,
                 std::size_t max_rank = TCX_HIP_MAX_RANK) {
  Strided out;
  out.strides.resize(strides.size());
  const std::size_t rank = shape.size();
  std::size_t merged_ok = 0;  // leading entries of out that may still absorb a neighbour
  for (std::size_t a = 0; a < rank; ++a) {
    const bool tail = a + keep >= rank;
    if (!tail && shape[a] == 1) continue;
    bool merge = !tail && merged_ok == out.shape.size() && !out.shape.empty();
    for (std::size_t o = 0; merge && o < strides.size(); ++o)
      merge = out.strides[o].back() == strides[o][a] * shape[a];
    if (merge) {
      out.shape.back() *= shape[a];
      for (std::size_t o = 0; o < strides.size(); ++o) out.strides[o].back() = strides[o][a];
      continue;
    }
    out.shape.push_back(shape[a]);
    for (std::size_t o = 0; o < strides.size(); ++o) out.strides[o].push_back(strides[o][a]);
    if (!tail) merged_ok = out.shape.size();
  }
  if (out.shape.size() > max_rank)
    throw std::invalid_argument("HIP broadcast metadata exceeds rank " + std::to_string(max_rank));
  return out;
}

Shape broadcast_strides(const Shape& from, const Shape& to) { return make_broadcast_plan(from, to).lhs_strides; }

// ------------------------------------------------------------ reductions
struct RowDims {
  Shape output_shape;
  Dim outer, reduce, inner;
};

Dim normalize_axis(Dim axis, std::size_t rank) {
  if (rank == 0) {
    if (axis == 0 || axis == -1) return 0;
    throw std::invalid_argument("reduction axis is out of range");
  }
  const Dim r = static_cast<Dim>(rank);
  if (axis < 0) axis += r;
  if (axis < 0 || axis >= r) throw std::invalid_argument("reduction axis is out of range");
  return axis;
}

// (outer, reduce, inner) of a single-axis op (cpu_backend.cpp:93-123).
RowDims row_dims(const Shape& shape, Dim axis) {
  const Dim a = normalize_axis(axis, shape.size());
  if (shape.empty()) return {{}, 1, 1, 1};
  RowDims d{{}, 1, shape[static_cast<std::size_t>(a)], contiguous_strides(shape)[static_cast<std::size_t>(a)]};
  for (std::size_t i = 0; i < shape.size(); ++i) {
    if (static_cast<Dim>(i) < a) d.outer *= shape[i];
    if (static_cast<Dim>(i) != a) d.output_shape.push_back(shape[i]);
  }
  return d;
}

int reduce_code(OpKind kind) {
  switch (kind) {
    case OpKind::kSum: return TCX_REDUCE_SUM;
    case OpKind::kMax: return TCX_REDUCE_MAX;
    case OpKind::kMean: return TCX_REDUCE_MEAN;
    case OpKind::kMin: return TCX_REDUCE_MIN;
    case OpKind::kArgmax: return TCX_REDUCE_ARGMAX;
    default: throw std::invalid_argument("unsupported reduction");
  }
}

// One GEMM through tcx_hip_gemm_f32_ws: shapes that run faster with K split
// over several blocks get their workspace from the thread's pool (without it,
// when that allocation fails, the GEMM runs unsplit), held until the stream
// has run the call.
void run_gemm(const float* lhs, const float* rhs, float* out, const tcx_hip_gemm_desc_t& d, Stream& s,
              const char* what) {
  const std::size_t ws = tcx_hip_gemm_workspace_bytes(&d);
  std::shared_ptr<HipBuffer> workspace;
  if (ws) {
    auto created = HipBuffer::create(ws);
    if (created) workspace = created.move_value();
  }
  ok_or_throw(tcx_hip_gemm_f32_ws(lhs, rhs, out, &d, workspace ? workspace->data() : nullptr, workspace ? ws : 0, s),
              what);
  if (workspace) ok_or_throw(tcx_hip_stream_synchronize(s), what);
}

// Guards tcx_hip_reduce_noalloc's scratch, one per device: a call holds it
// from launch until its stream has finished. Only one call at a time uses it;
// a call that finds it taken runs on a workspace of its own instead of
// waiting, so concurrent segmented reductions never queue behind each other.
std::mutex reduce_scratch_mutex;

void run_rows(int code, const Tensor& x, const Tensor& out, Dim outer, Dim reduce, Dim inner, Stream& s) {
  const int dtype = tcx_dtype(x.dtype);
  const std::size_t ws = tcx_hip_reduce_workspace_bytes(code, dtype, outer, reduce, inner);
  if (ws != 0 && ws <= TCX_HIP_REDUCE_NOALLOC_MAX_WORKSPACE) {
    // Segmented rows (a full-tensor sum, few long rows): the partials go to
    // the library's static scratch when it is free, so no workspace is
    // allocated per call.
    std::unique_lock lock(reduce_scratch_mutex, std::try_to_lock);
    if (lock.owns_lock()) {
      ok_or_throw(tcx_hip_reduce_noalloc(code, dtype, device_ptr(x), out_ptr(out), outer, reduce, inner, s),
                  "HIP reduction");
      ok_or_throw(tcx_hip_stream_synchronize(s), "HIP reduction");
      return;
    }
  }
  std::shared_ptr<HipBuffer> workspace;
  if (ws) {
    auto created = HipBuffer::create(ws);
    if (!created) throw std::runtime_error(created.status().message());
    workspace = created.move_value();
  }
  ok_or_throw(tcx_hip_reduce(code, dtype, device_ptr(x), out_ptr(out), outer, reduce, inner,
                             workspace ? workspace->data() : nullptr, ws, s),
              "HIP reduction");
  if (workspace) ok_or_throw(tcx_hip_stream_synchronize(s), "HIP reduction");
}

// An axis selection over a contiguous shape, folded: size-1 axes are dropped
// (they move no offset) and neighbouring axes that are both reduced or both
// kept are merged (row-major order over two adjacent axes is row-major order
// over their product). The reference's element order, kept axes row-major
// and reduced axes row-major in axis order (make_reduction_plan,
// shape.cpp:140-173; cpu_backend.cpp:1102-1153), is the same before and after,
// and so is every argmax index.
struct FoldedAxes {
  Shape extent;
  std::vector<bool> reduced;
};

FoldedAxes fold_axes(const Shape& shape, const std::vector<bool>& selected) {
  FoldedAxes f;
  for (std::size_t i = 0; i < shape.size(); ++i) {
    if (shape[i] == 1) continue;
    if (!f.extent.empty() && f.reduced.back() == selected[i]) {
      f.extent.back() *= shape[i];  // bounded by numel(shape)
    } else {
      f.extent.push_back(shape[i]);
      f.reduced.push_back(selected[i]);
    }
  }
  return f;
}

// Reduction over an axis selection into a non-empty output. After folding, a
// selection that is one run of axes is an (outer, reduce, inner) reduction
// with the same element order; any other runs the general metadata kernel
// over the folded axes, kept first.
// Selections of several reduced runs with at most this many elements per
// output run the metadata kernel: one lane per output, the reference's
// element order (bit-exact sums), the same bound as a single run's exact
// order in the reduction kernels.
constexpr Dim kExactSelectionMax = 64;

// Selections of several reduced runs (after folding) with more elements per
// output. sum / mean / max / min fold one reduced run at a time, innermost
// first, through the (outer, reduce, inner) kernels, so every pass streams
// its input with the row or column kernels and the first pass, over the whole
// tensor, leaves a tensor R times smaller; max / min and int32 sums are exact
// in any order, float32 sums take this fixed order (the reductions' sum bar),
// and mean divides the sum once by float(count), as the reference
// (cpu_backend.cpp:1102-1153). argmax, whose index runs over the selected
// axes in row-major order, gathers them innermost ([kept..., reduced...],
// one strided copy of at most TCX_HIP_MAX_RANK folded axes) and takes one row
// argmax per output. Returns false, having launched nothing, for an argmax
// over more folded axes than the gather takes.
bool reduce_runs(int code, const Tensor& x, const Tensor& out, const FoldedAxes& f, Dim count, Stream& s) {
  std::vector<Tensor> held;  // intermediates, alive until the stream has run
  if (code == TCX_REDUCE_ARGMAX) {
    if (f.extent.size() > TCX_HIP_MAX_RANK) return false;
    const Shape strides = contiguous_strides(f.extent);
    Shape shape, in_strides;
    for (int pass = 0; pass < 2; ++pass)
      for (std::size_t i = 0; i < f.extent.size(); ++i)
        if (f.reduced[i] == (pass == 1)) {
          shape.push_back(f.extent[i]);
          in_strides.push_back(strides[i]);
        }
    Tensor gathered = make_tensor(x.dtype, Shape{numel(f.extent)});
    ok_or_throw(tcx_hip_gather_strided(static_cast<int>(dtype_size(x.dtype)), device_ptr(x), out_ptr(gathered),
                                       static_cast<int32_t>(shape.size()), shape.data(), in_strides.data(), 0, s),
                "HIP reduction gather");
    run_rows(code, gathered, out, numel(f.extent) / count, count, 1, s);
    ok_or_throw(tcx_hip_stream_synchronize(s), "HIP reduction");
    return true;
  }
  const int pass_code = code == TCX_REDUCE_MEAN ? TCX_REDUCE_SUM : code;
  Shape extent = f.extent;
  std::vector<bool> reduced = f.reduced;
  Tensor cur = x;
  for (;;) {
    std::size_t k = extent.size();
    while (!reduced[k - 1]) --k;
    --k;  // the innermost reduced run
    Dim outer = 1, inner = 1;
    for (std::size_t i = 0; i < k; ++i) outer *= extent[i];
    for (std::size_t i = k + 1; i < extent.size(); ++i) inner *= extent[i];
    const bool last = std::count(reduced.begin(), reduced.end(), true) == 1;
    if (last) {
      run_rows(pass_code, cur, out, outer, extent[k], inner, s);
      break;
    }
    Tensor next = make_tensor(x.dtype, Shape{outer * inner});
    run_rows(pass_code, cur, next, outer, extent[k], inner, s);
    held.push_back(next);
    cur = next;
    // Drop the run; its kept neighbours merge.
    extent.erase(extent.begin() + static_cast<std::ptrdiff_t>(k));
    reduced.erase(reduced.begin() + static_cast<std::ptrdiff_t>(k));
    if (k > 0 && k < extent.size() && !reduced[k - 1] && !reduced[k]) {
      extent[k - 1] *= extent[k];
      extent.erase(extent.begin() + static_cast<std::ptrdiff_t>(k));
      reduced.erase(reduced.begin() + static_cast<std::ptrdiff_t>(k));
    }
  }
  if (code == TCX_REDUCE_MEAN)
    ok_or_throw(tcx_hip_scalar_op(TCX_SCALAR_DIVIDE, TCX_FLOAT32, out_ptr(out), out_ptr(out), numel(out.shape),
                                  static_cast<double>(count), 0, s),
                "HIP reduction mean");
  if (!held.empty()) ok_or_throw(tcx_hip_stream_synchronize(s), "HIP reduction");
  return true;
}

void run_selection(int code, const Tensor& x, const Tensor& out, const Shape& axes, const ReductionPlan& plan,
                   Stream& s) {
  const Dim groups = numel(plan.output_shape);
  if (plan.reduction_size == 0) {  // an empty selected axis: sum 0, mean NaN
    run_rows(code, x, out, groups, 0, 1, s);
    return;
  }
  const Dim rank = static_cast<Dim>(x.shape.size());
  std::vector<bool> selected(x.shape.size(), false);
  for (Dim a : axes) selected[static_cast<std::size_t>(a < 0 ? a + rank : a)] = true;
  const FoldedAxes f = fold_axes(x.shape, selected);
  const auto runs = std::count(f.reduced.begin(), f.reduced.end(), true);
  if (runs <= 1) {
    Dim outer = 1, reduce = 1, inner = 1;
    bool seen = false;
    for (std::size_t i = 0; i < f.extent.size(); ++i) {
      if (f.reduced[i]) {
        reduce = f.extent[i];
        seen = true;
      } else if (seen) {
        inner *= f.extent[i];
      } else {
        outer *= f.extent[i];
      }
    }
    run_rows(code, x, out, outer, reduce, inner, s);
    return;
  }
  if (plan.reduction_size > kExactSelectionMax && reduce_runs(code, x, out, f, plan.reduction_size, s)) return;
  // Every folded axis has extent >= 2, so a folded rank above the kernel's
  // metadata capacity would need more than 2^40 elements.
  if (f.extent.size() > TCX_HIP_MAX_FOLDED_RANK)
    throw std::invalid_argument("HIP reduction metadata exceeds the folded rank limit");
  const Shape strides = contiguous_strides(f.extent);
  std::vector<std::int64_t> meta;
  int32_t kept = 0;
  for (int pass = 0; pass < 2; ++pass)
    for (std::size_t i = 0; i < f.extent.size(); ++i)
      if (f.reduced[i] == (pass == 1)) {
        meta.push_back(f.extent[i]);
        meta.push_back(strides[i]);
        kept += pass == 0;
      }
  ok_or_throw(tcx_hip_reduce_axes(code, tcx_dtype(x.dtype), device_ptr(x), out_ptr(out), meta.data(), kept,
                                  static_cast<int32_t>(f.extent.size()), groups, plan.reduction_size, s),
              "HIP reduction");
}

Tensor reduce(const OpDesc& op, const Tensor& x, Stream& s) {
  if (x.dtype == DType::kBool) throw std::invalid_argument("numeric reductions do not support bool tensors");
  (void)device_ptr(x);
  const int code = reduce_code(op.kind);
  if (op.reduction_axes) {
    const auto plan = make_reduction_plan(x.shape, *op.reduction_axes);
    if (op.kind == OpKind::kMean && x.dtype != DType::kFloat32)
      throw std::invalid_argument("mean only supports float32 tensors");
    if (op.kind == OpKind::kMax && plan.reduction_size == 0)
      throw std::invalid_argument("max reduction requires non-empty axes");
    if (op.reduction_axes->empty()) {
      auto copy = clone(x);
      if (!copy) throw std::runtime_error(copy.status().message());
      return copy.move_value();
    }
    Tensor out = make_tensor(x.dtype, plan.output_shape);
    if (numel(plan.output_shape) != 0) run_selection(code, x, out, *op.reduction_axes, plan, s);
    return out;
  }
  const RowDims d = row_dims(x.shape, op.axis);
  if (op.kind == OpKind::kMax && d.reduce == 0) throw std::invalid_argument("max reduction requires a non-empty axis");
  if (op.kind == OpKind::kMean && x.dtype != DType::kFloat32)
    throw std::invalid_argument("mean only supports float32 tensors");
  Tensor out = make_tensor(x.dtype, d.output_shape);
  if (numel(d.output_shape) != 0) run_rows(code, x, out, d.outer, d.reduce, d.inner, s);
  return out;
}

// min / argmax with the reference math plan (core/math.cpp:39-56).
Tensor argext(const OpDesc& op, const Tensor& x, Stream& s) {
  if (x.dtype != DType::kFloat32 && x.dtype != DType::kInt32)
    throw std::invalid_argument("math operations require float32 or int32 tensors");
  (void)device_ptr(x);
  const Shape axes = op.reduction_axes.value_or(x.shape.empty() ? Shape{} : Shape{op.axis});
  if (x.shape.empty() && !op.reduction_axes && op.axis != 0 && op.axis != -1)
    throw std::invalid_argument("reduction axis out of range");
  const auto plan = make_reduction_plan(x.shape, axes);
  if (plan.reduction_size == 0) throw std::invalid_argument("min/argmax require a non-empty reduction");
  DType out_dtype = x.dtype;
  if (op.kind == OpKind::kArgmax) {
    Dim extent = 1;
    for (Dim a : axes) {
      if (a < 0) a += static_cast<Dim>(x.shape.size());
      const Dim e = x.shape[static_cast<std::size_t>(a)];
      if (e > std::numeric_limits<std::int32_t>::max() / extent)
        throw std::invalid_argument("argmax index range exceeds int32");
      extent *= e;
    }
    out_dtype = DType::kInt32;
  }
  Tensor out = make_tensor(out_dtype, plan.output_shape);
  if (numel(plan.output_shape) == 0) return out;
  const int code = reduce_code(op.kind);
  if (axes.empty()) {
    // No reduced axes: every element is its own group of one.
    ok_or_throw(tcx_hip_reduce(code, tcx_dtype(x.dtype), device_ptr(x), out_ptr(out), numel(x.shape), 1, 1,
                               nullptr, 0, s),
                "HIP reduction");
    return out;
  }
  run_selection(code, x, out, axes, plan, s);
  return out;
}

// ------------------------------------------------------------ row ops
float checked_epsilon(double eps) {
  const float rounded = static_cast<float>(eps);
  if (!std::isfinite(eps) || eps < 0.0 || eps > static_cast<double>(std::numeric_limits<float>::max()) ||
      (eps > 0.0 && rounded == 0.0F))
    throw std::invalid_argument("epsilon must be finite and non-negative and representable as float32");
  return rounded;
}

Tensor row_op(const OpDesc& op, const Tensor& x, const Tensor* gamma, const Tensor* beta, Stream& s) {
  const RowDims d = row_dims(x.shape, op.axis);
  const char* name = op.kind == OpKind::kSoftmax ? "softmax" : op.kind == OpKind::kRmsNorm ? "rmsnorm" : "layernorm";
  float eps = 0.F;
  if (op.kind != OpKind::kSoftmax) eps = checked_epsilon(op.epsilon);
  if (x.dtype != DType::kFloat32) throw std::invalid_argument(std::string(name) + " only supports float32 tensors");
  const float* xp = f32(x);
  const float* g = gamma ? f32(*gamma) : nullptr;
  const float* b = beta ? f32(*beta) : nullptr;
  Tensor out = make_tensor(DType::kFloat32, x.shape);
  if (numel(x.shape) == 0) return out;
  auto* o = static_cast<float*>(out_ptr(out));
  // Strided rows with few columns split their rows over blocks, with the
  // split statistics in a workspace held until the stream has finished.
  const std::size_t ws = tcx_hip_rownorm_workspace_bytes(d.outer, d.reduce, d.inner);
  std::shared_ptr<HipBuffer> workspace;
  if (ws) {
    auto created = HipBuffer::create(ws);
    if (!created) throw std::runtime_error(created.status().message());
    workspace = created.move_value();
  }
  void* wp = workspace ? workspace->data() : nullptr;
  int rc = TCX_OK;
  if (op.kind == OpKind::kSoftmax)
    rc = tcx_hip_softmax_f32_ws(xp, o, d.outer, d.reduce, d.inner, wp, ws, s);
  else if (op.kind == OpKind::kRmsNorm)
    rc = tcx_hip_rmsnorm_f32_ws(xp, g, o, d.outer, d.reduce, d.inner, eps, wp, ws, s);
  else
    rc = tcx_hip_layernorm_f32_ws(xp, g, b, o, d.outer, d.reduce, d.inner, eps, wp, ws, s);
  ok_or_throw(rc, name);
  if (workspace) ok_or_throw(tcx_hip_stream_synchronize(s), name);
  return out;
}

// kAffineRmsNorm / kAffineLayerNorm with the validation of
// core/inference.cpp:103-122, computed in one fused pass.
Tensor affine_norm(const OpDesc& op, std::span<const Tensor> inputs, Stream& s) {
  const bool rms = op.kind == OpKind::kAffineRmsNorm;
  if (inputs.size() != 1U + op.has_weight + op.has_bias || (rms && op.has_bias))
    throw std::invalid_argument("invalid affine normalization parameters");
  for (const Tensor& t : inputs) {
    if (t.dtype != DType::kFloat32) throw std::invalid_argument("inference values require float32 tensors");
    (void)device_ptr(t);
  }
  const Tensor& x = inputs[0];
  Dim axis = op.axis;
  if (x.shape.empty()) {
    if (axis != 0 && axis != -1) throw std::invalid_argument("normalization axis out of range");
    axis = 0;
  } else {
    if (axis < 0) axis += static_cast<Dim>(x.shape.size());
    if (axis < 0 || axis >= static_cast<Dim>(x.shape.size()))
      throw std::invalid_argument("normalization axis out of range");
  }
  const Shape expected = x.shape.empty() ? Shape{} : Shape{x.shape[static_cast<std::size_t>(axis)]};
  for (std::size_t i = 1; i < inputs.size(); ++i)
    if (inputs[i].shape != expected) throw std::invalid_argument("affine parameters must match the normalized axis");
  const float narrowed = static_cast<float>(op.epsilon);
  if (!std::isfinite(op.epsilon) || !std::isfinite(narrowed) || op.epsilon < 0 || (op.epsilon > 0 && narrowed == 0))
    throw std::invalid_argument("epsilon must be finite, non-negative and representable as float32");
  OpDesc base{rms ? OpKind::kRmsNorm : OpKind::kLayerNorm, op.axis, op.epsilon};
  const Tensor* gamma = op.has_weight ? &inputs[1] : nullptr;
  const Tensor* beta = op.has_bias ? &inputs[op.has_weight ? 2 : 1] : nullptr;
  return row_op(base, x, gamma, beta, s);
}

// ------------------------------------------------------------ matmul / linear
Tensor matmul(const Tensor& lhs, const Tensor& rhs, Stream& s) {
  if (lhs.dtype != DType::kFloat32 || rhs.dtype != DType::kFloat32)
    throw std::invalid_argument("matmul only supports float32 tensors");
  const float* a = f32(lhs);
  const float* b = f32(rhs);
  const MatmulPlan plan = make_matmul_plan(lhs.shape, rhs.shape);
  Tensor out = make_tensor(DType::kFloat32, plan.output_shape);
  if (numel(plan.output_shape) == 0) return out;
  // Batch axes folded: size-1 axes move no offset, and neighbouring axes that
  // both operands walk contiguously (or both broadcast) are one axis. The
  // batch index order, and so the output layout, is unchanged.
  const Strided batch =
      compress(plan.batch_shape, {plan.lhs_batch_strides, plan.rhs_batch_strides}, 0, TCX_HIP_MAX_FOLDED_RANK);
  auto* c = static_cast<float*>(out_ptr(out));
  tcx_hip_gemm_desc_t d{};
  d.m = plan.m;
  d.n = plan.n;
  d.k = plan.k;
  d.batch_count = 1;
  if (batch.shape.size() == 1 && batch.strides[1][0] == 0 && batch.strides[0][0] == plan.m * plan.k) {
    // Batches that only walk the lhs contiguously (rhs shared) are one taller
    // GEMM: rows of consecutive batches are adjacent in both lhs and out.
    d.m = plan.m * batch.shape[0];
    run_gemm(a, b, c, d, s, "HIP matmul");
    return out;
  }
  // The last TCX_HIP_MAX_BATCH_RANK folded axes go to the kernel; any axes in
  // front of them (alternating broadcast patterns only) are walked here, one
  // launch per index.
  const std::size_t rank = batch.shape.size();
  const std::size_t lead = rank > TCX_HIP_MAX_BATCH_RANK ? rank - TCX_HIP_MAX_BATCH_RANK : 0;
  d.batch_rank = static_cast<int32_t>(rank - lead);
  for (std::size_t i = lead; i < rank; ++i) {
    d.batch_shape[i - lead] = batch.shape[i];
    d.lhs_batch_strides[i - lead] = batch.strides[0][i];
    d.rhs_batch_strides[i - lead] = batch.strides[1][i];
    d.batch_count *= batch.shape[i];
  }
  const Dim launches = numel(Shape(batch.shape.begin(), batch.shape.begin() + static_cast<std::ptrdiff_t>(lead)));
  for (Dim index = 0; index < launches; ++index) {
    Dim rest = index, lhs_off = 0, rhs_off = 0;
    for (std::size_t i = lead; i-- > 0;) {
      const Dim coord = rest % batch.shape[i];
      rest /= batch.shape[i];
      lhs_off += coord * batch.strides[0][i];
      rhs_off += coord * batch.strides[1][i];
    }
    run_gemm(a + lhs_off, b + rhs_off, c + index * d.batch_count * plan.m * plan.n, d, s, "HIP matmul");
  }
  return out;
}

// y = act(x @ weight^T + bias) for x (..., in) and weight (out, in), writing
// into `out` (contiguous (..., out)). One NT GEMM with the bias and activation
// in its epilogue: the kLinear composite of core/inference.cpp:89-102 without
// the transposed weight copy.
void linear_into(const Tensor& x, const Tensor& w, const Tensor* bias, int act, const Tensor& out, Stream& s) {
  tcx_hip_gemm_desc_t d{};
  d.k = w.shape[1];
  d.n = w.shape[0];
  d.m = numel(out.shape) / d.n;  // callers pass a non-empty output, so n > 0
  d.batch_count = 1;
  d.rhs_transposed = 1;
  d.bias = bias ? f32(*bias) : nullptr;
  d.activation = act;
  run_gemm(f32(x), f32(w), static_cast<float*>(out_ptr(out)), d, s, "HIP linear");
}

Shape linear_shape(std::span<const Tensor> inputs) {
  if (inputs.size() < 2 || inputs.size() > 3)
    throw std::invalid_argument("linear requires input, weight and optional bias");
  for (const Tensor& t : inputs) {
    if (t.dtype != DType::kFloat32) throw std::invalid_argument("inference values require float32 tensors");
    (void)device_ptr(t);
  }
  const Tensor& x = inputs[0];
  const Tensor& w = inputs[1];
  if (x.shape.empty() || w.shape.size() != 2 || x.shape.back() != w.shape[1])
    throw std::invalid_argument("linear requires (..., in_features) and (out_features, in_features)");
  if (inputs.size() == 3 && inputs[2].shape != Shape{w.shape[0]})
    throw std::invalid_argument("linear bias must have shape (out_features,)");
  Shape shape = x.shape;
  shape.back() = w.shape[0];
  (void)numel(shape);
  return shape;
}

Tensor linear(std::span<const Tensor> inputs, Stream& s) {
  const Shape shape = linear_shape(inputs);
  Tensor out = make_tensor(DType::kFloat32, shape);
  if (numel(shape) == 0) return out;
  linear_into(inputs[0], inputs[1], inputs.size() == 3 ? &inputs[2] : nullptr, TCX_ACT_NONE, out, s);
  return out;
}


// ------------------------------------------------------------ elementwise
Tensor unary(const OpDesc& op, const Tensor& x, Stream& s) {
  const int code = op.kind == OpKind::kExp ? TCX_UNARY_EXP : op.kind == OpKind::kGelu ? TCX_UNARY_GELU : TCX_UNARY_SILU;
  if (x.dtype != DType::kFloat32) {
    const char* name = code == TCX_UNARY_EXP ? "exp" : code == TCX_UNARY_GELU ? "gelu" : "silu";
    throw std::invalid_argument(std::string(name) + " only supports float32 tensors");
  }
  const float* xp = f32(x);
  Tensor out = make_tensor(DType::kFloat32, x.shape);
  ok_or_throw(tcx_hip_unary_f32(code, xp, static_cast<float*>(out_ptr(out)), numel(x.shape), s), "HIP unary");
  return out;
}

Tensor binary(const OpDesc& op, const Tensor& lhs, const Tensor& rhs, Stream& s) {
  if (lhs.dtype == DType::kBool || rhs.dtype == DType::kBool)
    throw std::invalid_argument("arithmetic does not support bool tensors");
  if (lhs.dtype != rhs.dtype) throw std::invalid_argument("dtype mismatch for binary operation");
  const int code = op.kind == OpKind::kAdd        ? TCX_BINARY_ADD
                   : op.kind == OpKind::kSubtract ? TCX_BINARY_SUBTRACT
                   : op.kind == OpKind::kMultiply ? TCX_BINARY_MULTIPLY
                                                  : TCX_BINARY_DIVIDE;
  if (code == TCX_BINARY_DIVIDE && lhs.dtype != DType::kFloat32)
    throw std::invalid_argument("division only supports float32 tensors");
  const void* l = device_ptr(lhs);
  const void* r = device_ptr(rhs);
  const BroadcastPlan plan = make_broadcast_plan(lhs.shape, rhs.shape);
  Tensor out = make_tensor(lhs.dtype, plan.output_shape);
  if (numel(plan.output_shape) == 0) return out;
  // Row-vector bias on float32 addition: the fused bias kernel, same rounding.
  const Shape& os = plan.output_shape;
  if (code == TCX_BINARY_ADD && lhs.dtype == DType::kFloat32 && lhs.shape == os && !os.empty() &&
      rhs.shape == Shape{os.back()}) {
    const Dim cols = os.back();
    ok_or_throw(tcx_hip_bias_act_f32(static_cast<const float*>(l), static_cast<const float*>(r),
                                     static_cast<float*>(out_ptr(out)), numel(os) / cols, cols, TCX_ACT_NONE, s),
                "HIP add");
    return out;
  }
  // Size-1 axes dropped and axes both operands walk contiguously merged: any
  // rank folds to at most one axis per change of broadcast pattern.
  const Strided m = compress(os, {plan.lhs_strides, plan.rhs_strides}, 0, TCX_HIP_MAX_FOLDED_RANK);
  ok_or_throw(tcx_hip_binary(code, tcx_dtype(lhs.dtype), l, r, out_ptr(out), static_cast<int32_t>(m.shape.size()),
                             m.shape.data(), m.strides[0].data(), m.strides[1].data(), s),
              "HIP arithmetic");
  return out;
}

Tensor fill(const Tensor& descriptor, double value, Stream& s) {
  if (descriptor.dtype == DType::kInt32 && !is_int32_representable(value))
    throw std::invalid_argument("fill value must be an integer in int32 range");
  const int dtype = descriptor.dtype == DType::kBool ? TCX_BOOL : tcx_dtype(descriptor.dtype);
  Tensor out = make_tensor(descriptor.dtype, descriptor.shape);
  ok_or_throw(tcx_hip_fill(dtype, out_ptr(out), numel(descriptor.shape), value, s), "HIP fill");
  return out;
}


// ------------------------------------------------------------ math extension
// log / sqrt / abs, clip and topk with the plans of core/math.cpp:13-71.
void require_math_dtype(const Tensor& t) {
  if (t.dtype != DType::kFloat32 && t.dtype != DType::kInt32)
    throw std::invalid_argument("math operations require float32 or int32 tensors");
}

Tensor math_unary(const OpDesc& op, const Tensor& x, Stream& s) {
  require_math_dtype(x);
  const int code = op.kind == OpKind::kLog ? TCX_MATH_LOG : op.kind == OpKind::kSqrt ? TCX_MATH_SQRT : TCX_MATH_ABS;
  if (code != TCX_MATH_ABS && x.dtype != DType::kFloat32)
    throw std::invalid_argument("log/sqrt only support float32 tensors");
  const void* xp = device_ptr(x);
  Tensor out = make_tensor(x.dtype, x.shape);
  ok_or_throw(tcx_hip_math_unary(code, tcx_dtype(x.dtype), xp, out_ptr(out), numel(x.shape), s), "HIP math");
  return out;
}

Tensor clip(std::span<const Tensor> inputs, Stream& s) {
  if (inputs.size() != 3) throw std::invalid_argument("invalid math operation or input count");
  for (const Tensor& t : inputs) {
    require_math_dtype(t);
    if (t.dtype != inputs[0].dtype) throw std::invalid_argument("math input dtypes must match");
    (void)device_ptr(t);
  }
  Shape shape = inputs[0].shape;
  for (const Tensor& t : inputs) shape = make_broadcast_plan(shape, t.shape).output_shape;
  Tensor out = make_tensor(inputs[0].dtype, shape);
  if (numel(shape) == 0) return out;
  const Strided m = compress(shape, {broadcast_strides(inputs[0].shape, shape), broadcast_strides(inputs[1].shape, shape),
                                     broadcast_strides(inputs[2].shape, shape)});
  ok_or_throw(tcx_hip_clip(tcx_dtype(inputs[0].dtype), device_ptr(inputs[0]), device_ptr(inputs[1]),
                           device_ptr(inputs[2]), out_ptr(out), static_cast<int32_t>(m.shape.size()), m.shape.data(),
                           m.strides[0].data(), m.strides[1].data(), m.strides[2].data(), s),
              "HIP clip");
  return out;
}

std::pair<Tensor, Tensor> topk(const OpDesc& op, const Tensor& x, Stream& s) {
  require_math_dtype(x);
  if (x.shape.empty()) throw std::invalid_argument("topk requires rank >= 1");
  Dim axis = op.axis;
  if (axis < 0) axis += static_cast<Dim>(x.shape.size());
  if (axis < 0 || axis >= static_cast<Dim>(x.shape.size())) throw std::invalid_argument("topk axis out of range");
  const Dim reduce = x.shape[static_cast<std::size_t>(axis)];
  if (reduce > std::numeric_limits<std::int32_t>::max()) throw std::invalid_argument("topk index range exceeds int32");
  if (op.k < 0 || op.k > reduce) throw std::invalid_argument("topk k must be between zero and the axis size");
  Shape shape = x.shape;
  shape[static_cast<std::size_t>(axis)] = op.k;
  (void)numel(shape);
  const void* xp = device_ptr(x);
  Tensor values = make_tensor(x.dtype, shape);
  Tensor indices = make_tensor(DType::kInt32, shape);
  if (numel(shape) == 0) return {std::move(values), std::move(indices)};
  Dim outer = 1, inner = 1;
  for (Dim a = 0; a < static_cast<Dim>(x.shape.size()); ++a) {
    if (a < axis) outer *= x.shape[static_cast<std::size_t>(a)];
    if (a > axis) inner *= x.shape[static_cast<std::size_t>(a)];
  }
  ok_or_throw(tcx_hip_topk(tcx_dtype(x.dtype), xp, out_ptr(values), static_cast<int32_t*>(out_ptr(indices)), outer,
                           reduce, inner, op.k, op.largest ? 1 : 0, op.sorted ? 1 : 0, s),
              "HIP topk");
  return {std::move(values), std::move(indices)};
}

// ------------------------------------------------------------ inference primitives
// kEmbedding with make_embedding_plan (core/inference.cpp:47-57).
Tensor embedding(std::span<const Tensor> inputs, Stream& s) {
  if (inputs.size() != 2) throw std::invalid_argument("embedding requires indices and weight");
  const Tensor& indices = inputs[0];
  const Tensor& weight = inputs[1];
  if (indices.dtype != DType::kInt32) throw std::invalid_argument("embedding indices must be int32");
  if (weight.dtype != DType::kFloat32) throw std::invalid_argument("inference values require float32 tensors");
  if (weight.shape.size() != 2) throw std::invalid_argument("embedding weight must have rank 2");
  Shape shape = indices.shape;
  shape.push_back(weight.shape[1]);
  (void)numel(shape);
  const auto* ip = static_cast<const int32_t*>(device_ptr(indices));
  const float* wp = f32(weight);
  Tensor out = make_tensor(DType::kFloat32, shape);
  const Dim count = numel(indices.shape);
  if (count == 0) return out;
  Tensor flag = make_tensor(DType::kInt32, Shape{1});
  ok_or_throw(tcx_hip_embedding_f32(ip, wp, static_cast<float*>(out_ptr(out)), count, weight.shape[0], weight.shape[1],
                                    static_cast<int32_t*>(out_ptr(flag)), s),
              "HIP embedding");
  return out;
}

float checked_scale(double scale) {
  const float narrowed = static_cast<float>(scale);
  if (!std::isfinite(scale) || !std::isfinite(narrowed) || (scale != 0 && narrowed == 0))
    throw std::invalid_argument("attention scale must be finite and representable as float32");
  return narrowed;
}

struct AttentionSoftmaxPlan {
  Shape shape;
  int mask_kind;
  float scale;
};

// make_attention_softmax_plan (core/inference.cpp:59-84).
AttentionSoftmaxPlan attention_softmax_plan(const OpDesc& op, std::span<const Tensor> inputs) {
  if (inputs.empty() || inputs.size() > 2)
    throw std::invalid_argument("attention softmax requires scores and optional mask");
  if (inputs[0].dtype != DType::kFloat32) throw std::invalid_argument("inference values require float32 tensors");
  (void)numel(inputs[0].shape);
  if (inputs[0].shape.size() < 2 || op.attention_shape.size() < 2)
    throw std::invalid_argument("attention scores must have rank >= 2");
  const Shape& shape = op.attention_shape;
  if (make_broadcast_plan(inputs[0].shape, shape).output_shape != shape)
    throw std::invalid_argument("attention scores cannot broadcast to target");
  int mask_kind = TCX_MASK_NONE;
  if (inputs.size() == 2) {
    const Tensor& mask = inputs[1];
    if (mask.dtype != DType::kBool && mask.dtype != DType::kFloat32)
      throw std::invalid_argument("attention mask must be bool or float32");
    if (make_broadcast_plan(mask.shape, shape).output_shape != shape)
      throw std::invalid_argument("attention mask cannot broadcast to scores");
    mask_kind = mask.dtype == DType::kBool ? TCX_MASK_BOOL : TCX_MASK_ADDITIVE;
  }
  (void)numel(shape);
  return {shape, mask_kind, checked_scale(op.attention_scale.value_or(1.0))};
}

void attention_softmax_into(const OpDesc& op, const AttentionSoftmaxPlan& plan, const Tensor& scores,
                            const Tensor* mask, const Tensor& out, Stream& s) {
  std::vector<Shape> strides{broadcast_strides(scores.shape, plan.shape)};
  strides.push_back(mask ? broadcast_strides(mask->shape, plan.shape) : Shape(plan.shape.size(), 0));
  const Strided m = compress(plan.shape, strides, 2);
  tcx_hip_attention_softmax_desc_t d{};
  d.rank = static_cast<int32_t>(m.shape.size());
  for (std::size_t i = 0; i < m.shape.size(); ++i) {
    d.shape[i] = m.shape[i];
    d.score_strides[i] = m.strides[0][i];
    d.mask_strides[i] = m.strides[1][i];
  }
  d.mask_kind = plan.mask_kind;
  d.causal = op.causal ? 1 : 0;
  d.scale = plan.scale;
  ok_or_throw(tcx_hip_attention_softmax_f32(f32(scores), mask ? device_ptr(*mask) : nullptr,
                                            static_cast<float*>(out_ptr(out)), &d, s),
              "HIP attention softmax");
}

Tensor attention_softmax(const OpDesc& op, std::span<const Tensor> inputs, Stream& s) {
  const AttentionSoftmaxPlan plan = attention_softmax_plan(op, inputs);
  for (const Tensor& t : inputs) (void)device_ptr(t);
  Tensor out = make_tensor(DType::kFloat32, plan.shape);
  if (numel(plan.shape) == 0) return out;
  attention_softmax_into(op, plan, inputs[0], inputs.size() == 2 ? &inputs[1] : nullptr, out, s);
  return out;
}

// scores[b, i, j] = sum_f q[b, i, f] * k[b, j, f] over broadcast batches: one
// NT GEMM reading K in place (the reference transposes K first).
Tensor attention_scores(const Tensor& q, const Tensor& k, Stream& s) {
  const Shape qb(q.shape.begin(), q.shape.end() - 2), kb(k.shape.begin(), k.shape.end() - 2);
  const Dim rows = q.shape[q.shape.size() - 2], columns = k.shape[k.shape.size() - 2], features = q.shape.back();
  const BroadcastPlan bp = make_broadcast_plan(qb, kb);
  Shape shape = bp.output_shape;
  shape.push_back(rows);
  shape.push_back(columns);
  Tensor out = make_tensor(DType::kFloat32, shape);
  if (numel(shape) == 0) return out;
  Shape ql = bp.lhs_strides, kl = bp.rhs_strides;
  for (Dim& v : ql) v *= rows * features;
  for (Dim& v : kl) v *= columns * features;
  const Strided m = compress(bp.output_shape, {ql, kl});
  if (m.shape.size() > TCX_HIP_MAX_BATCH_RANK) throw std::invalid_argument("HIP attention supports 8 batch axes");
  tcx_hip_gemm_desc_t d{};
  d.m = rows;
  d.n = columns;
  d.k = features;
  d.rhs_transposed = 1;
  d.batch_rank = static_cast<int32_t>(m.shape.size());
  d.batch_count = numel(m.shape);
  for (std::size_t i = 0; i < m.shape.size(); ++i) {
    d.batch_shape[i] = m.shape[i];
    d.lhs_batch_strides[i] = m.strides[0][i];
    d.rhs_batch_strides[i] = m.strides[1][i];
  }
  run_gemm(f32(q), f32(k), static_cast<float*>(out_ptr(out)), d, s, "HIP attention scores");
  return out;
}

// kAttention with the validation of core/inference.cpp:123-161: scores, the
// attention softmax, then probabilities @ V, each a native launch.
Tensor attention(const OpDesc& op, std::span<const Tensor> inputs, Stream& s) {
  if (op.kind != OpKind::kAttention || inputs.size() < 3 || inputs.size() > 4)
    throw std::invalid_argument("attention requires query, key, value and optional mask");
  for (std::size_t i = 0; i < 3; ++i) {
    if (inputs[i].dtype != DType::kFloat32) throw std::invalid_argument("inference values require float32 tensors");
    (void)numel(inputs[i].shape);
    if (inputs[i].shape.size() < 2) throw std::invalid_argument("attention tensors require rank >= 2");
  }
  const Tensor& q = inputs[0];
  const Tensor& k = inputs[1];
  const Tensor& v = inputs[2];
  const Dim features = q.shape.back(), rows = q.shape[q.shape.size() - 2], columns = k.shape[k.shape.size() - 2];
  if (features <= 0 || features != k.shape.back() || columns != v.shape[v.shape.size() - 2])
    throw std::invalid_argument(
        "attention query/key features and key/value sequence sizes must match; features must be positive");
  Shape batch;
  for (std::size_t i = 0; i < 3; ++i) {
    const Shape& input = inputs[i].shape;
    const std::size_t rank = std::max(batch.size(), input.size() - 2);
    Shape merged(rank, 1);
    for (std::size_t a = 0; a < rank; ++a) {
      const Dim left = a < rank - batch.size() ? 1 : batch[a - (rank - batch.size())];
      const Dim right = a < rank - (input.size() - 2) ? 1 : input[a - (rank - (input.size() - 2))];
      if (left != right && left != 1 && right != 1) throw std::invalid_argument("attention batch dimensions cannot broadcast");
      merged[a] = left == 1 ? right : left;
    }
    batch = std::move(merged);
  }
  Shape scores = batch;
  scores.push_back(rows);
  scores.push_back(columns);
  Shape shape = batch;
  shape.push_back(rows);
  shape.push_back(v.shape.back());
  (void)numel(scores);
  (void)numel(shape);
  OpDesc softmax{OpKind::kAttentionSoftmax};
  softmax.attention_shape = scores;
  softmax.causal = op.causal;
  softmax.attention_scale =
      checked_scale(op.attention_scale.value_or(1.0 / std::sqrt(static_cast<double>(features))));
  // Validate the mask against the scores before any launch, also for empty outputs.
  Tensor descriptor = q;
  descriptor.shape = scores;
  descriptor.strides = contiguous_strides(scores);
  std::vector<Tensor> preview{descriptor};
  if (inputs.size() == 4) preview.push_back(inputs[3]);
  const AttentionSoftmaxPlan plan = attention_softmax_plan(softmax, preview);
  for (const Tensor& t : inputs) (void)device_ptr(t);
  if (numel(shape) == 0) return make_tensor(DType::kFloat32, shape);
  // Unmasked attention over matching batches with 32/64/128 features: the
  // fused kernel, scores never materialised.
  const Shape qb(q.shape.begin(), q.shape.end() - 2);
  if (inputs.size() == 3 && qb == Shape(k.shape.begin(), k.shape.end() - 2) &&
      qb == Shape(v.shape.begin(), v.shape.end() - 2) &&
      tcx_hip_flash_attention_supported(features, v.shape.back()) &&
      aligned16(device_ptr(q)) && aligned16(device_ptr(k)) && aligned16(device_ptr(v))) {
    Tensor out = make_tensor(DType::kFloat32, shape);
    ok_or_throw(tcx_hip_flash_attention_f32(f32(q), f32(k), f32(v), static_cast<float*>(out_ptr(out)), numel(qb),
                                            rows, columns, features, *softmax.attention_scale, op.causal ? 1 : 0,
                                            s),
                "HIP attention");
    return out;
  }
  if (columns == 0) {  // no keys: every output row is an empty sum
    Tensor zeros;
    zeros.dtype = DType::kFloat32;
    zeros.shape = shape;
    return fill(zeros, 0.0, s);
  }
  const Tensor product = attention_scores(q, k, s);
  Tensor probabilities = make_tensor(DType::kFloat32, scores);
  attention_softmax_into(softmax, plan, product, inputs.size() == 4 ? &inputs[3] : nullptr, probabilities, s);
  return matmul(probabilities, v, s);
}

// ------------------------------------------------------------ layout, casts, scalars
// kNegate / k*Scalar / kCast / kTranspose / kSlice / kConcat with the checks of
// cpu_backend.cpp:801-930 and the plans of core/shape.cpp.
int element_bytes(DType dtype) { return static_cast<int>(dtype_size(dtype)); }

// Scratch device memory that outlives no call (flags, counts, offsets).
std::shared_ptr<HipBuffer> scratch(std::size_t bytes) {
  auto created = HipBuffer::create(bytes);
  if (!created) {
    const Status& st = created.status();
    if (st.code() == StatusCode::kUnavailable) throw Unavailable(st.message());
    throw std::runtime_error(st.message());
  }
  return created.move_value();
}

Tensor scalar_op(const OpDesc& op, const Tensor& x, Stream& s) {
  if (x.dtype == DType::kBool) throw std::invalid_argument("numeric operations do not support bool");
  const int code = op.kind == OpKind::kNegate           ? TCX_SCALAR_NEGATE
                   : op.kind == OpKind::kAddScalar      ? TCX_SCALAR_ADD
                   : op.kind == OpKind::kSubtractScalar ? TCX_SCALAR_SUBTRACT
                   : op.kind == OpKind::kMultiplyScalar ? TCX_SCALAR_MULTIPLY
                                                        : TCX_SCALAR_DIVIDE;
  if (x.dtype == DType::kInt32 && code != TCX_SCALAR_NEGATE) {
    if (code == TCX_SCALAR_DIVIDE) throw std::invalid_argument("division only supports float32 tensors");
    if (!is_int32_representable(op.scalar_value))
      throw std::invalid_argument("arithmetic scalar must be an integer in int32 range");
  }
  const void* xp = device_ptr(x);
  Tensor out = make_tensor(x.dtype, x.shape);
  ok_or_throw(tcx_hip_scalar_op(code, tcx_dtype(x.dtype), xp, out_ptr(out), numel(x.shape), op.scalar_value,
                                op.scalar_left ? 1 : 0, s),
              "HIP scalar arithmetic");
  return out;
}

int any_dtype(DType d) { return d == DType::kBool ? TCX_BOOL : tcx_dtype(d); }

Tensor cast(const OpDesc& op, const Tensor& x, Stream& s) {
  const DType to = op.target_dtype;
  if (to != DType::kFloat32 && to != DType::kInt32 && to != DType::kBool)
    throw std::invalid_argument("unsupported cast target dtype");
  const void* xp = device_ptr(x);
  Tensor out = make_tensor(to, x.shape);
  const Dim n = numel(x.shape);
  if (n == 0) return out;
  std::shared_ptr<HipBuffer> flag;
  if (x.dtype == DType::kFloat32 && to == DType::kInt32) flag = scratch(sizeof(std::int32_t));
  ok_or_throw(tcx_hip_cast(any_dtype(x.dtype), any_dtype(to), xp, out_ptr(out), n,
                           flag ? static_cast<std::int32_t*>(flag->data()) : nullptr, s),
              "HIP cast");
  return out;
}

// A strided gather of x through `plan`, with size-1 axes dropped and
// contiguous runs merged to fit the kernel's metadata.
Tensor gather(const Tensor& x, const TransposePlan& plan, Stream& s) {
  const void* xp = device_ptr(x);
  Tensor out = make_tensor(x.dtype, plan.output_shape);
  if (numel(plan.output_shape) == 0) return out;
  const Strided m = compress(plan.output_shape, {plan.input_strides});
  ok_or_throw(tcx_hip_gather_strided(element_bytes(x.dtype), xp, out_ptr(out), static_cast<int32_t>(m.shape.size()),
                                     m.shape.data(), m.strides[0].data(), plan.offset, s),
              "HIP gather");
  return out;
}

Tensor concat(const OpDesc& op, std::span<const Tensor> inputs, Stream& s) {
  std::vector<Shape> shapes;
  for (const Tensor& t : inputs) {
    if (t.dtype != inputs[0].dtype) throw std::invalid_argument("concat dtypes must match");
    (void)device_ptr(t);
    shapes.push_back(t.shape);
  }
  const ConcatPlan plan = make_concat_plan(shapes, op.axis);
  Tensor out = make_tensor(inputs[0].dtype, plan.output_shape);
  if (numel(plan.output_shape) == 0) return out;
  const Dim out_block = plan.output_shape[plan.axis] * plan.inner;
  Dim outer = 1;
  for (std::size_t a = 0; a < plan.axis; ++a) outer *= plan.output_shape[a];
  Dim offset = 0;
  for (const Tensor& t : inputs) {
    const Dim block = t.shape[plan.axis] * plan.inner;
    ok_or_throw(tcx_hip_copy_blocks(element_bytes(t.dtype), device_ptr(t), out_ptr(out), outer, block, out_block,
                                    offset, s),
                "HIP concat");
    offset += block;
  }
  return out;
}

// ------------------------------------------------------------ predicates
int predicate_code(OpKind kind) {
  switch (kind) {
    case OpKind::kEqual: return TCX_PRED_EQUAL;
    case OpKind::kNotEqual: return TCX_PRED_NOT_EQUAL;
    case OpKind::kLess: return TCX_PRED_LESS;
    case OpKind::kLessEqual: return TCX_PRED_LESS_EQUAL;
    case OpKind::kGreater: return TCX_PRED_GREATER;
    case OpKind::kGreaterEqual: return TCX_PRED_GREATER_EQUAL;
    case OpKind::kLogicalAnd: return TCX_PRED_LOGICAL_AND;
    case OpKind::kLogicalOr: return TCX_PRED_LOGICAL_OR;
    case OpKind::kLogicalXor: return TCX_PRED_LOGICAL_XOR;
    case OpKind::kLogicalNot: return TCX_PRED_LOGICAL_NOT;
    default: return TCX_PRED_WHERE;
  }
}

Tensor predicate(const OpDesc& op, std::span<const Tensor> inputs, Stream& s) {
  const PredicatePlan plan = make_predicate_plan(op, inputs);
  std::vector<const void*> ptrs;
  for (const Tensor& t : inputs) ptrs.push_back(device_ptr(t));
  Tensor out = make_tensor(plan.output_dtype, plan.output_shape);
  if (numel(plan.output_shape) == 0) return out;
  std::vector<Shape> strides = plan.input_strides;
  while (strides.size() < 3) strides.push_back(Shape(plan.output_shape.size(), 0));
  const Strided m = compress(plan.output_shape, strides);
  tcx_hip_broadcast3_t d{};
  d.rank = static_cast<int32_t>(m.shape.size());
  for (std::size_t a = 0; a < m.shape.size(); ++a) {
    d.shape[a] = m.shape[a];
    for (int k = 0; k < 3; ++k) d.strides[k][a] = m.strides[static_cast<std::size_t>(k)][a];
  }
  const bool where = op.kind == OpKind::kWhere;
  const DType compared = where ? inputs[1].dtype : inputs[0].dtype;
  if (compared == DType::kInt32) d.flags = TCX_PRED_FLAG_INT32;
  ok_or_throw(tcx_hip_predicate(predicate_code(op.kind), element_bytes(compared), ptrs[0],
                                ptrs.size() > 1 ? ptrs[1] : nullptr, ptrs.size() > 2 ? ptrs[2] : nullptr, out_ptr(out),
                                &d, s),
              "HIP predicate");
  return out;
}

Tensor bool_reduce(const OpDesc& op, const Tensor& x, Stream& s) {
  if (x.dtype != DType::kBool) throw std::invalid_argument("any/all require bool tensors");
  const ReductionPlan plan = make_boolean_reduction_plan(op, x.shape);
  const void* xp = device_ptr(x);
  Tensor out = make_tensor(DType::kBool, plan.output_shape);
  const Dim groups = numel(plan.output_shape);
  if (groups == 0) return out;
  if (x.shape.size() > TCX_HIP_MAX_RANK) throw std::invalid_argument("HIP boolean reductions support rank <= 8");
  ok_or_throw(tcx_hip_bool_reduce(op.kind == OpKind::kAll ? 1 : 0, static_cast<const uint8_t*>(xp),
                                  static_cast<uint8_t*>(out_ptr(out)), plan.index_metadata.data(),
                                  static_cast<int32_t>(x.shape.size()), groups, plan.reduction_size, s),
              "HIP boolean reduction");
  return out;
}

// masked_select: counts per chunk, host offsets, then index compaction and a
// row gather (cpu_predicate.cpp:72-96).
Tensor masked_select(const Tensor& x, const Tensor& mask, Stream& s) {
  const MaskedSelectPlan plan = make_masked_select_plan(x, mask);
  const void* xp = device_ptr(x);
  const auto* mp = static_cast<const uint8_t*>(device_ptr(mask));
  const Dim n = numel(mask.shape);
  Dim total = 0;
  std::vector<std::int64_t> offsets;
  std::shared_ptr<HipBuffer> counts_dev;
  if (n > 0) {
    const Dim chunks = tcx_hip_mask_chunks(n);
    counts_dev = scratch(static_cast<std::size_t>(chunks) * sizeof(std::int64_t));
    auto* counts = static_cast<std::int64_t*>(counts_dev->data());
    ok_or_throw(tcx_hip_mask_count(mp, n, counts, s), "HIP mask count");
    offsets.resize(static_cast<std::size_t>(chunks));
    ok_or_throw(tcx_hip_memcpy_d2h(offsets.data(), counts, offsets.size() * sizeof(std::int64_t), s),
                "HIP mask count copy");
    for (std::int64_t& c : offsets) {  // counts -> exclusive offsets
      const std::int64_t here = c;
      c = total;
      total += here;
    }
  }
  Shape shape{total};
  shape.insert(shape.end(), plan.tail_shape.begin(), plan.tail_shape.end());
  Tensor out = make_tensor(x.dtype, shape);
  if (total == 0) return out;
  ok_or_throw(tcx_hip_memcpy_h2d(counts_dev->data(), offsets.data(), offsets.size() * sizeof(std::int64_t), s),
              "HIP mask offset copy");
  auto index = scratch(static_cast<std::size_t>(total) * sizeof(std::int64_t));
  ok_or_throw(tcx_hip_masked_select(element_bytes(x.dtype), xp, mp, n, plan.block_size,
                                    static_cast<const std::int64_t*>(counts_dev->data()), total,
                                    static_cast<std::int64_t*>(index->data()), out_ptr(out), s),
              "HIP masked select");
  synchronize(s);  // the scratch buffers are released on return
  return out;
}

// ------------------------------------------------------------ kernel class
Status execute_builtin_kernel(const BackendExecution& e) {
  if (Status s = validate_kernel_execution_contract(e); !s.ok()) return s;
  const auto& target = *e.compilation_target;
  if (target.artifact_kind != KernelArtifactKind::kStaticLibrary || target.artifact != kStaticArtifact)
    return Status(StatusCode::kInvalidArgument, "HIP kernels must name the tensorcx_hip static library");
  if (target.entry_point != "linear_bias_act" && target.entry_point != "bias_act")
    return Status(StatusCode::kInvalidArgument, "unknown HIP built-in kernel entry point");
  std::vector<const Tensor*> tensors;
  std::vector<std::uint32_t> scalars;
  for (const KernelArgument& a : e.kernel_arguments) {
    if (a.kind == KernelArgumentKind::kTensor)
      tensors.push_back(a.tensor);
    else
      scalars.push_back(a.uint32_value);
  }
  if (e.outputs.size() != 1) return Status(StatusCode::kInvalidArgument, "HIP built-in kernels write one output");
  const Tensor& out = e.outputs[0];
  if (out.dtype != DType::kFloat32) return Status(StatusCode::kInvalidArgument, "HIP built-in kernels write float32");
  (void)device_ptr(out);
  if (scalars.size() != 1 || scalars[0] > TCX_ACT_GELU)
    return Status(StatusCode::kInvalidArgument, "HIP built-in kernels take one activation code");
  const int act = static_cast<int>(scalars[0]);
  Stream s;
  if (target.entry_point == "linear_bias_act") {
    if (tensors.size() != 3) return Status(StatusCode::kInvalidArgument, "linear_bias_act takes x, weight, bias");
    const Tensor inputs[3] = {*tensors[0], *tensors[1], *tensors[2]};
    if (linear_shape(inputs) != out.shape)
      return Status(StatusCode::kInvalidArgument, "linear_bias_act output shape mismatch");
    if (numel(out.shape) != 0) linear_into(inputs[0], inputs[1], &inputs[2], act, out, s);
  } else if (target.entry_point == "bias_act") {
    if (tensors.size() != 2) return Status(StatusCode::kInvalidArgument, "bias_act takes x and bias");
    const Tensor& x = *tensors[0];
    const Tensor& b = *tensors[1];
    if (x.shape.empty() || b.shape != Shape{x.shape.back()} || out.shape != x.shape)
      return Status(StatusCode::kInvalidArgument, "bias_act requires x (..., n), bias (n,) and a matching output");
    const Dim cols = x.shape.back();
    if (numel(x.shape) != 0)
      ok_or_throw(tcx_hip_bias_act_f32(f32(x), f32(b), static_cast<float*>(out_ptr(out)), numel(x.shape) / cols, cols,
                                       act, s),
                  "HIP bias_act");
  }
  if (s.used()) synchronize(s);
  return Status::Ok();
}

}  // namespace

// ------------------------------------------------------------ public API
Expected<std::shared_ptr<HipBuffer>> HipBuffer::create(std::size_t bytes) {
  ProfileScope span(ProfileCategory::kAllocation, "hip_allocate", "hip", bytes);
  std::shared_ptr<HipBuffer> buffer(new HipBuffer());
  const int rc = tcx_hip_allocate(bytes, &buffer->data_, &buffer->owner_);
  if (rc != TCX_OK) return status_from_code(rc, "HIP allocation");
  buffer->bytes_ = bytes;
  return buffer;
}

Expected<std::shared_ptr<HipBuffer>> HipBuffer::borrow(void* data, std::size_t bytes, std::shared_ptr<void> owner) {
  if (!owner || (bytes != 0 && data == nullptr))
    return Status(StatusCode::kInvalidArgument, "borrowed HIP storage requires an owner and data");
  const int rc = tcx_hip_borrow_check(data, bytes);
  if (rc != TCX_OK) return status_from_code(rc, "HIP borrow");
  std::shared_ptr<HipBuffer> buffer(new HipBuffer());
  buffer->data_ = bytes ? data : nullptr;
  buffer->bytes_ = bytes;
  buffer->external_ = std::move(owner);
  return buffer;
}

StorageIdentity HipBuffer::storage_identity() const {
  static const char device0 = 0;
  return {&device0, reinterpret_cast<std::uintptr_t>(data_), bytes_};
}

HipBuffer::~HipBuffer() {
  if (external_) return;  // the external owner's deleter runs when external_ goes
  ProfileScope span(ProfileCategory::kDeallocation, "hip_release", "hip", bytes_);
  if (exported_.load(std::memory_order_relaxed)) tcx_hip_release_uncached(data_, bytes_, owner_);
  else tcx_hip_release(data_, bytes_, owner_);
}

bool available() { return tcx_hip_init() == TCX_OK; }

Expected<DeviceInfo> device_info() {
  tcx_hip_device_info_t raw{};
  const int rc = tcx_hip_device_info(0, &raw);
  if (rc != TCX_OK) return status_from_code(rc, "HIP device info");
  DeviceInfo info;
  info.name = raw.name;
  info.arch = raw.arch;
  info.compute_units = raw.compute_units;
  info.clock_khz = raw.clock_khz;
  info.memory_clock_khz = raw.memory_clock_khz;
  info.memory_bus_width = raw.memory_bus_width;
  info.l2_bytes = raw.l2_bytes;
  info.runtime_version = raw.runtime_version;
  info.driver_version = raw.driver_version;
  info.free_bytes = raw.free_bytes;
  info.total_bytes = raw.total_bytes;
  return info;
}

Expected<std::string> device_name() {
  auto info = device_info();
  if (!info) return info.status();
  return info.value().name;
}

Expected<Tensor> empty(Shape shape, DType dtype) {
  try {
    if (dtype != DType::kFloat32 && dtype != DType::kInt32 && dtype != DType::kBool)
      return Status(StatusCode::kInvalidArgument, "HIP tensors support float32, int32 and bool");
    const auto bytes = byte_size(shape, dtype);
    if (const int rc = tcx_hip_init(); rc != TCX_OK) return status_from_code(rc, "HIP device");
    auto buffer = HipBuffer::create(bytes);
    if (!buffer) return buffer.status();
    Shape strides = contiguous_strides(shape);
    return Tensor{dtype, std::move(shape), std::move(strides), Device{"hip", 0},
                  std::static_pointer_cast<Buffer>(buffer.move_value()), 0};
  } catch (const std::invalid_argument& error) {
    return Status(StatusCode::kInvalidArgument, error.what());
  }
}

Expected<Tensor> from_host(const void* host, DType dtype, Shape shape) {
  auto created = empty(std::move(shape), dtype);
  if (!created) return created.status();
  Tensor t = created.move_value();
  const std::size_t bytes = t.buffer->nbytes();
  if (bytes) {
    ProfileScope span(ProfileCategory::kCopy, "host_to_device", "hip", bytes);
    tcx_stream_t s = nullptr;
    int rc = tcx_hip_stream(&s);
    if (rc == TCX_OK) rc = tcx_hip_memcpy_h2d(out_ptr(t), host, bytes, s);
    if (rc != TCX_OK) return status_from_code(rc, "HIP host to device copy");
  }
  return t;
}

Status to_host(const Tensor& tensor, void* host, std::size_t bytes) {
  try {
    const void* src = device_ptr(tensor);
    const auto need = static_cast<std::size_t>(numel(tensor.shape)) * dtype_size(tensor.dtype);
    if (bytes != need) return Status(StatusCode::kInvalidArgument, "host buffer size does not match the tensor");
    if (need == 0) return Status::Ok();
    ProfileScope span(ProfileCategory::kCopy, "device_to_host", "hip", need);
    tcx_stream_t s = nullptr;
    int rc = tcx_hip_stream(&s);
    if (rc == TCX_OK) rc = tcx_hip_memcpy_d2h(host, src, need, s);
    return status_from_code(rc, "HIP device to host copy");
  } catch (const std::invalid_argument& error) {
    return Status(StatusCode::kInvalidArgument, error.what());
  }
}

Expected<Tensor> clone(const Tensor& tensor) {
  try {
    const void* src = device_ptr(tensor);
    auto created = empty(tensor.shape, tensor.dtype);
    if (!created) return created.status();
    Tensor t = created.move_value();
    const std::size_t bytes = t.buffer->nbytes();
    if (bytes) {
      tcx_stream_t s = nullptr;
      int rc = tcx_hip_stream(&s);
      if (rc == TCX_OK) rc = tcx_hip_memcpy_d2d(out_ptr(t), src, bytes, s);
      if (rc != TCX_OK) return status_from_code(rc, "HIP device copy");
    }
    return t;
  } catch (const std::invalid_argument& error) {
    return Status(StatusCode::kInvalidArgument, error.what());
  }
}

Expected<Tensor> borrow(void* data, DType dtype, Shape shape, std::shared_ptr<void> owner) {
  try {
    if (dtype != DType::kFloat32 && dtype != DType::kInt32 && dtype != DType::kBool)
      return Status(StatusCode::kInvalidArgument, "HIP tensors support float32, int32 and bool");
    const auto bytes = byte_size(shape, dtype);
    if (bytes && reinterpret_cast<std::uintptr_t>(data) % dtype_size(dtype))
      return Status(StatusCode::kInvalidArgument, "borrowed HIP pointer is misaligned");
    auto buffer = HipBuffer::borrow(data, bytes, std::move(owner));
    if (!buffer) return buffer.status();
    Shape strides = contiguous_strides(shape);
    return Tensor{dtype, std::move(shape), std::move(strides), Device{"hip", 0},
                  std::static_pointer_cast<Buffer>(buffer.move_value()), 0};
  } catch (const std::invalid_argument& error) {
    return Status(StatusCode::kInvalidArgument, error.what());
  }
}

Expected<void*> export_storage(const Tensor& tensor) {
  try {
    void* data = device_ptr(tensor);
    static_cast<HipBuffer*>(tensor.buffer.get())->mark_exported();
    return data;
  } catch (const std::invalid_argument& error) {
    return Status(StatusCode::kInvalidArgument, error.what());
  }
}

Status HipBackend::execute(const BackendExecution& e) {
  ProfileScope dispatch(ProfileCategory::kDispatch, "execute", "hip", std::nullopt,
                        e.op_class == BackendOpClass::kPrimitive ? std::optional<OpKind>(e.op.kind) : std::nullopt);
  try {
    if (e.op_class == BackendOpClass::kKernel) return execute_builtin_kernel(e);
    if (Status contract = validate_primitive_execution_contract(e, "hip"); !contract.ok()) return contract;
    if (e.op.kind == OpKind::kFill && e.outputs[0].device.index != 0)
      return Status(StatusCode::kInvalidArgument, "HIP fill requires device index 0");
    // Validate every input before touching the device.
    if (e.op.kind != OpKind::kFill)
      for (const Tensor& t : e.inputs) (void)device_ptr(t);
    Stream s;
    DeviceInterval<> interval("hip_kernels");
    auto interval_at = [&](auto mark) noexcept {
      if (!interval.active()) return;
      try {
        mark(static_cast<tcx_stream_t>(s));
      } catch (const std::exception&) {
        interval.fail();
      }
    };
    interval_at([&](tcx_stream_t stream) { interval.start(stream); });
    Tensor result;
    switch (e.op.kind) {
      case OpKind::kFill: result = fill(e.outputs[0], e.op.scalar_value, s); break;
      case OpKind::kMatmul: result = matmul(e.inputs[0], e.inputs[1], s); break;
      case OpKind::kLinear: result = linear(e.inputs, s); break;
      case OpKind::kSum:
      case OpKind::kMax:
      case OpKind::kMean: result = reduce(e.op, e.inputs[0], s); break;
      case OpKind::kMin:
      case OpKind::kArgmax: result = argext(e.op, e.inputs[0], s); break;
      case OpKind::kSoftmax:
      case OpKind::kRmsNorm:
      case OpKind::kLayerNorm: result = row_op(e.op, e.inputs[0], nullptr, nullptr, s); break;
      case OpKind::kAffineRmsNorm:
      case OpKind::kAffineLayerNorm: result = affine_norm(e.op, e.inputs, s); break;
      case OpKind::kExp:
      case OpKind::kGelu:
      case OpKind::kSilu: result = unary(e.op, e.inputs[0], s); break;
      case OpKind::kAdd:
      case OpKind::kSubtract:
      case OpKind::kMultiply:
      case OpKind::kDivide: result = binary(e.op, e.inputs[0], e.inputs[1], s); break;
      case OpKind::kLog:
      case OpKind::kSqrt:
      case OpKind::kAbs: result = math_unary(e.op, e.inputs[0], s); break;
      case OpKind::kClip: result = clip(e.inputs, s); break;
      case OpKind::kTopK: {
        auto [values, indices] = topk(e.op, e.inputs[0], s);
        interval_at([&](tcx_stream_t stream) { interval.stop(stream); });
        if (s.used()) synchronize(s);
        e.outputs[0] = std::move(values);
        e.outputs[1] = std::move(indices);
        return Status::Ok();
      }
      case OpKind::kEmbedding: result = embedding(e.inputs, s); break;
      case OpKind::kAttentionSoftmax: result = attention_softmax(e.op, e.inputs, s); break;
      case OpKind::kAttention: result = attention(e.op, e.inputs, s); break;
      case OpKind::kNegate:
      case OpKind::kAddScalar:
      case OpKind::kSubtractScalar:
      case OpKind::kMultiplyScalar:
      case OpKind::kDivideScalar: result = scalar_op(e.op, e.inputs[0], s); break;
      case OpKind::kCast: result = cast(e.op, e.inputs[0], s); break;
      case OpKind::kTranspose: result = gather(e.inputs[0], make_transpose_plan(e.inputs[0].shape, e.op.axes), s); break;
      case OpKind::kSlice:
        result = gather(e.inputs[0],
                        make_slice_plan(e.inputs[0].shape, e.op.slice_starts, e.op.slice_steps, e.op.slice_shape), s);
        break;
      case OpKind::kConcat: result = concat(e.op, e.inputs, s); break;
      case OpKind::kEqual:
      case OpKind::kNotEqual:
      case OpKind::kLess:
      case OpKind::kLessEqual:
      case OpKind::kGreater:
      case OpKind::kGreaterEqual:
      case OpKind::kLogicalAnd:
      case OpKind::kLogicalOr:
      case OpKind::kLogicalXor:
      case OpKind::kLogicalNot:
      case OpKind::kWhere: result = predicate(e.op, e.inputs, s); break;
      case OpKind::kAny:
      case OpKind::kAll: result = bool_reduce(e.op, e.inputs[0], s); break;
      case OpKind::kMaskedSelect: result = masked_select(e.inputs[0], e.inputs[1], s); break;
      default:
        return Status(StatusCode::kInvalidArgument, "unsupported HIP backend execution operation");
    }
    interval_at([&](tcx_stream_t stream) { interval.stop(stream); });
    if (s.used()) synchronize(s);  // nothing to wait for when nothing was launched
    e.outputs[0] = std::move(result);  // publish only after the work completed
    return Status::Ok();
  } catch (const std::invalid_argument& error) {
    return Status(StatusCode::kInvalidArgument, error.what());
  } catch (const Unavailable& error) {
    return Status(StatusCode::kUnavailable, error.what());
  } catch (const std::exception& error) {
    return Status(StatusCode::kInternal, error.what());
  }
}

}  // namespace tensorcx::hip
