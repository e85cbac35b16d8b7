// Python binding of the hip device: the hip counterpart of the reference's
// per-device overload block (reference bindings/python_module.cpp:1660-1716)
// and its shared templates (:800-958). Every op builds a BackendExecution,
// releases the GIL, calls HipBackend::execute and maps the Status to a Python
// exception the way throw_status does (python_module.cpp:402-414):
// kInvalidArgument -> ValueError, anything else -> RuntimeError.

#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <array>
#include <cstring>
#include <optional>
#include <string>
#include <vector>

#include "hip_binding.h"
#include "tensorcx/backends/hip/hip_backend.h"
#include "tensorcx/core/profiling.h"

namespace py = pybind11;
using namespace tensorcx;

using tcx_bind::HipTensor;
using tcx_bind::throw_status;

namespace {

DType parse_dtype(const std::string& name) {
  if (name == "float32") return DType::kFloat32;
  if (name == "int32") return DType::kInt32;
  if (name == "bool") return DType::kBool;
  throw py::value_error("unsupported dtype: " + name);
}

Shape to_shape(const std::vector<std::int64_t>& dims) { return Shape(dims.begin(), dims.end()); }

HipTensor run(OpDesc op, std::vector<Tensor> inputs) {
  std::array<Tensor, 1> outputs{};
  Status status;
  {
    py::gil_scoped_release release;
    BackendExecution e{BackendOpClass::kPrimitive, std::move(op), inputs, outputs, std::nullopt, std::nullopt, {}};
    hip::HipBackend backend;
    status = backend.execute(e);
  }
  if (!status.ok()) throw_status(status);
  return HipTensor{std::move(outputs[0])};
}

std::pair<HipTensor, HipTensor> run2(OpDesc op, std::vector<Tensor> inputs) {
  std::array<Tensor, 2> outputs{};
  Status status;
  {
    py::gil_scoped_release release;
    BackendExecution e{BackendOpClass::kPrimitive, std::move(op), inputs, outputs, std::nullopt, std::nullopt, {}};
    hip::HipBackend backend;
    status = backend.execute(e);
  }
  if (!status.ok()) throw_status(status);
  return {HipTensor{std::move(outputs[0])}, HipTensor{std::move(outputs[1])}};
}

HipTensor unary(OpKind kind, const HipTensor& x) { return run(OpDesc{kind}, {x.tensor}); }

HipTensor axis_op(OpKind kind, const HipTensor& x, std::int64_t axis, double eps = 1e-5) {
  OpDesc op{kind};
  op.axis = axis;
  op.epsilon = eps;
  return run(op, {x.tensor});
}

HipTensor axes_op(OpKind kind, const HipTensor& x, const std::vector<std::int64_t>& axes) {
  OpDesc op{kind};
  op.reduction_axes = to_shape(axes);
  return run(op, {x.tensor});
}

// Built-in fused kernels through BackendOpClass::kKernel (the unchanged ABI's
// route for backend-provided kernels); the output is preallocated here.
HipTensor builtin(const std::string& entry, std::vector<const HipTensor*> args, std::uint32_t act, Shape out_shape) {
  auto created = hip::empty(std::move(out_shape), DType::kFloat32);
  if (!created) throw_status(created.status());
  std::array<Tensor, 1> outputs{created.move_value()};
  std::vector<KernelArgument> kargs;
  for (const HipTensor* t : args) kargs.push_back(KernelArgument{KernelArgumentKind::kTensor, &t->tensor, 0});
  kargs.push_back(KernelArgument{KernelArgumentKind::kUInt32, nullptr, act});
  Status status;
  {
    py::gil_scoped_release release;
    BackendExecution e{BackendOpClass::kKernel, OpDesc{},
                       {}, outputs, LaunchConfig{1, 1, 1, 1, 1, 1},
                       CompilationTarget{KernelArtifactKind::kStaticLibrary, hip::kStaticArtifact, entry}, kargs};
    hip::HipBackend backend;
    status = backend.execute(e);
  }
  if (!status.ok()) throw_status(status);
  return HipTensor{std::move(outputs[0])};
}

py::array to_numpy(const HipTensor& t) {
  std::vector<py::ssize_t> shape(t.tensor.shape.begin(), t.tensor.shape.end());
  py::array out;
  if (t.tensor.dtype == DType::kFloat32)
    out = py::array_t<float>(shape);
  else if (t.tensor.dtype == DType::kInt32)
    out = py::array_t<std::int32_t>(shape);
  else
    out = py::array_t<bool>(shape);
  const std::size_t bytes = static_cast<std::size_t>(out.nbytes());
  Status status;
  {
    void* dst = out.mutable_data();
    py::gil_scoped_release release;
    status = hip::to_host(t.tensor, dst, bytes);
  }
  if (!status.ok()) throw_status(status);
  return out;
}

HipTensor from_numpy(py::array array) {
  DType dtype;
  py::array contiguous;
  if (py::isinstance<py::array_t<float>>(array)) {
    dtype = DType::kFloat32;
    contiguous = py::array_t<float, py::array::c_style | py::array::forcecast>(array);
  } else if (py::isinstance<py::array_t<std::int32_t>>(array)) {
    dtype = DType::kInt32;
    contiguous = py::array_t<std::int32_t, py::array::c_style | py::array::forcecast>(array);
  } else if (py::isinstance<py::array_t<bool>>(array)) {
    dtype = DType::kBool;
    contiguous = py::array_t<bool, py::array::c_style | py::array::forcecast>(array);
  } else {
    throw py::value_error("hip tensors are created from float32, int32 or bool arrays");
  }
  Shape shape;
  for (py::ssize_t i = 0; i < contiguous.ndim(); ++i) shape.push_back(contiguous.shape(i));
  Expected<Tensor> created = Status();
  {
    const void* src = contiguous.data();
    py::gil_scoped_release release;
    created = hip::from_host(src, dtype, std::move(shape));
  }
  if (!created) throw_status(created.status());
  return HipTensor{created.move_value()};
}

struct PoolHandle {
  tcx_hip_pool_t* pool{nullptr};
  PoolHandle(std::size_t bytes, std::size_t blocks) {
    const int rc = tcx_hip_pool_create(bytes, blocks, nullptr, &pool);
    if (rc != TCX_OK) {
      if (rc == TCX_INVALID_ARGUMENT) throw py::value_error(tcx_hip_last_error());
      throw std::runtime_error(tcx_hip_last_error());
    }
  }
  ~PoolHandle() { tcx_hip_pool_destroy(pool); }
  void check(int rc) {
    if (rc == TCX_OK) return;
    if (rc == TCX_INVALID_ARGUMENT) throw py::value_error(tcx_hip_last_error());
    throw std::runtime_error(tcx_hip_last_error());
  }
};

}  // namespace

PYBIND11_MODULE(_core, m) {
  m.doc() = "tensor.cx hip device (MI355X / gfx950)";

  py::class_<HipTensor>(m, "HipTensor")
      .def_property_readonly("shape", [](const HipTensor& t) { return py::tuple(py::cast(std::vector<std::int64_t>(t.tensor.shape.begin(), t.tensor.shape.end()))); })
      .def_property_readonly("strides", [](const HipTensor& t) { return py::tuple(py::cast(std::vector<std::int64_t>(t.tensor.strides.begin(), t.tensor.strides.end()))); })
      .def_property_readonly("dtype", [](const HipTensor& t) { return std::string(dtype_name(t.tensor.dtype)); })
      .def_property_readonly("device", [](const HipTensor&) { return std::string("hip"); })
      .def_property_readonly("nbytes", [](const HipTensor& t) { return numel(t.tensor.shape) * static_cast<std::int64_t>(dtype_size(t.tensor.dtype)); })
      .def("numpy", &to_numpy);

  m.def("is_available", [] { return hip::available(); });
  m.def("device_info", [] {
    auto info = hip::device_info();
    if (!info) throw_status(info.status());
    const auto& d = info.value();
    py::dict out;
    out["name"] = d.name;
    out["arch"] = d.arch;
    out["compute_units"] = d.compute_units;
    out["clock_khz"] = d.clock_khz;
    out["memory_clock_khz"] = d.memory_clock_khz;
    out["memory_bus_width"] = d.memory_bus_width;
    out["l2_bytes"] = d.l2_bytes;
    out["runtime_version"] = d.runtime_version;
    out["driver_version"] = d.driver_version;
    out["free_bytes"] = d.free_bytes;
    out["total_bytes"] = d.total_bytes;
    return out;
  });
  m.def("from_numpy", &from_numpy);
  m.def("empty", [](std::vector<std::int64_t> shape, const std::string& dtype) {
    auto t = hip::empty(to_shape(shape), parse_dtype(dtype));
    if (!t) throw_status(t.status());
    return HipTensor{t.move_value()};
  });
  m.def("fill", [](std::vector<std::int64_t> shape, const std::string& dtype, double value) {
    Shape s = to_shape(shape);
    OpDesc op{OpKind::kFill};
    op.scalar_value = value;
    std::array<Tensor, 1> outputs{Tensor{parse_dtype(dtype), s, contiguous_strides(s), Device{"hip", 0}, nullptr, 0}};
    Status status;
    {
      py::gil_scoped_release release;
      BackendExecution e{BackendOpClass::kPrimitive, op, {}, outputs, std::nullopt, std::nullopt, {}};
      hip::HipBackend backend;
      status = backend.execute(e);
    }
    if (!status.ok()) throw_status(status);
    return HipTensor{std::move(outputs[0])};
  });
  m.def("reshape", [](const HipTensor& x, std::vector<std::int64_t> shape) {
    Shape s = to_shape(shape);
    if (numel(s) != numel(x.tensor.shape)) throw py::value_error("reshape size mismatch");
    Tensor t = x.tensor;
    t.shape = s;
    t.strides = contiguous_strides(s);
    return HipTensor{std::move(t)};
  });
  // True for the same storage range, False for disjoint storage; a partial
  // overlap is an error (python_module.cpp:914-919).
  m.def("_shares_storage", [](const HipTensor& a, const HipTensor& b) {
    if (!a.tensor.buffer || !b.tensor.buffer) return false;
    const StorageRelation relation = a.tensor.buffer->storage_relation(*b.tensor.buffer);
    if (relation == StorageRelation::kPartialOverlap)
      throw py::value_error("kernel arguments have unsupported partial storage overlap");
    return relation == StorageRelation::kSameRange;
  });
  tcx_bind::bind_dlpack(m);

  m.def("matmul", [](const HipTensor& a, const HipTensor& b) { return run(OpDesc{OpKind::kMatmul}, {a.tensor, b.tensor}); });
  m.def("linear", [](const HipTensor& x, const HipTensor& w, std::optional<const HipTensor*> b) {
    std::vector<Tensor> in{x.tensor, w.tensor};
    if (b && *b) in.push_back((*b)->tensor);
    return run(OpDesc{OpKind::kLinear}, std::move(in));
  }, py::arg("x"), py::arg("weight"), py::arg("bias") = py::none());
  m.def("linear_act", [](const HipTensor& x, const HipTensor& w, const HipTensor& b, std::uint32_t act) {
    Shape shape = x.tensor.shape;
    if (shape.empty() || w.tensor.shape.size() != 2) throw py::value_error("linear requires (..., in_features) and (out_features, in_features)");
    shape.back() = w.tensor.shape[0];
    return builtin("linear_bias_act", {&x, &w, &b}, act, shape);
  });
  m.def("bias_act", [](const HipTensor& x, const HipTensor& b, std::uint32_t act) {
    return builtin("bias_act", {&x, &b}, act, x.tensor.shape);
  });

  for (const auto& [name, kind] : std::vector<std::pair<const char*, OpKind>>{
           {"sum", OpKind::kSum}, {"max", OpKind::kMax}, {"mean", OpKind::kMean}}) {
    const OpKind k = kind;
    m.def(name, [k](const HipTensor& x, std::int64_t axis) { return axis_op(k, x, axis); }, py::arg("x"), py::arg("axis") = 0);
    m.def((std::string("_") + name + "_axes").c_str(),
          [k](const HipTensor& x, std::vector<std::int64_t> axes) { return axes_op(k, x, axes); });
  }
  m.def("_min_axes", [](const HipTensor& x, std::vector<std::int64_t> axes) { return axes_op(OpKind::kMin, x, axes); });
  m.def("_argmax_axes", [](const HipTensor& x, std::vector<std::int64_t> axes) { return axes_op(OpKind::kArgmax, x, axes); });
  m.def("softmax", [](const HipTensor& x, std::int64_t axis) { return axis_op(OpKind::kSoftmax, x, axis); }, py::arg("x"), py::arg("axis"));
  m.def("rmsnorm", [](const HipTensor& x, std::int64_t axis, double eps) { return axis_op(OpKind::kRmsNorm, x, axis, eps); },
        py::arg("x"), py::arg("axis"), py::arg("eps") = 1e-5);
  m.def("layernorm", [](const HipTensor& x, std::int64_t axis, double eps) { return axis_op(OpKind::kLayerNorm, x, axis, eps); },
        py::arg("x"), py::arg("axis"), py::arg("eps") = 1e-5);
  m.def("_affine_norm", [](const HipTensor& x, std::optional<const HipTensor*> w, std::optional<const HipTensor*> b,
                           std::int64_t axis, double eps, bool rms) {
    OpDesc op{rms ? OpKind::kAffineRmsNorm : OpKind::kAffineLayerNorm};
    op.axis = axis;
    op.epsilon = eps;
    std::vector<Tensor> in{x.tensor};
    if (w && *w) {
      op.has_weight = true;
      in.push_back((*w)->tensor);
    }
    if (b && *b) {
      op.has_bias = true;
      in.push_back((*b)->tensor);
    }
    return run(op, std::move(in));
  });
  m.def("exp", [](const HipTensor& x) { return unary(OpKind::kExp, x); });
  m.def("gelu", [](const HipTensor& x) { return unary(OpKind::kGelu, x); });
  m.def("silu", [](const HipTensor& x) { return unary(OpKind::kSilu, x); });
  for (const auto& [name, kind] : std::vector<std::pair<const char*, OpKind>>{
           {"add", OpKind::kAdd}, {"subtract", OpKind::kSubtract}, {"multiply", OpKind::kMultiply},
           {"divide", OpKind::kDivide}}) {
    const OpKind k = kind;
    m.def(name, [k](const HipTensor& a, const HipTensor& b) { return run(OpDesc{k}, {a.tensor, b.tensor}); });
  }

  m.def("log", [](const HipTensor& x) { return unary(OpKind::kLog, x); });
  m.def("sqrt", [](const HipTensor& x) { return unary(OpKind::kSqrt, x); });
  m.def("abs", [](const HipTensor& x) { return unary(OpKind::kAbs, x); });
  m.def("_clip", [](const HipTensor& x, const HipTensor& lo, const HipTensor& hi) {
    return run(OpDesc{OpKind::kClip}, {x.tensor, lo.tensor, hi.tensor});
  });
  m.def("_topk", [](const HipTensor& x, std::int64_t k, std::int64_t axis, bool largest, bool sorted) {
    OpDesc op{OpKind::kTopK};
    op.k = k;
    op.axis = axis;
    op.largest = largest;
    op.sorted = sorted;
    return run2(op, {x.tensor});
  });
  m.def("embedding", [](const HipTensor& ids, const HipTensor& w) {
    return run(OpDesc{OpKind::kEmbedding}, {ids.tensor, w.tensor});
  });
  m.def("_attention", [](const HipTensor& q, const HipTensor& k, const HipTensor& v,
                         std::optional<const HipTensor*> mask, bool causal, std::optional<double> scale) {
    OpDesc op{OpKind::kAttention};
    op.causal = causal;
    op.attention_scale = scale;
    std::vector<Tensor> in{q.tensor, k.tensor, v.tensor};
    if (mask && *mask) in.push_back((*mask)->tensor);
    return run(op, std::move(in));
  }, py::arg("q"), py::arg("k"), py::arg("v"), py::arg("mask") = py::none(), py::arg("causal") = false,
     py::arg("scale") = py::none());
  m.def("_attention_softmax", [](const HipTensor& scores, std::optional<const HipTensor*> mask,
                                 std::vector<std::int64_t> shape, bool causal, std::optional<double> scale) {
    OpDesc op{OpKind::kAttentionSoftmax};
    op.attention_shape = to_shape(shape);
    op.causal = causal;
    op.attention_scale = scale;
    std::vector<Tensor> in{scores.tensor};
    if (mask && *mask) in.push_back((*mask)->tensor);
    return run(op, std::move(in));
  }, py::arg("scores"), py::arg("mask"), py::arg("shape"), py::arg("causal") = false, py::arg("scale") = py::none());

  // Scalar arithmetic, casts and layout (the reference's _core names).
  m.def("negative", [](const HipTensor& x) { return unary(OpKind::kNegate, x); });
  for (const auto& [name, kind] : std::vector<std::pair<const char*, OpKind>>{
           {"add_scalar", OpKind::kAddScalar}, {"subtract_scalar", OpKind::kSubtractScalar},
           {"multiply_scalar", OpKind::kMultiplyScalar}, {"divide_scalar", OpKind::kDivideScalar}}) {
    const OpKind k = kind;
    m.def(name, [k](const HipTensor& x, double value, bool scalar_left) {
      OpDesc op{k};
      op.scalar_value = value;
      op.scalar_left = scalar_left;
      return run(op, {x.tensor});
    }, py::arg("x"), py::arg("value"), py::arg("scalar_left") = false);
  }
  m.def("astype", [](const HipTensor& x, const std::string& dtype) {
    OpDesc op{OpKind::kCast};
    op.target_dtype = parse_dtype(dtype);
    return run(op, {x.tensor});
  });
  m.def("transpose", [](const HipTensor& x, std::vector<std::int64_t> axes) {
    OpDesc op{OpKind::kTranspose};
    op.axes = to_shape(axes);
    return run(op, {x.tensor});
  });
  m.def("_slice", [](const HipTensor& x, std::vector<std::int64_t> starts, std::vector<std::int64_t> steps,
                     std::vector<std::int64_t> lengths) {
    OpDesc op{OpKind::kSlice};
    op.slice_starts = to_shape(starts);
    op.slice_steps = to_shape(steps);
    op.slice_shape = to_shape(lengths);
    return run(op, {x.tensor});
  });
  m.def("_concat", [](const HipTensor& first, const std::vector<const HipTensor*>& rest, std::int64_t axis) {
    OpDesc op{OpKind::kConcat};
    op.axis = axis;
    std::vector<Tensor> in{first.tensor};
    for (const HipTensor* t : rest) in.push_back(t->tensor);
    return run(op, std::move(in));
  });
  for (const auto& [name, kind] : std::vector<std::pair<const char*, OpKind>>{
           {"equal", OpKind::kEqual}, {"not_equal", OpKind::kNotEqual}, {"less", OpKind::kLess},
           {"less_equal", OpKind::kLessEqual}, {"greater", OpKind::kGreater},
           {"greater_equal", OpKind::kGreaterEqual}, {"logical_and", OpKind::kLogicalAnd},
           {"logical_or", OpKind::kLogicalOr}, {"logical_xor", OpKind::kLogicalXor}}) {
    const OpKind k = kind;
    m.def(name, [k](const HipTensor& a, const HipTensor& b) { return run(OpDesc{k}, {a.tensor, b.tensor}); });
  }
  m.def("logical_not", [](const HipTensor& x) { return unary(OpKind::kLogicalNot, x); });
  m.def("where", [](const HipTensor& c, const HipTensor& a, const HipTensor& b) {
    return run(OpDesc{OpKind::kWhere}, {c.tensor, a.tensor, b.tensor});
  });
  m.def("_any_axes", [](const HipTensor& x, std::vector<std::int64_t> axes) { return axes_op(OpKind::kAny, x, axes); });
  m.def("_all_axes", [](const HipTensor& x, std::vector<std::int64_t> axes) { return axes_op(OpKind::kAll, x, axes); });
  m.def("masked_select", [](const HipTensor& x, const HipTensor& mask) {
    return run(OpDesc{OpKind::kMaskedSelect}, {x.tensor, mask.tensor});
  });

  // Runtime profiling sessions (the reference's _profile_begin/_profile_end).
  m.def("_profile_begin", [](std::int64_t max_events, bool device_timing) {
    if (max_events < 1 || max_events > 100000) throw py::value_error("max_events must be an integer in [1, 100000]");
    try {
      return begin_profile(static_cast<std::size_t>(max_events), device_timing);
    } catch (const std::invalid_argument& error) {
      throw py::value_error(error.what());
    }
  });
  m.def("_profile_end", [](std::uint64_t token) {
    const ProfileResult r = end_profile(token);
    auto op_name = [](const std::optional<OpKind>& op) -> py::object {
      return op ? py::object(py::str(profile_operation_name(*op))) : py::object(py::none());
    };
    py::list events;
    for (const ProfileEvent& e : r.events) {
      py::dict d;
      d["id"] = e.id;
      d["parent_id"] = e.parent_id;
      d["start_ns"] = e.start_ns;
      d["duration_ns"] = e.duration_ns;
      d["self_ns"] = e.self_ns;
      d["category"] = profile_category_name(e.category);
      d["name"] = e.name;
      d["backend"] = e.backend;
      d["bytes"] = e.bytes ? py::object(py::int_(*e.bytes)) : py::object(py::none());
      d["operation"] = op_name(e.operation);
      events.append(d);
    }
    py::list device_events;
    for (const auto& e : r.device_events) {
      py::dict d;
      d["id"] = e.id;
      d["host_event_id"] = e.host_event_id;
      d["name"] = e.name;
      d["backend"] = e.backend;
      d["operation"] = op_name(e.operation);
      d["elapsed_ms"] = e.elapsed_ms ? py::object(py::float_(*e.elapsed_ms)) : py::object(py::none());
      d["error"] = e.error ? py::object(py::str(e.error)) : py::object(py::none());
      device_events.append(d);
    }
    py::dict out;
    out["elapsed_ns"] = r.elapsed_ns;
    out["dropped_events"] = r.dropped_events;
    out["events"] = events;
    out["device_timing"] = r.device_timing;
    out["dropped_device_events"] = r.dropped_device_events;
    out["device_events"] = device_events;
    return out;
  });

  py::class_<PoolHandle>(m, "MemoryPool")
      .def(py::init<std::size_t, std::size_t>(), py::arg("max_cached_bytes"), py::arg("max_cached_blocks") = 64)
      .def("enter", [](PoolHandle& p) { p.check(tcx_hip_pool_enter(p.pool)); })
      .def("exit", [](PoolHandle& p) { p.check(tcx_hip_pool_exit(p.pool)); })
      .def("trim", [](PoolHandle& p) { p.check(tcx_hip_pool_trim(p.pool)); })
      .def("stats", [](PoolHandle& p) {
        tcx_hip_pool_stats_t s{};
        p.check(tcx_hip_pool_stats(p.pool, &s));
        py::dict d;
        d["max_cached_bytes"] = s.max_cached_bytes;
        d["max_cached_blocks"] = s.max_cached_blocks;
        d["cached_bytes"] = s.cached_bytes;
        d["cached_blocks"] = s.cached_blocks;
        d["in_use_bytes"] = s.in_use_bytes;
        d["peak_in_use_bytes"] = s.peak_in_use_bytes;
        d["peak_cached_bytes"] = s.peak_cached_bytes;
        d["hits"] = s.hits;
        d["misses"] = s.misses;
        d["allocation_calls"] = s.allocation_calls;
        d["free_calls"] = s.free_calls;
        d["allocation_failures"] = s.allocation_failures;
        d["oom_retries"] = s.oom_retries;
        d["uncached_returns"] = s.uncached_returns;
        d["readiness_failures"] = s.readiness_failures;
        d["free_failures"] = s.free_failures;
        d["failed_free_bytes"] = s.failed_free_bytes;
        d["active"] = s.active != 0;
        return d;
      });
}
