// DLPack exchange for hip tensors (device kDLROCM, id 0) and host arrays
// (kDLCPU): the hip counterpart of the reference's bindings/dlpack.cpp, with
// the same contract (docs/DLPACK.md: contiguous float32 / int32 / bool,
// legacy and 1.0 versioned capsules, copy=None/False shares, copy=True makes
// an independent same-device copy, read-only input needs copy=True, the
// producer's deleter runs exactly once, BufferError for unsupported input).
//
// Import borrows the memory: the capsule's managed tensor becomes the owner
// of a HipBuffer (or the base of a NumPy view for host memory) and is
// released when the last tensor sharing it goes away. Export hands out the
// tensor's own storage, which from then on bypasses pool caches, because the
// consumer may still use it on streams this library cannot see.

#include <Python.h>
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>

#include <cstdint>
#include <limits>
#include <memory>
#include <optional>
#include <string>
#include <utility>
#include <vector>

#include "dlpack_abi.h"
#include "hip_binding.h"
#include "tensorcx/backends/hip/hip_backend.h"

namespace py = pybind11;
using namespace tensorcx;

namespace tcx_bind {
namespace {

constexpr const char* kLegacyName = "dltensor";
constexpr const char* kVersionedName = "dltensor_versioned";

[[noreturn]] void buffer_error(const std::string& message) {
  PyErr_SetString(PyExc_BufferError, message.c_str());
  throw py::error_already_set();
}

dl::DataType dl_type(DType dtype) {
  if (dtype == DType::kFloat32) return {dl::kFloat, 32, 1};
  if (dtype == DType::kInt32) return {dl::kInt, 32, 1};
  return {dl::kBool, 8, 1};
}

// ------------------------------------------------------------------ export
// Everything a capsule of ours owns: both managed-tensor records (one is
// used), the shape/stride arrays they point into, and the storage owner.
struct Export {
  dl::ManagedTensor legacy{};
  dl::ManagedTensorVersioned versioned{};
  std::vector<std::int64_t> shape, strides;
  Tensor device_owner;             // hip storage
  PyObject* host_owner = nullptr;  // strong reference to a host array

  Export() = default;
  Export(const Export&) = delete;
  Export& operator=(const Export&) = delete;
  ~Export() {
    // Consumers may call the deleter from threads without the GIL.
    if (host_owner != nullptr && Py_IsInitialized()) {
      const PyGILState_STATE gil = PyGILState_Ensure();
      Py_DECREF(host_owner);
      PyGILState_Release(gil);
    }
  }
};

void delete_legacy(dl::ManagedTensor* self) { delete static_cast<Export*>(self->manager_ctx); }
void delete_versioned(dl::ManagedTensorVersioned* self) { delete static_cast<Export*>(self->manager_ctx); }

// A capsule dropped before anyone consumed it still owns its tensor; a
// consumed one was renamed and belongs to its consumer.
void drop_capsule(PyObject* capsule) {
  if (PyCapsule_IsValid(capsule, kVersionedName)) {
    auto* t = static_cast<dl::ManagedTensorVersioned*>(PyCapsule_GetPointer(capsule, kVersionedName));
    if (t->deleter) t->deleter(t);
  } else if (PyCapsule_IsValid(capsule, kLegacyName)) {
    auto* t = static_cast<dl::ManagedTensor*>(PyCapsule_GetPointer(capsule, kLegacyName));
    if (t->deleter) t->deleter(t);
  }
}

py::object make_capsule(std::unique_ptr<Export> state, void* data, std::int64_t count, dl::Device device,
                        DType dtype, bool versioned, bool copied) {
  if (state->shape.size() > static_cast<std::size_t>(std::numeric_limits<std::int32_t>::max()))
    buffer_error("DLPack rank is too large");
  const dl::Tensor description{count ? data : nullptr, device, static_cast<std::int32_t>(state->shape.size()),
                               dl_type(dtype), state->shape.data(), state->strides.data(), 0};
  void* payload;
  const char* name;
  if (versioned) {
    state->versioned.version = {1, 0};
    state->versioned.manager_ctx = state.get();
    state->versioned.deleter = delete_versioned;
    state->versioned.flags = copied ? dl::kFlagIsCopied : 0;
    state->versioned.dl_tensor = description;
    payload = &state->versioned;
    name = kVersionedName;
  } else {
    state->legacy.manager_ctx = state.get();
    state->legacy.deleter = delete_legacy;
    state->legacy.dl_tensor = description;
    payload = &state->legacy;
    name = kLegacyName;
  }
  PyObject* capsule = PyCapsule_New(payload, name, drop_capsule);
  if (capsule == nullptr) throw py::error_already_set();
  state.release();  // the capsule (or its consumer) now owns it
  return py::reinterpret_steal<py::object>(capsule);
}

py::object export_hip(const HipTensor& input, bool versioned, bool copy) {
  Tensor tensor = input.tensor;
  if (copy) {
    std::optional<Expected<Tensor>> cloned;
    {
      py::gil_scoped_release release;
      cloned.emplace(hip::clone(tensor));
    }
    if (!*cloned) buffer_error(cloned->status().message());
    tensor = cloned->move_value();
  }
  auto data = hip::export_storage(tensor);
  if (!data) buffer_error(data.status().message());
  auto state = std::make_unique<Export>();
  state->shape.assign(tensor.shape.begin(), tensor.shape.end());
  state->strides.assign(tensor.strides.begin(), tensor.strides.end());
  const std::int64_t count = numel(tensor.shape);
  const DType dtype = tensor.dtype;
  state->device_owner = std::move(tensor);
  return make_capsule(std::move(state), data.value(), count, dl::Device{dl::kROCM, 0}, dtype, versioned, copy);
}

DType host_dtype(const py::array& array) {
  if (py::isinstance<py::array_t<float>>(array)) return DType::kFloat32;
  if (py::isinstance<py::array_t<std::int32_t>>(array)) return DType::kInt32;
  if (py::isinstance<py::array_t<bool>>(array)) return DType::kBool;
  buffer_error("DLPack requires float32, int32 or bool");
}

py::object export_host(py::array array, bool versioned, bool copy) {
  const DType dtype = host_dtype(array);
  if (!(array.flags() & py::array::c_style)) buffer_error("DLPack requires C-contiguous input");
  if (copy) array = py::module_::import("numpy").attr("array")(array, py::arg("copy") = true);
  auto state = std::make_unique<Export>();
  std::int64_t count = 1;
  for (py::ssize_t a = 0; a < array.ndim(); ++a) {
    state->shape.push_back(array.shape(a));
    state->strides.push_back(array.strides(a) / array.itemsize());
    count *= array.shape(a);
  }
  void* data = const_cast<void*>(array.data());
  state->host_owner = array.release().ptr();  // the reference taken over by Export
  return make_capsule(std::move(state), data, count, dl::Device{dl::kCPU, 0}, dtype, versioned, copy);
}

// ------------------------------------------------------------------ import
struct Consumed {
  dl::Tensor description;
  std::uint64_t flags;
  std::shared_ptr<void> owner;  // runs the producer's deleter once, when dropped
};

// Takes ownership of an unconsumed capsule (renaming it, so it cannot be
// consumed twice) before any check, so a rejected descriptor is still
// released exactly once.
Consumed consume(py::handle capsule) {
  PyObject* object = capsule.ptr();
  if (PyCapsule_IsValid(object, kVersionedName)) {
    auto* t = static_cast<dl::ManagedTensorVersioned*>(PyCapsule_GetPointer(object, kVersionedName));
    if (PyCapsule_SetName(object, "used_dltensor_versioned") != 0) throw py::error_already_set();
    std::shared_ptr<void> owner(t, [](void* p) {
      auto* managed = static_cast<dl::ManagedTensorVersioned*>(p);
      if (managed->deleter) managed->deleter(managed);
    });
    if (t->version.major != 1) buffer_error("unsupported DLPack major version");
    if (t->flags & ~(dl::kFlagReadOnly | dl::kFlagIsCopied)) buffer_error("unsupported DLPack flags");
    return {t->dl_tensor, t->flags, std::move(owner)};
  }
  if (PyCapsule_IsValid(object, kLegacyName)) {
    auto* t = static_cast<dl::ManagedTensor*>(PyCapsule_GetPointer(object, kLegacyName));
    if (PyCapsule_SetName(object, "used_dltensor") != 0) throw py::error_already_set();
    std::shared_ptr<void> owner(t, [](void* p) {
      auto* managed = static_cast<dl::ManagedTensor*>(p);
      if (managed->deleter) managed->deleter(managed);
    });
    return {t->dl_tensor, 0, std::move(owner)};
  }
  buffer_error("expected an unconsumed DLPack capsule");
}

py::dtype numpy_dtype(DType dtype) {
  if (dtype == DType::kFloat32) return py::dtype::of<float>();
  if (dtype == DType::kInt32) return py::dtype::of<std::int32_t>();
  return py::dtype::of<bool>();
}

py::object import_capsule(py::handle capsule, bool copy, bool forbid_copy, int expected_type, int expected_id) {
  Consumed consumed = consume(capsule);
  const dl::Tensor& t = consumed.description;
  if (forbid_copy && (consumed.flags & dl::kFlagIsCopied)) buffer_error("producer copied despite copy=False");
  if (!copy && (consumed.flags & dl::kFlagReadOnly)) buffer_error("read-only DLPack input requires copy=True");
  if (expected_type >= 0 && (t.device.device_type != expected_type || t.device.device_id != expected_id))
    buffer_error("DLPack capsule device differs from producer device");
  const bool host = t.device.device_type == dl::kCPU;
  if ((!host && t.device.device_type != dl::kROCM) || t.device.device_id != 0)
    buffer_error("DLPack supports CPU and ROCm device 0 only");
  if (t.dtype.lanes != 1) buffer_error("DLPack vector lanes are unsupported");
  DType dtype;
  if (t.dtype.code == dl::kFloat && t.dtype.bits == 32) dtype = DType::kFloat32;
  else if (t.dtype.code == dl::kInt && t.dtype.bits == 32) dtype = DType::kInt32;
  else if (t.dtype.code == dl::kBool && t.dtype.bits == 8) dtype = DType::kBool;
  else buffer_error("DLPack requires float32, int32 or bool");
  if (t.ndim < 0 || (t.ndim > 0 && t.shape == nullptr)) buffer_error("invalid DLPack shape");
  Shape shape(t.shape, t.shape + t.ndim);
  std::uint64_t count = 1;
  for (const Dim d : shape) {
    if (d < 0) buffer_error("invalid DLPack shape");
    if (d != 0 && count > std::numeric_limits<std::uint64_t>::max() / static_cast<std::uint64_t>(d))
      buffer_error("DLPack element count overflow");
    count *= static_cast<std::uint64_t>(d);
  }
  const Shape canonical = contiguous_strides(shape);
  // Strides of size-1 axes (or of any axis of an empty tensor) never change
  // which elements are reachable.
  if (count != 0 && t.strides != nullptr) {
    for (std::int32_t a = 0; a < t.ndim; ++a)
      if (shape[a] > 1 && t.strides[a] != canonical[a]) buffer_error("DLPack requires C-contiguous input");
  }
  const std::size_t element = dtype_size(dtype);
  if (count > std::numeric_limits<std::size_t>::max() / element) buffer_error("DLPack byte size overflow");
  const std::size_t bytes = static_cast<std::size_t>(count) * element;
  auto address = reinterpret_cast<std::uintptr_t>(t.data);
  if (t.byte_offset > std::numeric_limits<std::uintptr_t>::max() - address)
    buffer_error("DLPack pointer offset overflow");
  address += t.byte_offset;
  if (bytes != 0 && (t.data == nullptr || address % element != 0 ||
                     bytes > std::numeric_limits<std::uintptr_t>::max() - address))
    buffer_error("DLPack requires an aligned, non-null data range");
  void* data = bytes ? reinterpret_cast<void*>(address) : nullptr;

  if (host) {
    // A NumPy view whose base keeps the producer's tensor alive. Empty views
    // get a placeholder address (never read) so that they keep it alive too.
    static std::int64_t placeholder = 0;
    auto* keep = new std::shared_ptr<void>(std::move(consumed.owner));
    py::capsule base(keep, [](void* p) { delete static_cast<std::shared_ptr<void>*>(p); });
    std::vector<py::ssize_t> dims(shape.begin(), shape.end()), steps;
    for (const Dim s : canonical) steps.push_back(static_cast<py::ssize_t>(s * static_cast<Dim>(element)));
    py::array view(numpy_dtype(dtype), dims, steps, data ? data : &placeholder, base);
    if (copy) return view.attr("copy")();
    return std::move(view);
  }

  // Device memory: the pointer check and the wait for producer work run
  // without the GIL; a failed borrow releases the owner after the GIL is back.
  std::shared_ptr<void> keep = consumed.owner;
  std::optional<Expected<Tensor>> borrowed;
  {
    py::gil_scoped_release release;
    borrowed.emplace(hip::borrow(data, dtype, std::move(shape), std::move(consumed.owner)));
  }
  if (!*borrowed) {
    keep.reset();
    buffer_error(borrowed->status().message());
  }
  keep.reset();
  Tensor tensor = borrowed->move_value();
  if (copy) {
    std::optional<Expected<Tensor>> cloned;
    {
      py::gil_scoped_release release;
      cloned.emplace(hip::clone(tensor));
    }
    if (!*cloned) buffer_error(cloned->status().message());
    tensor = cloned->move_value();
  }
  return py::cast(HipTensor{std::move(tensor)});
}

}  // namespace

void bind_dlpack(py::module_& module) {
  module.def("_to_dlpack", &export_hip, py::arg("input"), py::arg("versioned"), py::arg("copy"));
  module.def("_to_dlpack_host", &export_host, py::arg("input"), py::arg("versioned"), py::arg("copy"));
  module.def("_from_dlpack", &import_capsule, py::arg("capsule"), py::arg("copy"), py::arg("forbid_copy"),
             py::arg("expected_type"), py::arg("expected_id"));
}

}  // namespace tcx_bind
