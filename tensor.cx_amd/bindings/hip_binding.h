// Pieces shared by the translation units of the _core module.
#pragma once

#include <pybind11/pybind11.h>

#include "tensorcx/core/status.h"
#include "tensorcx/core/tensor.h"

namespace tcx_bind {

// The Python-visible hip tensor: one core Tensor on {"hip", 0}.
struct HipTensor {
  tensorcx::Tensor tensor;
};

// kInvalidArgument -> ValueError, anything else -> RuntimeError
// (reference bindings/python_module.cpp:402-414).
[[noreturn]] inline void throw_status(const tensorcx::Status& status) {
  if (status.code() == tensorcx::StatusCode::kInvalidArgument) throw pybind11::value_error(status.message());
  throw std::runtime_error(status.message());
}

// Registers _to_dlpack / _from_dlpack (hip_dlpack.cpp).
void bind_dlpack(pybind11::module_& module);

}  // namespace tcx_bind
