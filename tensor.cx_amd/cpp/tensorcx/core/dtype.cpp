#include "tensorcx/core/dtype.h"

#include <cmath>
#include <stdexcept>

namespace tensorcx {

std::string_view dtype_name(DType dtype) {
  switch (dtype) {
    case DType::kFloat32: return "float32";
    case DType::kInt32: return "int32";
    case DType::kBool: return "bool";
  }
  throw std::invalid_argument("unknown dtype");
}

std::size_t dtype_size(DType dtype) {
  switch (dtype) {
    case DType::kFloat32:
    case DType::kInt32: return 4;
    case DType::kBool: return 1;
  }
  throw std::invalid_argument("unknown dtype");
}

bool is_int32_representable(double value) {
  return std::isfinite(value) && std::trunc(value) == value && value >= -2147483648.0 &&
         value <= 2147483647.0;
}

}  // namespace tensorcx
