// Element types; enumerator order matches the reference (core/dtype.h:8-12).
#pragma once

#include <cstddef>
#include <string_view>

namespace tensorcx {

enum class DType {
  kFloat32,
  kInt32,
  kBool,
};

std::string_view dtype_name(DType dtype);
std::size_t dtype_size(DType dtype);
// True for finite, integral values in [INT32_MIN, INT32_MAX].
bool is_int32_representable(double value);

}  // namespace tensorcx
