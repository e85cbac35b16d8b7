// Operation descriptors. The OpKind enumerator order and the OpDesc fields
// match the reference's core/operation.h:12-93 exactly, because both are part
// of the backend execution ABI that the hip backend plugs into.
#pragma once

#include <cstddef>
#include <cstdint>
#include <optional>

#include "tensorcx/core/dtype.h"
#include "tensorcx/core/shape.h"

namespace tensorcx {

enum class OpKind {
  kFill,
  kAdd,
  kMultiply,
  kMatmul,
  kSum,
  kMax,
  kMean,
  kExp,
  kGelu,
  kSilu,
  kSoftmax,
  kRmsNorm,
  kLayerNorm,
  kSubtract,
  kDivide,
  kNegate,
  kAddScalar,
  kSubtractScalar,
  kMultiplyScalar,
  kDivideScalar,
  kCast,
  kTranspose,
  kSlice,
  kConcat,
  kEqual,
  kNotEqual,
  kLess,
  kLessEqual,
  kGreater,
  kGreaterEqual,
  kLogicalAnd,
  kLogicalOr,
  kLogicalXor,
  kLogicalNot,
  kWhere,
  kAny,
  kAll,
  kMaskedSelect,
  kLog, kSqrt, kAbs, kMin, kArgmax, kClip, kTopK,
  kLinear, kAffineRmsNorm, kAffineLayerNorm, kEmbedding, kAttention, kAttentionSoftmax,
};

enum class MatmulPreference {
  kAuto,
  kCustom,
  kOptimized,
};

// An op kind plus the attributes the primitives read: axis and epsilon for
// axis-wise ops, scalar_value for fill and scalar arithmetic, reduction_axes
// for multi-axis reductions, has_weight/has_bias for affine normalisation.
struct OpDesc {
  OpKind kind{OpKind::kFill};
  std::int64_t axis{0};
  double epsilon{1.0e-5};
  double scalar_value{0.0};
  MatmulPreference matmul_preference{MatmulPreference::kAuto};
  bool scalar_left{false};
  DType target_dtype{DType::kFloat32};
  Shape axes{};
  std::optional<Shape> reduction_axes{};
  Shape slice_starts{};
  Shape slice_steps{};
  Shape slice_shape{};
  Dim k{0};
  bool largest{true};
  bool sorted{true};
  bool has_weight{false}, has_bias{false}, causal{false};
  std::optional<double> attention_scale{};
  Shape attention_shape{};
};

struct PrimitiveOpSchema {
  std::size_t input_count{0};
  std::size_t output_count{0};
  bool variadic_inputs{false};  // input_count is then a minimum
};

std::optional<PrimitiveOpSchema> primitive_op_schema(OpKind kind);

}  // namespace tensorcx
