// Shape and dtype plans of the predicate family (comparisons, logical ops,
// where, any / all, masked_select), with the names and fields of the
// reference's core/predicate.h so backends validate requests identically.
#pragma once

#include <span>
#include <vector>

#include "tensorcx/core/operation.h"
#include "tensorcx/core/tensor.h"

namespace tensorcx {

bool is_comparison(OpKind kind);
bool is_logical(OpKind kind);
bool is_predicate_elementwise(OpKind kind);

struct PredicatePlan {
  Shape output_shape;
  std::vector<Shape> input_strides;  // broadcast strides, one per input
  DType output_dtype;
};
PredicatePlan make_predicate_plan(const OpDesc& op, std::span<const Tensor> inputs);
ReductionPlan make_boolean_reduction_plan(const OpDesc& op, const Shape& input);

struct MaskedSelectPlan {
  Shape tail_shape;  // input axes after the mask's
  Dim block_size;    // elements per selected entry (0 when nothing is addressed)
};
MaskedSelectPlan make_masked_select_plan(const Tensor& input, const Tensor& mask);
Dim broadcast_offset(Dim flat, const Shape& shape, const Shape& strides);

}  // namespace tensorcx
