// Shapes and the shape plans the hip backend needs. Names and plan fields
// follow the reference's core/shape.h:8-70 (numel, contiguous_strides,
// BroadcastPlan, MatmulPlan, ReductionPlan, TransposePlan, ConcatPlan) so
// plans mean the same thing on both sides of the backend boundary.
#pragma once

#include <cstdint>
#include <vector>

namespace tensorcx {

using Dim = std::int64_t;
using Shape = std::vector<Dim>;

// Element count; throws std::invalid_argument on a negative extent or overflow.
std::int64_t numel(const Shape& shape);
Shape contiguous_strides(const Shape& shape);

struct BroadcastPlan {
  Shape output_shape;
  Shape lhs_strides;
  Shape rhs_strides;
};
// Right-aligned NumPy broadcasting; broadcast and padded axes get stride 0.
BroadcastPlan make_broadcast_plan(const Shape& lhs, const Shape& rhs);

struct MatmulPlan {
  Shape output_shape;
  Shape batch_shape;
  Shape lhs_batch_strides;
  Shape rhs_batch_strides;
  Dim m, k, n;
};
// NumPy matmul: rank-1 operands are promoted and their axes dropped again,
// leading batch axes broadcast.
MatmulPlan make_matmul_plan(const Shape& lhs, const Shape& rhs);
Dim matmul_batch_offset(Dim batch, const Shape& shape, const Shape& strides);

struct ReductionPlan {
  Shape output_shape;
  // Extent/stride pairs: kept axes first, then reduced axes, each in axis order.
  Shape index_metadata;
  Dim reduction_size{1};
};
ReductionPlan make_reduction_plan(const Shape& input, const Shape& axes);

// A strided view of a contiguous input: output element i reads
// offset + sum over axes of index * input_strides.
struct TransposePlan {
  Shape output_shape;
  Shape input_strides;
  Dim offset{0};
};
// A full permutation of the axes (negative axes allowed, no repeats).
TransposePlan make_transpose_plan(const Shape& input, const Shape& axes);
// Per-axis start / step / length, every visited index in bounds.
TransposePlan make_slice_plan(const Shape& input, const Shape& starts, const Shape& steps, const Shape& lengths);

struct ConcatPlan {
  Shape output_shape;
  std::size_t axis;
  Dim inner;  // contiguous stride of the concatenation axis in the output
};
ConcatPlan make_concat_plan(const std::vector<Shape>& inputs, Dim axis);

}  // namespace tensorcx
